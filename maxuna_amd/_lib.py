"""ctypes binding of libmaxuna_moe.so (the C ABI declared in include/maxuna_moe.h).

The library is loaded from maxuna_amd/lib/ only.  There is no fallback: if the
library is missing every op raises, so a GPU run can never silently take a
non-native path.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmaxuna_moe.so"

# status codes (maxuna_moe.h)
MX_OK = 0
STATUS_NAMES = {
    1: "MX_ERR_NULL", 2: "MX_ERR_SHAPE", 3: "MX_ERR_DTYPE", 4: "MX_ERR_BLOCK", 5: "MX_ERR_XPR",
    6: "MX_ERR_SCRATCH", 7: "MX_ERR_OVERFLOW", 8: "MX_ERR_TOPK", 9: "MX_ERR_ALIGN", 10: "MX_ERR_HIP",
    11: "MX_ERR_IO", 12: "MX_ERR_FORMAT", 13: "MX_ERR_NOT_FOUND",
}


class MaxunaError(RuntimeError):
    """A validation or runtime error reported by the native library."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


class ExpertStackC(C.Structure):
    _fields_ = [
        ("data", C.c_void_p),
        ("base_off", C.c_uint64),
        ("dtype", C.c_int32),
        ("reserved", C.c_int32),
        ("n_expert", C.c_int64),
        ("n_out", C.c_int64),
        ("k", C.c_int64),
    ]


class Map0C(C.Structure):
    _fields_ = [
        ("buffer", C.c_void_p),
        ("bytes", C.c_size_t),
        ("n_expert", C.c_int64),
        ("t", C.c_int64),
        ("top_k", C.c_int64),
    ]


class MoeLayerC(C.Structure):
    _fields_ = [
        ("router", C.c_void_p),
        ("exp_probs_b", C.c_void_p),
        ("gate", ExpertStackC),
        ("up", ExpertStackC),
        ("down", ExpertStackC),
        ("shared_gate", ExpertStackC),
        ("shared_up", ExpertStackC),
        ("shared_down", ExpertStackC),
        ("hidden", C.c_int64),
        ("expert_ff", C.c_int64),
        ("top_k", C.c_int64),
        ("weights_scale", C.c_double),
        ("weights_norm", C.c_int32),
        ("mm_min_seq", C.c_int32),
        ("rms_alpha", C.c_void_p),
        ("rms_eps", C.c_float),
        ("reserved", C.c_int32),
    ]


class GgufTensorC(C.Structure):
    _fields_ = [
        ("name", C.c_char_p),
        ("ggml_type", C.c_int32),
        ("n_dims", C.c_int32),
        ("ne", C.c_int64 * 4),
        ("offset", C.c_uint64),
        ("nbytes", C.c_uint64),
    ]


P, I32, I64, U32, U64, F32, F64, SZ = (C.c_void_p, C.c_int32, C.c_int64, C.c_uint32, C.c_uint64,
                                       C.c_float, C.c_double, C.c_size_t)
SIGNATURES = {
    "mx_last_error": (C.c_char_p, []),
    "mx_version": (C.c_char_p, []),
    "mx_block_size": (I32, [I32]),
    "mx_type_size": (I32, [I32]),
    "mx_dequantize": (I32, [I32, P, I64, P, P]),
    "mx_mul_mv_id": (I32, [C.POINTER(ExpertStackC), P, I64, I64, I64, P, I64, I64, P, P]),
    "mx_mul_mv": (I32, [P, I32, I64, I64, P, I64, P, P]),
    "mx_map0_scratch_bytes": (SZ, [I64, I64, I64]),
    "mx_prepare_map0": (I32, [I64, P, I64, I64, P, SZ, P]),
    "mx_mul_mm_id_shared": (I32, [C.POINTER(ExpertStackC), P, I64, I64, I64, P, I64, I64,
                                  C.POINTER(Map0C), P, P]),
    "mx_mul_mm_id_workspace_bytes": (SZ, [I64, I64, I64, I64, I64]),
    "mx_mul_mm_id": (I32, [C.POINTER(ExpertStackC), P, I64, I64, I64, P, I64, I64, P, SZ, P, P]),
    "mx_check_ids": (I32, [P, I64, I64, I64, P, P]),
    "mx_silu_mul": (I32, [P, P, I64, P, P]),
    "mx_combine": (I32, [P, P, P, I64, I64, I64, P, P]),
    "mx_rms_norm": (I32, [P, P, I64, I64, F32, P, P]),
    "mx_route_logits": (I32, [P, P, I64, I64, I64, P, P]),
    "mx_route_from_logits": (I32, [P, P, I64, I64, I64, F64, I32, P, P, P]),
    "mx_moe_workspace_bytes": (SZ, [C.POINTER(MoeLayerC), I64]),
    "mx_moe_forward": (I32, [C.POINTER(MoeLayerC), P, I64, P, P, P, P, P, SZ, P]),
    "mx_moe_forward_noalloc": (I32, [C.POINTER(MoeLayerC), P, I64, P, P, P, P, P]),
    "mx_moe_forward_noalloc_max_bytes": (SZ, []),
    "mx_tensor_key": (U64, [U64, U32, U32]),
    "mx_gguf_open": (I32, [C.c_char_p, C.POINTER(P)]),
    "mx_gguf_close": (None, [P]),
    "mx_gguf_version": (U32, [P]),
    "mx_gguf_alignment": (U64, [P]),
    "mx_gguf_data_offset": (U64, [P]),
    "mx_gguf_tensor_count": (I64, [P]),
    "mx_gguf_tensor_at": (I32, [P, I64, C.POINTER(GgufTensorC)]),
    "mx_gguf_find_tensor": (I32, [P, C.c_char_p, C.POINTER(GgufTensorC)]),
    "mx_gguf_kv_type": (I32, [P, C.c_char_p]),
    "mx_gguf_get_int": (I32, [P, C.c_char_p, C.POINTER(I64)]),
    "mx_gguf_get_float": (I32, [P, C.c_char_p, C.POINTER(F64)]),
    "mx_gguf_get_string": (I32, [P, C.c_char_p, C.POINTER(C.c_char_p)]),
    "mx_gguf_get_array": (I32, [P, C.c_char_p, C.POINTER(I32), C.POINTER(U64)]),
    "mx_gguf_read_host": (I32, [P, C.POINTER(GgufTensorC), P, U64]),
    "mx_gguf_read": (I32, [P, C.POINTER(GgufTensorC), P, U64, P]),
    "mx_synth_blocks": (I32, [I32, U64, P, I64, P]),
}

# bench-only instrumentation (maxuna_amd/csrc/mx_instrument.h): exported by the
# library, not part of the boundary header
INSTRUMENT_SIGNATURES = {
    "mx_moe_forward_profiled": (I32, [C.POINTER(MoeLayerC), P, I64, P, P, P, P, P, SZ, P, P, I32, P]),
    "mx_moe_forward_repeat": (I32, [C.POINTER(MoeLayerC), P, I64, P, P, P, P, P, SZ, P, I32, I32]),
    "mx_probe_read": (I32, [P, I64, P, P]),
}

_lib = None


def lib() -> C.CDLL:
    """The loaded native library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m maxuna_amd.build` "
                "(maxuna_amd has no non-native fallback)")
        handle = C.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in {**SIGNATURES, **INSTRUMENT_SIGNATURES}.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != MX_OK:
        raise MaxunaError(status, lib().mx_last_error().decode(errors="replace"))
