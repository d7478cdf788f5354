"""ctypes wrapper of the CPU oracle (oracle/moe_oracle.c) -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this
module, and only as the checker.  It restates the reference's
`--moe-impl reference` semantics (ReferenceExperts, moe.rs:141-187; routing
moe.rs:84-119; shared SwiGLU moe.rs:369-374) on the host.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "lib" / "libmoe_oracle.so"

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
BLOCK = {Q8_0: 32, Q4_K: 256, Q5_K: 256, Q6_K: 256}
TSIZE = {Q8_0: 34, Q4_K: 144, Q5_K: 176, Q6_K: 210}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        P, I, I64, U64, F, D = C.c_void_p, C.c_int, C.c_int64, C.c_uint64, C.c_float, C.c_double
        sig = {
            "or_block_size": (I, [I]), "or_type_size": (I, [I]),
            "or_f16_to_f32": (F, [C.c_uint16]), "or_f32_to_f16": (C.c_uint16, [F]),
            "or_dequantize": (I, [I, P, I64, P]),
            "or_mix64": (U64, [U64]), "or_tensor_key": (U64, [U64, C.c_uint32, C.c_uint32]),
            "or_synth_blocks": (I, [I, U64, I64, I64, P]),
            "or_route_logits": (None, [P, P, I64, I64, I64, P]),
            "or_route_from_logits": (None, [P, P, I64, I64, I64, D, I, P, P]),
            "or_mul_mv_id": (I, [I, P, I64, I64, I64, P, I64, P, I64, I64, P]),
            "or_mul_mv": (I, [I, P, I64, I64, P, I64, P]),
            "or_map0": (I, [P, I64, I64, I64, P, P]),
            "or_silu_mul": (None, [P, P, I64, P]),
            "or_combine": (None, [P, P, P, I64, I64, I64, P]),
            "or_rmsnorm": (None, [P, P, I64, I64, F, P]),
            "or_reference_experts": (I, [I, P, I, P, I, P, I64, I64, I64, P, P, P, I64, I64, P]),
            "or_swiglu": (I, [I, P, I, P, I, P, I64, I64, P, I64, P]),
            "or_num_threads": (I, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _rc(rc: int, what: str):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with {rc}")


def row_bytes(dtype: int, k: int) -> int:
    return k // BLOCK[dtype] * TSIZE[dtype]


def dequantize(dtype: int, blocks: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    _rc(lib().or_dequantize(dtype, _p(blocks), n, _p(out)), "dequantize")
    return out


def synth_bytes(dtype: int, key: int, byte_off: int, nbytes: int) -> np.ndarray:
    out = np.empty(nbytes, dtype=np.uint8)
    _rc(lib().or_synth_blocks(dtype, key, byte_off, nbytes, _p(out)), "synth")
    return out


def expert_blocks(dtype: int, key: int, e: int, n_out: int, k: int) -> np.ndarray:
    """Raw bytes of expert e of a synthetic stack [*, n_out, k]."""
    eb = n_out * row_bytes(dtype, k)
    return synth_bytes(dtype, key, e * eb, eb)


def route_logits(x: np.ndarray, router_t: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    router_t = np.ascontiguousarray(router_t, np.float32)
    t, h = x.shape
    e = router_t.shape[1]
    out = np.empty((t, e), np.float32)
    lib().or_route_logits(_p(x), _p(router_t), t, h, e, _p(out))
    return out


def route_from_logits(logits: np.ndarray, bias: np.ndarray, top_k: int, scale: float, norm: bool):
    logits = np.ascontiguousarray(logits, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    t, e = logits.shape
    ids = np.empty((t, top_k), np.uint32)
    w = np.empty((t, top_k), np.float32)
    lib().or_route_from_logits(_p(logits), _p(bias), t, e, top_k, float(scale), 1 if norm else 0, _p(ids), _p(w))
    return ids, w


def _ptr_array(blocks: dict[int, np.ndarray], n_expert: int):
    arr = (C.c_void_p * n_expert)()
    for e, b in blocks.items():
        arr[e] = b.ctypes.data
    return arr


def mul_mv_id(dtype: int, experts: dict[int, np.ndarray], n_expert: int, n_out: int, k: int,
              x: np.ndarray, ids: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.uint32)
    t, xpr, _ = x.shape
    top_k = ids.shape[1]
    out = np.empty((t, top_k, n_out), np.float32)
    arr = _ptr_array(experts, n_expert)
    _rc(lib().or_mul_mv_id(dtype, C.cast(arr, C.c_void_p), n_expert, n_out, k, _p(x), xpr, _p(ids), t, top_k,
                           _p(out)), "mul_mv_id")
    return out


def map0(ids: np.ndarray, n_expert: int):
    ids = np.ascontiguousarray(ids, np.uint32)
    t, k = ids.shape
    tpe = np.empty(n_expert, np.int32)
    hids = np.full(n_expert * max(t, 1), -1, np.int32)
    lib().or_map0(_p(ids), t, k, n_expert, _p(tpe), _p(hids))
    return tpe, hids.reshape(n_expert, max(t, 1))


def silu_mul(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, np.float32)
    u = np.ascontiguousarray(u, np.float32)
    out = np.empty_like(g)
    lib().or_silu_mul(_p(g), _p(u), g.size, _p(out))
    return out


def combine(down: np.ndarray, col_l2: np.ndarray | None, w: np.ndarray) -> np.ndarray:
    down = np.ascontiguousarray(down, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    l2 = None if col_l2 is None else np.ascontiguousarray(col_l2, np.float32)
    s, k, n = down.shape
    out = np.empty((s, n), np.float32)
    lib().or_combine(_p(down), _p(l2), _p(w), s, k, n, _p(out))
    return out


def rmsnorm(x: np.ndarray, alpha: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    alpha = np.ascontiguousarray(alpha, np.float32)
    out = np.empty_like(x)
    lib().or_rmsnorm(_p(x), _p(alpha), x.shape[0], x.shape[1], float(eps), _p(out))
    return out


def reference_experts(gate_dt, gate: dict, up_dt, up: dict, down_dt, down: dict, n_expert: int, hidden: int,
                      ff: int, x: np.ndarray, ids: np.ndarray, w: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    ids = np.ascontiguousarray(ids, np.uint32)
    w = np.ascontiguousarray(w, np.float32)
    t, k = ids.shape
    out = np.empty((t, hidden), np.float32)
    ga, ua, da = (_ptr_array(d, n_expert) for d in (gate, up, down))
    _rc(lib().or_reference_experts(gate_dt, C.cast(ga, C.c_void_p), up_dt, C.cast(ua, C.c_void_p), down_dt,
                                   C.cast(da, C.c_void_p), n_expert, hidden, ff, _p(x), _p(ids), _p(w), t, k,
                                   _p(out)), "reference_experts")
    return out


def swiglu(gate_dt, gate: np.ndarray, up_dt, up: np.ndarray, down_dt, down: np.ndarray, hidden: int, ff: int,
           x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    t = x.shape[0]
    out = np.empty((t, hidden), np.float32)
    _rc(lib().or_swiglu(gate_dt, _p(gate), up_dt, _p(up), down_dt, _p(down), hidden, ff, _p(x), t, _p(out)),
        "swiglu")
    return out


def moe_layer(spec, keys: dict, router_t: np.ndarray, bias: np.ndarray, x: np.ndarray,
              ids: np.ndarray | None = None, w: np.ndarray | None = None):
    """MoeBlock::forward with the Reference runner (moe.rs:73-78, 141-187) for a
    synthetic layer: regenerates only the experts the ids select.  If ids/w are
    given they replace the oracle's own routing (for comparing expert math on
    identical routing).  Returns (out, ids, w)."""
    H, FF, E = spec.hidden, spec.ff, spec.n_expert
    if ids is None:
        logits = route_logits(x, router_t)
        ids, w = route_from_logits(logits, bias, spec.top_k, spec.weights_scale, spec.weights_norm)
    sel = sorted(set(int(e) for e in np.asarray(ids).ravel()))
    gdt, udt, ddt = int(spec.gate_dt), int(spec.up_dt), int(spec.down_dt)
    g = {e: expert_blocks(gdt, keys["gate_exps"], e, FF, H) for e in sel}
    u = {e: expert_blocks(udt, keys["up_exps"], e, FF, H) for e in sel}
    d = {e: expert_blocks(ddt, keys["down_exps"], e, H, FF) for e in sel}
    out = reference_experts(gdt, g, udt, u, ddt, d, E, H, FF, x, ids, w)
    if spec.shared:
        sg = expert_blocks(gdt, keys["gate_shexp"], 0, FF, H)
        su = expert_blocks(udt, keys["up_shexp"], 0, FF, H)
        sd = expert_blocks(ddt, keys["down_shexp"], 0, H, FF)
        out = out + swiglu(gdt, sg, udt, su, ddt, sd, H, FF, x)  # routed + shared, f32
    return out, ids, w
