"""Host-side mirror of the reference's `ops` dispatch layer for the MoE path.

Same names, argument meaning and error behaviour as src/ops/{mv_id,mm_id,
combine,silu_mul}.rs: shapes are validated (by the native library, before any
launch) and violations raise `MaxunaError` instead of faulting the GPU; outputs
are allocated by the callee and returned.  Every op runs a hand-written gfx950
kernel from libmaxuna_moe.so on the current torch stream.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from functools import lru_cache

import torch

from ._lib import Map0C, MaxunaError, check, lib
from .gguf import ExpertStack, GgmlDType

__all__ = [
    "MM_ID_MIN_SEQ", "mm_id_min_seq", "no_mm_id", "MaxunaError", "Map0Scratch",
    "mul_mv_id", "mul_mv", "mul_mm_id", "prepare_map0", "mul_mm_id_shared", "supported",
    "silu_mul", "combine", "dequantize", "route_logits", "route_from_logits", "rms_norm",
]

# Prefill token count at/above which the MoE uses the grouped GEMM (ops/mod.rs:31).
MM_ID_MIN_SEQ = 32


@lru_cache(maxsize=None)
def mm_id_min_seq() -> int:
    """`LAGUNA_MM_ID_MIN_SEQ=<n>` overrides MM_ID_MIN_SEQ; read once (ops/mod.rs:38-50)."""
    try:
        return int(os.environ["LAGUNA_MM_ID_MIN_SEQ"])
    except (KeyError, ValueError):
        return MM_ID_MIN_SEQ


@lru_cache(maxsize=None)
def no_mm_id() -> bool:
    """Presence-based `LAGUNA_NO_MM_ID`: forces mul_mv_id everywhere (ops/mod.rs:57-64)."""
    return "LAGUNA_NO_MM_ID" in os.environ


def _stream() -> C.c_void_p:
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _f32(t: torch.Tensor, name: str, rank: int) -> torch.Tensor:
    if t.dtype != torch.float32:
        raise MaxunaError(2, f"{name} must be f32, got {t.dtype}")
    if t.dim() != rank:
        raise MaxunaError(2, f"{name} must be rank-{rank}, got shape {tuple(t.shape)}")
    if not t.is_contiguous():
        raise MaxunaError(2, f"{name} must be contiguous")
    return t


def _u32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype not in (torch.uint32, torch.int32):
        raise MaxunaError(2, f"{name} must be u32, got {t.dtype}")
    if t.dim() != 2 or not t.is_contiguous():
        raise MaxunaError(2, f"{name} must be a contiguous rank-2 [t, top_k] tensor")
    return t


def supported(dtype: GgmlDType, top_k: int) -> bool:
    """Whether the grouped-GEMM path has kernels for this dtype/top_k (mm_id.rs:48-50)."""
    return dtype in (GgmlDType.Q4_K, GgmlDType.Q5_K, GgmlDType.Q6_K, GgmlDType.Q8_0) and 1 <= top_k <= 64


IDS_DUPLICATE = 1
IDS_OUT_OF_RANGE = 2


def check_ids(ids: torch.Tensor, n_expert: int, raise_on_error: bool = True) -> int:
    """Device-side validation of routing ids (mx_check_ids): the flag word,
    IDS_DUPLICATE | IDS_OUT_OF_RANGE.  Synchronises with the device; with
    raise_on_error a non-zero flag raises MaxunaError (fail-closed, as the
    reference's host validation is, dispatch.rs:812-847)."""
    _u32(ids, "ids")
    t, top_k = ids.shape
    flags = torch.empty(1, dtype=torch.int32, device=ids.device)
    check(lib().mx_check_ids(ids.data_ptr(), t, top_k, n_expert, flags.data_ptr(), _stream()))
    f = int(flags.item())
    if f and raise_on_error:
        what = [n for b, n in ((IDS_DUPLICATE, "a token repeats an expert id"),
                               (IDS_OUT_OF_RANGE, f"an expert id >= n_expert ({n_expert})")) if f & b]
        raise MaxunaError(2, "invalid routing ids: " + "; ".join(what))
    return f


def mul_mv_id(stack: ExpertStack, x: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """Quantised gather mat-vec (mv_id.rs:37-45).

    x: [t, x_per_row, k] f32 (x_per_row 1 for gate/up, top_k for down);
    ids: [t, top_k] u32.  Returns [t, top_k, n_out] f32."""
    _f32(x, "x", 3)
    _u32(ids, "ids")
    t, xpr, k = x.shape
    t_ids, top_k = ids.shape
    dst = torch.empty((t, top_k, stack.n_out), dtype=torch.float32, device=x.device)
    sc = stack.to_c()
    check(lib().mx_mul_mv_id(C.byref(sc), x.data_ptr(), t, xpr, k, ids.data_ptr(), t_ids, top_k,
                             dst.data_ptr(), _stream()))
    return dst


def mul_mv(weight: torch.Tensor, dtype: GgmlDType, n_out: int, k: int, x: torch.Tensor) -> torch.Tensor:
    """Plain quantised mat-vec (mv_id.rs:54-56).  weight: raw [n_out, k] blocks; x [t, k]."""
    _f32(x, "x", 2)
    t, kx = x.shape
    if kx != k:
        raise MaxunaError(2, f"x k ({kx}) does not match weight k ({k})")
    dst = torch.empty((t, n_out), dtype=torch.float32, device=x.device)
    check(lib().mx_mul_mv(weight.data_ptr(), int(dtype), n_out, k, x.data_ptr(), t, dst.data_ptr(),
                          _stream()))
    return dst


@dataclass
class Map0Scratch:
    """A prepared bucket map plus the geometry it was laid out for (dispatch.rs:752-757)."""

    buffer: torch.Tensor  # int32 words, layout in maxuna_moe.h
    n_expert: int
    t: int
    top_k: int

    def to_c(self) -> Map0C:
        return Map0C(self.buffer.data_ptr(), self.buffer.numel() * 4, self.n_expert, self.t, self.top_k)

    # views of the documented layout, for inspection
    def _layout(self):
        e, t, k = self.n_expert, self.t, self.top_k
        t_max = (t * k + 63) // 64 + e
        off = e
        n_tiles = off + e + 1
        dup = n_tiles + 1
        tiles = dup + 1
        lst = tiles + t_max
        return dict(tpe=0, off=off, n_tiles=n_tiles, dup=dup, tiles=tiles, list=lst, t_max=t_max)

    def counts(self) -> torch.Tensor:
        return self.buffer[: self.n_expert]

    def offsets(self) -> torch.Tensor:
        L = self._layout()
        return self.buffer[L["off"]: L["off"] + self.n_expert + 1]

    def pair_list(self) -> torch.Tensor:
        L = self._layout()
        return self.buffer[L["list"]: L["list"] + self.t * self.top_k]

    def dup_flag(self) -> int:
        return int(self.buffer[self._layout()["dup"]].item())


def prepare_map0(n_expert: int, ids: torch.Tensor) -> Map0Scratch:
    """Bucket (token, slot) pairs per expert once for all three projections (mm_id.rs:27-29)."""
    _u32(ids, "ids")
    t, top_k = ids.shape
    nbytes = lib().mx_map0_scratch_bytes(n_expert, t, top_k)
    buf = torch.empty(max(nbytes, 4) // 4, dtype=torch.int32, device=ids.device)
    check(lib().mx_prepare_map0(n_expert, ids.data_ptr(), t, top_k, buf.data_ptr(), buf.numel() * 4,
                                _stream()))
    return Map0Scratch(buf, n_expert, t, top_k)


def mul_mm_id_shared(stack: ExpertStack, x: torch.Tensor, ids: torch.Tensor,
                     scratch: Map0Scratch) -> torch.Tensor:
    """One grouped-GEMM projection against a prepared map (mm_id.rs:32-39)."""
    _f32(x, "x", 3)
    _u32(ids, "ids")
    t, xpr, k = x.shape
    t_ids, top_k = ids.shape
    dst = torch.empty((t, top_k, stack.n_out), dtype=torch.float32, device=x.device)
    sc, mc = stack.to_c(), scratch.to_c()
    check(lib().mx_mul_mm_id_shared(C.byref(sc), x.data_ptr(), t, xpr, k, ids.data_ptr(), t_ids, top_k,
                                    C.byref(mc), dst.data_ptr(), _stream()))
    return dst


def mul_mm_id(stack: ExpertStack, x: torch.Tensor, ids: torch.Tensor) -> torch.Tensor:
    """Self-contained grouped GEMM: its own bucket pass, then the GEMM (mm_id.rs:16-18)."""
    _f32(x, "x", 3)
    _u32(ids, "ids")
    t, xpr, k = x.shape
    t_ids, top_k = ids.shape
    ws_bytes = lib().mx_mul_mm_id_workspace_bytes(stack.n_expert, t, top_k, xpr, k)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=x.device)
    dst = torch.empty((t, top_k, stack.n_out), dtype=torch.float32, device=x.device)
    sc = stack.to_c()
    check(lib().mx_mul_mm_id(C.byref(sc), x.data_ptr(), t, xpr, k, ids.data_ptr(), t_ids, top_k,
                             ws.data_ptr(), ws.numel(), dst.data_ptr(), _stream()))
    return dst


def silu_mul(gate: torch.Tensor, up: torch.Tensor) -> torch.Tensor:
    """silu(gate) * up, one pass (silu_mul.rs:14-16)."""
    if gate.shape != up.shape:
        raise MaxunaError(2, f"gate {tuple(gate.shape)} and up {tuple(up.shape)} differ")
    if gate.dtype != torch.float32 or up.dtype != torch.float32:
        raise MaxunaError(2, "silu_mul operands must be f32")
    if not (gate.is_contiguous() and up.is_contiguous()):
        raise MaxunaError(2, "silu_mul operands must be contiguous")
    dst = torch.empty_like(gate)
    check(lib().mx_silu_mul(gate.data_ptr(), up.data_ptr(), gate.numel(), dst.data_ptr(), _stream()))
    return dst


def combine(down: torch.Tensor, col_l2: torch.Tensor | None, weights: torch.Tensor) -> torch.Tensor:
    """Weighted sum over top_k (combine.rs:16-18).  down [seq, top_k, n_out]; weights
    [seq, top_k]; col_l2 optional [seq, top_k, 1] (undoes the L2 rescale)."""
    _f32(down, "down", 3)
    seq, top_k, n_out = down.shape
    _f32(weights, "weights", 2)
    if tuple(weights.shape) != (seq, top_k):
        raise MaxunaError(2, f"weights shape {tuple(weights.shape)} must be [seq, top_k] = [{seq}, {top_k}]")
    if col_l2 is not None:
        _f32(col_l2, "col_l2", 3)
        if tuple(col_l2.shape) != (seq, top_k, 1):
            raise MaxunaError(2, f"col_l2 shape {tuple(col_l2.shape)} must be [seq, top_k, 1]")
    dst = torch.empty((seq, n_out), dtype=torch.float32, device=down.device)
    check(lib().mx_combine(down.data_ptr(), _ptr(col_l2), weights.data_ptr(), seq, top_k, n_out,
                           dst.data_ptr(), _stream()))
    return dst


def dequantize(blocks: torch.Tensor, dtype: GgmlDType, n: int) -> torch.Tensor:
    """Bit-exact dequantisation of n weights of raw blocks to f32."""
    out = torch.empty(n, dtype=torch.float32, device=blocks.device)
    check(lib().mx_dequantize(int(dtype), blocks.data_ptr(), n, out.data_ptr(), _stream()))
    return out


def route_logits(router: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """logits[t, e] = <x[t], router[e]> in f32 (moe.rs:84-87).  `router` is the GGUF
    `ffn_gate_inp` weight [n_expert, hidden] as stored (no transpose needed)."""
    _f32(x, "x", 2)
    _f32(router, "router", 2)
    t, hidden = x.shape
    if router.shape[1] != hidden:
        raise MaxunaError(2, f"router {tuple(router.shape)} does not match hidden {hidden}")
    n_expert = router.shape[0]
    out = torch.empty((t, n_expert), dtype=torch.float32, device=x.device)
    check(lib().mx_route_logits(x.data_ptr(), router.data_ptr(), t, hidden, n_expert, out.data_ptr(),
                                _stream()))
    return out


def route_from_logits(logits: torch.Tensor, bias: torch.Tensor, n_expert_used: int, scale: float,
                      norm: bool) -> tuple[torch.Tensor, torch.Tensor]:
    """Routing decision from pre-sigmoid logits (moe.rs:94-119).  Returns (ids u32 [t, k],
    weights f32 [t, k])."""
    _f32(logits, "logits", 2)
    t, n_expert = logits.shape
    if bias.numel() != n_expert:
        raise MaxunaError(2, f"bias has {bias.numel()} entries, expected {n_expert}")
    ids = torch.empty((t, n_expert_used), dtype=torch.uint32, device=logits.device)
    w = torch.empty((t, n_expert_used), dtype=torch.float32, device=logits.device)
    check(lib().mx_route_from_logits(logits.data_ptr(), bias.contiguous().data_ptr(), t, n_expert,
                                     n_expert_used, float(scale), 1 if norm else 0, ids.data_ptr(),
                                     w.data_ptr(), _stream()))
    return ids, w


def rms_norm(x: torch.Tensor, alpha: torch.Tensor, eps: float) -> torch.Tensor:
    """x / sqrt(mean(x^2) + eps) * alpha over the last dim."""
    _f32(x, "x", 2)
    rows, dim = x.shape
    out = torch.empty_like(x)
    check(lib().mx_rms_norm(x.data_ptr(), alpha.data_ptr(), rows, dim, float(eps), out.data_ptr(),
                            _stream()))
    return out
