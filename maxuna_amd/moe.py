"""The MoE block: routing, routed experts, shared expert (src/moe.rs:19-374).

`MoeBlock.forward` runs the whole block through one native entry point
(`mx_moe_forward`): the fused decode kernels below MM_ID_MIN_SEQ tokens, the
bucketed grouped GEMM at and above it.  `FusedExperts` and `SharedExpert`
compose the individual ops exactly as the reference's `FusedExperts::forward`
(moe.rs:221-323) does, for callers that drive the stages themselves.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import ops
from ._lib import MoeLayerC, check, lib
from .gguf import ExpertStack, null_stack

# F16's smallest positive normal: the routing-weight sum floor (moe.rs:12-14).
WEIGHTS_SUM_FLOOR = 6.103515625e-5


def route_logits(router: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """moe.rs:84-87 (router in its GGUF layout [n_expert, hidden])."""
    return ops.route_logits(router, x)


def route_from_logits(logits, bias, n_expert_used, scale, norm):
    """moe.rs:94-119."""
    return ops.route_from_logits(logits, bias, n_expert_used, scale, norm)


class SharedExpert:
    """The always-on SwiGLU expert `down(silu(gate(x)) * up(x))` (moe.rs:327-345, 369-374)."""

    def __init__(self, gate: ExpertStack, up: ExpertStack, down: ExpertStack):
        for s in (gate, up, down):
            if s.n_expert != 1:
                raise ValueError("a shared expert stack has n_expert == 1")
        self.gate, self.up, self.down = gate, up, down

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        t = x.shape[0]
        ids = torch.zeros((t, 1), dtype=torch.uint32, device=x.device)
        xr = x.reshape(t, 1, -1).contiguous()
        g = ops.mul_mv_id(self.gate, xr, ids)
        u = ops.mul_mv_id(self.up, xr, ids)
        h = ops.silu_mul(g, u)
        return ops.mul_mv_id(self.down, h, ids).reshape(t, -1)


class FusedExperts:
    """Routed experts evaluated from the stacked GGUF layout (moe.rs:194-324)."""

    def __init__(self, gate: ExpertStack, up: ExpertStack, down: ExpertStack):
        if not (gate.n_expert == up.n_expert == down.n_expert):
            raise ValueError(f"MoE expert stacks disagree on n_expert: gate={gate.n_expert}, "
                             f"up={up.n_expert}, down={down.n_expert}")
        self.gate, self.up, self.down = gate, up, down

    def forward(self, x: torch.Tensor, ids: torch.Tensor, weights: torch.Tensor) -> torch.Tensor:
        seq, hidden = x.shape
        top_k = ids.shape[1]
        use_mm = (seq >= ops.mm_id_min_seq() and not ops.no_mm_id()
                  and all(ops.supported(s.dtype, top_k) for s in (self.gate, self.up, self.down)))
        map0 = ops.prepare_map0(self.gate.n_expert, ids) if use_mm else None

        def matmul(stack, xx):
            if map0 is not None:
                return ops.mul_mm_id_shared(stack, xx, ids, map0)
            return ops.mul_mv_id(stack, xx, ids)

        x_g = x.reshape(seq, 1, hidden).contiguous()
        gate = matmul(self.gate, x_g)
        up = matmul(self.up, x_g)
        act = ops.silu_mul(gate, up)
        # The grouped GEMM stages the activation in f16 with an exact per-row
        # power-of-two scale, so no L2 rescale pass is needed on either path.
        down = matmul(self.down, act)
        return ops.combine(down, None, weights.contiguous())


@dataclass
class MoeConfig:
    """MoE hyper-parameters (config.rs:35-42)."""

    n_expert_used: int
    expert_weights_scale: float = 1.0
    expert_weights_norm: bool = True


class MoeBlock:
    """One MoE FFN block: `routed(x, route(x)) + shared(x)` (moe.rs:28-79)."""

    def __init__(self, router: torch.Tensor, exp_probs_b: torch.Tensor, gate: ExpertStack,
                 up: ExpertStack, down: ExpertStack, cfg: MoeConfig,
                 shared: SharedExpert | None = None, rms_alpha: torch.Tensor | None = None,
                 rms_eps: float = 1e-6):
        self.router = router.contiguous()  # [n_expert, hidden], ffn_gate_inp as stored
        self.exp_probs_b = exp_probs_b.contiguous()
        self.experts = FusedExperts(gate, up, down)
        self.shared = shared
        self.cfg = cfg
        self.rms_alpha = rms_alpha
        self.rms_eps = rms_eps
        self._ws = None
        self._c = self._layer_struct()

    @property
    def hidden(self) -> int:
        return self.router.shape[1]

    def _layer_struct(self) -> MoeLayerC:
        e = self.experts
        sh = self.shared
        return MoeLayerC(
            self.router.data_ptr(), self.exp_probs_b.data_ptr(),
            e.gate.to_c(), e.up.to_c(), e.down.to_c(),
            sh.gate.to_c() if sh else null_stack(), sh.up.to_c() if sh else null_stack(),
            sh.down.to_c() if sh else null_stack(),
            self.hidden, e.gate.n_out, self.cfg.n_expert_used, float(self.cfg.expert_weights_scale),
            1 if self.cfg.expert_weights_norm else 0,
            -1 if ops.no_mm_id() else ops.mm_id_min_seq(),
            self.rms_alpha.data_ptr() if self.rms_alpha is not None else None,
            float(self.rms_eps), 0)

    def workspace(self, t: int, device) -> torch.Tensor:
        need = lib().mx_moe_workspace_bytes(C.byref(self._c), t)
        if self._ws is None or self._ws.numel() < need:
            # no state lives in the workspace between calls (every forward
            # initialises what it reads); zeroed only for tidiness
            self._ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=device)
        return self._ws

    def route(self, x_normed: torch.Tensor):
        """(ids [t, k] u32, weights [t, k] f32) (moe.rs:62-71)."""
        logits = route_logits(self.router, x_normed)
        return route_from_logits(logits, self.exp_probs_b, self.cfg.n_expert_used,
                                 self.cfg.expert_weights_scale, self.cfg.expert_weights_norm)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
                return_routing: bool = False):
        """out = residual + MoE(x') with x' = RMSNorm(x) if rms_alpha is set, else x."""
        if x.dtype != torch.float32 or x.dim() != 2 or not x.is_contiguous():
            raise ops.MaxunaError(2, "x must be a contiguous f32 [t, hidden] tensor")
        t = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        ids = torch.empty((t, self.cfg.n_expert_used), dtype=torch.uint32, device=x.device)
        w = torch.empty((t, self.cfg.n_expert_used), dtype=torch.float32, device=x.device)
        ws = self.workspace(t, x.device)
        check(lib().mx_moe_forward(C.byref(self._c), x.data_ptr(), t,
                                   residual.data_ptr() if residual is not None else None,
                                   out.data_ptr(), ids.data_ptr(), w.data_ptr(), ws.data_ptr(),
                                   ws.numel(), ops._stream()))
        return (out, ids, w) if return_routing else out

    def forward_noalloc(self, x: torch.Tensor, residual: torch.Tensor | None = None,
                        out: torch.Tensor | None = None, return_routing: bool = False):
        """`forward` through mx_moe_forward_noalloc: the library's own device-resident
        scratch is the workspace (no allocation by the call, for callers that cannot
        allocate); MaxunaError if this t needs more than that scratch holds.  Calls
        that overlap on one GPU share the scratch and race."""
        if x.dtype != torch.float32 or x.dim() != 2 or not x.is_contiguous():
            raise ops.MaxunaError(2, "x must be a contiguous f32 [t, hidden] tensor")
        t = x.shape[0]
        if out is None:
            out = torch.empty_like(x)
        ids = torch.empty((t, self.cfg.n_expert_used), dtype=torch.uint32, device=x.device)
        w = torch.empty((t, self.cfg.n_expert_used), dtype=torch.float32, device=x.device)
        check(lib().mx_moe_forward_noalloc(C.byref(self._c), x.data_ptr(), t,
                                           residual.data_ptr() if residual is not None else None,
                                           out.data_ptr(), ids.data_ptr(), w.data_ptr(), ops._stream()))
        return (out, ids, w) if return_routing else out
