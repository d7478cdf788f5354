"""Seeded synthetic MoE layers for the benchmark configurations (no checkpoints).

Weights are generated on the device by the library's counter-based generator
(`mx_synth_blocks`): byte j of a tensor is byte (j & 7) of
mix64(key + (j/8 + 1) * GAMMA) (splitmix64 finaliser), after which each
block's f16 scale fields are set to f16(0.001 + 0.009 u).  Dense f32 inputs
(x, router, selection bias) are N(0, sigma) from a counter-based Box-Muller over
the same mixer, generated on the host with numpy and uploaded.  Every tensor is
addressed by (seed, layer, tensor id), so any expert can be regenerated
independently (the CPU checker regenerates only the experts a token selects).
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np
import torch

from ._lib import check, lib
from .gguf import ExpertStack, GgmlDType
from .moe import MoeBlock, MoeConfig, SharedExpert

GAMMA = 0x9E3779B97F4A7C15
MASK = (1 << 64) - 1

TENSOR_IDS = {
    "router": 0, "bias": 1, "x": 2, "rms": 3,
    "gate_exps": 10, "up_exps": 11, "down_exps": 12,
    "gate_shexp": 20, "up_shexp": 21, "down_shexp": 22,
}


def mix64(z: int) -> int:
    z &= MASK
    z ^= z >> 30; z = (z * 0xBF58476D1CE4E5B9) & MASK
    z ^= z >> 27; z = (z * 0x94D049BB133111EB) & MASK
    z ^= z >> 31
    return z


def tensor_key(seed: int, layer: int, tensor_id: int) -> int:
    a = mix64(seed + GAMMA)
    b = mix64(((layer << 16) | tensor_id) + 2 * GAMMA)
    return mix64(a ^ b)


def _mix64_np(z: np.ndarray) -> np.ndarray:
    z = z ^ (z >> np.uint64(30)); z = z * np.uint64(0xBF58476D1CE4E5B9)
    z = z ^ (z >> np.uint64(27)); z = z * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def normal(key: int, n: int, sigma: float, offset: int = 0) -> np.ndarray:
    """n samples of N(0, sigma) as f32: Box-Muller on two mixed counters per sample."""
    i = np.arange(offset, offset + n, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h1 = _mix64_np(np.uint64(key) + (np.uint64(2) * i + np.uint64(1)) * np.uint64(GAMMA))
        h2 = _mix64_np(np.uint64(key) + (np.uint64(2) * i + np.uint64(2)) * np.uint64(GAMMA))
    u1 = ((h1 >> np.uint64(11)).astype(np.float64) + 1.0) * 2.0**-53
    u2 = (h2 >> np.uint64(11)).astype(np.float64) * 2.0**-53
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (sigma * z).astype(np.float32)


def synth_stack(dtype: GgmlDType, n_expert: int, n_out: int, k: int, key: int, device="cuda") -> ExpertStack:
    st = ExpertStack.empty(dtype, n_expert, n_out, k, device=device)
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    check(lib().mx_synth_blocks(int(dtype), key, st.buffer.data_ptr(), st.nbytes, stream))
    return st


@dataclass
class LayerSpec:
    """One synthetic MoE layer shape (C1 is Laguna-shaped)."""

    hidden: int
    ff: int
    n_expert: int
    top_k: int
    gate_dt: GgmlDType
    down_dt: GgmlDType
    shared: bool
    router_sigma: float = 0.02
    bias_sigma: float = 0.1
    weights_scale: float = 1.0
    weights_norm: bool = True

    @property
    def up_dt(self) -> GgmlDType:
        return self.gate_dt

    def expert_bytes(self) -> int:
        """Bytes of one expert's gate + up + down."""
        from .gguf import row_bytes
        return 2 * self.ff * row_bytes(self.gate_dt, self.hidden) + self.hidden * row_bytes(self.down_dt, self.ff)


# The BASELINE.json configurations (0-indexed, as that file cross-references them).
CONFIGS = {
    "C0": dict(spec=LayerSpec(1024, 512, 64, 4, GgmlDType.Q4_K, GgmlDType.Q4_K, shared=False,
                              bias_sigma=0.0), t=1, layers=1),
    "C1": dict(spec=LayerSpec(4096, 1536, 256, 10, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True), t=1, layers=1),
    "C2": dict(spec=LayerSpec(4096, 1536, 256, 10, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True), t=16, layers=1),
    "C3": dict(spec=LayerSpec(4096, 1536, 256, 10, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True,
                              bias_sigma=0.5), t=2048, layers=1),
    "C4": dict(spec=LayerSpec(4096, 1536, 256, 10, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True), t=1, layers=48),
}


@dataclass
class SynthLayer:
    spec: LayerSpec
    seed: int
    layer: int
    block: MoeBlock
    router: np.ndarray          # host copy [n_expert, hidden] (GGUF ffn_gate_inp layout)
    bias: np.ndarray            # host copy [n_expert]
    keys: dict = field(default_factory=dict)

    @property
    def router_t(self) -> np.ndarray:
        """[hidden, n_expert], the reference's pre-transposed router (moe.rs:43)."""
        return np.ascontiguousarray(self.router.T)


def build_layer(spec: LayerSpec, seed: int, layer: int = 0, device="cuda", rms: bool = False) -> SynthLayer:
    """Allocates and fills one layer on the device."""
    key = lambda name: tensor_key(seed, layer, TENSOR_IDS[name])  # noqa: E731
    # router ~ N(0, sigma) in the GGUF ffn_gate_inp layout [n_expert, hidden]
    router = normal(key("router"), spec.n_expert * spec.hidden, spec.router_sigma).reshape(spec.n_expert, spec.hidden)
    bias = (normal(key("bias"), spec.n_expert, spec.bias_sigma) if spec.bias_sigma > 0
            else np.zeros(spec.n_expert, dtype=np.float32))
    keys = {n: key(n) for n in TENSOR_IDS}
    gate = synth_stack(spec.gate_dt, spec.n_expert, spec.ff, spec.hidden, keys["gate_exps"], device)
    up = synth_stack(spec.up_dt, spec.n_expert, spec.ff, spec.hidden, keys["up_exps"], device)
    down = synth_stack(spec.down_dt, spec.n_expert, spec.hidden, spec.ff, keys["down_exps"], device)
    shared = None
    if spec.shared:
        shared = SharedExpert(
            synth_stack(spec.gate_dt, 1, spec.ff, spec.hidden, keys["gate_shexp"], device),
            synth_stack(spec.up_dt, 1, spec.ff, spec.hidden, keys["up_shexp"], device),
            synth_stack(spec.down_dt, 1, spec.hidden, spec.ff, keys["down_shexp"], device))
    # RMSNorm weight = 1 (declared for the C4 chain)
    alpha = torch.ones(spec.hidden, dtype=torch.float32, device=device) if rms else None
    block = MoeBlock(torch.from_numpy(router).to(device), torch.from_numpy(bias).to(device), gate, up, down,
                     MoeConfig(spec.top_k, spec.weights_scale, spec.weights_norm), shared=shared,
                     rms_alpha=alpha, rms_eps=1e-6)
    return SynthLayer(spec, seed, layer, block, router, bias, keys)


def make_x(spec: LayerSpec, seed: int, t: int, layer: int = 0, sigma: float = 1.0) -> np.ndarray:
    return normal(tensor_key(seed, layer, TENSOR_IDS["x"]), t * spec.hidden, sigma).reshape(t, spec.hidden)
