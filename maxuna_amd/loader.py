"""Builds MoE blocks from a GGUF file (the reference's model load of the FFN
half, src/moe.rs:42-60, 128-137, 333-339; config keys config.rs:124-130)."""
from __future__ import annotations

import torch

from .gguf import GgufFile
from .moe import MoeBlock, MoeConfig, SharedExpert


def moe_config(gf: GgufFile, arch: str = "laguna") -> MoeConfig:
    """n_expert_used, expert_weights_scale (default 2.5), expert_weights_norm
    (default true) -- config.rs:125-129."""
    return MoeConfig(gf.get_int(f"{arch}.expert_used_count"),
                     gf.get_float(f"{arch}.expert_weights_scale", 2.5),
                     gf.get_bool(f"{arch}.expert_weights_norm", True))


def load_moe_block(gf: GgufFile, layer: int, device="cuda", arch: str = "laguna",
                   with_norm: bool = False) -> MoeBlock:
    """MoE block of decoder layer `layer`: router `ffn_gate_inp` [n_expert, hidden]
    as stored, `exp_probs_b` (`.weight` or `.bias`, gguf.rs:671-687), expert
    stacks `ffn_{gate,up,down}_exps`, and the shared expert
    `ffn_{gate,up,down}_shexp` when present (moe.rs:333-339).  with_norm adds the
    FFN RMSNorm `ffn_norm` (eps `attention.layer_norm_rms_epsilon`, default
    1e-6), so forward computes residual + MoE(RMSNorm(x)) (model.rs:340-351)."""
    p = f"blk.{layer}."
    router = gf.dense_f32(p + "ffn_gate_inp.weight", device)
    bias_name = p + "exp_probs_b.weight" if p + "exp_probs_b.weight" in gf.tensors else p + "exp_probs_b.bias"
    bias = gf.dense_f32(bias_name, device).reshape(-1)
    gate = gf.expert_stack(p + "ffn_gate_exps.weight", device)
    up = gf.expert_stack(p + "ffn_up_exps.weight", device)
    down = gf.expert_stack(p + "ffn_down_exps.weight", device)
    n_expert = gf.get_int(f"{arch}.expert_count", gate.n_expert)
    if gate.n_expert != n_expert or router.shape[0] != n_expert or bias.numel() != n_expert:
        raise ValueError(f"layer {layer}: expert count mismatch (metadata {n_expert}, gate {gate.n_expert}, "
                         f"router {router.shape[0]}, bias {bias.numel()})")
    shared = None
    if p + "ffn_gate_shexp.weight" in gf.tensors:
        shared = SharedExpert(gf.expert_stack(p + "ffn_gate_shexp.weight", device),
                              gf.expert_stack(p + "ffn_up_shexp.weight", device),
                              gf.expert_stack(p + "ffn_down_shexp.weight", device))
    alpha = None
    eps = gf.get_float(f"{arch}.attention.layer_norm_rms_epsilon", 1e-6)
    if with_norm:
        alpha = gf.dense_f32(p + "ffn_norm.weight", device).reshape(-1)
    return MoeBlock(router, bias, gate, up, down, moe_config(gf, arch), shared=shared, rms_alpha=alpha,
                    rms_eps=eps)


def export_layer(path, layers, arch: str = "laguna", extra_metadata: dict | None = None) -> None:
    """Writes synthetic layers (maxuna_amd.synth.SynthLayer) as a GGUF file with
    the reference's tensor names: the inverse of load_moe_block."""
    from .gguf import GGML_F32, GGUF_BOOL, GGUF_F32, GGUF_STRING, GGUF_U32, write_gguf
    spec = layers[0].spec
    meta = {
        "general.architecture": (GGUF_STRING, arch),
        f"{arch}.expert_count": (GGUF_U32, spec.n_expert),
        f"{arch}.expert_used_count": (GGUF_U32, spec.top_k),
        f"{arch}.expert_feed_forward_length": (GGUF_U32, spec.ff),
        f"{arch}.embedding_length": (GGUF_U32, spec.hidden),
        f"{arch}.expert_weights_scale": (GGUF_F32, float(spec.weights_scale)),
        f"{arch}.expert_weights_norm": (GGUF_BOOL, bool(spec.weights_norm)),
        f"{arch}.attention.layer_norm_rms_epsilon": (GGUF_F32, 1e-6),
    }
    meta.update(extra_metadata or {})
    tensors = []
    for li, lay in enumerate(layers):
        b = lay.block
        p = f"blk.{li}."
        tensors.append((p + "ffn_gate_inp.weight", GGML_F32, tuple(b.router.shape), b.router.cpu().numpy().tobytes()))
        tensors.append((p + "exp_probs_b.bias", GGML_F32, (spec.n_expert,), b.exp_probs_b.cpu().numpy().tobytes()))
        tensors.append((p + "ffn_norm.weight", GGML_F32, (spec.hidden,),
                        torch.ones(spec.hidden, dtype=torch.float32).numpy().tobytes()))
        e = b.experts
        for nm, st in (("ffn_gate_exps", e.gate), ("ffn_up_exps", e.up), ("ffn_down_exps", e.down)):
            tensors.append((p + nm + ".weight", int(st.dtype), (st.n_expert, st.n_out, st.k),
                            st.buffer[st.base_off:st.base_off + st.nbytes].cpu().numpy().tobytes()))
        if b.shared is not None:
            for nm, st in (("ffn_gate_shexp", b.shared.gate), ("ffn_up_shexp", b.shared.up),
                           ("ffn_down_shexp", b.shared.down)):
                tensors.append((p + nm + ".weight", int(st.dtype), (st.n_out, st.k),
                                st.buffer[st.base_off:st.base_off + st.nbytes].cpu().numpy().tobytes()))
    write_gguf(path, meta, tensors)
