"""End-to-end MoE block parity on the BASELINE configurations.

The GPU block (router + routed experts + shared expert, decode or grouped-GEMM
path) is compared with the oracle's `MoeBlock::forward` under the Reference
runner (moe.rs:73-78, 141-187) on identical seeded inputs:
  * expert ids and order must match exactly, except on tokens whose top-k
    boundary the oracle itself decides by less than 1e-5 (f32 logit rounding
    can flip such a near-tie; the number of exempted tokens is asserted small);
  * the output is compared to the oracle evaluated with the GPU's routing, to
    rel-L2 <= 1e-3 and max-abs <= 1e-2 * rms(out).
At full prefill size (t = 2048) the oracle checks all 2048 token rows of both
the grouped-GEMM path and the decode path.
"""
import numpy as np
import pytest
import torch

from maxuna_amd import ops
from maxuna_amd.moe import FusedExperts
from maxuna_amd.synth import CONFIGS, LayerSpec, build_layer, make_x
from maxuna_amd.gguf import GgmlDType
from tests.gpu_util import assert_close, check_ids, dev_f32, host, rel_l2, selection_margin

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


def run_block(layer, x):
    out, ids, w = layer.block.forward(dev_f32(x), return_routing=True)
    return host(out), host(ids), host(w)


def oracle_check(orc, layer, x, out, ids, w, what, max_flips=None):
    spec = layer.spec
    logits = orc.route_logits(x, layer.router_t)
    oid, ow = orc.route_from_logits(logits, layer.bias, spec.top_k, spec.weights_scale, spec.weights_norm)
    margin = selection_margin(logits, layer.bias, spec.top_k)
    flips = check_ids(ids, oid, margin)
    if max_flips is not None:
        assert flips <= max_flips, f"{what}: {flips} near-tie tokens"
    same = np.all(ids == oid, axis=1)
    assert np.allclose(w[same], ow[same], rtol=1e-5, atol=1e-7), f"{what}: routing weights"
    want, _, _ = orc.moe_layer(spec, layer.keys, layer.router_t, layer.bias, x, ids=ids, w=w)
    return assert_close(out, want, what=what)


@pytest.mark.parametrize("name", ["C0", "C1"])
def test_decode_layer(dev, orc, name):
    cfg = CONFIGS[name]
    _log(f"{name} decode")
    layer = build_layer(cfg["spec"], seed=1000 + int(name[1]))
    for seed in range(3):
        x = make_x(cfg["spec"], 7 + seed, cfg["t"])
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"{name} seed={seed}", max_flips=0)


@pytest.mark.parametrize("t", [2, 4, 5, 16, 31])
def test_verify_block(dev, orc, t):
    """C2: speculative verify blocks below MM_ID_MIN_SEQ: t < 16 on the decode
    kernels ((token, slot) pairs walked in expert order), t = 16 and 31 on the
    16-pair MFMA tiles."""
    cfg = CONFIGS["C2"]
    _log(f"C2 t={t}")
    layer = build_layer(cfg["spec"], seed=1002)
    x = make_x(cfg["spec"], 11, t)
    out, ids, w = run_block(layer, x)
    oracle_check(orc, layer, x, out, ids, w, f"C2 t={t}", max_flips=1)


SWEEP_SPEC = LayerSpec(1024, 512, 64, 4, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True)


@pytest.mark.parametrize("t", [1, 2, 3, 15, 16, 17, 31, 32, 33, 63, 64, 65, 100, 128, 129, 300, 512, 513])
def test_t_sweep_across_path_boundaries(dev, orc, t):
    """One shared-expert layer (Q4_K gate/up, Q6_K down; hidden 1024, ff 512,
    64 experts, top-4 + shared: 5 slots) at every t on either side of the path
    boundaries: t = 1 (top-k in the gate/up blocks), 2..15 (mat-vecs in expert
    order), 16..512 (16-pair MFMA tiles, up to 2560 pairs), 129 and up (the
    unfused router), 513 and up (grouped GEMM), against the oracle."""
    _log(f"sweep t={t}")
    layer = build_layer(SWEEP_SPEC, seed=1020)
    x = make_x(SWEEP_SPEC, 40 + t, t)
    out, ids, w = run_block(layer, x)
    oracle_check(orc, layer, x, out, ids, w, f"sweep t={t}", max_flips=max(1, t // 16))


WIDE_SPEC = LayerSpec(7168, 2048, 64, 8, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True)


@pytest.mark.parametrize("t", [1, 4])
def test_wide_hidden_decode(dev, orc, t):
    """hidden 7168 (DeepSeek-shaped rows: 112 Q4_K groups): the generic gate/up
    kernel in its wide geometry (a whole wave per row, tail groups masked), at
    t = 1 and on the expert-ordered verify path, against the oracle."""
    _log(f"wide hidden t={t}")
    layer = build_layer(WIDE_SPEC, seed=1030)
    x = make_x(WIDE_SPEC, 60 + t, t)
    out, ids, w = run_block(layer, x)
    oracle_check(orc, layer, x, out, ids, w, f"wide t={t}", max_flips=1)


SHAPES = {
    "h2048_ff768_q4q6": LayerSpec(2048, 768, 64, 8, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True),
    "h5120_ff1536_q5q6": LayerSpec(5120, 1536, 32, 6, GgmlDType.Q5_K, GgmlDType.Q6_K, shared=True),
    "h3072_ff2048_q8q8": LayerSpec(3072, 2048, 32, 4, GgmlDType.Q8_0, GgmlDType.Q8_0, shared=False),
    "h6144_ff2816_q6q4": LayerSpec(6144, 2816, 16, 4, GgmlDType.Q6_K, GgmlDType.Q4_K, shared=True),
    "h7168_ff2048_q4q5": LayerSpec(7168, 2048, 32, 8, GgmlDType.Q4_K, GgmlDType.Q5_K, shared=False),
    # Q6_K down of ff 1536 with hidden not a multiple of 256 output rows: the
    # compiled down kernels' row tiles do not divide it, so it takes the generic one
    "h1056_ff1536_q8q6": LayerSpec(1056, 1536, 16, 4, GgmlDType.Q8_0, GgmlDType.Q6_K, shared=True),
}


@pytest.mark.parametrize("name", list(SHAPES))
@pytest.mark.parametrize("t", [1, 5])
def test_model_shapes(dev, orc, name, t):
    """Layer shapes beyond the Laguna one (hidden 2048 to 7168, ff 768 to 2816,
    mixed quant types, with and without a shared expert): whichever decode
    kernels, geometry and router each shape selects, against the oracle."""
    spec = SHAPES[name]
    _log(f"shape {name} t={t}")
    layer = build_layer(spec, seed=1040)
    x = make_x(spec, 70 + t, t)
    out, ids, w = run_block(layer, x)
    oracle_check(orc, layer, x, out, ids, w, f"{name} t={t}", max_flips=1)


def test_verify_block_no_shared(dev, orc):
    """Expert-ordered verify without a shared expert (C0 shape, t = 20)."""
    cfg = CONFIGS["C0"]
    _log("C0 t=20")
    layer = build_layer(cfg["spec"], seed=1010)
    x = make_x(cfg["spec"], 12, 20)
    out, ids, w = run_block(layer, x)
    oracle_check(orc, layer, x, out, ids, w, "C0 t=20", max_flips=1)


def test_prefill_grouped_gemm_small(dev, orc):
    """C3 layer at t = 96 (16-pair MFMA tiles) and t = 240 (the grouped GEMM, past
    the tiles' 2560 pairs) against the oracle."""
    cfg = CONFIGS["C3"]
    layer = build_layer(cfg["spec"], seed=1003)
    for t in (96, 240):
        _log(f"C3 t={t}")
        x = make_x(cfg["spec"], 13, t)
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"C3 t={t}", max_flips=2)


def test_prefill_full_size_all_rows(dev, orc):
    """C3 at its full size t = 2048 (skewed bias): every one of the 2048 output
    rows of the grouped-GEMM path is held to the contract's tolerance (rel-L2 and
    max-abs) against the oracle on the same routing, and every token's ids are
    checked against the oracle's own routing.  The decode path (mul_mv_id through
    the reference-shaped ops, same routing) is held to the same bar on all rows."""
    cfg = CONFIGS["C3"]
    spec = cfg["spec"]
    _log("C3 t=2048")
    layer = build_layer(spec, seed=1004)
    x = make_x(spec, 17, 2048)
    out, ids, w = run_block(layer, x)
    counts = np.bincount(ids.ravel(), minlength=spec.n_expert)
    assert counts.max() > 4 * counts.mean()  # the skewed bias really is imbalanced
    _log("C3 t=2048: oracle on all rows")
    want, _, _ = orc.moe_layer(spec, layer.keys, layer.router_t, layer.bias, x, ids=ids, w=w)
    assert_close(out, want, what="C3 all rows vs oracle")
    logits = orc.route_logits(x, layer.router_t)
    oid, _ = orc.route_from_logits(logits, layer.bias, spec.top_k, 1.0, True)
    check_ids(ids, oid, selection_margin(logits, layer.bias, spec.top_k))
    xd = dev_f32(x)
    # decode path on the same routing, through the reference-shaped ops
    gate, up, down = layer.block.experts.gate, layer.block.experts.up, layer.block.experts.down
    ids_d = torch.from_numpy(ids.astype(np.int64)).to(torch.int32).cuda().view(torch.uint32)
    w_d = dev_f32(w)
    xg = xd.reshape(2048, 1, -1)
    act = ops.silu_mul(ops.mul_mv_id(gate, xg, ids_d), ops.mul_mv_id(up, xg, ids_d))
    routed = ops.combine(ops.mul_mv_id(down, act, ids_d), None, w_d)
    mv = host(routed + layer.block.shared.forward(xd))
    assert_close(mv, want, what="C3 decode path (all rows) vs oracle")


@pytest.mark.parametrize("gate_dt,down_dt", [(GgmlDType.Q8_0, GgmlDType.Q8_0), (GgmlDType.Q6_K, GgmlDType.Q4_K),
                                             (GgmlDType.Q4_K, GgmlDType.Q8_0)], ids=["q8q8", "q6q4", "q4q8"])
def test_weight_types(dev, orc, gate_dt, down_dt):
    """Every weight type in both matrices: decode at t = 1 (per-slot down
    workgroups) and the grouped GEMM at t = 160 (the shared expert's pairs span
    two m-tiles, one partial; SwiGLU gate/up and plain down GEMM)."""
    spec = LayerSpec(768, 512, 32, 4, gate_dt, down_dt, shared=True)
    layer = build_layer(spec, seed=1040 + int(gate_dt) + int(down_dt))
    for t in (1, 160):
        _log(f"{gate_dt.name}/{down_dt.name} t={t}")
        x = make_x(spec, 41 + t, t)
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"{gate_dt.name}/{down_dt.name} t={t}", max_flips=1)


@pytest.mark.parametrize("gate_dt,down_dt", [(GgmlDType.Q5_K, GgmlDType.Q5_K), (GgmlDType.Q5_K, GgmlDType.Q6_K),
                                             (GgmlDType.Q4_K, GgmlDType.Q5_K)], ids=["q5q5", "q5q6", "q4q5"])
def test_q5_k_layers(dev, orc, gate_dt, down_dt):
    """Q5_K experts (the UD-Q4_K_XL mixes): decode (t = 1), expert-ordered verify
    (t = 12) and the grouped GEMM (t = 64), shared expert included."""
    spec = LayerSpec(1024, 512, 64, 6, gate_dt, down_dt, shared=True)
    layer = build_layer(spec, seed=1020 + int(gate_dt) + int(down_dt))
    for t in (1, 12, 64):
        _log(f"q5 {gate_dt.name}/{down_dt.name} t={t}")
        x = make_x(spec, 31 + t, t)
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"{gate_dt.name}/{down_dt.name} t={t}", max_flips=1)


def test_fused_experts_ops_match_block(dev, orc):
    """FusedExperts composed from the individual ops == the block's fused kernels."""
    spec = LayerSpec(1024, 512, 64, 4, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=False)
    layer = build_layer(spec, seed=1005)
    for t in (1, 40):
        _log(f"fused-vs-ops t={t}")
        x = make_x(spec, 19 + t, t)
        out, ids, w = run_block(layer, x)
        fe = layer.block.experts
        ids_d = torch.from_numpy(ids.astype(np.int64)).to(torch.int32).cuda().view(torch.uint32)
        got = host(FusedExperts(fe.gate, fe.up, fe.down).forward(dev_f32(x), ids_d, dev_f32(w)))
        assert_close(got, out, rel=2e-6 if t == 1 else 1e-3, what=f"ops vs block t={t}")


def test_chain_with_rmsnorm_and_residual(dev, orc):
    """C4 shape on 3 layers: x <- x + MoE(RMSNorm(x)) per layer (model.rs:340-351)."""
    spec = CONFIGS["C4"]["spec"]
    layers = [build_layer(spec, seed=2000, layer=i, rms=True) for i in range(3)]
    x0 = make_x(spec, 23, 1)
    xd = dev_f32(x0)
    for i, L in enumerate(layers):
        _log(f"chain layer {i}")
        L.block.forward(xd, residual=xd, out=xd)
    got = host(xd)
    x = x0.copy()
    for L in layers:
        xn = orc.rmsnorm(x, np.ones(spec.hidden, np.float32), 1e-6)
        y, _, _ = orc.moe_layer(spec, L.keys, L.router_t, L.bias, xn)
        x = (x + y).astype(np.float32)
    assert_close(got, x, what="3-layer chain")


def test_rmsnorm_verify_tiles(dev, orc):
    """A 20-token block with the FFN RMSNorm on the MFMA verify tiles: the f16 x
    rows come from the normalised rows (a separate conversion after the router,
    which writes them), not from the router's own f16 rows."""
    spec = CONFIGS["C4"]["spec"]
    layer = build_layer(spec, seed=2001, rms=True)
    x = make_x(spec, 24, 20)
    out, ids, w = layer.block.forward(dev_f32(x), residual=dev_f32(x), return_routing=True)
    out, ids, w = host(out), host(ids), host(w)
    xn = orc.rmsnorm(x, np.ones(spec.hidden, np.float32), 1e-6)
    logits = orc.route_logits(xn, layer.router_t)
    oid, _ = orc.route_from_logits(logits, layer.bias, spec.top_k, spec.weights_scale, spec.weights_norm)
    assert check_ids(ids, oid, selection_margin(logits, layer.bias, spec.top_k)) <= 1
    y, _, _ = orc.moe_layer(spec, layer.keys, layer.router_t, layer.bias, xn, ids=ids, w=w)
    assert_close(out, (x + y).astype(np.float32), what="rmsnorm verify t=20")


def test_wide_rows(dev, orc):
    """hidden = 5120 and ff = 2304: Q4_K rows too wide for the fused decode
    kernels' LDS ring.  Decode (t = 1) and verify (t = 6) take the f32 gather
    mat-vec path, chosen before any launch; the grouped GEMM (t = 48) converts
    rows to f16 in its any-width form (k > 4096) and the partial register-cached
    form (ff = 2304)."""
    spec = LayerSpec(5120, 2304, 16, 4, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True)
    layer = build_layer(spec, seed=1041)
    for t in (1, 6, 48):
        _log(f"wide rows t={t}")
        x = make_x(spec, 57 + t, t)
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"wide rows t={t}", max_flips=1)


def test_decode_in_block_topk_odd_expert_count(dev, orc):
    """t = 1 with 4096-wide Q4_K gate/up rows: the gate/up blocks run the top-k
    themselves (no k_decode_select launch) and one of them writes ids and weights.
    100 experts leave a partial group of 8 in the pruned selection; scale 2.5."""
    spec = LayerSpec(4096, 512, 100, 8, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True, weights_scale=2.5)
    layer = build_layer(spec, seed=1071)
    for seed in range(3):
        _log(f"in-block top-k seed={seed}")
        x = make_x(spec, 81 + seed, 1)
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"in-block top-k seed={seed}", max_flips=0)


def test_prefill_ragged_router_tiles(dev, orc):
    """Prefill at t = 500 with 96 experts (3000 pairs: the grouped GEMM): the
    MFMA router's 32-token and 64-expert tiles and the GEMM's m-tiles are all
    left partly filled."""
    spec = LayerSpec(1024, 512, 96, 6, GgmlDType.Q4_K, GgmlDType.Q4_K, shared=False)
    layer = build_layer(spec, seed=1061)
    _log("ragged prefill t=500")
    x = make_x(spec, 71, 500)
    out, ids, w = run_block(layer, x)
    oracle_check(orc, layer, x, out, ids, w, "ragged prefill t=500", max_flips=3)


def test_laguna_geometry(dev, orc):
    """The shipped Laguna layer geometry (reference/config.json: hidden 3072,
    moe_intermediate_size 1024, shared_expert_intermediate_size 1024, 256 experts,
    top-10) with the GGUF's expert_weights_scale 2.5 and norm on.  ff = 1024 has 32
    Q4_K groups per gate/up row and 4 Q6_K blocks per down row, so decode takes the
    generic slot kernels (not the ff = 1536 compile-time forms); t = 6 is a
    verify block on them, t = 16 and 64 run the MFMA verify tiles and t = 240
    the grouped GEMM."""
    spec = LayerSpec(3072, 1024, 256, 10, GgmlDType.Q4_K, GgmlDType.Q6_K, shared=True, weights_scale=2.5)
    layer = build_layer(spec, seed=1051)
    for t in (1, 6, 16, 64, 240):
        _log(f"laguna geometry t={t}")
        x = make_x(spec, 61 + t, t)
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"laguna t={t}", max_flips=2)


def test_chain_full_depth_48_layers(dev, orc):
    """C4 at its stated depth: 48 C1-shaped layers, x <- x + MoE(RMSNorm(x))
    (model.rs:340-351), each layer built, run and freed in turn on the GPU while
    the oracle steps the same chain on the host.  Per layer the expert ids must
    match the oracle's own routing of its own x (near-ties excepted); the oracle
    then steps with the GPU's routing so a flip cannot cascade.  The final
    residual stream is held to the contract tolerance."""
    spec = CONFIGS["C4"]["spec"]
    x0 = make_x(spec, 23, 1)
    xd = dev_f32(x0)
    x = x0.copy()
    ones = np.ones(spec.hidden, np.float32)
    flips = 0
    for i in range(48):
        L = build_layer(spec, seed=2000, layer=i, rms=True)
        out, ids, w = L.block.forward(xd, residual=xd, out=xd, return_routing=True)
        ids, w = host(ids), host(w)
        xn = orc.rmsnorm(x, ones, 1e-6)
        logits = orc.route_logits(xn, L.router_t)
        oid, _ = orc.route_from_logits(logits, L.bias, spec.top_k, 1.0, True)
        flips += check_ids(ids, oid, selection_margin(logits, L.bias, spec.top_k))
        y, _, _ = orc.moe_layer(spec, L.keys, L.router_t, L.bias, xn, ids=ids, w=w)
        x = (x + y).astype(np.float32)
        if i % 8 == 7:
            _log(f"chain layer {i}: rel-L2 so far {rel_l2(host(xd), x):.2e}")
        del L
    assert flips <= 1
    assert_close(host(xd), x, what="48-layer chain")


def test_decode_down_compiled_shape_matches_generic(dev):
    """The C1 shape's down rows (Q6_K, expert_ff 1536, 16-byte-aligned stacks) run
    a kernel with compile-time geometry; the same weights placed 2 bytes off
    16-byte alignment (Q6_K needs 2) take the generic slot-per-wave kernel.  Both
    perform the same operations in the same order, so the outputs must be
    bit-identical (t = 1 and 3: the slot-per-wave path; t = 6 and 12: the
    per-(slot, row tile) verify path).  At t = 16 both run the MFMA verify tiles,
    whose Q6_K copies take the 16-byte span around each block: the 2-byte offset
    moves the expert's last block across a chunk boundary, and the results must
    not change."""
    from maxuna_amd.gguf import ExpertStack
    from maxuna_amd.moe import MoeBlock, SharedExpert

    spec = CONFIGS["C1"]["spec"]
    layer = build_layer(spec, seed=1077)
    blk = layer.block

    def shifted(st):
        buf = torch.empty(st.nbytes + 16, dtype=torch.uint8, device=st.buffer.device)
        buf[2:2 + st.nbytes].copy_(st.buffer[st.base_off:st.base_off + st.nbytes])
        return ExpertStack(buf, st.dtype, st.n_expert, st.n_out, st.k, base_off=2)

    e, sh = blk.experts, blk.shared
    other = MoeBlock(blk.router, blk.exp_probs_b, e.gate, e.up, shifted(e.down), blk.cfg,
                     shared=SharedExpert(sh.gate, sh.up, shifted(sh.down)))
    for t in (1, 3, 6, 12, 16):
        x = dev_f32(make_x(spec, 300 + t, t))
        a = host(blk.forward(x))
        b = host(other.forward(x))
        _log(f"down compiled vs generic t={t}: max |diff| {np.abs(a - b).max()}")
        assert np.array_equal(a, b), f"t={t}: compiled-shape down kernel differs from the generic kernel"


def test_workspace_contents_do_not_matter(dev):
    """The workspace carries no state between calls: a forward whose workspace
    was filled with 0xFF bytes, or with random bytes, is bit-identical to one
    whose workspace was zeroed -- for a decode token (t = 1), MFMA verify tiles
    (t = 16, and t = 64 past mm_min_seq) and a grouped-GEMM block (t = 240)."""
    spec = CONFIGS["C2"]["spec"]
    layer = build_layer(spec, seed=1305)
    blk = layer.block
    gen = torch.Generator(device="cuda").manual_seed(5)
    for t in (1, 16, 64, 240):
        _log(f"workspace fill t={t}")
        x = dev_f32(make_x(spec, 700 + t, t))
        ws = blk.workspace(t, x.device)
        ws.zero_()
        want, wid, ww = blk.forward(x, return_routing=True)
        for fill in ("ff", "random"):
            if fill == "ff":
                ws.fill_(0xFF)
            else:
                ws.copy_(torch.randint(0, 256, ws.shape, dtype=torch.uint8, device=x.device, generator=gen))
            got, gid, gw = blk.forward(x, return_routing=True)
            assert np.array_equal(host(got).view(np.uint32), host(want).view(np.uint32)), f"t={t} {fill}: out"
            assert np.array_equal(host(gid), host(wid)), f"t={t} {fill}: ids"
            assert np.array_equal(host(gw).view(np.uint32), host(ww).view(np.uint32)), f"t={t} {fill}: w"


def test_decode_down_q6_hidden_off_the_verify_tile(dev, orc):
    """Q6_K down rows of expert_ff 1536 at a hidden that is a multiple of the
    16-row tile but not of the verify kernel's 256-row tile (Q8_0 gate/up rows
    allow hidden = 1056): t > 4 must take the generic down kernel, checked
    against the oracle."""
    spec = LayerSpec(1056, 1536, 16, 4, GgmlDType.Q8_0, GgmlDType.Q6_K, shared=True)
    layer = build_layer(spec, seed=1306)
    for t in (6, 12):
        _log(f"hidden 1056 Q6_K down t={t}")
        x = make_x(spec, 800 + t, t)
        out, ids, w = run_block(layer, x)
        oracle_check(orc, layer, x, out, ids, w, f"hidden 1056 t={t}")


def test_router_expert_groups_bit_identical(dev):
    """Blocks of more than 4 tokens run the fused router with four experts per
    workgroup (the token rows loaded once for four router rows); every logit is
    the same sum in the same order, so the routing of the first tokens must be
    bit-identical to a 4-token block's (one expert per workgroup)."""
    spec = CONFIGS["C2"]["spec"]
    layer = build_layer(spec, seed=1003)
    x = make_x(spec, 21, 16)
    _, ids16, w16 = run_block(layer, x)
    _, ids4, w4 = run_block(layer, x[:4])
    assert np.array_equal(ids16[:4], ids4)
    assert np.array_equal(w16[:4].view(np.uint32), w4.view(np.uint32))
