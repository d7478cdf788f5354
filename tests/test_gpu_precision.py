"""Activation precision of the decode kernels, wide rows, and id validation.

The decode kernels carry each activation value on a 24-bit grid per scale group
-- the aligned 128-value block (32-value group when k % 128 != 0) -- with a
power-of-two scale, three int8 digit planes and exact int32 plane sums: every
value to within 2^-23 * (1 + 2^-8) of its group's largest magnitude.
That is the width of the reference's f32 `y` (mv.metal:227-275), so the
decode outputs match the f32 oracle to f32-class error -- well inside the
contract's rel-L2 1e-3 -- also when a group holds a large outlier channel next
to unit-scale values, the case a block grid handles worst.  The tests below
assert rel-L2 <= 2e-6 (a 16-bit grid misses that by an order of magnitude on
the outlier inputs) and the contract bound on whole layers.  Verify blocks of
16 to 31 tokens run the 16-pair MFMA tiles instead (f16 operands, like the
grouped GEMM): those are held to the contract bound.
"""
import numpy as np
import pytest
import torch

from maxuna_amd import ops
from maxuna_amd.gguf import GgmlDType
from maxuna_amd.synth import CONFIGS, LayerSpec, build_layer, make_x
from tests.gpu_util import assert_close, check_ids, dev_f32, dev_u32, host, rel_l2, selection_margin, upload_stack

pytestmark = pytest.mark.gpu

DTYPES = [GgmlDType.Q4_K, GgmlDType.Q5_K, GgmlDType.Q6_K, GgmlDType.Q8_0]
F32_CLASS = 2e-6


def _log(msg):
    print(msg, flush=True)


def outlier_x(rng, shape, factor=1000.0):
    """N(0,1) values with one channel per 32-value group scaled by `factor`."""
    x = rng.standard_normal(shape).astype(np.float32)
    k = shape[-1]
    ch = np.arange(0, k, 32) + (np.arange(k // 32) * 7) % 32
    x[..., ch] *= np.float32(factor)
    return x


def _stack(orc, dt, n_expert, n_out, k, seed):
    blocks = {e: orc.expert_blocks(int(dt), seed, e, n_out, k) for e in range(n_expert)}
    return blocks, upload_stack(dt, blocks, n_expert, n_out, k)


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: d.name)
@pytest.mark.parametrize("kind", ["normal", "outlier", "tiny_and_huge"])
def test_mv_id_f32_class_accuracy(dev, orc, dt, kind):
    """mul_mv_id (LDS-ring kernel, k = 1536 and 4096) against the f32 oracle."""
    rng = np.random.default_rng(7)
    for k in (1536, 4096):
        _log(f"mv_id precision {dt.name} {kind} k={k}")
        blocks, st = _stack(orc, dt, 8, 96, k, 0xA11 + k)
        shape = (2, 4, k)
        if kind == "normal":
            x = rng.standard_normal(shape).astype(np.float32)
        elif kind == "outlier":
            x = outlier_x(rng, shape)
        else:  # groups spanning many binades, plus an all-zero group and a denormal-scale group
            x = (rng.standard_normal(shape) * np.exp2(rng.integers(-40, 40, shape))).astype(np.float32)
            x[..., :32] = 0.0
            x[..., 32:64] = rng.standard_normal(32).astype(np.float32) * np.float32(1e-41)
        ids = np.stack([rng.choice(8, 4, replace=False) for _ in range(2)]).astype(np.uint32)
        got = host(ops.mul_mv_id(st, dev_f32(x), dev_u32(ids)))
        want = orc.mul_mv_id(int(dt), blocks, 8, 96, k, x, ids)
        r = rel_l2(got, want)
        _log(f"  rel-L2 {r:.2e}")
        assert r <= F32_CLASS, f"{dt.name} {kind} k={k}: rel-L2 {r:.3e}"


def test_decode_layer_outlier_channels(dev, orc):
    """C1 layer at t = 1 and a verify block at t = 12 (both on the decode kernels)
    with one channel x1000 per 32-group: f32-class agreement with the oracle (same
    routing)."""
    spec = CONFIGS["C1"]["spec"]
    layer = build_layer(spec, seed=1101)
    rng = np.random.default_rng(11)
    for t in (1, 12):
        _log(f"C1 outlier t={t}")
        x = outlier_x(rng, (t, spec.hidden))
        out, ids, w = layer.block.forward(dev_f32(x), return_routing=True)
        out, ids, w = host(out), host(ids), host(w)
        logits = orc.route_logits(x, layer.router_t)
        oid, _ = orc.route_from_logits(logits, layer.bias, spec.top_k, 1.0, True)
        check_ids(ids, oid, selection_margin(logits, layer.bias, spec.top_k))
        want, _, _ = orc.moe_layer(spec, layer.keys, layer.router_t, layer.bias, x, ids=ids, w=w)
        assert_close(out, want, what=f"C1 outlier t={t}")
        r = rel_l2(out, want)
        assert r <= 1e-5, f"t={t}: rel-L2 {r:.3e} is not f32-class"


@pytest.mark.parametrize("dt,k", [(GgmlDType.Q4_K, 5120), (GgmlDType.Q6_K, 20480), (GgmlDType.Q8_0, 24576)],
                         ids=["q4k-5120", "q6k-20480", "q8-24576"])
def test_mv_id_wide_rows(dev, orc, dt, k):
    """Rows wider than the LDS-ring kernel holds take the f32 mat-vec (any k)."""
    _log(f"mv_id wide {dt.name} k={k}")
    rng = np.random.default_rng(k)
    blocks, st = _stack(orc, dt, 3, 40, k, 0xB0 + k)
    x = rng.standard_normal((2, 1, k)).astype(np.float32)
    ids = np.array([[2, 0], [1, 2]], np.uint32)
    got = host(ops.mul_mv_id(st, dev_f32(x), dev_u32(ids)))
    want = orc.mul_mv_id(int(dt), blocks, 3, 40, k, x, ids)
    assert rel_l2(got, want) <= F32_CLASS


def test_workspace_reuse_across_t(dev, orc):
    """One block's workspace serves calls of any t in any order: a grouped-GEMM
    call (t = 240), MFMA verify tiles (t = 64) and then verify blocks on the
    decode kernels (t = 12, 3) must each match the oracle."""
    spec = CONFIGS["C2"]["spec"]
    layer = build_layer(spec, seed=1102)
    for t, seed in ((240, 1), (64, 5), (12, 2), (3, 3), (12, 4)):
        _log(f"workspace reuse t={t}")
        x = make_x(spec, 300 + seed, t)
        out, ids, w = layer.block.forward(dev_f32(x), return_routing=True)
        out, ids, w = host(out), host(ids), host(w)
        want, _, _ = orc.moe_layer(spec, layer.keys, layer.router_t, layer.bias, x, ids=ids, w=w)
        assert_close(out, want, what=f"reuse t={t}")


def test_check_ids(dev):
    _log("check_ids")
    ok = np.array([[0, 1, 2], [3, 4, 5]], np.uint32)
    assert ops.check_ids(dev_u32(ok), 8) == 0
    dup = np.array([[0, 1, 0], [3, 4, 5]], np.uint32)
    assert ops.check_ids(dev_u32(dup), 8, raise_on_error=False) == ops.IDS_DUPLICATE
    oor = np.array([[0, 1, 2], [3, 8, 5]], np.uint32)
    assert ops.check_ids(dev_u32(oor), 8, raise_on_error=False) == ops.IDS_OUT_OF_RANGE
    both = np.array([[9, 9, 2]] * 3000, np.uint32)
    assert ops.check_ids(dev_u32(both), 8, raise_on_error=False) == 3
    with pytest.raises(ops.MaxunaError, match="repeats an expert id"):
        ops.check_ids(dev_u32(dup), 8)
    # beyond 65536 pairs the check runs as a grid of blocks: clean ids, then one bad
    # token near the end of each kind (the flag word is cleared by the call itself)
    rng = np.random.default_rng(3)
    big = np.stack([rng.choice(64, 8, replace=False) for _ in range(20000)]).astype(np.uint32)
    assert ops.check_ids(dev_u32(big), 64) == 0
    for row, bad, want in ((19_999, [5, 5, 1, 2, 3, 4, 6, 7], ops.IDS_DUPLICATE),
                           (17_123, [0, 1, 2, 3, 4, 5, 6, 64], ops.IDS_OUT_OF_RANGE)):
        b2 = big.copy()
        b2[row] = bad
        assert ops.check_ids(dev_u32(b2), 64, raise_on_error=False) == want
    assert ops.check_ids(dev_u32(big), 64) == 0


def test_verify_tiles_outlier_channels(dev, orc):
    """Verify blocks of 16 and 31 tokens run the 16-pair MFMA tiles (f16 operands,
    per-row power-of-two scales, like the grouped GEMM): the contract bound on the
    outlier inputs, not f32-class."""
    spec = CONFIGS["C1"]["spec"]
    layer = build_layer(spec, seed=1101)
    rng = np.random.default_rng(12)
    for t in (16, 31):
        _log(f"C1 outlier verify tiles t={t}")
        x = outlier_x(rng, (t, spec.hidden))
        out, ids, w = layer.block.forward(dev_f32(x), return_routing=True)
        out, ids, w = host(out), host(ids), host(w)
        logits = orc.route_logits(x, layer.router_t)
        oid, _ = orc.route_from_logits(logits, layer.bias, spec.top_k, 1.0, True)
        check_ids(ids, oid, selection_margin(logits, layer.bias, spec.top_k))
        want, _, _ = orc.moe_layer(spec, layer.keys, layer.router_t, layer.bias, x, ids=ids, w=w)
        r = assert_close(out, want, what=f"C1 outlier verify tiles t={t}")
        _log(f"  {r}")


def test_no_mm_id_keeps_verify_blocks_on_the_mat_vecs(dev, orc):
    """mm_min_seq < 0 (LAGUNA_NO_MM_ID: mul_mv_id everywhere, ops/mod.rs:57-64)
    keeps a 16-token block on the decode kernels: f32-class again."""
    spec = CONFIGS["C1"]["spec"]
    layer = build_layer(spec, seed=1101)
    layer.block._c.mm_min_seq = -1
    rng = np.random.default_rng(13)
    x = outlier_x(rng, (16, spec.hidden))
    out, ids, w = layer.block.forward(dev_f32(x), return_routing=True)
    out, ids, w = host(out), host(ids), host(w)
    want, _, _ = orc.moe_layer(spec, layer.keys, layer.router_t, layer.bias, x, ids=ids, w=w)
    r = rel_l2(out, want)
    _log(f"no-mm-id t=16: rel-L2 {r:.2e}")
    assert r <= 1e-5, f"rel-L2 {r:.3e} is not f32-class"
