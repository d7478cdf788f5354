"""GPU parity of the individual kernels against the CPU oracle (same seeded inputs).

Integer/byte/index work is compared bit-exactly (synthetic blocks, dequantised
values, expert ids and order, bucket lists); floating-point outputs to the
contract tolerance rel-L2 <= 1e-3 and max-abs <= 1e-2 * rms(out).
"""
import numpy as np
import pytest
import torch

from maxuna_amd import ops
from maxuna_amd.gguf import ExpertStack, GgmlDType
from maxuna_amd.synth import synth_stack
from tests._pack import pack_q4_k, pack_q6_k, pack_q8_0
from tests.gpu_util import (assert_close, dev_f32, dev_u32, host, rel_l2, upload_stack)

pytestmark = pytest.mark.gpu

DTYPES = [GgmlDType.Q4_K, GgmlDType.Q5_K, GgmlDType.Q6_K, GgmlDType.Q8_0]


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: d.name)
def test_synth_blocks_match_oracle(dev, orc, dt):
    _log(f"synth {dt.name}")
    key = 0x1234_5678_9ABC
    st = synth_stack(dt, 5, 24, 512, key)
    got = host(st.buffer)
    want = orc.synth_bytes(int(dt), key, 0, st.nbytes)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: d.name)
def test_dequantize_bit_exact(dev, orc, dt):
    _log(f"dequant {dt.name}")
    n = 64 * 1024
    st = synth_stack(dt, 1, n // 1024, 1024, 99)
    got = host(ops.dequantize(st.buffer, dt, n))
    want = orc.dequantize(int(dt), host(st.buffer), n)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # encoder-built blocks with known closed forms, incl. high-bit scales and q = 32 (Q6_K)
    rng = np.random.default_rng(0)
    if dt is GgmlDType.Q4_K:
        blk = np.concatenate([pack_q4_k(0.0123, 0.0071, [int(v) for v in rng.integers(0, 64, 8)],
                                        [int(v) for v in rng.integers(0, 64, 8)], rng.integers(0, 16, 256))
                              for _ in range(8)])
        nw = 8 * 256
    elif dt is GgmlDType.Q6_K:
        blk = np.concatenate([pack_q6_k(0.0123, [int(v) for v in rng.integers(-128, 128, 16)],
                                        rng.integers(0, 64, 256)) for _ in range(8)])
        nw = 8 * 256
    else:
        blk = np.concatenate([pack_q8_0(0.0123, rng.integers(-128, 128, 32)) for _ in range(8)])
        nw = 8 * 32
    got = host(ops.dequantize(torch.from_numpy(blk).cuda(), dt, nw))
    want = orc.dequantize(int(dt), blk, nw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _mv_case(orc, dt, n_expert, n_out, k, t, top_k, xpr, ids, seed, base_off=0):
    rng = np.random.default_rng(seed)
    key = int(rng.integers(0, 2**62))
    blocks = {e: orc.expert_blocks(int(dt), key, e, n_out, k) for e in range(n_expert)}
    st = upload_stack(dt, blocks, n_expert, n_out, k, base_off=base_off)
    x = rng.uniform(-1, 1, (t, xpr, k)).astype(np.float32)
    got = host(ops.mul_mv_id(st, dev_f32(x), dev_u32(ids)))
    want = orc.mul_mv_id(int(dt), blocks, n_expert, n_out, k, x, ids)
    return got, want, st, x, blocks


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: d.name)
def test_mul_mv_id_shared_and_per_slot(dev, orc, dt):
    rng = np.random.default_rng(1)
    for (t, top_k, xpr) in [(3, 2, 1), (5, 4, 4)]:
        _log(f"mv_id {dt.name} t={t} k={top_k} xpr={xpr}")
        ids = rng.integers(0, 4, (t, top_k)).astype(np.uint32)
        got, want, *_ = _mv_case(orc, dt, 4, 8, 256, t, top_k, xpr, ids, 0x100 + t)
        assert_close(got, want, what=f"{dt.name} xpr={xpr}")


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: d.name)
def test_mul_mv_id_repeated_ids_ragged_rows(dev, orc, dt):
    _log(f"mv_id ragged {dt.name}")
    ids = np.ones((4, 3), np.uint32)
    got, want, *_ = _mv_case(orc, dt, 4, 8, 256, 4, 3, 1, ids, 0x300)
    assert_close(got, want, what="repeated ids")
    # n_out = 100 (ragged tail), k = 512 (two super-blocks), nonzero base_off
    rng = np.random.default_rng(2)
    ids = rng.integers(0, 3, (2, 2)).astype(np.uint32)
    got, want, *_ = _mv_case(orc, dt, 3, 100, 512, 2, 2, 2, ids, 0x400, base_off=16 if dt in (GgmlDType.Q4_K, GgmlDType.Q5_K) else 2)
    assert_close(got, want, what="ragged")


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: d.name)
@pytest.mark.parametrize("k", [1024, 1536, 4096])
def test_mul_mv_id_production_widths(dev, orc, dt, k):
    _log(f"mv_id widths {dt.name} k={k}")
    rng = np.random.default_rng(k)
    ids = np.stack([rng.choice(16, 10, replace=False) for _ in range(2)]).astype(np.uint32)
    got, want, *_ = _mv_case(orc, dt, 16, 200, k, 2, 10, 10, ids, k)
    assert_close(got, want, what=f"k={k}")


def test_mul_mv_plain(dev, orc):
    _log("mul_mv")
    rng = np.random.default_rng(3)
    dt = GgmlDType.Q6_K
    blk = orc.expert_blocks(int(dt), 555, 0, 300, 768)
    x = rng.standard_normal((3, 768)).astype(np.float32)
    got = host(ops.mul_mv(torch.from_numpy(blk).cuda(), dt, 300, 768, dev_f32(x)))
    w = orc.dequantize(int(dt), blk, 300 * 768).reshape(300, 768).astype(np.float64)
    assert_close(got, x.astype(np.float64) @ w.T, what="mul_mv")


def test_mul_mv_q6_compiled_rows(dev, orc):
    """Q6_K rows of k = 1536, 2048, 3072 (the lm_head width) and 4096 take the
    compile-time mat-vec when n_out is a whole number of row batches.  Checked
    against the oracle, and against the generic LDS-ring kernel on the same rows
    (one more row makes n_out odd, which selects the generic kernel): bit-identical
    where both use the same lane geometry (k = 1536, 3072)."""
    rng = np.random.default_rng(31)
    dt = GgmlDType.Q6_K
    for k, n in ((3072, 1000), (1536, 500), (4096, 260), (2048, 300)):
        _log(f"mul_mv q6 k={k} n={n}")
        rb = k // 256 * 210
        blk = orc.expert_blocks(int(dt), 777 + k, 0, n + 1, k)
        x = rng.standard_normal((2, k)).astype(np.float32)
        got = host(ops.mul_mv(torch.from_numpy(blk[: n * rb].copy()).cuda(), dt, n, k, dev_f32(x)))
        gen = host(ops.mul_mv(torch.from_numpy(blk).cuda(), dt, n + 1, k, dev_f32(x)))[:, :n]
        w = orc.dequantize(int(dt), blk, (n + 1) * k).reshape(n + 1, k)[:n].astype(np.float64)
        want = x.astype(np.float64) @ w.T
        assert_close(got, want, what=f"mul_mv q6 k={k}")
        assert_close(gen, want, what=f"mul_mv generic k={k}")
        if k in (1536, 3072):
            assert np.array_equal(got.view(np.uint32), gen.view(np.uint32)), f"k={k}: compiled != generic"


def test_route_from_logits_bit_exact(dev, orc):
    _log("route_from_logits")
    rng = np.random.default_rng(4)
    t, E, K = 96, 256, 10
    logits = rng.standard_normal((t, E)).astype(np.float32)
    logits[:8, 20:40] = logits[:8, 5:6]  # exact ties -> lower index first
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    bias[20:40] = bias[5]
    for scale, norm in [(1.0, True), (2.5, True), (1.0, False)]:
        ids, w = ops.route_from_logits(dev_f32(logits), dev_f32(bias), K, scale, norm)
        oid, ow = orc.route_from_logits(logits, bias, K, scale, norm)
        assert np.array_equal(host(ids), oid)
        assert np.allclose(host(w), ow, rtol=2e-6, atol=0)


def test_route_pruned_topk_edge_cases(dev, orc):
    """The pruned top-k (group maxima -> threshold -> candidate ranks) against a
    full stable sort: expert counts that are not multiples of the 8-expert
    group, fewer groups than top_k, top_k = 32, heavy ties, -0.0 / +0.0."""
    rng = np.random.default_rng(44)
    for E, K in [(20, 7), (37, 17), (8, 8), (1000, 32), (1024, 1), (256, 10), (64, 32)]:
        _log(f"pruned top-k E={E} K={K}")
        t = 24
        logits = rng.standard_normal((t, E)).astype(np.float32)
        logits[:6] = np.round(logits[:6] * 2) / 2  # many exact ties
        logits[6:9] = 0.25  # every score tied
        logits[9, : E // 2] = -0.0
        logits[9, E // 2:] = 0.0
        bias = np.zeros(E, np.float32)
        if E > 16:
            bias[: E // 3] = (rng.standard_normal(E // 3) * 0.1).astype(np.float32)
        ids, w = ops.route_from_logits(dev_f32(logits), dev_f32(bias), K, 1.0, True)
        oid, ow = orc.route_from_logits(logits, bias, K, 1.0, True)
        assert np.array_equal(host(ids), oid), (E, K)
        assert np.allclose(host(w), ow, rtol=2e-6, atol=0)
        # all scores tied: the order is the bias order, ties -> lower id
        p = np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-0.25)))
        want6 = np.argsort(-(p + bias), kind="stable")[:K]
        assert host(ids)[6].tolist() == want6.tolist()


def test_route_kats_on_device(dev, orc):
    """The reference's routing known-answer tests (moe.rs:405-484) on the GPU."""
    row = np.array([[2.0, -2.0, 0.0, 1.0, -1.0, 3.0, 0.5, -0.5]], np.float32)
    cases = [([0, 0, 0, 0, 0, 0, 0.2, 0], [5, 0, 6]), ([0, 0, 0, 0, 0, -1.0, 0, 0], [0, 3, 6])]
    for bias, exp in cases:
        ids, _ = ops.route_from_logits(dev_f32(row), dev_f32(np.array(bias, np.float32)), 3, 2.5, True)
        assert host(ids).tolist() == [exp]
    ids, _ = ops.route_from_logits(dev_f32(np.zeros((1, 8), np.float32)), dev_f32(np.zeros(8, np.float32)), 3, 2.5, True)
    assert host(ids).tolist() == [[0, 1, 2]]
    _, w = ops.route_from_logits(dev_f32(np.full((1, 8), -30.0, np.float32)), dev_f32(np.zeros(8, np.float32)), 3,
                                 2.5, True)
    p = 1.0 / (1.0 + np.exp(30.0))
    assert np.allclose(host(w), p / 6.103515625e-5 * 2.5, rtol=1e-3)


def test_route_logits(dev, orc):
    """t < 8: one block per expert (t = 1 and 7, hidden 7168 as well); t >= 8 with
    hidden % 128 == 0: the LDS-staged MFMA kernel; hidden 1040 (% 16 only): the
    register-fed MFMA kernel (the two MFMA kernels form the same sums in the same
    order); hidden 1036 at t = 9: the tiled f32 kernel."""
    _log("route_logits")
    rng = np.random.default_rng(5)
    for t, hidden, n_expert in ((1, 1024, 256), (1, 7168, 256), (7, 4096, 64), (70, 1024, 256), (45, 1040, 100),
                                (45, 1024, 100), (9, 1036, 60)):
        x = rng.standard_normal((t, hidden)).astype(np.float32)
        r = (rng.standard_normal((n_expert, hidden)) * 0.02).astype(np.float32)  # [n_expert, hidden]
        got = host(ops.route_logits(dev_f32(r), dev_f32(x)))
        assert_close(got, orc.route_logits(x, np.ascontiguousarray(r.T)), rel=1e-5, what=f"logits t={t} h={hidden}")


def _distinct_ids(rng, t, k, E):
    return np.stack([rng.choice(E, k, replace=False) for _ in range(t)]).astype(np.uint32)


def test_map0_matches_oracle(dev, orc):
    rng = np.random.default_rng(6)
    # E = 2000 takes the scan fallback of the fill pass (slot table too large for LDS)
    for t, k, E in [(1, 4, 64), (48, 10, 32), (300, 10, 256), (2048, 10, 256), (8192, 2, 296), (9000, 3, 64),
                    (70, 8, 300), (50, 20, 64), (100, 4, 2000)]:
        _log(f"map0 t={t} k={k} E={E}")
        ids = _distinct_ids(rng, t, k, E)
        m = ops.prepare_map0(E, dev_u32(ids))
        tpe, hids = orc.map0(ids, E)
        assert np.array_equal(host(m.counts()), tpe)
        offs = host(m.offsets())
        lst = host(m.pair_list())
        assert offs[-1] == t * k
        for e in range(E):
            assert np.array_equal(lst[offs[e]:offs[e + 1]], hids[e, :tpe[e]]), e
        assert m.dup_flag() == 0
    for E in (4, 2000):  # both fill passes flag a repeated id (1) and an out-of-range id (2)
        ids = np.array([[1, 1, 2]], np.uint32)
        assert ops.prepare_map0(E, dev_u32(ids)).dup_flag() == 1
        ids = np.array([[0, 2], [3, E]], np.uint32)
        m = ops.prepare_map0(E, dev_u32(ids))
        assert m.dup_flag() == 2
        assert np.array_equal(host(m.pair_list())[:3], [0, 1, 2])  # the bad pair (token 1, slot 1) is dropped


@pytest.mark.parametrize("dt", DTYPES, ids=lambda d: d.name)
def test_mul_mm_id_matches_oracle(dev, orc, dt):
    rng = np.random.default_rng(7)
    n_expert, n_out, k = 16, 96, 512
    key = int(rng.integers(0, 2**62))
    blocks = {e: orc.expert_blocks(int(dt), key, e, n_out, k) for e in range(n_expert)}
    st = upload_stack(dt, blocks, n_expert, n_out, k)
    # (600, 8): about 300 pairs per expert, so experts span several 128-pair m-tiles
    for t, top_k in [(16, 2), (64, 10), (130, 4), (600, 8)]:
        for xpr in (1, top_k):
            _log(f"mm_id {dt.name} t={t} k={top_k} xpr={xpr}")
            ids = _distinct_ids(rng, t, top_k, n_expert)
            x = (rng.standard_normal((t, xpr, k)) * 10.0 ** rng.integers(-3, 4)).astype(np.float32)
            got = host(ops.mul_mm_id(st, dev_f32(x), dev_u32(ids)))
            want = orc.mul_mv_id(int(dt), blocks, n_expert, n_out, k, x, ids)
            assert_close(got, want, what=f"mm {dt.name} t={t} xpr={xpr}")


def test_mul_mm_id_prefill_size(dev, orc):
    """The reference-API projections at prefill size (t = 2048, top-10; gate/up-like
    Q4_K [1536 x 4096] with one x row per token, down-like Q6_K [4096 x 1536] with
    one per pair): 64 sampled tokens against the oracle (rows are independent), and
    the shared-map form bitwise equal to the self-contained one on every row."""
    rng = np.random.default_rng(23)
    t, top_k, n_expert = 2048, 10, 64
    for dt, n_out, k, xpr in ((GgmlDType.Q4_K, 1536, 4096, 1), (GgmlDType.Q6_K, 4096, 1536, top_k)):
        _log(f"mm_id prefill size {dt.name} [{n_out} x {k}] xpr={xpr}")
        key = int(rng.integers(0, 2**62))
        blocks = {e: orc.expert_blocks(int(dt), key, e, n_out, k) for e in range(n_expert)}
        st = upload_stack(dt, blocks, n_expert, n_out, k)
        ids = _distinct_ids(rng, t, top_k, n_expert)
        x = rng.standard_normal((t, xpr, k)).astype(np.float32)
        xd, idd = dev_f32(x), dev_u32(ids)
        got = host(ops.mul_mm_id(st, xd, idd))
        shared = host(ops.mul_mm_id_shared(st, xd, idd, ops.prepare_map0(n_expert, idd)))
        assert np.array_equal(got.view(np.uint32), shared.view(np.uint32))
        sub = np.sort(rng.choice(t, 64, replace=False))
        want = orc.mul_mv_id(int(dt), blocks, n_expert, n_out, k, np.ascontiguousarray(x[sub]),
                             np.ascontiguousarray(ids[sub]))
        assert_close(got[sub], want, what=f"mm prefill size {dt.name}")
        del st, xd


def test_mul_mm_id_fallback_tiles(dev, orc):
    """Q8_0 with K = 288 (not whole 256-weight super-blocks) runs the fallback tiles,
    which take each 128-pair m-tile of the map as two 64-pair halves."""
    rng = np.random.default_rng(17)
    dt, n_expert, n_out, k = GgmlDType.Q8_0, 8, 72, 288
    key = int(rng.integers(0, 2**62))
    blocks = {e: orc.expert_blocks(int(dt), key, e, n_out, k) for e in range(n_expert)}
    st = upload_stack(dt, blocks, n_expert, n_out, k)
    for t, top_k in [(5, 3), (200, 4)]:
        for xpr in (1, top_k):
            _log(f"mm_id fallback t={t} k={top_k} xpr={xpr}")
            ids = _distinct_ids(rng, t, top_k, n_expert)
            x = (rng.standard_normal((t, xpr, k)) * 10.0 ** rng.integers(-3, 4)).astype(np.float32)
            xd, idd = dev_f32(x), dev_u32(ids)
            got = host(ops.mul_mm_id(st, xd, idd))
            want = orc.mul_mv_id(int(dt), blocks, n_expert, n_out, k, x, ids)
            assert_close(got, want, what=f"mm fallback t={t} xpr={xpr}")
            shared = host(ops.mul_mm_id_shared(st, xd, idd, ops.prepare_map0(n_expert, idd)))
            assert np.array_equal(got.view(np.uint32), shared.view(np.uint32))


def test_shared_map0_matches_self_contained(dev, orc):
    """mm_id.rs:394-437: one map reused by several projections is bitwise equal to the
    self-contained form; no host sync between producing the map and consuming it."""
    _log("shared map0")
    rng = np.random.default_rng(8)
    n_expert, n_out, k, t, top_k = 32, 64, 256, 48, 10
    st = synth_stack(GgmlDType.Q4_K, n_expert, n_out, k, 0x91)
    ids = dev_u32(_distinct_ids(rng, t, top_k, n_expert))
    scratch = ops.prepare_map0(n_expert, ids)
    outs = []
    for xpr in (1, top_k):
        x = dev_f32(rng.uniform(-1, 1, (t, xpr, k)).astype(np.float32))
        outs.append((ops.mul_mm_id(st, x, ids), ops.mul_mm_id_shared(st, x, ids, scratch)))
    for owned, shared in outs:
        assert np.array_equal(host(owned).view(np.uint32), host(shared).view(np.uint32))


def test_silu_mul_and_combine(dev, orc):
    _log("silu_mul/combine")
    rng = np.random.default_rng(9)
    g = (rng.standard_normal((4, 10, 1536)) * 8).astype(np.float32)
    u = rng.standard_normal((4, 10, 1536)).astype(np.float32)
    got = host(ops.silu_mul(dev_f32(g), dev_f32(u)))
    want = orc.silu_mul(g, u)
    assert np.allclose(got, want, rtol=3e-7, atol=1e-37)
    down = (rng.standard_normal((4, 10, 4096)) * 10.0 ** rng.integers(-6, 4, (4, 10, 4096))).astype(np.float32)
    w = rng.uniform(0, 1, (4, 10)).astype(np.float32)
    l2 = rng.uniform(0.5, 2, (4, 10, 1)).astype(np.float32)
    for col in (None, l2):
        got = host(ops.combine(dev_f32(down), None if col is None else dev_f32(col), dev_f32(w)))
        want = orc.combine(down, col, w)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))  # same order, same roundings


def test_rms_norm(dev, orc):
    rng = np.random.default_rng(10)
    x = rng.standard_normal((3, 4096)).astype(np.float32)
    a = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    got = host(ops.rms_norm(dev_f32(x), dev_f32(a), 1e-6))
    assert np.allclose(got, orc.rmsnorm(x, a, 1e-6), rtol=2e-6, atol=1e-7)


def test_shape_errors_do_not_launch(dev):
    st = synth_stack(GgmlDType.Q4_K, 4, 8, 256, 1)
    x = torch.zeros((16, 1, 256), device="cuda")
    ids = torch.zeros((8, 2), dtype=torch.uint32, device="cuda")
    with pytest.raises(ops.MaxunaError, match="ids t"):
        ops.mul_mm_id(st, x, ids)
    with pytest.raises(ops.MaxunaError, match="does not match expert stack k"):
        ops.mul_mv_id(st, torch.zeros((1, 1, 512), device="cuda"), torch.zeros((1, 2), dtype=torch.uint32,
                                                                                device="cuda"))
