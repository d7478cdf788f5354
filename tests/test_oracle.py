"""Pins the CPU oracle (oracle/moe_oracle.c) before it is trusted as the checker.

Each test checks the oracle against something it does not share code with:
the reference's own known-answer tests (routing, moe.rs:405-500), closed forms
on blocks built by an independent encoder (tests/_pack.py), numpy's IEEE half
conversion, brute force on small inputs, and permutation invariants.
"""
import math

import numpy as np
import pytest

from tests._pack import (pack_q4_k, pack_q5_k, pack_q6_k, pack_q8_0, q4_k_values, q6_k_values, f16_bits)

Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14

# sigmoid of the reference's fixed logit row [2,-2,0,1,-1,3,0.5,-0.5] (moe.rs:384-387)
S2, S1, S3, S05 = 0.8807970779778823, 0.7310585786300049, 0.9525741268224334, 0.6224593312018546
LOGITS_ROW = np.array([[2.0, -2.0, 0.0, 1.0, -1.0, 3.0, 0.5, -0.5]], np.float32)


# ---- IEEE half ------------------------------------------------------------------------
def test_f16_to_f32_all_patterns(orc):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().or_f16_to_f32(int(b)) for b in bits], np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(got[fin].view(np.uint32), ref[fin].view(np.uint32))
    assert np.all(np.isnan(got[np.isnan(ref)]))


def test_f32_to_f16_round_to_nearest_even(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-9, 5, 20000),
        np.array([0.0, -0.0, 65504.0, 65520.0, 1e-8, 6.1035156e-05, 5.96e-8, 2.98e-8, 1.0009765625], np.float32),
    ]).astype(np.float32)
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.lib().or_f32_to_f16(float(v)) for v in vals], np.uint16)
    assert np.array_equal(got, ref)


# ---- dequantisation: closed forms on encoder-built blocks ---------------------------------
def test_q4_k_integer_grid_exact(orc):
    rng = np.random.default_rng(2)
    for trial in range(20):
        d = [1.0, 0.5, 2.0, 0.25][trial % 4]
        dmin = [0.5, 1.0, 0.125, 0.0][trial % 4]
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        m = [int(v) for v in rng.integers(0, 64, 8)]
        q = rng.integers(0, 16, 256)
        blk = pack_q4_k(d, dmin, sc, m, q)
        got = orc.dequantize(Q4_K, blk, 256)
        assert np.array_equal(got.astype(np.float64), q4_k_values(d, dmin, sc, m, q)), trial


def test_q4_k_single_subblock_scale_moves_only_its_weights(orc):
    q = np.full(256, 3)
    base = orc.dequantize(Q4_K, pack_q4_k(1.0, 0.0, [1] * 8, [0] * 8, q), 256)
    for j in range(8):
        sc = [1] * 8
        sc[j] = 2 + 16 * (j >= 4) * 2  # j >= 4 exercises the high-bit packing
        got = orc.dequantize(Q4_K, pack_q4_k(1.0, 0.0, sc, [0] * 8, q), 256)
        changed = np.nonzero(got != base)[0]
        assert np.array_equal(changed, np.arange(32 * j, 32 * j + 32)), j


def test_q4_k_special_cases(orc):
    z = orc.dequantize(Q4_K, np.zeros(144, np.uint8), 256)
    assert np.all(z == 0)
    # q = 0 -> -dmin*m
    got = orc.dequantize(Q4_K, pack_q4_k(1.0, 0.5, [5] * 8, list(range(8)), np.zeros(256, int)), 256)
    assert np.array_equal(got, (-0.5 * (np.arange(256) // 32)).astype(np.float32))


def test_q4_k_rounding_order(orc):
    """y = fl(fl(d*sc)*q) - fl(dmin*m): a fused or reassociated form differs on these."""
    rng = np.random.default_rng(3)
    d, dmin = 0.0033378601, 0.0071563721  # arbitrary f16 values
    d = float(np.float16(d)); dmin = float(np.float16(dmin))
    sc = [int(v) for v in rng.integers(1, 64, 8)]
    m = [int(v) for v in rng.integers(1, 64, 8)]
    q = rng.integers(0, 16, 256)
    got = orc.dequantize(Q4_K, pack_q4_k(d, dmin, sc, m, q), 256)
    j = np.arange(256) // 32
    f = np.float32
    d1 = f(d) * np.array(sc, f)[j]
    m1 = f(dmin) * np.array(m, f)[j]
    exp = (d1 * q.astype(f)) - m1
    assert np.array_equal(got.view(np.uint32), exp.astype(f).view(np.uint32))
    # sanity: the exact value is within 1 ulp-ish of both
    assert np.allclose(got, q4_k_values(d, dmin, sc, m, q), rtol=1e-6, atol=1e-6)


def test_q5_k_integer_grid_exact(orc):
    """d*sc_j*q - dmin*m_j with q in 0..31 (the fifth bit from qh)."""
    rng = np.random.default_rng(20)
    for trial in range(20):
        d = [1.0, 0.5, 2.0, 0.25][trial % 4]
        dmin = [0.5, 1.0, 0.125, 0.0][trial % 4]
        sc = [int(v) for v in rng.integers(0, 64, 8)]
        m = [int(v) for v in rng.integers(0, 64, 8)]
        q = rng.integers(0, 32, 256)
        got = orc.dequantize(Q5_K, pack_q5_k(d, dmin, sc, m, q), 256)
        assert np.array_equal(got.astype(np.float64), q4_k_values(d, dmin, sc, m, q)), trial


def test_q5_k_each_high_bit_moves_only_its_weight(orc):
    q = np.full(256, 5)
    base = orc.dequantize(Q5_K, pack_q5_k(1.0, 0.0, [3] * 8, [0] * 8, q), 256)
    for w in [0, 31, 32, 63, 64, 100, 159, 200, 255]:
        q2 = q.copy()
        q2[w] += 16
        got = orc.dequantize(Q5_K, pack_q5_k(1.0, 0.0, [3] * 8, [0] * 8, q2), 256)
        changed = np.nonzero(got != base)[0]
        assert changed.tolist() == [w], w
        assert got[w] - base[w] == 48.0  # 16 * d * sc


def test_q5_k_special_cases_and_rounding(orc):
    assert np.all(orc.dequantize(Q5_K, np.zeros(176, np.uint8), 256) == 0)
    rng = np.random.default_rng(21)
    d, dmin = float(np.float16(0.0047)), float(np.float16(0.0061))
    sc = [int(v) for v in rng.integers(1, 64, 8)]
    m = [int(v) for v in rng.integers(1, 64, 8)]
    q = rng.integers(0, 32, 256)
    got = orc.dequantize(Q5_K, pack_q5_k(d, dmin, sc, m, q), 256)
    j = np.arange(256) // 32
    f = np.float32
    exp = (f(d) * np.array(sc, f)[j] * q.astype(f)) - f(dmin) * np.array(m, f)[j]
    assert np.array_equal(got.view(np.uint32), exp.astype(f).view(np.uint32))


def test_q6_k_integer_grid_exact(orc):
    rng = np.random.default_rng(4)
    for trial in range(20):
        d = [1.0, 0.5, 0.25, 2.0][trial % 4]
        sc = [int(v) for v in rng.integers(-128, 128, 16)]
        q = rng.integers(0, 64, 256)
        got = orc.dequantize(Q6_K, pack_q6_k(d, sc, q), 256)
        assert np.array_equal(got.astype(np.float64), q6_k_values(d, sc, q)), trial
    # q = 32 -> 0 whatever the scale
    got = orc.dequantize(Q6_K, pack_q6_k(0.37, [-77] * 16, np.full(256, 32)), 256)
    assert np.all(got == 0)


def test_q6_k_each_scale_owns_16_weights(orc):
    q = np.full(256, 33)
    base = orc.dequantize(Q6_K, pack_q6_k(1.0, [1] * 16, q), 256)
    for j in range(16):
        sc = [1] * 16
        sc[j] = -3
        got = orc.dequantize(Q6_K, pack_q6_k(1.0, sc, q), 256)
        assert np.array_equal(np.nonzero(got != base)[0], np.arange(16 * j, 16 * j + 16)), j


def test_q8_0_exact(orc):
    rng = np.random.default_rng(5)
    qs = rng.integers(-128, 128, 32)
    assert np.array_equal(orc.dequantize(Q8_0, pack_q8_0(1.0, qs), 32), qs.astype(np.float32))
    d = float(np.float16(0.0123))
    got = orc.dequantize(Q8_0, pack_q8_0(d, qs), 32)
    assert np.array_equal(got, (qs.astype(np.float32) * np.float32(d)).astype(np.float32))


# ---- routing: the reference's known-answer tests (moe.rs:405-500) ------------------------
def _close(got, exp, tol):
    for g, e in zip(np.ravel(got), np.ravel(exp)):
        assert abs(float(g) - e) <= tol, (g, e)


def test_routing_positive_bias_displaces(orc):
    bias = np.array([0, 0, 0, 0, 0, 0, 0.2, 0], np.float32)
    ids, w = orc.route_from_logits(LOGITS_ROW, bias, 3, 2.5, True)
    assert ids.tolist() == [[5, 0, 6]]
    sel = [S3, S2, S05]
    _close(w, [p / sum(sel) * 2.5 for p in sel], 1e-5)


def test_routing_negative_bias_excludes(orc):
    bias = np.array([0, 0, 0, 0, 0, -1.0, 0, 0], np.float32)
    ids, w = orc.route_from_logits(LOGITS_ROW, bias, 3, 2.5, True)
    assert ids.tolist() == [[0, 3, 6]]
    sel = [S2, S1, S05]
    _close(w, [p / sum(sel) * 2.5 for p in sel], 1e-5)


def test_routing_ties_pick_lowest_indices(orc):
    ids, _ = orc.route_from_logits(np.zeros((1, 8), np.float32), np.zeros(8, np.float32), 3, 2.5, True)
    assert ids.tolist() == [[0, 1, 2]]


def test_routing_clamps_tiny_denominator(orc):
    _, w = orc.route_from_logits(np.full((1, 8), -30.0, np.float32), np.zeros(8, np.float32), 3, 2.5, True)
    p = 1.0 / (1.0 + math.exp(30.0))
    exp = p / 6.103515625e-5 * 2.5
    _close(w, [exp] * 3, exp * 1e-3)


def test_router_matmul_identity(orc):
    logits = orc.route_logits(LOGITS_ROW, np.eye(8, dtype=np.float32))
    _close(logits, LOGITS_ROW.ravel(), 1e-6)


def test_routing_scale_one_and_no_norm(orc):
    bias = np.zeros(8, np.float32)
    _, w = orc.route_from_logits(LOGITS_ROW, bias, 2, 1.0, False)
    _close(w, [S3, S2], 1e-6)  # unnormalised, unscaled sigmoid probs


def test_routing_matches_brute_force_sort(orc):
    rng = np.random.default_rng(6)
    logits = rng.standard_normal((50, 256)).astype(np.float32)
    # include exact ties
    logits[:, 100:110] = logits[:, 10:11]
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    bias[100:110] = bias[10]
    ids, w = orc.route_from_logits(logits, bias, 10, 1.0, True)
    for r in range(50):
        p = (1.0 / (np.exp(-logits[r].astype(np.float64)) + 1.0)).astype(np.float32)
        sel = p + bias
        order = sorted(range(256), key=lambda e: (-float(sel[e]), e))
        assert ids[r].tolist() == order[:10]
        pw = p[order[:10]].astype(np.float64)
        assert np.allclose(w[r], pw / pw.sum(), rtol=1e-6)


# ---- generator ---------------------------------------------------------------------------
def test_tensor_key_matches_python(orc):
    from maxuna_amd.synth import tensor_key, mix64
    for seed, layer, tid in [(0, 0, 0), (1, 2, 3), (123456789, 47, 12), (2**63 + 5, 65535, 22)]:
        assert orc.lib().or_tensor_key(seed, layer, tid) == tensor_key(seed, layer, tid)
        assert orc.lib().or_mix64(seed) == mix64(seed)


@pytest.mark.parametrize("dt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_synth_ranges_are_consistent(orc, dt):
    key = 0xDEADBEEF
    ts = orc.TSIZE[dt]
    whole = orc.synth_bytes(dt, key, 0, ts * 40)
    for a, b in [(0, ts), (3, 5 * ts + 7), (ts * 7 + 1, ts * 39)]:
        assert np.array_equal(orc.synth_bytes(dt, key, a, b - a), whole[a:b])
    # scale fields decode to f16 values in [0.001, 0.01]
    blocks = whole.reshape(40, ts)
    offs = {Q4_K: [0, 2], Q5_K: [0, 2], Q6_K: [208], Q8_0: [0]}[dt]
    for o in offs:
        v = blocks[:, o:o + 2].copy().view(np.float16).astype(np.float32).ravel()
        assert np.all(v >= np.float16(0.001)) and np.all(v <= np.float16(0.01))


def test_normal_generator_moments():
    from maxuna_amd.synth import normal
    z = normal(42, 200000, 1.0)
    assert z.dtype == np.float32
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1.0) < 0.01
    assert np.array_equal(normal(42, 10, 1.0, offset=5), z[5:15])


# ---- mat-vec / bucket / elementwise ----------------------------------------------------------
def _rand_stack(rng, dt, n_expert, n_out, k):
    from oracle.oracle import row_bytes
    key = int(rng.integers(0, 2**62))
    return {e: orc_expert(dt, key, e, n_out, k) for e in range(n_expert)}, key


def orc_expert(dt, key, e, n_out, k):
    from oracle import oracle as o
    return o.expert_blocks(dt, key, e, n_out, k)


@pytest.mark.parametrize("dt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_mul_mv_id_brute_force(orc, dt):
    rng = np.random.default_rng(7)
    n_expert, n_out, k, t, top_k = 4, 8, 256, 3, 2
    stack, _ = _rand_stack(rng, dt, n_expert, n_out, k)
    deq = {e: orc.dequantize(dt, b, n_out * k).reshape(n_out, k).astype(np.float64) for e, b in stack.items()}
    ids = rng.integers(0, n_expert, (t, top_k)).astype(np.uint32)
    for xpr in (1, top_k):
        x = rng.uniform(-1, 1, (t, xpr, k)).astype(np.float32)
        got = orc.mul_mv_id(dt, stack, n_expert, n_out, k, x, ids)
        for tok in range(t):
            for s in range(top_k):
                xr = x[tok, 0 if xpr == 1 else s].astype(np.float64)
                assert np.allclose(got[tok, s], deq[int(ids[tok, s])] @ xr, rtol=1e-6, atol=1e-6)


def test_map0_invariants(orc):
    rng = np.random.default_rng(8)
    for t, k, E in [(1, 4, 64), (37, 10, 256), (300, 8, 32)]:
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(t)]).astype(np.uint32)
        tpe, hids = orc.map0(ids, E)
        assert tpe.sum() == t * k
        seen = []
        for e in range(E):
            lst = hids[e, :tpe[e]]
            toks = lst // k
            assert np.all(np.diff(toks) > 0)                 # tokens ascending
            assert np.all(ids.ravel()[lst] == e)              # each entry routes to e
            seen.extend(lst.tolist())
        assert sorted(seen) == list(range(t * k))            # a permutation of all pairs


def test_silu_mul_closed_form(orc):
    rng = np.random.default_rng(9)
    g = (rng.standard_normal(4096) * 10).astype(np.float32)
    u = rng.standard_normal(4096).astype(np.float32)
    got = orc.silu_mul(g, u).astype(np.float64)
    gd = g.astype(np.float64)
    exp = gd / (1 + np.exp(-gd)) * u.astype(np.float64)
    assert np.allclose(got, exp, rtol=4e-7, atol=1e-30)


def test_combine_closed_form(orc):
    rng = np.random.default_rng(10)
    down = (rng.standard_normal((3, 10, 64)) * 10.0 ** rng.integers(-6, 4, (3, 10, 64))).astype(np.float32)
    w = rng.uniform(0, 1, (3, 10)).astype(np.float32)
    got = orc.combine(down, None, w)
    exp = np.zeros((3, 64), np.float32)
    for k in range(10):
        exp = (exp + (down[:, k] * w[:, k:k + 1]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(got, exp)
    l2 = rng.uniform(0.5, 2, (3, 10, 1)).astype(np.float32)
    got = orc.combine(down, l2, w)
    exp = np.zeros((3, 64), np.float32)
    for k in range(10):
        d = (down[:, k] * l2[:, k]).astype(np.float32) * np.float32(2.0 ** -15)
        exp = (exp + (d * w[:, k:k + 1]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(got, exp)


def test_rmsnorm_closed_form(orc):
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4, 4096)).astype(np.float32)
    a = rng.uniform(0.5, 1.5, 4096).astype(np.float32)
    got = orc.rmsnorm(x, a, 1e-6)
    xd = x.astype(np.float64)
    exp = xd / np.sqrt((xd ** 2).mean(1, keepdims=True) + 1e-6) * a
    assert np.allclose(got, exp, rtol=1e-5)


# ---- ReferenceExperts wiring (structure of moe.rs:522-609) ----------------------------------
@pytest.mark.parametrize("dt", [Q4_K, Q5_K, Q6_K, Q8_0])
def test_reference_experts_matches_per_token_oracle(orc, dt):
    rng = np.random.default_rng(12)
    n_expert, ff, hidden, seq, top_k = 4, 256, 256, 3, 2
    g, _ = _rand_stack(rng, dt, n_expert, ff, hidden)
    u, _ = _rand_stack(rng, dt, n_expert, ff, hidden)
    d, _ = _rand_stack(rng, dt, n_expert, hidden, ff)
    x = rng.uniform(-1, 1, (seq, hidden)).astype(np.float32)
    ids = np.array([[0, 3], [1, 2], [3, 0]], np.uint32)
    w = np.array([[0.5, 0.25], [1.5, 0.75], [0.1, 0.9]], np.float32)
    got = orc.reference_experts(dt, g, dt, u, dt, d, n_expert, hidden, ff, x, ids, w)
    deq = lambda st, e, r, c: orc.dequantize(dt, st[e], r * c).reshape(r, c).astype(np.float64)  # noqa
    for tok in range(seq):
        acc = np.zeros(hidden)
        for s in range(top_k):
            e = int(ids[tok, s])
            xg = deq(g, e, ff, hidden) @ x[tok]
            xu = deq(u, e, ff, hidden) @ x[tok]
            h = xg / (1 + np.exp(-xg)) * xu
            acc += (deq(d, e, hidden, ff) @ h) * w[tok, s]
        tol = 1e-3 * np.maximum(np.abs(acc), 1.0)
        assert np.all(np.abs(got[tok] - acc) <= tol)


def test_swiglu_closed_form(orc):
    rng = np.random.default_rng(13)
    hidden, ff = 256, 512
    key = 77
    gb = orc.expert_blocks(Q8_0, key, 0, ff, hidden)
    ub = orc.expert_blocks(Q8_0, key, 1, ff, hidden)
    db = orc.expert_blocks(Q8_0, key, 2, hidden, ff)
    x = rng.standard_normal((4, hidden)).astype(np.float32)
    got = orc.swiglu(Q8_0, gb, Q8_0, ub, Q8_0, db, hidden, ff, x)
    G = orc.dequantize(Q8_0, gb, ff * hidden).reshape(ff, hidden).astype(np.float64)
    U = orc.dequantize(Q8_0, ub, ff * hidden).reshape(ff, hidden).astype(np.float64)
    D = orc.dequantize(Q8_0, db, ff * hidden).reshape(hidden, ff).astype(np.float64)
    g = x @ G.T
    exp = ((g / (1 + np.exp(-g))) * (x @ U.T)) @ D.T
    assert np.allclose(got, exp, rtol=1e-4, atol=1e-4 * np.abs(exp).max())
