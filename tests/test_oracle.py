"""Pins the CPU oracle against the reference's own known answers.

Sources of truth, in order: the literal cases of peregrine's unit tests
(quant.rs:39-76, lib.rs:1651-1697), the same LCG-drawn inputs those tests use
(idot.rs:558-693, matmul.rs:202-348) with their assertions, brute-force integer
arithmetic in numpy (an independent computation), and closed forms.
"""
import math

import numpy as np
import pytest

from peregrine_amd import qt
from tests.refcases import GROUPED_CASES, LENS, Lcg


# ---------------- activation quantisation (quant.rs:39-76) ----------------

def test_qrow_roundtrip_literal(orc):
    x = np.array([0.5, -1.25, 3.0, -0.001, 2.7, -3.0], np.float32)
    q, s = orc.qrow_i8(x)
    assert q[2] == 127 and q[5] == -127
    assert np.all(np.abs(x - q.astype(np.float32) * s) <= s)


def test_qrow_all_zero(orc):
    q, s = orc.qrow_i8(np.zeros(8, np.float32))
    assert s == np.float32(1e-12) and not q.any()


def test_qrow_ties_to_even(orc):
    q, s = orc.qrow_i8(np.array([127.0, 1.5, 2.5, -1.5], np.float32))
    assert s == 1.0 and list(q[1:]) == [2, 2, -2]


def test_qrow_uses_reciprocal_multiply(orc):
    # x * (1/s) and x / s differ for some inputs; the reference multiplies.
    rng = np.random.default_rng(7)
    for _ in range(50):
        x = rng.standard_normal(64).astype(np.float32) * np.float32(rng.uniform(0.1, 10))
        q, s = orc.qrow_i8(x)
        inv = np.float32(1.0) / s
        assert np.array_equal(q, np.rint(x * inv).astype(np.int8))


def test_quant_rows_blocks_equal_per_slice(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((3, 100)).astype(np.float32)
    q, sx = orc.quant_rows(x, 32)
    assert sx.shape == (3, 4)
    for r in range(3):
        for b in range(4):
            qq, ss = orc.qrow_i8(x[r, 32 * b:32 * b + 32])
            assert ss == sx[r, b] and np.array_equal(qq, q[r, 32 * b:32 * b + 32])


# ---------------- integer dots (idot.rs:558-693) ----------------

def test_i8_dot_lcg_cases(orc):
    rng = Lcg(0x1234_5678)
    for n in LENS:
        w = np.array([rng.i8_full() for _ in range(n)], np.int8)
        x = np.array([rng.i8_127() for _ in range(n)], np.int8)
        assert orc.dot_i8i8(w, x) == int(np.dot(w.astype(np.int64), x.astype(np.int64)))


def test_i4_dot_lcg_cases_pack_unpack(orc):
    rng = Lcg(0x9E37_79B9)
    for n in LENS:
        vals = np.array([rng.nib() for _ in range(n)], np.int32)
        w4 = qt.pack_i4(vals)
        x = np.array([rng.i8_127() for _ in range(n)], np.int8)
        hand = int(np.dot(vals.astype(np.int64), x.astype(np.int64)))
        assert orc.dot_i4i8(w4, x) == hand, n
        if orc.have_avx2():
            assert orc.dot_i4i8_avx2(w4, x) == hand, n


def test_i4_dot_nibble_order_is_low_first(orc):
    # a single +1 in the low nibble of byte 0 must hit element 0, not element 1
    w4 = np.array([0x8 + 1 | (0x8 << 4)], np.uint8)
    assert orc.dot_i4i8(w4, np.array([5, 100], np.int8)) == 5
    w4 = np.array([0x8 | ((0x8 + 1) << 4)], np.uint8)
    assert orc.dot_i4i8(w4, np.array([5, 100], np.int8)) == 100


def test_i4_grouped_lcg_cases_exact(orc):
    rng = Lcg(0xDEAD_BEEF)
    for n, gs in GROUPED_CASES:
        vals = np.array([rng.nib() for _ in range(n)], np.int32)
        w4 = qt.pack_i4(vals)
        x = np.array([rng.i8_127() for _ in range(n)], np.int8)
        ng = -(-n // gs)
        scales = np.array([np.float32(0.01) + np.float32(0.05) * np.float32(g) for g in range(ng)], np.float32)
        hand = np.float32(0.0)
        for g in range(ng):
            a, b = g * gs, min((g + 1) * gs, n)
            d = int(np.dot(vals[a:b].astype(np.int64), x[a:b].astype(np.int64)))
            hand = np.float32(hand + np.float32(scales[g] * np.float32(d)))
        got = orc.dot_i4i8_grouped(w4, x, scales, gs)
        assert got.tobytes() == hand.tobytes(), (n, gs)


# ---------------- matmuls (matmul.rs:202-348) ----------------

def _perrow_expect(dots, sc, sx):
    # (f32)d * sc * sx evaluated left to right, in f32
    return (dots.astype(np.float32) * sc[None, :]).astype(np.float32) * sx[:, None]


def test_int8_matmul_matches_scalar_definition(orc):
    s_n, i_n, o_n = 3, 70, 5
    rng = Lcg(0xABCD)
    xf = rng.fvec(s_n * i_n).reshape(s_n, i_n)
    wf = rng.fvec(o_n * i_n).reshape(o_n, i_n)
    q8, sc8 = qt.quant_i8_rows(wf)
    xq, sx = orc.quant_rows(xf, 0)
    y = orc.linear(xq, sx, 0, orc.Tensor(q8, sc8, 1, i_n, o_n))
    dots = xq.astype(np.int64) @ q8.astype(np.int64).T
    assert np.array_equal(y, _perrow_expect(dots, sc8, sx[:, 0]))


def test_int4_matmul_matches_scalar_definition(orc):
    s_n, i_n, o_n = 2, 96, 4
    rng = Lcg(0x0F0F)
    xf = rng.fvec(s_n * i_n).reshape(s_n, i_n)
    wf = rng.fvec(o_n * i_n).reshape(o_n, i_n)
    q4, sc4 = qt.quant_i4_rows(wf)
    xq, sx = orc.quant_rows(xf, 0)
    y = orc.linear(xq, sx, 0, orc.Tensor(q4, sc4, 2, i_n, o_n))
    vals = qt.unpack_i4(q4, i_n).astype(np.int64)
    dots = xq.astype(np.int64) @ vals.T
    assert np.array_equal(y, _perrow_expect(dots, sc4, sx[:, 0]))


def test_grouped_matmul_matches_definition_and_beats_perrow(orc):
    s_n, i_n, o_n, gs = 2, 128, 4, 32
    rng = Lcg(0x6D6D)
    xf = rng.fvec(s_n * i_n).reshape(s_n, i_n)
    wf = rng.fvec(o_n * i_n).reshape(o_n, i_n)
    q4, sc4 = qt.quant_i4_grouped(wf, gs)
    xq, sx = orc.quant_rows(xf, 0)
    y = orc.linear(xq, sx, 0, orc.Tensor(q4, sc4, 4, i_n, o_n, gs))
    vals = qt.unpack_i4(q4, i_n).astype(np.int64)
    for s in range(s_n):
        for o in range(o_n):
            acc = np.float32(0)
            for g in range(i_n // gs):
                d = int(np.dot(vals[o, g * gs:(g + 1) * gs], xq[s, g * gs:(g + 1) * gs].astype(np.int64)))
                acc = np.float32(acc + np.float32(sc4[o, g] * np.float32(d)))
            assert y[s, o].tobytes() == np.float32(acc * sx[s, 0]).tobytes()
    qr, sr = qt.quant_i4_rows(wf)
    yr = orc.linear(xq, sx, 0, orc.Tensor(qr, sr, 2, i_n, o_n))
    ref = xf.astype(np.float64) @ wf.astype(np.float64).T
    assert np.abs(y - ref).sum() <= np.abs(yr - ref).sum()


def test_int8_matmul_approximates_f32(orc):
    s_n, i_n, o_n = 4, 128, 6
    rng = Lcg(0x5151)
    xf = rng.fvec(s_n * i_n).reshape(s_n, i_n)
    wf = rng.fvec(o_n * i_n).reshape(o_n, i_n)
    q8, sc8 = qt.quant_i8_rows(wf)
    xq, sx = orc.quant_rows(xf, 0)
    y = orc.linear(xq, sx, 0, orc.Tensor(q8, sc8, 1, i_n, o_n))
    ref = xf.astype(np.float64) @ wf.astype(np.float64).T
    assert np.all(np.abs(y - ref) < 0.02 * i_n)


@pytest.mark.parametrize("fmt", [1, 2, 4, 8])
@pytest.mark.parametrize("ga", [0, 32])
def test_linear_tracks_dequantised_product(orc, fmt, ga):
    # guards index/layout mistakes (transposed operand, wrong group) that the
    # exact tests on the same formula would not see
    rng = np.random.default_rng(fmt * 10 + ga)
    S, I, O = 3, 256, 40
    x = rng.standard_normal((S, I)).astype(np.float32)
    if fmt in (2, 4):
        v = rng.integers(-8, 8, (O, I))
        q = qt.pack_i4(v)
    else:
        v = rng.integers(-127, 128, (O, I))
        q = v.astype(np.int8)
    gs = 64 if fmt in (4, 8) else 0
    ns = O * (I // gs) if gs else O
    sc = np.exp(rng.normal(np.log(0.01), 0.5, ns)).astype(np.float32)
    wdeq = v.astype(np.float64) * (np.repeat(sc.reshape(O, -1), gs, axis=1) if gs else sc[:, None])
    xq, sx = orc.quant_rows(x, ga)
    y = orc.linear(xq, sx, ga, orc.Tensor(q, sc, fmt, I, O, gs))
    ref = x.astype(np.float64) @ wdeq.T
    assert np.max(np.abs(y - ref)) <= 0.02 * np.max(np.abs(ref))
    # the integer part is exact regardless of fp order
    d = orc.block_dots(xq, orc.Tensor(q, sc, fmt, I, O, gs))
    brute = np.einsum("sbk,obk->sob", xq.reshape(S, I // 32, 32).astype(np.int64),
                      v.reshape(O, I // 32, 32).astype(np.int64))
    assert np.array_equal(d, brute)


def test_grouped_mode_a_equals_reference_grouped_dot(orc):
    # fmt 4 with ga=0 must be dot_i4i8_grouped * sx exactly (matmul.rs:93-106)
    rng = np.random.default_rng(3)
    I, O, gs = 96, 3, 32
    v = rng.integers(-8, 8, (O, I))
    q = qt.pack_i4(v)
    sc = rng.uniform(0.001, 0.1, (O, I // gs)).astype(np.float32)
    x = rng.standard_normal((1, I)).astype(np.float32)
    xq, sx = orc.quant_rows(x, 0)
    y = orc.linear(xq, sx, 0, orc.Tensor(q, sc, 4, I, O, gs))
    for o in range(O):
        gd = orc.dot_i4i8_grouped(q[o], xq[0], sc[o], gs)
        assert y[0, o].tobytes() == np.float32(gd * sx[0, 0]).tobytes()


# ---------------- SwiGLU (math.rs:108-118, mlp.rs:21-26) ----------------

def test_silu_closed_form(orc):
    assert orc.silu(0.0) == 0.0
    assert orc.silu(-200.0) == 0.0 and math.copysign(1, orc.silu(-200.0)) < 0
    for v in np.linspace(-20, 20, 401, dtype=np.float32):
        exact = float(v) / (1.0 + math.exp(-float(v)))
        got = float(orc.silu(v))
        assert abs(got - exact) <= 2 * np.spacing(np.float32(abs(exact)) + np.float32(1e-30))


def test_silu_matches_glibc_expf_exactly(orc):
    # the oracle's SiLU calls glibc's expf, which is what Rust's f32::exp
    # (math.rs:108-111) calls on Linux: no input may differ.
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.expf.restype = ctypes.c_float
    libm.expf.argtypes = [ctypes.c_float]
    xs = np.random.default_rng(0).uniform(-20, 20, 20000).astype(np.float32)
    diff = 0
    for v in xs:
        ref = np.float32(v / np.float32(np.float32(1.0) + np.float32(libm.expf(float(-v)))))
        diff += ref.tobytes() != orc.silu(v).tobytes()
    assert diff == 0


def test_expert_swiglu_tracks_f64(orc):
    rng = np.random.default_rng(11)
    D, I, S = 128, 64, 3
    def mk(o, i):
        v = rng.integers(-8, 8, (o, i))
        sc = np.exp(rng.normal(np.log(0.05), 0.3, (o, i // 32))).astype(np.float32)
        return orc.Tensor(qt.pack_i4(v), sc, 4, i, o, 32), v * np.repeat(sc, 32, axis=1).astype(np.float64)
    (g, gd), (u, ud), (d, dd) = mk(I, D), mk(I, D), mk(D, I)
    x = rng.standard_normal((S, D)).astype(np.float32)
    for ga in (0, 32):
        y, h = orc.expert_swiglu(x, g, u, d, ga, want_h=True)
        gg, uu = x @ gd.T, x @ ud.T
        hh = gg / (1 + np.exp(-gg)) * uu
        ref = hh @ dd.T
        assert np.max(np.abs(h - hh)) <= 0.03 * np.max(np.abs(hh))
        assert np.max(np.abs(y - ref)) <= 0.05 * np.max(np.abs(ref))


# ---------------- routing (router.rs:52-170, 420-445) ----------------

def test_route_sigmoid_ties_lowest_index_and_weights(orc):
    logits = np.array([[0.0, 2.0, 2.0, -1.0]], np.float32)
    idx, w, keff = orc.route_sigmoid(logits, np.zeros(4, np.float32), 2, norm_topk=False)
    assert list(idx[0]) == [1, 2] and keff[0] == 2
    sig = np.float32(1.0) / (np.float32(1.0) + np.float32(math.exp(-2.0)))
    assert w[0, 0] == sig and w[0, 1] == sig


def test_route_sigmoid_bias_selects_but_weight_is_sigmoid(orc):
    logits = np.array([[1.0, 0.0]], np.float32)
    idx, w, _ = orc.route_sigmoid(logits, np.array([0.0, 5.0], np.float32), 1, norm_topk=False,
                                  routed_scale=2.0)
    assert idx[0, 0] == 1
    assert np.isclose(w[0, 0], 2.0 * 0.5)


def test_route_sigmoid_normalises(orc):
    rng = np.random.default_rng(2)
    logits = rng.standard_normal((5, 16)).astype(np.float32)
    idx, w, keff = orc.route_sigmoid(logits, np.zeros(16, np.float32), 4, True, 2.5)
    assert np.allclose(w.sum(1), 2.5, rtol=1e-6)
    for s in range(5):
        assert len(set(idx[s])) == 4
        top = np.argsort(-logits[s], kind="stable")[:4]
        assert sorted(idx[s]) == sorted(top)


def test_negligible_tail_reference_cases(orc):
    """router.rs:531-554: only a trailing run under min_share is dropped, at
    most kept-1, and degenerate rows are left alone."""
    w = np.array([0.9, 0.05, 0.03, 0.02], np.float32)
    assert orc.negligible_tail(w, 4, 0.06) == 3
    assert orc.negligible_tail(w, 4, 0.04) == 2
    assert orc.negligible_tail(w, 4, 0.01) == 0
    assert orc.negligible_tail(np.array([0.5, 0.01, 0.48, 0.01], np.float32), 4, 0.05) == 1
    assert orc.negligible_tail(np.full(4, 0.25, np.float32), 4, 0.99) == 3
    assert orc.negligible_tail(np.array([1.0], np.float32), 1, 0.99) == 0
    assert orc.negligible_tail(np.array([0.0, 0.0], np.float32), 2, 0.5) == 0
    assert orc.negligible_tail(np.array([np.nan, 1.0], np.float32), 2, 0.5) == 0


def test_route_truncates_and_renormalises_to_the_original_scale(orc):
    """router.rs:557-584: logits 6 and -6 (x = 1 through router weights 6, -6),
    k = 2, renormalised, routed_scale 2.5: min_share 0.05 drops the negligible
    expert and the survivor still carries the whole routed_scale."""
    logits = np.array([[6.0, -6.0]], np.float32)
    bias = np.zeros(2, np.float32)
    i_off, w_off, k_off = orc.route_sigmoid(logits, bias, 2, True, 2.5, 0.0)
    i_on, w_on, k_on = orc.route_sigmoid(logits, bias, 2, True, 2.5, 0.05)
    assert k_off[0] == 2 and k_on[0] == 1
    assert i_on[0, 0] == i_off[0, 0] == 0
    assert abs(float(w_on[0, :1].sum()) - 2.5) < 1e-5 and abs(float(w_off[0, :2].sum()) - 2.5) < 1e-5
    assert i_on[0, 1] == 0 and w_on[0, 1] == 0.0


def test_route_softmax_topk_equals_renormalised_softmax(orc):
    rng = np.random.default_rng(4)
    logits = rng.standard_normal((6, 160)).astype(np.float32)
    idx, w = orc.route_softmax_topk(logits, 8)
    for s in range(6):
        p = np.exp(logits[s].astype(np.float64) - logits[s].max())
        p /= p.sum()
        top = np.argsort(-logits[s], kind="stable")[:8]
        assert list(idx[s]) == list(top)
        ref = p[top] / p[top].sum()
        assert np.allclose(w[s], ref, rtol=1e-6, atol=0)


def test_batch_union_first_seen_order(orc):
    idx = np.array([[5, 3], [3, 7], [1, 5]], np.int32)
    assert list(orc.batch_union(idx, 8)) == [5, 3, 7, 1]


# ---------------- expert table, ReduceLayout, combine ----------------

def test_reduce_layout_golden(orc):
    # crates/peregrine-cuda/src/lib.rs:1651-1697
    rp, ri = orc.reduce_layout_build(np.array([0, 1, 0, 1, 0]), 2)
    assert list(rp) == [0, 3, 5] and list(ri) == [0, 2, 4, 1, 3]
    rp, ri = orc.reduce_layout_build(np.array([2, 0, 2, 1, 1, 2, 0]), 3)
    assert list(np.diff(rp)) == [2, 2, 3]
    for s in range(3):
        seg = ri[rp[s]:rp[s + 1]]
        assert list(seg) == sorted(seg)
    assert orc.reduce_layout_build(np.array([0, 3]), 2) is None


def test_grouped_reduce_order_and_closed_form(orc):
    rng = np.random.default_rng(5)
    y = rng.standard_normal((5, 7)).astype(np.float32)
    rw = rng.uniform(0, 1, 5).astype(np.float32)
    rp, ri = orc.reduce_layout_build(np.array([0, 1, 0, 1, 0]), 2)
    out = orc.grouped_reduce(y, rp, ri, rw, 2)
    exp0 = np.float32(0)
    for k in (0, 2, 4):
        exp0 = (exp0 + (rw[k] * y[k]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(out[0], exp0)
    assert np.allclose(out[1], rw[1] * y[1] + rw[3] * y[3], rtol=1e-6)


def test_expert_table_invariants(orc):
    idx = np.array([[5, 3], [3, 7], [1, 5], [7, 3]], np.int32)
    t = orc.expert_table(idx, 8)
    assert list(t["uexp"]) == [5, 3, 7, 1]
    assert list(t["off"]) == [0, 2, 5, 7, 8]
    assert list(t["row_tok"]) == [0, 2, 0, 1, 3, 1, 3, 2]
    # token 1 routes [3, 7]; union ranks 3->1, 7->2
    assert list(t["tok_rows"][1]) == [3, 5]
    # token 3 routes [7, 3] but adds expert 3 (rank 1) before 7 (rank 2)
    assert list(t["tok_rows"][3]) == [4, 6]
    rng = np.random.default_rng(6)
    idx = np.stack([rng.choice(40, 6, replace=False) for _ in range(100)]).astype(np.int32)
    t = orc.expert_table(idx, 40)
    assert t["off"][-1] == idx.size
    for u in range(t["n_u"]):
        toks = t["row_tok"][t["off"][u]:t["off"][u + 1]]
        assert np.all(np.diff(toks) > 0)
        assert np.all(idx[toks, t["row_kk"][t["off"][u]:t["off"][u + 1]]] == t["uexp"][u])


# ---------------- whole layer ----------------

def _tiny_layer(orc, seed, E=6, D=64, I=64, fmt=4):
    rng = np.random.default_rng(seed)
    experts = []
    for _ in range(E):
        trip = []
        for (o, i) in ((I, D), (I, D), (D, I)):
            v = rng.integers(-8, 8, (o, i))
            sc = np.exp(rng.normal(np.log(0.01), 0.5, (o, i // 32))).astype(np.float32)
            trip.append(orc.Tensor(qt.pack_i4(v), sc, fmt, i, o, 32))
        experts.append(tuple(trip))
    return experts, rng


@pytest.mark.parametrize("ga", [0, 32])
def test_moe_forward_serial_parallel_simd_subset_identical(orc, ga):
    experts, rng = _tiny_layer(orc, 9)
    S, k = 10, 3
    x = rng.standard_normal((S, 64)).astype(np.float32)
    idx, w = orc.route_softmax_topk(rng.standard_normal((S, 6)).astype(np.float32), k)
    a = orc.moe_forward(x, idx, w, experts, ga)
    b = orc.moe_forward(x, idx, w, experts, ga, nthreads=4)
    c = orc.moe_forward(x, idx, w, experts, ga, simd=orc.have_avx2())
    d = orc.moe_forward(x, idx, w, experts, ga, subset=np.array([7, 2]))
    assert np.array_equal(a, b) and np.array_equal(a, c)
    assert np.array_equal(d[[2, 7]], a[[2, 7]]) and not d[0].any()


def test_moe_forward_matches_per_expert_scatter(orc):
    # the layer equals Mlp::swiglu per expert plus the union-order scatter
    experts, rng = _tiny_layer(orc, 12)
    S, k = 7, 2
    x = rng.standard_normal((S, 64)).astype(np.float32)
    idx, w = orc.route_softmax_topk(rng.standard_normal((S, 6)).astype(np.float32), k)
    out = orc.moe_forward(x, idx, w, experts, 0)
    ref = np.zeros_like(out)
    for e in orc.batch_union(idx, 6):
        rows = [s for s in range(S) if e in idx[s]]
        y = orc.expert_swiglu(x[rows], *experts[e], 0)
        for r, s in enumerate(rows):
            kk = list(idx[s]).index(e)
            ref[s] = (ref[s] + (w[s, kk] * y[r]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(out, ref)
