"""GPU parity: the HIP lane through its C ABI against the CPU oracle.

Bars: per-block int32 dots bit-exact; fp32 outputs
within 1e-5 of the oracle, max-abs normalised. The kernels evaluate every f32
epilogue in the oracle's order, so most cases are asserted bit-identical.
"""
import sys

import numpy as np
import pytest

from peregrine_amd import qt, synth

pytestmark = pytest.mark.gpu

TOL = 1e-5


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


def nerr(got, ref):
    ref = np.asarray(ref, np.float64)
    den = max(np.max(np.abs(ref)), 1e-30)
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref)) / den)


@pytest.fixture(scope="module")
def hip():
    from peregrine_amd import hip as h
    assert h.probe_device_count() >= 1
    assert h.init([0]) == 1
    yield h
    h.set_arm(-1)
    h.set_act_group(0)
    h.set_debug_dots(0, 0)


def _experts(rng, n, D, I, fmt, gs, orc, hip):
    gpu, ora = [], []
    for _ in range(n):
        trip = synth.make_expert(rng, D, I, fmt, gs)
        gpu.append(hip.GpuExpert.upload_grouped(0, trip[0][:2], trip[1][:2], trip[2][:2], D, I, fmt, gs))
        shp = ((I, D), (I, D), (D, I))
        ora.append(tuple(orc.Tensor(t[0], t[1], fmt, i, o, gs) for t, (o, i) in zip(trip, shp)))
    return gpu, ora


def test_probe_init_meminfo(hip):
    assert hip.device_count() == 1
    free, total = hip.mem_info(0)
    assert total > 100e9 and 0 < free <= total


def test_init_rejects_bad_ordinal_lists(hip):
    """A list naming a missing device or one device twice is refused as a
    whole and leaves the contexts of the earlier init in place."""
    say("init validation")
    assert hip.init([0, 0]) == 0
    assert hip.init([hip.probe_device_count()]) == 0
    assert hip.init([-1]) == 0
    assert hip.device_count() == 1
    free, total = hip.mem_info(0)
    assert 0 < free <= total


FORMATS = [(qt.FMT_I4G, 32), (qt.FMT_I4G, 128), (qt.FMT_I4, 0), (qt.FMT_I8G, 32), (qt.FMT_I8, 0)]


@pytest.mark.parametrize("fmt,gs", FORMATS)
@pytest.mark.parametrize("ga", [0, 32])
@pytest.mark.parametrize("arm", [2, 0])
def test_expert_group_matches_oracle(hip, orc, fmt, gs, ga, arm):
    say("expert_group", fmt, gs, ga, arm)
    rng = np.random.default_rng(100 + fmt * 7 + gs + ga + arm)
    D, I = 320, 192   # not multiples of the 64-row tile: exercises padding
    gpu, ora = _experts(rng, 3, D, I, fmt, gs or 32, orc, hip)
    rows = [1, 3, 34]
    x = rng.standard_normal((sum(rows), D)).astype(np.float32)
    hip.set_act_group(ga)
    hip.set_arm(arm)
    y, used = hip.expert_group_tiled(gpu, rows, x, D)
    assert used.value == arm
    r0 = 0
    for e, n in enumerate(rows):
        ref = orc.expert_swiglu(x[r0:r0 + n], *ora[e], ga)
        assert nerr(y[r0:r0 + n], ref) <= TOL, (e, nerr(y[r0:r0 + n], ref))
        assert np.array_equal(y[r0:r0 + n], ref), f"expert {e}: not bit-identical"
        r0 += n


@pytest.mark.parametrize("arm", [2, 0])
@pytest.mark.parametrize("fmt", [qt.FMT_I4G, qt.FMT_I8G])
def test_block_dots_bit_exact(hip, orc, arm, fmt):
    say("block dots", arm, fmt)
    rng = np.random.default_rng(7 + arm + fmt)
    D, I = 256, 128
    gpu, ora = _experts(rng, 2, D, I, fmt, 32, orc, hip)
    rows = [2, 3]
    R = sum(rows)
    x = rng.standard_normal((R, D)).astype(np.float32)
    nbd, nbi = D // 32, I // 32
    dgu = hip.DeviceBuffer(R * 2 * I * nbd * 4)
    ddn = hip.DeviceBuffer(R * D * nbi * 4)
    hip.set_act_group(32)
    hip.set_arm(arm)
    hip.set_debug_dots(dgu.ptr, ddn.ptr)
    try:   # with the dump on, the MFMA arm runs its register-prefetch kernel
        y = hip.expert_group(gpu, rows, x, D)
    finally:
        hip.set_debug_dots(0, 0)
    gu = dgu.download(np.int32, (R, 2, I, nbd))
    dn = ddn.download(np.int32, (R, D, nbi))
    r0 = 0
    for e, n in enumerate(rows):
        xq, sx = orc.quant_rows(x[r0:r0 + n], 32)
        assert np.array_equal(gu[r0:r0 + n, 0], orc.block_dots(xq, ora[e][0]))
        assert np.array_equal(gu[r0:r0 + n, 1], orc.block_dots(xq, ora[e][1]))
        _, h = orc.expert_swiglu(x[r0:r0 + n], *ora[e], 32, want_h=True)
        hq, _ = orc.quant_rows(h, 32)
        assert np.array_equal(dn[r0:r0 + n], orc.block_dots(hq, ora[e][2]))
        assert np.array_equal(y[r0:r0 + n], orc.expert_swiglu(x[r0:r0 + n], *ora[e], 32))
        r0 += n


@pytest.mark.parametrize("ga", [0, 32])
def test_expert_group_reduce(hip, orc, ga):
    say("expert_group_reduce", ga)
    rng = np.random.default_rng(21 + ga)
    D, I = 256, 128
    gpu, ora = _experts(rng, 3, D, I, qt.FMT_I4G, 32, orc, hip)
    rows = [2, 1, 3]
    x = rng.standard_normal((6, D)).astype(np.float32)
    dst = [0, 1, 0, 1, 0, 1]
    rw = rng.uniform(0.1, 1.0, 6).astype(np.float32)
    lay = hip.ReduceLayout.build(dst, 2)
    assert list(lay.row_ptr) == [0, 3, 6]
    hip.set_act_group(ga)
    hip.set_arm(-1)
    out = hip.expert_group_reduce(gpu, rows, x, D, lay, rw, 2)
    y = hip.expert_group(gpu, rows, x, D)
    ref = orc.grouped_reduce(y, lay.row_ptr, lay.row_idx, rw, 2)
    assert np.array_equal(out, ref)
    # repeat: no atomics, so the result is bit-stable
    assert np.array_equal(out, hip.expert_group_reduce(gpu, rows, x, D, lay, rw, 2))


@pytest.mark.parametrize("rows", [[96], [70, 70, 5], [64] * 5])
@pytest.mark.parametrize("fmt,gs", [(qt.FMT_I4G, 32), (qt.FMT_I4, 0)])
@pytest.mark.parametrize("ga", [0, 32])
@pytest.mark.parametrize("graph", [0, 1])
def test_expert_group_weight_reuse_shapes(hip, orc, rows, fmt, gs, ga, graph):
    """int4 expert_group / expert_group_reduce shapes with two or more M tiles
    per expert (the weight-reuse dispatch, XCD-ordered work items) and a grid
    of exactly the M tiles: odd tile counts, 5 experts x 2 tiles, eager and
    through the graph cache, bit-identical to the oracle. The mapped output
    staging buffer is shared by every call, so an unwritten slab would return
    an earlier call's values and fail the comparison."""
    import os
    say("expert_group weight reuse", rows, fmt, gs, ga, graph)
    rng = np.random.default_rng(0x5EED + sum(rows) + fmt + ga + graph)
    D, I = 1536, 640   # gate/up: 5 slabs of 128 channels; down: 6 slabs of 256
    gpu, ora = _experts(rng, len(rows), D, I, fmt, gs or 32, orc, hip)
    R = sum(rows)
    x = rng.standard_normal((R, D)).astype(np.float32)
    dst = rng.integers(0, 7, R).astype(np.int32)
    rw = rng.uniform(0.1, 1.0, R).astype(np.float32)
    lay = hip.ReduceLayout.build(dst, 7)
    hip.set_act_group(ga)
    hip.set_arm(2)
    old = os.environ.get("COLI_HIP_GRAPH")
    os.environ["COLI_HIP_GRAPH"] = str(graph)
    offs = np.concatenate([[0], np.cumsum(rows)])
    ref = np.concatenate([orc.expert_swiglu(x[offs[e]:offs[e + 1]], *ora[e], ga) for e in range(len(rows))])
    ref_out = orc.grouped_reduce(ref, lay.row_ptr, lay.row_idx, rw, 7)
    try:
        for _ in range(2):   # graph: capture, then replay
            y = hip.expert_group(gpu, rows, x, D)
            for e in range(len(rows)):
                a, b = offs[e], offs[e + 1]
                assert np.array_equal(y[a:b], ref[a:b]), f"expert {e}: not bit-identical, err {nerr(y[a:b], ref[a:b])}"
            assert np.array_equal(hip.expert_group_reduce(gpu, rows, x, D, lay, rw, 7), ref_out)
    finally:
        hip.set_arm(-1)
        if old is None:
            os.environ.pop("COLI_HIP_GRAPH", None)
        else:
            os.environ["COLI_HIP_GRAPH"] = old


def test_expert_group_error_paths(hip, orc):
    say("error paths")
    rng = np.random.default_rng(3)
    gpu, _ = _experts(rng, 2, 64, 64, qt.FMT_I4G, 32, orc, hip)
    x = np.zeros((2, 64), np.float32)
    with pytest.raises(hip.HipError):
        hip.expert_group(gpu, [1, 0], x[:1], 64)
    with pytest.raises(hip.HipError):
        hip.expert_group(gpu, [1], x, 64)
    with pytest.raises(hip.HipError):
        hip.expert_group(gpu, [1, 1], x[:1], 64)
    with pytest.raises(hip.HipError):
        hip.expert_group([gpu[0]] * 257, [1] * 257, np.zeros((257, 64), np.float32), 64)
    q, sc, _ = synth.make_tensor(rng, 64, 64, qt.FMT_I4G, 32)
    with pytest.raises(hip.HipError):
        hip._upload(0, q, sc, qt.FMT_I4G, 64, 64, 48)     # unsupported group size
    with pytest.raises(hip.HipError):
        hip._upload(0, q, sc, 3, 64, 64, 0)                # int2 not resident here
    with pytest.raises(hip.HipError):
        hip.GpuExpert.upload(0, None, None, None, 64, 64)
    assert hip.ReduceLayout.build([0, 2], 2) is None
    # an expert whose down shape disagrees is rejected before any launch
    other, _ = _experts(rng, 1, 64, 32, qt.FMT_I4G, 32, orc, hip)
    mixed = hip.GpuExpert(gpu[0].gate, gpu[0].up, other[0].down, 64, 64)
    try:
        with pytest.raises(hip.HipError):
            hip.expert_group([mixed], [1], x[:1], 64)
    finally:
        mixed.gate = mixed.up = mixed.down = None


def test_tensor_update_changes_results(hip, orc):
    say("tensor_update")
    rng = np.random.default_rng(5)
    D, I = 128, 64
    gpu, ora = _experts(rng, 1, D, I, qt.FMT_I4, 0, orc, hip)
    x = rng.standard_normal((1, D)).astype(np.float32)
    hip.set_act_group(0)
    y0 = hip.expert_group(gpu, [1], x, D)
    q, sc, _ = synth.make_tensor(rng, I, D, qt.FMT_I4, 0)
    from peregrine_amd._lib import lib
    import ctypes as C
    assert lib.coli_hip_tensor_update(gpu[0].gate, C.c_void_p(q.ctypes.data), C.c_void_p(sc.ctypes.data)) == 1
    y1 = hip.expert_group(gpu, [1], x, D)
    ref = orc.expert_swiglu(x, orc.Tensor(q, sc, qt.FMT_I4, D, I), ora[0][1], ora[0][2], 0)
    assert not np.array_equal(y0, y1) and np.array_equal(y1, ref)


# ------------------------------------------------------------ device-resident MoE layer

def _layer_case(hip, orc, rng, E, D, I, S, k, fmt=qt.FMT_I4G, gs=32, zipf=False):
    gpu, ora = _experts(rng, E, D, I, fmt, gs, orc, hip)
    eset = hip.ExpertSet(gpu)
    x = rng.standard_normal((S, D)).astype(np.float32)
    logits = synth.zipf_logits(rng, S, E) if zipf else synth.normal_logits(rng, S, E)
    return gpu, ora, eset, x, logits


def _run_layer(hip, eset, x, logits, k, ga, arm):
    S, D = x.shape
    E = logits.shape[1]
    bx = hip.DeviceBuffer.from_array(x)
    bl = hip.DeviceBuffer.from_array(logits)
    bids = hip.DeviceBuffer(S * k * 4)
    bw = hip.DeviceBuffer(S * k * 4)
    bout = hip.DeviceBuffer(S * D * 4)
    hip.route_softmax_topk_dev(0, bl.ptr, S, E, k, bids.ptr, bw.ptr)
    hip.moe_forward_dev(eset, bx.ptr, S, bids.ptr, bw.ptr, k, bout.ptr, ga, arm)
    hip.pipe_sync(0)
    return (bout.download(np.float32, (S, D)), bids.download(np.int32, (S, k)), bw.download(np.float32, (S, k)))


def test_router_matches_oracle(hip, orc):
    say("router")
    rng = np.random.default_rng(8)
    for S, E, k in ((1, 160, 8), (37, 256, 8), (5, 7, 3)):
        logits = synth.normal_logits(rng, S, E)
        logits[0, 3] = logits[0, 5] = np.max(logits[0]) + 1.0   # a tie: lower index first
        bl = hip.DeviceBuffer.from_array(logits)
        bids, bw = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4)
        hip.route_softmax_topk_dev(0, bl.ptr, S, E, k, bids.ptr, bw.ptr)
        hip.pipe_sync(0)
        idx, w = orc.route_softmax_topk(logits, k)
        assert np.array_equal(bids.download(np.int32, (S, k)), idx)
        assert np.array_equal(bw.download(np.float32, (S, k)), w)
        assert list(idx[0][:2]) == [3, 5]


def _adversarial_logits(rng, E):
    """Rows that stress the greedy selection: many equal values, NaN and
    -inf (fewer than k valid), +inf, signed zeros, nothing valid."""
    L = rng.integers(-2, 3, size=(5, E)).astype(np.float32)       # row 0: heavy ties
    L[1] = -np.inf
    L[1, rng.choice(E, 5, replace=False)] = rng.standard_normal(5).astype(np.float32)
    L[1, 0] = np.nan
    L[2] = 0.0
    L[2, 1::3] = -0.0
    L[2, E - 1] = np.inf
    L[3] = -np.inf                                                   # nothing valid
    L[4] = rng.standard_normal(E).astype(np.float32)
    L[4, E // 2] = np.nan
    return L


def test_router_adversarial_matches_oracle(hip, orc):
    say("router adversarial")
    rng = np.random.default_rng(81)
    for E, k in ((200, 8), (64, 8), (256, 16), (9, 4)):
        logits = _adversarial_logits(rng, E)
        S = logits.shape[0]
        bl = hip.DeviceBuffer.from_array(logits)
        bids, bw = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4)
        hip.route_softmax_topk_dev(0, bl.ptr, S, E, k, bids.ptr, bw.ptr)
        hip.pipe_sync(0)
        idx, w = orc.route_softmax_topk(logits, k)
        assert np.array_equal(bids.download(np.int32, (S, k)), idx), E
        # +inf as the top logit makes exp(inf - inf) NaN on both sides
        np.testing.assert_array_equal(bw.download(np.float32, (S, k)), w, err_msg=str(E))
        assert np.all(idx[3] == 0) and np.all(w[3] == 0)


@pytest.mark.parametrize("fused", [1, 0])
@pytest.mark.parametrize("E,D,I,k,ga", [(200, 320, 192, 8, 32), (256, 100, 64, 6, 0), (5, 264, 96, 3, 32),
                                         (160, 5120, 1536, 8, 32)])
def test_one_token_router_paths_match_oracle(hip, orc, fused, E, D, I, k, ga):
    """One token with router logits: the router inside the gate/up GEMV
    (fused=1) and the separate router launch (fused=0) both equal the oracle,
    over normal and adversarial logits, eager and replayed from a graph."""
    say("one-token router", fused, E, D, I, k, ga)
    rng = np.random.default_rng(500 + E + D + fused)
    n_exp = E if D < 1024 else 12
    gpu, ora = _experts(rng, n_exp, D, I, qt.FMT_I4G, 32, orc, hip)
    eset = hip.ExpertSet([gpu[e % n_exp] for e in range(E)])
    ora_full = [ora[e % n_exp] for e in range(E)]
    cases = [synth.normal_logits(rng, 1, E)] + [row[None, :] for row in _adversarial_logits(rng, E)]
    bx = hip.DeviceBuffer(D * 4)
    bl = hip.DeviceBuffer(E * 4)
    bids, bw, bout = hip.DeviceBuffer(k * 4), hip.DeviceBuffer(k * 4), hip.DeviceBuffer(D * 4)
    hip.set_fused_route(fused)
    try:
        def body():
            hip.moe_forward_logits_dev(eset, bx.ptr, 1, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, ga, -1)

        def check(x, logits, tag):
            ids, w = orc.route_softmax_topk(logits, k)
            assert np.array_equal(bids.download(np.int32, (1, k)), ids), tag
            np.testing.assert_array_equal(bw.download(np.float32, (1, k)), w, err_msg=str(tag))   # NaN == NaN
            ref = orc.moe_forward(x, ids, w, ora_full, ga)
            got = bout.download(np.float32, (1, D))
            np.testing.assert_array_equal(got, ref, err_msg=str(tag))

        for ci, logits in enumerate(cases):
            x = rng.standard_normal((1, D)).astype(np.float32)
            bx.upload(x)
            bl.upload(logits)
            body()
            hip.pipe_sync(0)
            check(x, logits, ("eager", ci))
        g = hip.capture(0, body)
        for ci, logits in enumerate(cases[:3]):
            x = rng.standard_normal((1, D)).astype(np.float32)
            bx.upload(x)
            bl.upload(logits)
            g.launch()
            check(x, logits, ("graph", ci))
    finally:
        hip.set_fused_route(-1)


@pytest.mark.parametrize("fmt,gs", FORMATS)
@pytest.mark.parametrize("ga", [0, 32])
def test_one_token_fused_combine(hip, orc, fmt, gs, ga):
    """One token: the down GEMV that also applies the router weights equals
    the separate down + combine launches and the oracle bit for bit, for odd
    and even k, a hidden size that is not a multiple of 16, and shapes past
    its limits (k > 8, K > 1536: the separate launches then run)."""
    say("fused combine", fmt, gs, ga)
    rng = np.random.default_rng(1500 + fmt * 5 + gs + ga)
    for E, D, I, k in ((9, 100, 96, 3), (20, 320, 192, 8), (18, 256, 4608, 16), (4, 64, 64, 1), (6, 96, 1536, 2),
                       (10, 64, 1600, 4)):
        gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, 1, k, fmt=fmt, gs=gs or 32)
        outs = []
        for fc in (1, 0):
            hip.set_fused_combine(fc)
            try:
                out, ids, w = _run_layer(hip, eset, x, logits, k, ga, 2)
            finally:
                hip.set_fused_combine(-1)
            outs.append(out)
        ref = orc.moe_forward(x, ids, w, ora, ga)
        assert np.array_equal(outs[0], outs[1]), (E, D, I, k)
        assert np.array_equal(outs[0], ref), (E, D, I, k, nerr(outs[0], ref))


@pytest.mark.parametrize("ga", [0, 32])
@pytest.mark.parametrize("arm", [2, 0])
def test_moe_layer_matches_oracle(hip, orc, ga, arm):
    say("moe layer", ga, arm)
    rng = np.random.default_rng(40 + ga + arm)
    E, D, I, S, k = 12, 256, 192, 19, 4
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k, zipf=True)
    out, ids, w = _run_layer(hip, eset, x, logits, k, ga, arm)
    ref = orc.moe_forward(x, ids, w, ora, ga)
    assert nerr(out, ref) <= TOL
    assert np.array_equal(out, ref)
    # the device-built expert-offset table equals the oracle's
    t = hip.last_table(0, E, S * k)
    o = orc.expert_table(ids, E)
    assert t["n_u"] == o["n_u"] and np.array_equal(t["uexp"], o["uexp"]) and np.array_equal(t["off"], o["off"])
    assert np.array_equal(t["row_tok"], o["row_tok"])
    assert np.array_equal(t["tok_rows"].reshape(S, k), o["tok_rows"])


@pytest.mark.parametrize("S,arm", [(1, -1), (1, 0), (6, 2), (6, -1)])
@pytest.mark.parametrize("ga", [32, 0])
def test_moe_layer_fused_router_matches_oracle(hip, orc, S, arm, ga):
    """Router fused with the x quantisation; one token on the GEMV arm runs
    without an expert table."""
    say("fused router layer", S, arm, ga)
    rng = np.random.default_rng(300 + S + arm + ga)
    E, D, I, k = 20, 320, 192, 6
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k)
    bx, bl = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(logits)
    bids, bw, bout = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * D * 4)
    for rep in range(3):   # repeats: no state may carry over between calls
        hip.moe_forward_logits_dev(eset, bx.ptr, S, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, ga, arm)
        hip.pipe_sync(0)
        out = bout.download(np.float32, (S, D))
        ids, w = orc.route_softmax_topk(logits, k)
        assert np.array_equal(bids.download(np.int32, (S, k)), ids)
        assert np.array_equal(bw.download(np.float32, (S, k)), w)
        ref = orc.moe_forward(x, ids, w, ora, ga)
        assert np.array_equal(out, ref), (rep, nerr(out, ref))


@pytest.mark.parametrize("ga", [32, 0])
@pytest.mark.parametrize("fmt,gs", FORMATS)
def test_mfma_dense_and_streaming_dispatches(hip, orc, ga, fmt, gs):
    """MFMA dispatches with many rows per expert (full 32-row tiles; two or
    more tiles per expert, so the weight copies stay cacheable) and with
    under two (ragged tiles, non-temporal copies) equal the oracle bit for bit."""
    say("mfma dense/streaming", ga, fmt, gs)
    rng = np.random.default_rng(610 + ga + fmt)
    for E, S, k in ((3, 100, 2), (16, 9, 3)):   # 67 rows per expert, then under 2
        gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, 288, 160, S, k, fmt=fmt, gs=gs or 32)
        out, ids, w = _run_layer(hip, eset, x, logits, k, ga, 2)
        ref = orc.moe_forward(x, ids, w, ora, ga)
        assert np.array_equal(out, ref), (E, S, k, nerr(out, ref))


@pytest.mark.parametrize("fmt,D", [(qt.FMT_I4G, 5120), (qt.FMT_I4G, 6400), (qt.FMT_I4G, 7680), (qt.FMT_I4G, 8320),
                                   (qt.FMT_I8G, 768), (qt.FMT_I8G, 2048), (qt.FMT_I8G, 5120), (qt.FMT_I8G, 8320)])
def test_mfma_staging_tiers(hip, orc, fmt, D):
    """Per-32 activation scales with a hidden size at each gate/up staging
    tier of the MFMA arm: three blocks ahead at three workgroups per CU, two
    ahead at three, the deep tier at two, and the register-prefetch kernel
    past them; bit-identical to the oracle."""
    say("mfma tiers", fmt, D)
    rng = np.random.default_rng(720 + D + fmt)
    E, I, S, k = 3, 64, 40, 2
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k, fmt=fmt)
    out, ids, w = _run_layer(hip, eset, x, logits, k, 32, 0)
    ref = orc.moe_forward(x, ids, w, ora, 32)
    assert np.array_equal(out, ref), nerr(out, ref)


def test_moe_layer_arms_agree_and_repeat(hip, orc):
    say("arms agree")
    rng = np.random.default_rng(77)
    E, D, I, S, k = 10, 192, 128, 6, 3
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k)
    a, _, _ = _run_layer(hip, eset, x, logits, k, 32, 2)
    b, _, _ = _run_layer(hip, eset, x, logits, k, 32, 0)
    c, _, _ = _run_layer(hip, eset, x, logits, k, 32, 0)
    assert np.array_equal(a, b) and np.array_equal(b, c)


@pytest.mark.parametrize("ga", [32, 0])
def test_decode_layer_full_shape(hip, orc, ga):
    """BASELINE config 2 shape (D=5120, I=1536, top-8) with 16 resident experts."""
    say("decode full shape", ga)
    rng = np.random.default_rng(2024 + ga)
    E, D, I, S, k = 16, 5120, 1536, 1, 8
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k)
    out, ids, w = _run_layer(hip, eset, x, logits, k, ga, -1)
    ref = orc.moe_forward(x, ids, w, ora, ga)
    assert nerr(out, ref) <= TOL, nerr(out, ref)


def test_batched_layer_full_width_sampled(hip, orc):
    """BASELINE config 3 widths (64 tokens, Zipf top-8), checked on 6 sampled tokens."""
    say("batched 64 tokens")
    rng = np.random.default_rng(64)
    E, D, I, S, k = 24, 5120, 1536, 64, 8
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k, zipf=True)
    out, ids, w = _run_layer(hip, eset, x, logits, k, 32, -1)
    sub = np.array([0, 5, 17, 33, 48, 63])
    ref = orc.moe_forward(x, ids, w, ora, 32, subset=sub, nthreads=8)
    assert nerr(out[sub], ref[sub]) <= TOL


def test_prefill_layer_full_width_sampled(hip, orc):
    """BASELINE config 4 widths (2048 tokens, Zipf top-8; about 680 rows per
    expert, so every expert spans many M tiles and the weight copies stay
    cacheable), checked on 6 sampled tokens."""
    say("prefill 2048 tokens")
    rng = np.random.default_rng(2048)
    E, D, I, S, k = 24, 5120, 1536, 2048, 8
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k, zipf=True)
    out, ids, w = _run_layer(hip, eset, x, logits, k, 32, -1)
    sub = np.array([0, 1, 511, 1024, 1777, 2047])
    ref = orc.moe_forward(x, ids, w, ora, 32, subset=sub, nthreads=8)
    assert nerr(out[sub], ref[sub]) <= TOL


@pytest.mark.parametrize("S,k,E", [(3, 2, 8), (1, 2, 8), (300, 8, 20)])
def test_graph_replay_matches_eager(hip, orc, S, k, E):
    """Replays of a captured layer equal eager runs, with eager work and
    synchronisations between the replays (S = 1: the one-token path; S = 300,
    k = 8: the three-launch expert table)."""
    say("graph replay", S, k, E)
    rng = np.random.default_rng(91 + S)
    D, I = 256, 128
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k)
    bx = hip.DeviceBuffer.from_array(x)
    bl = hip.DeviceBuffer.from_array(logits)
    bids, bw, bout = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * D * 4)

    def body():
        hip.route_softmax_topk_dev(0, bl.ptr, S, E, k, bids.ptr, bw.ptr)
        hip.moe_forward_dev(eset, bx.ptr, S, bids.ptr, bw.ptr, k, bout.ptr, 32, -1)

    body()   # eager first: reserves every scratch buffer the capture will bake in
    hip.pipe_sync(0)
    eager = bout.download(np.float32, (S, D))
    g = hip.capture(0, body)
    for rep in range(4):
        x2 = rng.standard_normal((S, D)).astype(np.float32)
        bx.upload(x2)
        g.launch()
        got = bout.download(np.float32, (S, D))
        body()
        hip.pipe_sync(0)
        assert np.array_equal(got, bout.download(np.float32, (S, D))), rep
    bx.upload(x)
    g.launch()
    assert np.array_equal(bout.download(np.float32, (S, D)), eager)


def test_graph_refused_after_scratch_growth(hip, orc):
    """A captured layer holds the addresses of the library's scratch buffers.
    Once a larger eager call reallocates them, launching the old graph is
    refused on the host (nothing runs), and a fresh capture replays the
    eager result."""
    say("graph refused after scratch growth")
    rng = np.random.default_rng(4321)
    E, D, I, S, k = 8, 256, 128, 3, 2
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k)
    bx, bl = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(logits)
    bids, bw, bout = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * D * 4)

    def body():
        hip.route_softmax_topk_dev(0, bl.ptr, S, E, k, bids.ptr, bw.ptr)
        hip.moe_forward_dev(eset, bx.ptr, S, bids.ptr, bw.ptr, k, bout.ptr, 32, -1)

    body()
    hip.pipe_sync(0)
    eager = bout.download(np.float32, (S, D))
    g = hip.capture(0, body)
    g.launch()
    assert np.array_equal(bout.download(np.float32, (S, D)), eager)
    # 65536 rows: more than any other call in the suite, so the row tables grow
    big_x = rng.standard_normal((8192, D)).astype(np.float32)
    _run_layer(hip, eset, big_x, synth.normal_logits(rng, 8192, E), 8, 32, -1)
    with pytest.raises(hip.HipError):
        g.launch()
    g2 = hip.capture(0, body)
    g2.launch()
    assert np.array_equal(bout.download(np.float32, (S, D)), eager)


def test_greedy_argmax_token_identical(hip, orc):
    """Random-init MoE-only stack (embedding -> 3 MoE layers with residual ->
    lm_head argmax); the GPU and the oracle generate the same tokens."""
    say("greedy argmax")
    rng = np.random.default_rng(0xC0FFEE)
    V, D, I, E, k, L, B, steps = 64, 128, 64, 8, 2, 3, 4, 12
    emb = rng.standard_normal((V, D)).astype(np.float32)
    head = rng.standard_normal((V, D)).astype(np.float32)
    layers = []
    for _ in range(L):
        gpu, ora = _experts(rng, E, D, I, qt.FMT_I4G, 32, orc, hip)
        router = (rng.standard_normal((E, D)) * 0.1).astype(np.float32)
        layers.append((hip.ExpertSet(gpu), gpu, ora, router))
    tok_g = rng.integers(0, V, B)
    tok_o = tok_g.copy()
    seq_g, seq_o = [], []
    for _ in range(steps):
        for side in ("gpu", "ora"):
            tok = tok_g if side == "gpu" else tok_o
            x = emb[tok].copy()
            for eset, gpu, ora, router in layers:
                logits = orc.matmul_f32(x, router, D, E)
                if side == "gpu":
                    out, _, _ = _run_layer(hip, eset, x, logits, k, 0, -1)
                else:
                    ids, w = orc.route_softmax_topk(logits, k)
                    out = orc.moe_forward(x, ids, w, ora, 0)
                x = (x + out).astype(np.float32)
            nxt = np.argmax(orc.matmul_f32(x, head, D, V), axis=1)
            if side == "gpu":
                tok_g = nxt
                seq_g.append(nxt)
            else:
                tok_o = nxt
                seq_o.append(nxt)
    assert np.array_equal(np.array(seq_g), np.array(seq_o))


@pytest.mark.parametrize("ga,arm,B", [(32, -1, 1), (0, -1, 1), (32, 2, 4), (0, 0, 4), (32, -1, 64), (0, -1, 64)])
def test_greedy_argmax_baseline_width(hip, orc, ga, arm, B):
    """Greedy decoding at the BASELINE decode widths (generate_is_deterministic_greedy,
    model.rs:5354-5366, restated on a MoE-only stack): D=5120, I=1536, two
    MoE layers of 160 expert slots aliasing 12 distinct experts each, top-8
    from the device router on host-computed router logits, residual, lm_head
    argmax, 8 steps. Batch 1 runs the one-token decode path (automatic arm:
    GEMV with the fused router), batch 4 forces each arm, batch 64 takes the
    automatic MFMA arm. Every layer output and every generated token equals
    the oracle's."""
    say("greedy argmax baseline width", ga, arm, B)
    rng = np.random.default_rng(0xC0FFEE + ga + B)
    V, D, I, E, n_dist, k, L, steps = 96, 5120, 1536, 160, 12, 8, 2, 8
    emb = rng.standard_normal((V, D)).astype(np.float32)
    head = rng.standard_normal((V, D)).astype(np.float32)
    layers = []
    for _ in range(L):
        gpu, ora = _experts(rng, n_dist, D, I, qt.FMT_I4G, 32, orc, hip)
        router = (rng.standard_normal((E, D)) * 0.02).astype(np.float32)
        layers.append((hip.ExpertSet([gpu[e % n_dist] for e in range(E)]), [ora[e % n_dist] for e in range(E)],
                       router))
    bx, bl = hip.DeviceBuffer(B * D * 4), hip.DeviceBuffer(B * E * 4)
    bids, bw, bout = hip.DeviceBuffer(B * k * 4), hip.DeviceBuffer(B * k * 4), hip.DeviceBuffer(B * D * 4)
    tok = rng.integers(0, V, B)
    seq_g, seq_o = [], []
    tok_g, tok_o = tok.copy(), tok.copy()
    for step in range(steps):
        xg, xo = emb[tok_g].copy(), emb[tok_o].copy()
        for li, (eset, ora, router) in enumerate(layers):
            lg = orc.matmul_f32(xg, router, D, E)
            bx.upload(xg)
            bl.upload(lg)
            hip.moe_forward_logits_dev(eset, bx.ptr, B, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, ga, arm)
            hip.pipe_sync(0)
            og = bout.download(np.float32, (B, D))
            lo = orc.matmul_f32(xo, router, D, E)
            ids, w = orc.route_softmax_topk(lo, k)
            oo = orc.moe_forward(xo, ids, w, ora, ga, nthreads=16, simd=orc.have_avx2())
            assert np.array_equal(og, oo), (step, li, nerr(og, oo))
            xg = (xg + og).astype(np.float32)
            xo = (xo + oo).astype(np.float32)
        tok_g = np.argmax(orc.matmul_f32(xg, head, D, V), axis=1)
        tok_o = np.argmax(orc.matmul_f32(xo, head, D, V), axis=1)
        seq_g.append(tok_g)
        seq_o.append(tok_o)
    assert np.array_equal(np.array(seq_g), np.array(seq_o))
    # the stack is not degenerate: the batch's tokens differ
    if B > 1:
        assert len(np.unique(np.array(seq_g))) > 1


@pytest.mark.parametrize("arm", [-1, 0, 2])
def test_golden_layer_bit_exact(hip, arm):
    """The committed fixture (tests/golden/moe_layer_small.npz): device
    routing, table, both activation-scale modes and every arm reproduce the
    stored oracle outputs bit-for-bit."""
    import os
    say("golden layer", arm)
    f = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "moe_layer_small.npz"))
    E, D, I, S, k = (int(v) for v in f["dims"])
    gpu = [hip.GpuExpert.upload_grouped(0, (f[f"e{e}_gate_q"], f[f"e{e}_gate_s"]),
                                        (f[f"e{e}_up_q"], f[f"e{e}_up_s"]),
                                        (f[f"e{e}_down_q"], f[f"e{e}_down_s"]), D, I, qt.FMT_I4G, 32)
           for e in range(E)]
    eset = hip.ExpertSet(gpu)
    bx, bl = hip.DeviceBuffer.from_array(f["x"]), hip.DeviceBuffer.from_array(f["logits"])
    bids, bw, bout = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * D * 4)
    for ga in (0, 32):
        hip.moe_forward_logits_dev(eset, bx.ptr, S, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, ga, arm)
        hip.pipe_sync(0)
        assert np.array_equal(bids.download(np.int32, (S, k)), f["ids"])
        assert bw.download(np.float32, (S, k)).tobytes() == f["w"].tobytes()
        assert bout.download(np.float32, (S, D)).tobytes() == f[f"y_ga{ga}"].tobytes(), ga


@pytest.mark.parametrize("S,k,E", [(600, 8, 40), (300, 16, 24), (1100, 1, 12), (512, 8, 256), (500, 8, 160), (256, 16, 512), (4096, 1, 7)])
def test_expert_table_many_passes(hip, orc, S, k, E):
    """The device-built expert-offset table for batches that take several
    placement passes (and multi-word token masks) equals the oracle's, and the
    layer output stays bit-identical."""
    say("table many passes", S, k, E)
    rng = np.random.default_rng(900 + S + k)
    D, I = 64, 32
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k, zipf=True)
    out, ids, w = _run_layer(hip, eset, x, logits, k, 32, 0)
    t = hip.last_table(0, E, S * k)
    o = orc.expert_table(ids, E)
    assert t["n_u"] == o["n_u"] and np.array_equal(t["uexp"], o["uexp"]) and np.array_equal(t["off"], o["off"])
    assert np.array_equal(t["row_tok"], o["row_tok"])
    assert np.array_equal(t["tok_rows"].reshape(S, k), o["tok_rows"])
    sub = np.arange(0, S, max(1, S // 40))
    ref = orc.moe_forward(x, ids, w, ora, 32, subset=sub, nthreads=8)
    assert np.array_equal(out[sub], ref[sub])


@pytest.mark.parametrize("S,k,E", [(300, 6, 20), (40, 16, 5), (513, 3, 300), (600, 16, 512)])
def test_expert_table_duplicate_and_invalid_ids(hip, orc, S, k, E):
    """Caller-supplied ids with repeated experts inside a token and ids out of
    range (skipped): table and layer equal the oracle's."""
    say("table duplicate/invalid ids", S, k, E)
    rng = np.random.default_rng(1300 + S + k)
    D, I = 64, 32
    n_exp = min(E, 24)
    gpu, ora = _experts(rng, n_exp, D, I, qt.FMT_I4G, 32, orc, hip)
    eset = hip.ExpertSet([gpu[e % n_exp] for e in range(E)])
    ora_full = [ora[e % n_exp] for e in range(E)]
    ids = rng.integers(-2, E + 2, size=(S, k)).astype(np.int32)
    ids[::7, 1:] = ids[::7, :1]            # every seventh token: one expert in every slot
    w = rng.random((S, k)).astype(np.float32)
    x = rng.standard_normal((S, D)).astype(np.float32)
    bx, bids, bw = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(ids), hip.DeviceBuffer.from_array(w)
    bout = hip.DeviceBuffer(S * D * 4)
    hip.moe_forward_dev(eset, bx.ptr, S, bids.ptr, bw.ptr, k, bout.ptr, 32, 0)
    hip.pipe_sync(0)
    out = bout.download(np.float32, (S, D))
    t = hip.last_table(0, E, S * k)
    o = orc.expert_table(ids, E)
    assert t["n_u"] == o["n_u"] and np.array_equal(t["uexp"], o["uexp"]) and np.array_equal(t["off"], o["off"])
    assert np.array_equal(t["row_tok"], o["row_tok"])
    assert np.array_equal(t["tok_rows"].reshape(S, k), o["tok_rows"])
    ref = orc.moe_forward(x, ids, w, ora_full, 32)
    assert np.array_equal(out, ref), nerr(out, ref)


@pytest.mark.parametrize("arm", [2, -1, 0])
def test_one_token_caller_ids(hip, orc, arm):
    """One token with caller-supplied ids: out-of-range ids are skipped and a
    repeated expert adds both rows in slot order, as in the oracle (these ids
    go through the table, never straight to the expert descriptors)."""
    say("one token caller ids", arm)
    rng = np.random.default_rng(1700 + arm)
    E, D, I, k = 10, 96, 64, 4
    gpu, ora = _experts(rng, E, D, I, qt.FMT_I4G, 32, orc, hip)
    eset = hip.ExpertSet(gpu)
    x = rng.standard_normal((1, D)).astype(np.float32)
    bx, bout = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer(D * 4)
    for ids in ([[3, -1, 3, 12]], [[0, 1, 2, 3]], [[-5, 10, 11, -1]], [[7, 7, 7, 7]]):
        ids = np.array(ids, np.int32)
        w = rng.random((1, k)).astype(np.float32)
        bids, bw = hip.DeviceBuffer.from_array(ids), hip.DeviceBuffer.from_array(w)
        hip.moe_forward_dev(eset, bx.ptr, 1, bids.ptr, bw.ptr, k, bout.ptr, 32, arm)
        hip.pipe_sync(0)
        ref = orc.moe_forward(x, ids, w, ora, 32)
        np.testing.assert_array_equal(bout.download(np.float32, (1, D)), ref, err_msg=str(ids))


@pytest.mark.parametrize("min_share,norm,scale", [(0.0, True, 2.5), (0.05, True, 1.0), (0.02, False, 1.7)])
def test_sigmoid_router_matches_oracle(hip, orc, min_share, norm, scale):
    """The reference router (router.rs:52-170) on the device equals the
    oracle bit-for-bit: bias-augmented selection, ties, NaN and -inf logits,
    the negligible tail and renormalisation."""
    say("sigmoid router", min_share, norm, scale)
    rng = np.random.default_rng(31)
    S, E, k = 37, 160, 8
    logits = rng.standard_normal((S, E)).astype(np.float32) * 3
    logits[0, 5] = logits[0, 9] = 4.0          # ties go to the lower index
    logits[1, :] = np.nan                      # nothing selectable
    logits[2, : E - 3] = np.nan                # fewer than k selectable
    logits[3, 7] = -np.inf
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    bl, bb = hip.DeviceBuffer.from_array(logits), hip.DeviceBuffer.from_array(bias)
    bids, bw, bk = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * 4)
    hip.route_sigmoid_topk_dev(0, bl.ptr, bb.ptr, S, E, k, bids.ptr, bw.ptr, bk.ptr, norm, scale, min_share)
    hip.pipe_sync(0)
    ids, w, keff = orc.route_sigmoid(logits, bias, k, norm, scale, min_share)
    assert np.array_equal(bids.download(np.int32, (S, k)), ids)
    assert bw.download(np.float32, (S, k)).tobytes() == w.tobytes()
    assert np.array_equal(bk.download(np.int32, (S,)), keff)


@pytest.mark.parametrize("fmt", [qt.FMT_I4G, qt.FMT_I4, qt.FMT_I8])
def test_experts_from_qt_container(hip, orc, fmt, tmp_path):
    """The QT loader bridge: experts written to a model.safetensors container
    (some tensors kblock-tiled) are detected, read and uploaded; the expert
    group then equals the oracle on the row-major bytes, bit-for-bit."""
    from peregrine_amd import qtfile as Q
    say("qt container", fmt)
    rng = np.random.default_rng(700 + fmt)
    D, I, E = 256, 128, 3
    blobs, ora = [], []
    for e in range(E):
        trip = synth.make_expert(rng, D, I, fmt, 32)
        shp = ((I, D), (I, D), (D, I))
        ora.append(tuple(orc.Tensor(t[0], t[1], fmt, i, o, 32) for t, (o, i) in zip(trip, shp)))
        for m, (name, (o, i)) in enumerate(zip(("gate", "up", "down"), shp)):
            q = np.asarray(trip[m][0], np.uint8).reshape(-1)
            sc = np.asarray(trip[m][1], np.float32).reshape(-1)
            row_bytes = q.size // o
            if fmt == qt.FMT_I4G and (e + m) % 2 == 0:   # every other tensor kblock-tiled by group
                blobs.append((f"e{e}.{name}", "U8", [o, row_bytes], Q.to_kblock(q, o, 16), ("kblock", 16)))
            else:
                blobs.append((f"e{e}.{name}", "U8", [o, row_bytes], q))
            blobs.append((f"e{e}.{name}.qs", "F32", [sc.size], sc))
    Q.write_qt(str(tmp_path / "model.safetensors"), blobs)
    with Q.QtFile(str(tmp_path)) as f:
        gpu = [Q.upload_expert(0, f, f"e{e}.gate", f"e{e}.up", f"e{e}.down", D, I) for e in range(E)]
    rows = [2, 5, 1]
    x = rng.standard_normal((sum(rows), D)).astype(np.float32)
    hip.set_act_group(0)
    hip.set_arm(-1)
    y = hip.expert_group(gpu, rows, x, D)
    r0 = 0
    for e, n in enumerate(rows):
        ref = orc.expert_swiglu(x[r0:r0 + n], *ora[e], 0)
        assert np.array_equal(y[r0:r0 + n], ref), e
        r0 += n


@pytest.mark.parametrize("S,arm", [(1, 2), (5, 0), (5, 2)])
def test_limits_512_experts_top16(hip, orc, S, arm):
    """The largest supported dispatch: 512 experts, top-16 (the router runs
    16 logits per lane, the GEMV one-token path 16 rows, the table 16 slots),
    with router logits and with given ids; past the limits the calls fail."""
    say("limits", S, arm)
    rng = np.random.default_rng(5120 + S + arm)
    E, D, I, k = 512, 96, 64, 16
    n_real = 24   # 512 table entries over 24 distinct uploaded experts
    gpu, ora = _experts(rng, n_real, D, I, qt.FMT_I4G, 32, orc, hip)
    eset = hip.ExpertSet([gpu[e % n_real] for e in range(E)])
    ora_full = [ora[e % n_real] for e in range(E)]
    x = rng.standard_normal((S, D)).astype(np.float32)
    logits = synth.normal_logits(rng, S, E)
    bx, bl = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(logits)
    bids, bw, bout = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * D * 4)
    hip.moe_forward_logits_dev(eset, bx.ptr, S, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, 32, arm)
    hip.pipe_sync(0)
    ids, w = orc.route_softmax_topk(logits, k)
    assert np.array_equal(bids.download(np.int32, (S, k)), ids)
    assert np.array_equal(bw.download(np.float32, (S, k)), w)
    ref = orc.moe_forward(x, ids, w, ora_full, 32)
    assert np.array_equal(bout.download(np.float32, (S, D)), ref)
    # given ids (the second path), same result
    hip.moe_forward_dev(eset, bx.ptr, S, bids.ptr, bw.ptr, k, bout.ptr, 32, arm)
    hip.pipe_sync(0)
    assert np.array_equal(bout.download(np.float32, (S, D)), ref)
    # one past each limit is refused, with nothing launched
    b17 = hip.DeviceBuffer(S * 17 * 4)
    with pytest.raises(hip.HipError):
        hip.moe_forward_logits_dev(eset, bx.ptr, S, bl.ptr, 17, b17.ptr, b17.ptr, bout.ptr, 32, arm)
    big = hip.ExpertSet([gpu[e % n_real] for e in range(E + 1)])
    bl2 = hip.DeviceBuffer.from_array(synth.normal_logits(rng, S, E + 1))
    with pytest.raises(hip.HipError):
        hip.moe_forward_logits_dev(big, bx.ptr, S, bl2.ptr, k, bids.ptr, bw.ptr, bout.ptr, 32, arm)


# ------------------------------------------------------------ BASELINE configs 1 and 5 at size

@pytest.mark.parametrize("ga", [32, 0])
def test_single_expert_fused_down_combine_full_shape(hip, orc, ga):
    """one expert, one token, D=5120, I=1536, k=1. The down
    projection runs gemv_down_combine_kernel at its widest K (48 blocks =
    DC_MAXNB); bit-identical to the oracle (matmul.rs:93-106, mlp.rs:21-26)."""
    say("config 1 full shape", ga)
    rng = np.random.default_rng(5120 + ga)
    E, D, I, S, k = 1, 5120, 1536, 1, 1
    gpu, ora, eset, x, logits = _layer_case(hip, orc, rng, E, D, I, S, k)
    bx, bl = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(logits)
    bids, bw, bout = hip.DeviceBuffer(4), hip.DeviceBuffer(4), hip.DeviceBuffer(D * 4)
    for mode in (-1, 0):   # automatic (k = 1: fused) and the separate down + combine
        hip.set_fused_combine(mode)
        try:
            hip.moe_forward_logits_dev(eset, bx.ptr, 1, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, ga)
            hip.pipe_sync(0)
        finally:
            hip.set_fused_combine(-1)
        ids, w = bids.download(np.int32, (1, 1)), bw.download(np.float32, (1, 1))
        assert ids[0, 0] == 0 and w[0, 0] == 1.0
        out = bout.download(np.float32, (1, D))
        ref = orc.moe_forward(x, ids, w, ora, ga)
        assert np.array_equal(out, ref), (mode, nerr(out, ref))


def _cfg5_case(hip, orc, fmt, seed, n_dist=16):
    """BASELINE config 5 shape: D=6144, I=2048, 256 experts, 512 tokens,
    uniform top-8. The 256 expert slots alias n_dist distinct uploaded experts
    (device memory and host oracle time), so the dispatch has config 5's
    table, tile count and kernel instantiations (about 16 rows per expert:
    non-temporal weight copies)."""
    rng = np.random.default_rng(seed)
    E, D, I, S = 256, 6144, 2048, 512
    gpu, ora = _experts(rng, n_dist, D, I, fmt, 32, orc, hip)
    eset = hip.ExpertSet([gpu[e % n_dist] for e in range(E)])
    ora_full = [ora[e % n_dist] for e in range(E)]
    x = rng.standard_normal((S, D)).astype(np.float32)
    logits = synth.normal_logits(rng, S, E)
    return gpu, ora_full, eset, x, logits


@pytest.mark.parametrize("fmt", [qt.FMT_I4G, qt.FMT_I8G])
def test_large_layer_cfg5_sampled(hip, orc, fmt):
    """Config 5 through both device-resident entry points (router fused with
    the activation quant, then precomputed ids as the bench's later layers),
    int4 and int8 weights, sampled tokens bit-identical to the oracle
    (matmul.rs:61-72 int8, idot.rs:98-110 grouped)."""
    say("config 5", fmt)
    gpu, ora, eset, x, logits = _cfg5_case(hip, orc, fmt, 6144 + fmt)
    S, D, E, k = 512, 6144, 256, 8
    bx, bl = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(logits)
    bids, bw = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4)
    b1, b2 = hip.DeviceBuffer(S * D * 4), hip.DeviceBuffer(S * D * 4)
    hip.moe_forward_logits_dev(eset, bx.ptr, S, bl.ptr, k, bids.ptr, bw.ptr, b1.ptr, 32)
    hip.moe_forward_dev(eset, bx.ptr, S, bids.ptr, bw.ptr, k, b2.ptr, 32)
    hip.pipe_sync(0)
    ids, w = bids.download(np.int32, (S, k)), bw.download(np.float32, (S, k))
    ri, rw = orc.route_softmax_topk(logits, k)
    assert np.array_equal(ids, ri) and np.array_equal(w, rw)
    o1, o2 = b1.download(np.float32, (S, D)), b2.download(np.float32, (S, D))
    assert np.array_equal(o1, o2)
    sub = np.array([0, 1, 130, 257, 400, 511])
    ref = orc.moe_forward(x, ids, w, ora, 32, subset=sub, nthreads=8)
    assert np.array_equal(o1[sub], ref[sub]), nerr(o1[sub], ref[sub])
    assert np.all(np.isfinite(o1))


def _aliased_case(hip, orc, fmt, seed, E, D, I, S, n_dist, zipf):
    """E expert slots aliasing n_dist distinct uploaded experts, so a dispatch
    has the configuration's routing, expert-offset table and M-tile count."""
    rng = np.random.default_rng(seed)
    gpu, ora = _experts(rng, n_dist, D, I, fmt, 32, orc, hip)
    eset = hip.ExpertSet([gpu[e % n_dist] for e in range(E)])
    ora_full = [ora[e % n_dist] for e in range(E)]
    x = rng.standard_normal((S, D)).astype(np.float32)
    logits = synth.zipf_logits(rng, S, E) if zipf else synth.normal_logits(rng, S, E)
    return gpu, ora_full, eset, x, logits


@pytest.mark.parametrize("fmt", [qt.FMT_I4G, qt.FMT_I8G])
def test_batched_layer_cfg3_all_tokens(hip, orc, fmt):
    """BASELINE config 3 at its shape: 160 expert slots, 64 tokens, Zipf(1.1)
    top-8 (1-40 rows per expert), every token bit-identical to the oracle."""
    say("config 3, 160 slots", fmt)
    gpu, ora, eset, x, logits = _aliased_case(hip, orc, fmt, 3160 + fmt, 160, 5120, 1536, 64, 24, True)
    out, ids, w = _run_layer(hip, eset, x, logits, 8, 32, -1)
    ref = orc.moe_forward(x, ids, w, ora, 32, nthreads=8)
    assert np.array_equal(out, ref), nerr(out, ref)


def test_prefill_layer_cfg4_sampled(hip, orc):
    """BASELINE config 4 at its shape: 160 expert slots, 2048 tokens, Zipf(1.1)
    top-8 (16,384 rows, popular experts over many M tiles: weight-reuse
    dispatch), 64 sampled tokens bit-identical to the oracle."""
    say("config 4, 160 slots")
    gpu, ora, eset, x, logits = _aliased_case(hip, orc, qt.FMT_I4G, 4160, 160, 5120, 1536, 2048, 24, True)
    out, ids, w = _run_layer(hip, eset, x, logits, 8, 32, -1)
    sub = np.arange(0, 2048, 32)
    ref = orc.moe_forward(x, ids, w, ora, 32, subset=sub, nthreads=8)
    assert np.array_equal(out[sub], ref[sub]), nerr(out[sub], ref[sub])


@pytest.mark.parametrize("cfg", ["cfg4", "cfg5"])
def test_full_size_duplicate_tokens_agree(hip, orc, cfg):
    """A size-independent property over every token at full size: the second
    half of the batch repeats the first (same x, same logits), so each token
    and its copy take the same experts in the same order. Their rows sit at
    other positions of other M tiles (the copies extend every expert's row
    range), yet every output must agree bit for bit, and a sample of tokens
    must equal the oracle."""
    say("full-size duplicates", cfg)
    if cfg == "cfg4":
        E, D, I, S, n_dist, zipf = 160, 5120, 1536, 2048, 24, True
    else:
        E, D, I, S, n_dist, zipf = 256, 6144, 2048, 512, 16, False
    gpu, ora, eset, x, logits = _aliased_case(hip, orc, qt.FMT_I4G, 9000 + S, E, D, I, S, n_dist, zipf)
    h = S // 2
    x[h:] = x[:h]
    logits[h:] = logits[:h]
    out, ids, w = _run_layer(hip, eset, x, logits, 8, 32, -1)
    assert np.array_equal(ids[:h], ids[h:])
    assert np.array_equal(out[:h], out[h:])
    assert np.all(np.isfinite(out))
    sub = np.array([0, h - 1, h, S - 1])
    ref = orc.moe_forward(x, ids, w, ora, 32, subset=sub, nthreads=8)
    assert np.array_equal(out[sub], ref[sub]), nerr(out[sub], ref[sub])


def test_device_exp_equals_glibc_through_the_routers(hip, orc):
    """The kernels' exp (expf_glibc) against glibc's expf, through the two
    routers. Softmax: the top logit is 0 and the other 15 kept logits are the
    arguments d in [-104, 0], so the weights are exp(d) / sum, subnormal
    exp(d) included (d below -87.3). Sigmoid (no renormalisation): the
    weights are 1 / (1 + exp(-l)) for l in [-89, 104], exp's overflow
    included. Bit-identical to the oracle, which calls glibc's expf."""
    say("device exp sweep")
    rng = np.random.default_rng(2718)
    S, E, k = 8192, 16, 16
    d = np.linspace(-104.0, 0.0, S * (E - 1), dtype=np.float32)
    d = rng.permutation(d).reshape(S, E - 1)
    logits = np.concatenate([np.zeros((S, 1), np.float32), d], axis=1)
    bl = hip.DeviceBuffer.from_array(logits)
    bids, bw = hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4)
    hip.route_softmax_topk_dev(0, bl.ptr, S, E, k, bids.ptr, bw.ptr)
    hip.pipe_sync(0)
    ids, w = orc.route_softmax_topk(logits, k)
    assert np.array_equal(bids.download(np.int32, (S, k)), ids)
    assert bw.download(np.float32, (S, k)).tobytes() == w.tobytes()
    assert np.any((w > 0) & (w < np.finfo(np.float32).tiny))   # the subnormal range was reached

    lg = rng.permutation(np.linspace(-89.0, 104.0, S * E, dtype=np.float32)).reshape(S, E)
    bl2 = hip.DeviceBuffer.from_array(lg)
    zero = hip.DeviceBuffer.from_array(np.zeros(E, np.float32))
    bk = hip.DeviceBuffer(S * 4)
    hip.route_sigmoid_topk_dev(0, bl2.ptr, zero.ptr, S, E, k, bids.ptr, bw.ptr, bk.ptr, False, 1.0, 0.0)
    hip.pipe_sync(0)
    ids2, w2, _ = orc.route_sigmoid(lg, np.zeros(E, np.float32), k, False, 1.0, 0.0)
    assert np.array_equal(bids.download(np.int32, (S, k)), ids2)
    assert bw.download(np.float32, (S, k)).tobytes() == w2.tobytes()
