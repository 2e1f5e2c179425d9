"""Split-K decode GEMV (the GEMV arm with each (row, tile)'s K blocks spread
over several workgroups and the exact f32 chain run by the workgroup that
completes the tile's count). Bar: the same bits as the oracle
(idot.rs:82-88, matmul.rs:93-106, mlp.rs:21-26) at every split, every
weight format and both activation-scale modes, on repeated calls (the
per-tile counters reset themselves) and on graph replays."""
import sys

import numpy as np
import pytest

from peregrine_amd import qt, synth

pytestmark = pytest.mark.gpu

FORMATS = [(qt.FMT_I4G, 32), (qt.FMT_I4G, 128), (qt.FMT_I4, 0), (qt.FMT_I8G, 32), (qt.FMT_I8, 0)]
# workgroup targets: 0 = unsplit kernel, small = a few splits, large = one
# wave-pair of blocks per workgroup (the most splits the planner allows)
SPLITS = [0, 96, 2048, 1 << 20]


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip():
    from peregrine_amd import hip as h
    assert h.init([0]) == 1
    yield h
    h.set_gemv_split(-1)
    h.set_arm(-1)
    h.set_act_group(0)
    h.set_fused_combine(-1)
    h.set_fused_route(-1)


def _experts(rng, n, D, I, fmt, gs, orc, hip):
    gpu, ora = [], []
    for _ in range(n):
        trip = synth.make_expert(rng, D, I, fmt, gs)
        gpu.append(hip.GpuExpert.upload_grouped(0, trip[0][:2], trip[1][:2], trip[2][:2], D, I, fmt, gs))
        shp = ((I, D), (I, D), (D, I))
        ora.append(tuple(orc.Tensor(t[0], t[1], fmt, i, o, gs) for t, (o, i) in zip(trip, shp)))
    return gpu, ora


@pytest.mark.parametrize("fmt,gs", FORMATS)
@pytest.mark.parametrize("ga", [0, 32])
def test_expert_group_gemv_every_split(hip, orc, fmt, gs, ga):
    """expert_group on the GEMV arm (one row per expert): every split target
    gives the oracle's bits, three calls in a row each."""
    say("split expert_group", fmt, gs, ga)
    rng = np.random.default_rng(0x5A11 + fmt * 3 + gs + ga)
    D, I = 1088, 704   # gate/up 34 blocks, down 22; not multiples of 64 channels
    gpu, ora = _experts(rng, 4, D, I, fmt, gs or 32, orc, hip)
    rows = [1, 1, 1, 1]
    hip.set_act_group(ga)
    hip.set_arm(2)
    try:
        for sp in SPLITS:
            hip.set_gemv_split(sp)
            for rep in range(3):
                x = rng.standard_normal((4, D)).astype(np.float32)
                y = hip.expert_group(gpu, rows, x, D)
                for e in range(4):
                    ref = orc.expert_swiglu(x[e:e + 1], *ora[e], ga)
                    assert np.array_equal(y[e:e + 1], ref), (sp, rep, e)
    finally:
        hip.set_gemv_split(-1)
        hip.set_arm(-1)


def _one_token(hip, orc, rng, E, n_dist, D, I, k, fmt, gs):
    gpu, ora = _experts(rng, n_dist, D, I, fmt, gs, orc, hip)
    eset = hip.ExpertSet([gpu[e % n_dist] for e in range(E)])
    return eset, [ora[e % n_dist] for e in range(E)]


@pytest.mark.parametrize("ga", [32, 0])
@pytest.mark.parametrize("shape", ["cfg1", "cfg2"])
def test_one_token_full_shape_every_split(hip, orc, ga, shape):
    """BASELINE configs 1 (one expert, k = 1) and 2 (160 slots over 12
    distinct experts, top-8) at D=5120, I=1536: the layer through the router
    launch, split gate/up and split down with its tail combine, bit-identical
    to the oracle at every split and with the fused combine kernel."""
    say("split one token", shape, ga)
    E, n_dist, k = (1, 1, 1) if shape == "cfg1" else (160, 12, 8)
    D, I = 5120, 1536
    rng = np.random.default_rng(0xC0DE + ga + k)
    eset, ora = _one_token(hip, orc, rng, E, n_dist, D, I, k, qt.FMT_I4G, 32)
    bx, bl = hip.DeviceBuffer(D * 4), hip.DeviceBuffer(E * 4)
    bids, bw, bout = hip.DeviceBuffer(k * 4), hip.DeviceBuffer(k * 4), hip.DeviceBuffer(D * 4)
    try:
        for sp in SPLITS:
            for fc in (-1, 0, 1):
                hip.set_gemv_split(sp)
                hip.set_fused_combine(fc)
                x = rng.standard_normal((1, D)).astype(np.float32)
                logits = synth.normal_logits(rng, 1, E)
                bx.upload(x)
                bl.upload(logits)
                hip.moe_forward_logits_dev(eset, bx.ptr, 1, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, ga, -1)
                hip.pipe_sync(0)
                ids, w = orc.route_softmax_topk(logits, k)
                assert np.array_equal(bids.download(np.int32, (1, k)), ids)
                ref = orc.moe_forward(x, ids, w, ora, ga)
                got = bout.download(np.float32, (1, D))
                assert np.array_equal(got, ref), (sp, fc, float(np.max(np.abs(got - ref))))
    finally:
        hip.set_gemv_split(-1)
        hip.set_fused_combine(-1)


def test_split_graph_replays_match_oracle(hip, orc):
    """A captured one-token layer with split gate/up and down replays with new
    contents, the program's own work and synchronisations in between, every
    replay equal to the oracle (the per-tile counters are left zero by every
    dispatch, so replays need no clearing node)."""
    say("split graph replay")
    E, n_dist, D, I, k, ga = 40, 6, 2048, 768, 6, 32
    rng = np.random.default_rng(0x6A)
    eset, ora = _one_token(hip, orc, rng, E, n_dist, D, I, k, qt.FMT_I4G, 32)
    bx, bl = hip.DeviceBuffer(D * 4), hip.DeviceBuffer(E * 4)
    bids, bw, bout = hip.DeviceBuffer(k * 4), hip.DeviceBuffer(k * 4), hip.DeviceBuffer(D * 4)
    hip.set_gemv_split(4096)
    try:
        def body():
            hip.moe_forward_logits_dev(eset, bx.ptr, 1, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, ga, -1)

        body()   # eager first: scratch is sized before the capture records its addresses
        hip.pipe_sync(0)
        g = hip.capture(0, body)
        for rep in range(4):
            x = rng.standard_normal((1, D)).astype(np.float32)
            logits = synth.normal_logits(rng, 1, E)
            bx.upload(x)
            bl.upload(logits)
            g.launch()
            ids, w = orc.route_softmax_topk(logits, k)
            ref = orc.moe_forward(x, ids, w, ora, ga)
            assert np.array_equal(bout.download(np.float32, (1, D)), ref), rep
            body()   # eager work between replays
            hip.pipe_sync(0)
            assert np.array_equal(bout.download(np.float32, (1, D)), ref), rep
    finally:
        hip.set_gemv_split(-1)


def test_split_setter_rejects_bad_values(hip):
    with pytest.raises(hip.HipError):
        hip.set_gemv_split(-5)
    hip.set_gemv_split(0)
    hip.set_gemv_split(-1)
