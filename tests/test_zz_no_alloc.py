"""The no-allocation layer entry point (coli_hip_moe_forward_dev_noalloc)
against the allocating one (coli_hip_moe_forward_dev), through the C ABI:
bit-identical on two calls in a row, the second smaller, on both arms; a call
beyond the fixed scratch is refused. Collected last (it shares the device's
fixed scratch array with nothing else, but runs after the other GPU tests)."""
import sys

import numpy as np
import pytest

from peregrine_amd import qt, synth

pytestmark = pytest.mark.gpu


def say(*a):
    print("[case]", *a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def hip():
    from peregrine_amd import hip as h
    assert h.init([0]) == 1
    return h


def _layer(hip, rng, E, D, I):
    gpu = []
    for _ in range(E):
        trip = synth.make_expert(rng, D, I, qt.FMT_I4G, 32)
        gpu.append(hip.GpuExpert.upload_grouped(0, trip[0][:2], trip[1][:2], trip[2][:2], D, I))
    return gpu, hip.ExpertSet(gpu)


def _run(hip, fn, eset, x, ids, w, k, ga, arm):
    S, D = x.shape
    bx, bi, bw = (hip.DeviceBuffer.from_array(a) for a in (x, ids, w))
    bout = hip.DeviceBuffer(S * D * 4)
    fn(eset, bx.ptr, S, bi.ptr, bw.ptr, k, bout.ptr, ga, arm)
    hip.pipe_sync(0)
    return bout.download(np.float32, (S, D))


@pytest.mark.parametrize("arm,ga", [(-1, 32), (0, 0), (2, 32)])
def test_noalloc_matches_allocating_entry_point(hip, arm, ga):
    say("no-alloc", arm, ga)
    rng = np.random.default_rng(77 + arm + ga)
    E, D, I, k = 24, 1024, 512, 8
    _, eset = _layer(hip, rng, E, D, I)
    for S in (40, 3):   # the second call smaller: stale contents of the first must not leak
        x = rng.standard_normal((S, D)).astype(np.float32)
        ids, w = (np.ascontiguousarray(a) for a in synth_route(rng, S, E, k))
        want = _run(hip, hip.moe_forward_dev, eset, x, ids, w, k, ga, arm)
        got = _run(hip, hip.moe_forward_dev_noalloc, eset, x, ids, w, k, ga, arm)
        assert np.array_equal(got, want), (S, arm, ga)


def test_noalloc_decode_shape_and_limit(hip):
    """BASELINE config 2's shape (one token, top-8 of 160... here 16 resident
    experts) twice, then a batch whose scratch exceeds the fixed array."""
    say("no-alloc decode + limit")
    rng = np.random.default_rng(5120)
    E, D, I, k = 16, 5120, 1536, 8
    _, eset = _layer(hip, rng, E, D, I)
    for S in (2, 1):
        x = rng.standard_normal((S, D)).astype(np.float32)
        ids, w = synth_route(rng, S, E, k)
        want = _run(hip, hip.moe_forward_dev, eset, x, ids, w, k, 32, -1)
        got = _run(hip, hip.moe_forward_dev_noalloc, eset, x, ids, w, k, 32, -1)
        assert np.array_equal(got, want), S
    S = 400   # 3200 rows: about 90 MB of scratch at this width
    x = rng.standard_normal((S, D)).astype(np.float32)
    ids, w = synth_route(rng, S, E, k)
    with pytest.raises(hip.HipError):
        _run(hip, hip.moe_forward_dev_noalloc, eset, x, ids, w, k, 32, -1)


def test_noalloc_replayed_from_a_graph(hip):
    """What the entry point is for: a layer captured into a HIP graph with
    no allocation anywhere, replayed with new contents written into the same
    device buffers between replays; every replay equals the allocating entry
    point run eagerly on those contents."""
    say("no-alloc graph replay")
    rng = np.random.default_rng(6144)
    E, D, I, k, S = 24, 1024, 512, 8, 24
    _, eset = _layer(hip, rng, E, D, I)
    bx, bi, bw = hip.DeviceBuffer(S * D * 4), hip.DeviceBuffer(S * k * 4), hip.DeviceBuffer(S * k * 4)
    bout = hip.DeviceBuffer(S * D * 4)

    def contents():
        x = rng.standard_normal((S, D)).astype(np.float32)
        ids, w = synth_route(rng, S, E, k)
        bx.upload(x)
        bi.upload(ids)
        bw.upload(w)
        return x, ids, w

    def body():
        hip.moe_forward_dev_noalloc(eset, bx.ptr, S, bi.ptr, bw.ptr, k, bout.ptr, 32, -1)

    x, ids, w = contents()
    body()   # one eager call first, as for any captured layer
    hip.pipe_sync(0)
    # the allocating reference calls below reserve their scratch now, before
    # the capture (a later growth would make graph_launch refuse the graph)
    _run(hip, hip.moe_forward_dev, eset, x, ids, w, k, 32, -1)
    g = hip.capture(0, body)
    for rep in range(3):
        x, ids, w = contents()
        g.launch()
        hip.pipe_sync(0)
        got = bout.download(np.float32, (S, D))
        want = _run(hip, hip.moe_forward_dev, eset, x, ids, w, k, 32, -1)
        assert np.array_equal(got, want), rep


def synth_route(rng, S, E, k):
    logits = synth.normal_logits(rng, S, E)
    order = np.argsort(-logits, axis=1, kind="stable")[:, :k].astype(np.int32)
    sel = np.take_along_axis(logits, order, 1).astype(np.float64)
    w = np.exp(sel - sel[:, :1])
    w = (w / w.sum(1, keepdims=True)).astype(np.float32)
    return np.ascontiguousarray(order), np.ascontiguousarray(w)
