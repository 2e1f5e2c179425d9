"""The automatic expert-group graph cache (COLI_HIP_GRAPH=1) and the GEMV's
bounded-wait failure report, through the C ABI.

The cache tests mirror the reference's (crates/peregrine-cuda/src/lib.rs:
963-1059): a replay is bit-identical to eager, a grown scratch invalidates
graphs captured before it, and a replay at the same shape uses the current
expert weights.
"""
import contextlib
import os
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
    yield h
    h.set_arm(-1)
    h.set_act_group(0)
    h.set_spin_limit(0)
    os.environ.pop("COLI_HIP_GRAPH", None)


@contextlib.contextmanager
def graph_knob(on):
    old = os.environ.get("COLI_HIP_GRAPH")
    os.environ["COLI_HIP_GRAPH"] = "1" if on else "0"
    try:
        yield
    finally:
        if old is None:
            os.environ.pop("COLI_HIP_GRAPH", None)
        else:
            os.environ["COLI_HIP_GRAPH"] = old


def _expert(hip, seed, D, I, fmt=qt.FMT_I4G):
    rng = np.random.default_rng(seed)
    trip = synth.make_expert(rng, D, I, fmt, 32)
    return hip.GpuExpert.upload_grouped(0, trip[0][:2], trip[1][:2], trip[2][:2], D, I, fmt, 32)


@pytest.mark.parametrize("rows,ga", [([2], 0), ([1], 32), ([1, 1, 1], 32), ([40, 3], 32)])
def test_graph_cached_expert_group_matches_eager(hip, rows, ga):
    say("graph cache eager parity", rows, ga)
    D, I = 256, 128
    ex = [_expert(hip, 0x9001 + i, D, I) for i in range(len(rows))]
    x = np.random.default_rng(0x51DE).standard_normal((sum(rows), D)).astype(np.float32)
    hip.set_act_group(ga)
    with graph_knob(False):
        eager = hip.expert_group(ex, rows, x, D)
    before = hip.graph_cache_stats()
    with graph_knob(True):
        captured = hip.expert_group(ex, rows, x, D)
        replayed = hip.expert_group(ex, rows, x, D)
    after = hip.graph_cache_stats()
    assert np.array_equal(eager, captured)
    assert np.array_equal(eager, replayed)
    assert after.captures == before.captures + 1
    assert after.replays == before.replays + 1


def test_graph_cached_reduce_matches_eager(hip):
    say("graph cache reduce")
    D, I = 256, 128
    ex = [_expert(hip, 0x9100 + i, D, I) for i in range(3)]
    rows = [2, 1, 3]
    rng = np.random.default_rng(0x77)
    x = rng.standard_normal((6, D)).astype(np.float32)
    lay = hip.ReduceLayout.build([0, 1, 0, 1, 0, 1], 2)
    rw = rng.uniform(0.1, 1.0, 6).astype(np.float32)
    hip.set_act_group(0)
    with graph_knob(False):
        eager = hip.expert_group_reduce(ex, rows, x, D, lay, rw, 2)
    with graph_knob(True):
        for _ in range(3):
            assert np.array_equal(eager, hip.expert_group_reduce(ex, rows, x, D, lay, rw, 2))


def test_grown_scratch_invalidates_cached_graphs(hip):
    """Small shape captured, a much larger call reallocates scratch, the small
    shape again must not replay the stale graph. The large eager reference is
    taken last, so nothing sizes the scratch for it before the graphed calls."""
    say("graph cache invalidation")
    D, I = 64, 32
    big_rows = 6000   # larger than every other call in this process
    e = _expert(hip, 0x9002, D, I)
    rng = np.random.default_rng(0x6120)
    small = rng.standard_normal((1, D)).astype(np.float32)
    big = rng.standard_normal((big_rows, D)).astype(np.float32)
    hip.set_act_group(32)
    with graph_knob(False):
        want_small = hip.expert_group([e], [1], small, D)
    before = hip.graph_cache_stats()
    with graph_knob(True):
        hip.expert_group([e], [1], small, D)
        got_big = hip.expert_group([e], [big_rows], big, D)
        got_small = hip.expert_group([e], [1], small, D)
    after = hip.graph_cache_stats()
    with graph_knob(False):
        want_big = hip.expert_group([e], [big_rows], big, D)
    assert np.array_equal(want_big, got_big)
    assert np.array_equal(want_small, got_small)
    assert after.invalidations > before.invalidations


def test_replayed_graph_uses_current_expert_weights(hip):
    say("graph cache new weights")
    D, I, n = 64, 32, 2
    a, b = _expert(hip, 0xA1, D, I), _expert(hip, 0xB2, D, I)
    x = np.random.default_rng(0xD1FF).standard_normal((n, D)).astype(np.float32)
    hip.set_act_group(0)
    with graph_knob(False):
        want_a = hip.expert_group([a], [n], x, D)
        want_b = hip.expert_group([b], [n], x, D)
    assert not np.array_equal(want_a, want_b)
    before = hip.graph_cache_stats()
    with graph_knob(True):
        got_a = hip.expert_group([a], [n], x, D)
        got_b = hip.expert_group([b], [n], x, D)
    after = hip.graph_cache_stats()
    assert np.array_equal(want_a, got_a) and np.array_equal(want_b, got_b)
    assert after.replays >= before.replays + 1


@pytest.mark.parametrize("adapt", [1, 0])
def test_cache_probes_then_keeps_the_faster_way(hip, adapt):
    """After its capture a shape's calls alternate replay and eager launch
    (three timed probes each), then keep whichever was faster; a declined
    shape runs eagerly and counts as uncacheable. With COLI_HIP_GRAPH_ADAPT=0
    every call replays. Every call equals the eager result."""
    say("graph cache adaptive", adapt)
    D, I = 192, 96
    ex = [_expert(hip, 0x9300 + i, D, I) for i in range(3)]
    rows = [1, 2, 1 + adapt]   # a shape of its own per mode (a slot keeps its decision)
    x = np.random.default_rng(0xADA).standard_normal((sum(rows), D)).astype(np.float32)
    hip.set_act_group(32)
    with graph_knob(False):
        want = hip.expert_group(ex, rows, x, D)
    old = os.environ.get("COLI_HIP_GRAPH_ADAPT")
    os.environ["COLI_HIP_GRAPH_ADAPT"] = str(adapt)
    try:
        before = hip.graph_cache_stats()
        with graph_knob(True):
            for _ in range(12):
                assert np.array_equal(want, hip.expert_group(ex, rows, x, D))
        after = hip.graph_cache_stats()
    finally:
        if old is None:
            os.environ.pop("COLI_HIP_GRAPH_ADAPT", None)
        else:
            os.environ["COLI_HIP_GRAPH_ADAPT"] = old
    assert after.captures == before.captures + 1
    replays = after.replays - before.replays
    eager = after.uncacheable - before.uncacheable
    assert replays + eager == 11
    if adapt:
        assert replays >= 3 and eager >= 3            # both ways were probed
        assert replays in (3, 11 - 3)                 # then one way was kept for the remaining calls
    else:
        assert replays == 11 and eager == 0


def test_profiled_calls_are_uncacheable_and_time_phases(hip):
    say("graph cache uncacheable + phase stats")
    D, I = 256, 128
    e = _expert(hip, 0x9004, D, I)
    x = np.random.default_rng(3).standard_normal((4, D)).astype(np.float32)
    hip.reset_stats()
    hip.set_profile(True)
    try:
        before = hip.graph_cache_stats()
        with graph_knob(True):
            got = hip.expert_group([e], [4], x, D)
        after = hip.graph_cache_stats()
    finally:
        hip.set_profile(False)
    with graph_knob(False):
        assert np.array_equal(got, hip.expert_group([e], [4], x, D))
    assert after.uncacheable == before.uncacheable + 1 and after.captures == before.captures
    st = hip.group_stats()
    assert st.calls >= 1 and st.h2d_ms > 0 and st.d2h_ms > 0 and st.kernel_ms > 0


def test_gemv_wait_give_up_is_reported(hip, orc):
    """A GEMV bounded wait that gives up (forced from the host with a spin
    limit of one poll) fails the next synchronising call instead of returning
    wrong output silently; every kernel still runs to its end. With the
    default limit the same layer is then correct again."""
    say("gemv wait give-up")
    rng = np.random.default_rng(17)
    E, D, I, k = 8, 5120, 1536, 8
    gpu, ora = [], []
    for _ in range(E):
        trip = synth.make_expert(rng, D, I, qt.FMT_I4G, 32)
        gpu.append(hip.GpuExpert.upload_grouped(0, trip[0][:2], trip[1][:2], trip[2][:2], D, I))
        shp = ((I, D), (I, D), (D, I))
        ora.append(tuple(orc.Tensor(t[0], t[1], qt.FMT_I4G, i, o, 32) for t, (o, i) in zip(trip, shp)))
    eset = hip.ExpertSet(gpu)
    x = rng.standard_normal((1, D)).astype(np.float32)
    logits = synth.normal_logits(rng, 1, E)
    bx, bl = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(logits)
    bids, bw, bout = hip.DeviceBuffer(k * 4), hip.DeviceBuffer(k * 4), hip.DeviceBuffer(D * 4)
    hip.pipe_sync(0)
    hip.set_spin_limit(1)
    try:
        hip.moe_forward_logits_dev(eset, bx.ptr, 1, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, 32)
        with pytest.raises(hip.HipError):
            hip.pipe_sync(0)
        # host-buffer entry point: the same report through its own return code
        hip.set_arm(hip.ARM_GEMV)
        with pytest.raises(hip.HipError):
            hip.expert_group(gpu[:2], [1, 1], np.repeat(x, 2, 0), D)
    finally:
        hip.set_spin_limit(0)
        hip.set_arm(-1)
    hip.pipe_sync(0)   # the flag was cleared by the failing call
    hip.moe_forward_logits_dev(eset, bx.ptr, 1, bl.ptr, k, bids.ptr, bw.ptr, bout.ptr, 32)
    hip.pipe_sync(0)
    ids, w = bids.download(np.int32, (1, k)), bw.download(np.float32, (1, k))
    ref = orc.moe_forward(x, ids, w, ora, 32)
    assert np.array_equal(bout.download(np.float32, (1, D)), ref)
