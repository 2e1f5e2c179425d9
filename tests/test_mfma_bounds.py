"""CPU bounds check of the staged MFMA kernels' copy addresses.

tests/native/mfma_bounds.cpp walks every workgroup, wave, lane and K block of
a dispatch through the same index functions the kernels call
(peregrine_amd/csrc/mfma_map.h) and checks that every LDS-DMA copy of
activations, weights, weight scales and per-32 activation scales lies inside
its buffer, and that the workgroup -> (M tile, channel slab) maps, including
the XCD-aware order of weight-reuse dispatches, cover every item exactly once.
The expert tables are the ones the BASELINE configs produce (routing through
the oracle's router and table, as the device builds them) and the host call
order of expert_group (backend_cuda.cu:1035-1211)."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from peregrine_amd import synth

HERE = os.path.dirname(os.path.abspath(__file__))
MT = 32


class Geom(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("K", "Kp", "nb", "O", "Op", "ng", "gshift", "w4")]


def geom(K, O, w4, gs):
    Kp = -(-K // 32) * 32
    nb = Kp // 32
    if gs:
        gpb = gs // 32
        return Geom(K, Kp, nb, O, -(-O // 64) * 64, -(-nb // gpb), gpb.bit_length() - 1, int(w4))
    return Geom(K, Kp, nb, O, -(-O // 64) * 64, 1, 30, int(w4))


@pytest.fixture(scope="module")
def chk(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("mfmab") / "libmfma_bounds.so")
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", os.path.join(HERE, "native", "mfma_bounds.cpp"),
                    "-o", out], check=True)
    lib = ctypes.CDLL(out)
    ip = ctypes.POINTER(ctypes.c_int)
    lib.check_dispatch.restype = ctypes.c_long
    lib.check_dispatch.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(Geom), ctypes.c_int, ctypes.c_int, ip, ip, ip,
                                                        ip, ctypes.c_int, ip, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                                        ctypes.c_int]
    return lib


def tiles_from_groups(groups):
    """groups: [(descriptor index, rows)] in row order -> M-tile arrays."""
    mt_exp, mt_row0, mt_rend, mt_first = [], [], [], []
    r = 0
    for e, n in groups:
        t0 = len(mt_exp)
        for q in range(0, n, MT):
            mt_exp.append(e)
            mt_row0.append(r + q)
            mt_rend.append(r + n)
            mt_first.append(t0)
        r += n
    return [np.asarray(a, np.int32) for a in (mt_exp, mt_row0, mt_rend, mt_first)], r


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def run_check(chk, kind, gateup, xo, ga, g, tiles, R, grid_tiles, row_act, rows_x, n_desc, per_row):
    mt = tiles
    T = len(mt[0])
    x_stride = g.Kp
    sx_stride = g.nb if ga == 32 else 1
    grp_copy = int(ga == 32 or not per_row)
    n = chk.check_dispatch(kind, int(gateup), int(xo), int(ga == 32), grp_copy, ctypes.byref(g), T, grid_tiles,
                           _p(mt[0]), _p(mt[1]), _p(mt[2]), _p(mt[3]), R, _p(row_act), rows_x, x_stride, sx_stride,
                           n_desc)
    return n


def check_layer(chk, D, I, w4, gs, ga, tiles, R, grid_tiles, row_act, rows_x, n_desc, w_reuse):
    gg, gd = geom(D, I, w4, gs), geom(I, D, w4, gs)
    bad = {}
    for kind in (0, 1):   # 0: mfma_sa_kernel, 1: mfma_dma_kernel
        # the XO order is checked for every table, reuse or not: it must cover any n
        for xo in ((0, 1) if kind == 0 else (0,)):
            for gateup, g, ra, rx in ((True, gg, row_act, rows_x), (False, gd, None, R)):
                n = run_check(chk, kind, gateup, xo, ga, g, tiles, R, grid_tiles, ra, rx, n_desc, gs == 0)
                if n:
                    bad[(kind, xo, gateup)] = n
    return bad


def moe_tables(orc, S, E, k, logits):
    ids, _ = orc.route_softmax_topk(logits, k)
    t = orc.expert_table(ids, E)
    groups = [(int(e), int(t["off"][u + 1] - t["off"][u])) for u, e in enumerate(t["uexp"])]
    tiles, R = tiles_from_groups(groups)
    assert R == S * k
    tmax = -(-R // MT) + min(E, R)
    return tiles, R, tmax, t["row_tok"].astype(np.int32), R >= 2 * MT * E


CONFIGS = {
    "cfg3": dict(S=64, E=160, D=5120, I=1536, zipf=True),
    "cfg4": dict(S=2048, E=160, D=5120, I=1536, zipf=True),
    "cfg5": dict(S=512, E=256, D=6144, I=2048, zipf=False),
}


@pytest.mark.parametrize("name", sorted(CONFIGS))
@pytest.mark.parametrize("w4", [True, False], ids=["int4", "int8"])
def test_baseline_configs_copies_in_bounds(chk, orc, name, w4):
    c = CONFIGS[name]
    rng = np.random.default_rng(7)
    S, E = c["S"], c["E"]
    logits = synth.zipf_logits(rng, S, E) if c["zipf"] else synth.normal_logits(rng, S, E)
    tiles, R, tmax, row_tok, w_reuse = moe_tables(orc, S, E, 8, logits)
    for gs, ga in ((32, 32), (32, 0), (128, 0), (0, 0)):
        bad = check_layer(chk, c["D"], c["I"], w4, gs, ga, tiles, R, tmax, row_tok, S, E, w_reuse)
        assert not bad, (name, gs, ga, bad)


@pytest.mark.parametrize("rows", [[96], [70, 70, 5], [1, 3, 34], [64] * 3, [33], [200, 1, 31, 95]])
def test_expert_group_call_order_in_bounds(chk, rows):
    """expert_group: rows packed in call order, grid = exactly the M tiles
    (no spare workgroups), which is where an XCD order that needs spare
    workgroups would leave items unwritten."""
    tiles, R = tiles_from_groups(list(enumerate(rows)))
    T = len(tiles[0])
    for w4 in (True, False):
        for gs, ga in ((32, 32), (32, 0), (0, 0)):
            bad = check_layer(chk, 512, 320, w4, gs, ga, tiles, R, T, None, R, len(rows), True)
            assert not bad, (rows, w4, gs, ga, bad)


def test_xo_order_is_a_bijection_for_every_item_count(chk):
    """The XCD-aware order (the header's xo_item): workgroups L < n map onto
    distinct items covering [0, n), each XCD (L mod 8) takes a contiguous run
    of items, and L >= n idles."""
    for n in range(1, 700):
        items = [chk.xo_item_c(L, n) for L in range(n)]
        assert sorted(items) == list(range(n)), n
        for x in range(min(8, n)):
            run = sorted(items[x::8])
            assert run == list(range(run[0], run[0] + len(run))), (n, x)
        assert chk.xo_item_c(n, n) == -1


def test_checker_is_not_vacuous(chk):
    """A dispatch that would read past a buffer or skip an item is reported:
    an activation buffer one row short, a tile whose rows run past R, and a
    grid one M-tile row short of the tiles."""
    tiles, R = tiles_from_groups([(0, 40), (1, 70)])
    g = geom(256, 128, True, 32)
    T = len(tiles[0])
    assert run_check(chk, 0, True, 1, 32, g, tiles, R, T, None, R, 2, False) == 0
    assert run_check(chk, 0, True, 0, 32, g, tiles, R, T, None, R - 1, 2, False) > 0
    assert run_check(chk, 0, True, 0, 32, g, tiles, R - 1, T, None, R, 2, False) > 0
    assert run_check(chk, 0, True, 0, 32, g, tiles, R, T - 1, None, R, 2, False) > 0
    assert run_check(chk, 1, True, 0, 32, g, tiles, R, T, None, R, 1, False) > 0   # descriptor 1 of 1
