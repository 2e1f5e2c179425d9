"""The committed golden fixtures (tests/golden/make_golden.py) against the
CPU oracle: the reference's LCG dot cases with brute-force expected values,
and a small routed MoE layer whose outputs the GPU path must also reproduce
(tests/test_gpu_parity.py::test_golden_layer_bit_exact)."""
import os

import numpy as np

from peregrine_amd import qt
from tests.refcases import GROUPED_CASES, LENS

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_oracle_reproduces_lcg_dot_fixtures(orc):
    f = np.load(os.path.join(GOLD, "dots_lcg.npz"))
    for n in LENS:
        assert orc.dot_i4i8(f[f"i4_{n}_w"], f[f"i4_{n}_x"], n) == int(f[f"i4_{n}_dot"][0]), n
        assert orc.dot_i8i8(f[f"i8_{n}_w"], f[f"i8_{n}_x"]) == int(f[f"i8_{n}_dot"][0]), n
        # the fixture values are the brute force of the unpacked nibbles
        vals = qt.unpack_i4(f[f"i4_{n}_w"], n).astype(np.int64)
        assert int(np.dot(vals, f[f"i4_{n}_x"].astype(np.int64))) == int(f[f"i4_{n}_dot"][0])
    for n, gs in GROUPED_CASES:
        got = orc.dot_i4i8_grouped(f[f"g_{n}_{gs}_w"], f[f"g_{n}_{gs}_x"], f[f"g_{n}_{gs}_sc"], gs)
        assert np.float32(got).tobytes() == f[f"g_{n}_{gs}_val"][0].tobytes(), (n, gs)


def golden_layer_tensors(f, orc):
    E, D, I, S, k = (int(v) for v in f["dims"])
    shp = {"gate": (I, D), "up": (I, D), "down": (D, I)}
    return [tuple(orc.Tensor(f[f"e{e}_{m}_q"], f[f"e{e}_{m}_s"], qt.FMT_I4G, shp[m][1], shp[m][0], 32)
                  for m in ("gate", "up", "down")) for e in range(E)]


def test_oracle_reproduces_layer_fixture(orc):
    f = np.load(os.path.join(GOLD, "moe_layer_small.npz"))
    E, D, I, S, k = (int(v) for v in f["dims"])
    ids, w = orc.route_softmax_topk(f["logits"], k)
    assert np.array_equal(ids, f["ids"]) and w.tobytes() == f["w"].tobytes()
    experts = golden_layer_tensors(f, orc)
    for ga in (0, 32):
        y = orc.moe_forward(f["x"], f["ids"], f["w"], experts, ga)
        assert y.tobytes() == f[f"y_ga{ga}"].tobytes(), ga
