"""Host-side checks of bench.py (no GPU): the committed PMC summary gives a
traffic figure for every benchmarked workload's gate/up kernel, and the
algorithmic byte and op counts follow from the configuration's shapes."""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


@pytest.mark.parametrize("cfg_id,wfmt", [(1, "int4"), (2, "int4"), (3, "int4"), (4, "int4"), (5, "int4"), (5, "int8")])
def test_traffic_for_every_bench_workload(cfg_id, wfmt):
    cfg = dict(bench.CONFIGS[cfg_id])
    name = cfg["name"] + ("_int8" if wfmt == "int8" else "")
    t = bench.measured_traffic(name)
    assert isinstance(t, int)
    # at least the algorithmic bytes of the fewest distinct experts a step can touch
    gu_one, _, _, _ = bench.algorithmic(cfg, wfmt, 1)
    assert t >= min(cfg["k"], cfg["E"]) * gu_one * 0.99
    # and not absurdly above what every expert of the layer would read twice
    assert t <= 2 * cfg["E"] * gu_one


def test_traffic_unknown_workload_is_none():
    assert bench.measured_traffic("no_such_workload") is None


def test_algorithmic_counts():
    cfg = bench.CONFIGS[2]
    gu, layer, gu_ops, layer_ops = bench.algorithmic(cfg, "int4", 8)
    per_mat = 5120 * 1536 // 2 + 5120 * 1536 // 32 * 4
    assert gu == 8 * 2 * per_mat == 78643200
    assert layer == 8 * 3 * per_mat
    assert gu_ops == 2 * 2 * 8 * 5120 * 1536
    assert layer_ops == 3 * 2 * 8 * 5120 * 1536
    gu8, _, _, _ = bench.algorithmic(bench.CONFIGS[5], "int8", 1)
    assert gu8 == 2 * (6144 * 2048 + 6144 * 2048 // 32 * 4) == 28311552
