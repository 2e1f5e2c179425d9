"""Writes the golden fixtures of this directory (run from the repo root:
`python tests/golden/make_golden.py`).

The reference keeps no stored vectors for the expert path (its tests draw
inputs from an LCG, peregrine-kernels/src/idot.rs:558-693), so the fixtures
are made here:

- dots_lcg.npz: the reference's own LCG dot cases (seeds and lengths of
  idot.rs:590-693). Expected values come from a NumPy brute force (int64
  sums; the grouped case accumulates scales[g] * (f32)dot_g in f32 in group
  order, idot.rs:82-88), independent of the C oracle.
- moe_layer_small.npz: one routed MoE layer (6 int4 gs=32 experts, D=96,
  I=64, 5 tokens, top-2 softmax routing) with the oracle's outputs for both
  activation-scale modes. The GPU path must reproduce them bit-for-bit.

Fixtures are plain arrays (np.savez, no pickled objects)."""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

from peregrine_amd import qt, synth  # noqa: E402
from refcases import GROUPED_CASES, LENS, Lcg  # noqa: E402


def dots_lcg():
    out = {}
    rng = Lcg(0x9E37_79B9)   # idot.rs i4 scalar-vs-dispatch
    for n in LENS:
        vals = np.array([rng.nib() for _ in range(n)], np.int32)
        x = np.array([rng.i8_127() for _ in range(n)], np.int8)
        out[f"i4_{n}_w"] = qt.pack_i4(vals)
        out[f"i4_{n}_x"] = x
        out[f"i4_{n}_dot"] = np.array([np.dot(vals.astype(np.int64), x.astype(np.int64))], np.int64)
    rng = Lcg(0x1234_5678)   # idot.rs i8 scalar-vs-dispatch
    for n in LENS:
        w = np.array([rng.i8_full() for _ in range(n)], np.int8)
        x = np.array([rng.i8_full() for _ in range(n)], np.int8)
        out[f"i8_{n}_w"] = w
        out[f"i8_{n}_x"] = x
        out[f"i8_{n}_dot"] = np.array([np.dot(w.astype(np.int64), x.astype(np.int64))], np.int64)
    rng = Lcg(0xDEAD_BEEF)   # idot.rs:613-635 grouped: scales 0.01 + 0.05*g
    for n, gs in GROUPED_CASES:
        vals = np.array([rng.nib() for _ in range(n)], np.int32)
        x = np.array([rng.i8_127() for _ in range(n)], np.int8)
        ng = (n + gs - 1) // gs
        sc = np.array([np.float32(0.01) + np.float32(0.05) * np.float32(g) for g in range(ng)], np.float32)
        acc = np.float32(0.0)
        for g in range(ng):
            d = int(np.dot(vals[g * gs:(g + 1) * gs].astype(np.int64), x[g * gs:(g + 1) * gs].astype(np.int64)))
            acc = np.float32(acc + np.float32(sc[g] * np.float32(d)))
        out[f"g_{n}_{gs}_w"] = qt.pack_i4(vals)
        out[f"g_{n}_{gs}_x"] = x
        out[f"g_{n}_{gs}_sc"] = sc
        out[f"g_{n}_{gs}_val"] = np.array([acc], np.float32)
    return out


def moe_layer_small():
    from oracle import oracle as orc
    rng = np.random.default_rng(20240611)
    E, D, I, S, k = 6, 96, 64, 5, 2
    out = dict(dims=np.array([E, D, I, S, k], np.int32))
    ora = []
    for e in range(E):
        trip = synth.make_expert(rng, D, I, qt.FMT_I4G, 32)
        for m, name in enumerate(("gate", "up", "down")):
            out[f"e{e}_{name}_q"] = trip[m][0]
            out[f"e{e}_{name}_s"] = trip[m][1]
        shp = ((I, D), (I, D), (D, I))
        ora.append(tuple(orc.Tensor(t[0], t[1], qt.FMT_I4G, i, o, 32) for t, (o, i) in zip(trip, shp)))
    x = rng.standard_normal((S, D)).astype(np.float32)
    logits = synth.zipf_logits(rng, S, E)
    ids, w = orc.route_softmax_topk(logits, k)
    out.update(x=x, logits=logits, ids=ids.astype(np.int32), w=w.astype(np.float32))
    for ga in (0, 32):
        out[f"y_ga{ga}"] = orc.moe_forward(x, ids, w, ora, ga)
    return out


def main():
    np.savez(os.path.join(HERE, "dots_lcg.npz"), **dots_lcg())
    np.savez(os.path.join(HERE, "moe_layer_small.npz"), **moe_layer_small())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
