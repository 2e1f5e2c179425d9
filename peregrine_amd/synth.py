"""Seeded synthetic MoE workloads in the BASELINE distributions (host, numpy).

* activations x ~ N(0, 1) f32;
* int4 weights uniform in [-8, 7] packed as QT nibbles, int8 weights uniform
  in [-127, 127];
* one f32 scale per 32-weight block ~ lognormal(ln 0.01, 0.5);
* router logits ~ N(0, 1); Zipf(alpha) expert popularity enters as log p_e
  plus Gumbel noise, so top-k of the logits samples k experts without
  replacement with probability proportional to p_e.
"""
from __future__ import annotations

import numpy as np

from . import qt


def make_tensor(rng, o, i, fmt=qt.FMT_I4G, gs=32):
    grouped = fmt in (qt.FMT_I4G, qt.FMT_I8G)
    if fmt in (qt.FMT_I4, qt.FMT_I4G):
        v = rng.integers(-8, 8, (o, i), dtype=np.int8)
        q = qt.pack_i4(v)
    else:
        v = rng.integers(-127, 128, (o, i), dtype=np.int8)
        q = v
    ns = o * (-(-i // gs)) if grouped else o
    sc = np.exp(rng.normal(np.log(0.01), 0.5, ns)).astype(np.float32)
    return q, sc, v


def make_expert(rng, hidden, inter, fmt=qt.FMT_I4G, gs=32):
    """(gate, up, down) as (q, scales, values) triples; gate/up [inter][hidden]."""
    return (make_tensor(rng, inter, hidden, fmt, gs), make_tensor(rng, inter, hidden, fmt, gs),
            make_tensor(rng, hidden, inter, fmt, gs))


def zipf_logits(rng, s_n, e_n, alpha=1.1):
    p = 1.0 / np.arange(1, e_n + 1, dtype=np.float64) ** alpha
    p = p[rng.permutation(e_n)]
    g = rng.gumbel(size=(s_n, e_n))
    return (np.log(p / p.sum())[None, :] + g).astype(np.float32)


def normal_logits(rng, s_n, e_n):
    return rng.standard_normal((s_n, e_n)).astype(np.float32)
