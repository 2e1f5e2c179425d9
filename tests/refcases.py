"""Input generators of peregrine's own unit tests, restated in Python.

The reference keeps no stored vectors for this path; its tests draw inputs
from a fixed LCG (peregrine-kernels/src/idot.rs:558-573 and
peregrine-kernels/src/matmul.rs:153-162). Reproducing the generator reproduces
the reference's test inputs exactly, so the oracle can be held to the
reference's own assertions on the very same data.
"""
from __future__ import annotations

import numpy as np

MASK = (1 << 64) - 1

# idot.rs:590 — lengths exercising the SIMD body plus every tail remainder
LENS = [1, 7, 15, 16, 17, 31, 32, 33, 63, 64, 100, 257]
# idot.rs:616 — (n, gs) pairs of i4_grouped_scalar_matches_dispatch_and_hand
GROUPED_CASES = [(32, 16), (96, 32), (128, 128), (70, 16), (10, 16), (256, 64)]


class Lcg:
    def __init__(self, seed: int):
        self.s = seed & MASK

    def next(self) -> int:
        self.s = (self.s * 6364136223846793005 + 1442695040888963407) & MASK
        return self.s

    def i8_full(self) -> int:  # (next >> 33) as i8
        v = (self.next() >> 33) & 0xFF
        return v - 256 if v >= 128 else v

    def i8_127(self) -> int:  # ((next >> 33) as i32 % 255 - 127) as i8
        return ((self.next() >> 33) % 255) - 127

    def nib(self) -> int:  # (next >> 40) as i32 % 16 - 8
        return ((self.next() >> 40) % 16) - 8

    def f(self) -> np.float32:  # matmul.rs: (next>>40)/2^24*2-1 in f32
        v = np.float32(self.next() >> 40)
        return np.float32(v / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0))

    def fvec(self, n: int) -> np.ndarray:
        return np.array([self.f() for _ in range(n)], np.float32)
