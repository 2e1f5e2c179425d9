"""QT weight-format helpers on the host (numpy).

These restate peregrine-core's packers and quantizers so callers can produce
the byte payloads ``coli_hip_tensor_upload*`` accepts:

* ``pack_i4`` — element i is the low nibble of byte i/2 (even i) or the high
  nibble (odd i), stored biased as v+8 (peregrine-kernels/src/idot.rs:8-10,
  575-587).
* ``quant_i4_rows`` / ``quant_i4_grouped`` / ``quant_i8_rows`` —
  peregrine-core/src/pack.rs:492-542 and peregrine-kernels/src/matmul.rs:164-275.
* ``detect_group_size`` — peregrine-core/src/qt.rs:70-85.
"""
from __future__ import annotations

import numpy as np

FMT_F32, FMT_I8, FMT_I4, FMT_I2, FMT_I4G, FMT_I8G = 0, 1, 2, 3, 4, 8
GROUP_CANDIDATES = (16, 32, 48, 64, 96, 128, 192, 256)


def row_bytes(fmt: int, I: int) -> int:
    if fmt == FMT_F32:
        return 4 * I
    if fmt in (FMT_I8, FMT_I8G):
        return I
    if fmt in (FMT_I4, FMT_I4G):
        return (I + 1) // 2
    if fmt == FMT_I2:
        return (I + 3) // 4
    raise ValueError(f"unknown fmt {fmt}")


def pack_i4(vals: np.ndarray) -> np.ndarray:
    """Pack int values in [-8, 7] along the last axis into QT nibbles."""
    v = np.asarray(vals, dtype=np.int32)
    n = v.shape[-1]
    biased = ((v + 8) & 0x0F).astype(np.uint8)
    if n % 2:
        biased = np.concatenate([biased, np.zeros(v.shape[:-1] + (1,), np.uint8)], axis=-1)
    lo = biased[..., 0::2]
    hi = biased[..., 1::2]
    if n % 2:
        # the padding nibble of an odd row is 0, not a biased value
        hi = hi.copy()
        hi[..., -1] = 0
    return (lo | (hi << 4)).astype(np.uint8)


def unpack_i4(q: np.ndarray, n: int) -> np.ndarray:
    """Inverse of pack_i4: int8 values in [-8, 7], shape [..., n]."""
    q = np.asarray(q, dtype=np.uint8)
    lo = (q & 0x0F).astype(np.int16) - 8
    hi = (q >> 4).astype(np.int16) - 8
    out = np.empty(q.shape[:-1] + (q.shape[-1] * 2,), np.int16)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out[..., :n].astype(np.int8)


def quant_i4_rows(w: np.ndarray):
    """pack.rs:492-512: per-row scale amax/7 (floor 1e-12), RNE, clamp [-8,7]."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.max(np.abs(w), axis=1)
    s = np.maximum(amax / np.float32(7.0), np.float32(1e-12)).astype(np.float32)
    v = np.clip(np.rint(w / s[:, None]), -8, 7).astype(np.int32)
    return pack_i4(v), s


def quant_i4_grouped(w: np.ndarray, gs: int):
    """pack.rs:514-542: one scale per gs-element group, laid out sc[o*ng + g]."""
    w = np.asarray(w, dtype=np.float32)
    o_n, i_n = w.shape
    ng = -(-i_n // gs)
    sc = np.zeros((o_n, ng), np.float32)
    v = np.zeros((o_n, i_n), np.int32)
    for g in range(ng):
        a, b = g * gs, min((g + 1) * gs, i_n)
        amax = np.max(np.abs(w[:, a:b]), axis=1)
        s = np.maximum(amax / np.float32(7.0), np.float32(1e-12)).astype(np.float32)
        sc[:, g] = s
        v[:, a:b] = np.clip(np.rint(w[:, a:b] / s[:, None]), -8, 7)
    return pack_i4(v), sc


def quant_i8_rows(w: np.ndarray):
    """matmul.rs:164-180: per-row scale amax/127 (floor 1e-12), RNE."""
    w = np.asarray(w, dtype=np.float32)
    amax = np.max(np.abs(w), axis=1)
    s = np.maximum(amax / np.float32(127.0), np.float32(1e-12)).astype(np.float32)
    q = np.rint(w / s[:, None]).astype(np.int8)
    return q, s


def detect_group_size(o: int, i: int, ns: int) -> int:
    """qt.rs:70-85: the finest candidate group size whose scale count is ns."""
    if o <= 0 or ns <= o or i <= 0:
        return 0
    for gs in GROUP_CANDIDATES:
        if gs > i:
            break
        if ns == o * (-(-i // gs)):
            return gs
    return 0
