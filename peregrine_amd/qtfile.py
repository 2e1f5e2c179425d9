"""QT container loader bridge: peregrine's quantised ``model.safetensors``
expert weights straight into the HIP lane's device layout.

A quantised weight ``name`` is a ``U8`` payload plus a sibling ``name.qs``
``F32`` scale tensor; the format is inferred from the byte and scale counts
(peregrine-core/src/qt.rs:63-160). A payload may be stored "kblock"
(group-major) tiled, tagged ``layout: "kblock"`` with ``layout_gs_bytes``
(peregrine-core/src/pack.rs:316-353); reading permutes it back to row-major as
the reference reader does (peregrine-core/src/safetensors.rs:497-505), and the
upload then repacks into tiles on the device.

Formats this lane computes: int8 per row (fmt 1), int4 per row (fmt 2) and
grouped int4 (fmt 4) with gs in {32, 64, 128, 256}. Everything else the
container can hold (fmt 0 full precision, int2, int3-g64, int2-g64, grouped
int4 at gs 16/48/96/192) is reported with a clear error, as is a zstd payload:
this image has no zstd decoder.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass

import numpy as np

FMT_F32, FMT_I8, FMT_I4, FMT_I2, FMT_I4G, FMT_I3G64, FMT_UNKNOWN, FMT_I2G64 = 0, 1, 2, 3, 4, 5, 6, 7
LANE_FORMATS = (FMT_I8, FMT_I4, FMT_I4G)
LANE_GROUP_SIZES = (32, 64, 128, 256)


class QtError(RuntimeError):
    pass


# ---------------------------------------------------------------------------
# K-block tiling (pack.rs:316-353): native [o][g] blocks of gs_bytes <-> [g][o]
# ---------------------------------------------------------------------------

def to_kblock(b: np.ndarray, o: int, gs_bytes: int) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint8).reshape(-1)
    if o <= 0 or gs_bytes <= 0 or b.size % (o * gs_bytes):
        raise QtError(f"kblock: {b.size} bytes do not tile o={o} x gs_bytes={gs_bytes}")
    g = b.size // (o * gs_bytes)
    return np.ascontiguousarray(b.reshape(o, g, gs_bytes).transpose(1, 0, 2)).reshape(-1)


def from_kblock(b: np.ndarray, o: int, gs_bytes: int) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint8).reshape(-1)
    if o <= 0 or gs_bytes <= 0 or b.size % (o * gs_bytes):
        raise QtError(f"kblock: {b.size} bytes do not tile o={o} x gs_bytes={gs_bytes}")
    g = b.size // (o * gs_bytes)
    return np.ascontiguousarray(b.reshape(g, o, gs_bytes).transpose(1, 0, 2)).reshape(-1)


# ---------------------------------------------------------------------------
# Format detection (qt.rs:63-160)
# ---------------------------------------------------------------------------

def detect_group_size(o: int, i: int, ns: int) -> int:
    """qt.rs:71-86: the grouped-int4 group size whose ceil(I/gs) scales per
    row account for all ns scales, finest first; 0 when not grouped."""
    if o <= 0 or ns <= o or i <= 0:
        return 0
    for gs in (16, 32, 48, 64, 96, 128, 192, 256):
        if gs > i:
            break
        if ns == o * ((i + gs - 1) // gs):
            return gs
    return 0


@dataclass
class QtInfo:
    fmt: int
    o: int
    i: int
    gs: int
    scale_count: int


_DTYPE = {"F32": np.float32, "F16": np.float16, "U8": np.uint8, "I8": np.int8, "I32": np.int32}


class QtFile:
    """A single ``model.safetensors`` (a path to the file or to a directory
    holding it), memory-mapped; the header may carry the reference's
    ``compression``/``uncompressed_nbytes`` and ``layout``/``layout_gs_bytes``
    fields (pack.rs:358-395)."""

    def __init__(self, path: str):
        if os.path.isdir(path):
            path = os.path.join(path, "model.safetensors")
        self.path = path
        self._f = open(path, "rb")
        self._mm = mmap.mmap(self._f.fileno(), 0, access=mmap.ACCESS_READ)
        (hlen,) = struct.unpack("<Q", self._mm[:8])
        if 8 + hlen > len(self._mm):
            raise QtError(f"{path}: header length {hlen} past the end of the file")
        hdr = json.loads(bytes(self._mm[8:8 + hlen]).decode("utf-8"))
        self._base = 8 + hlen
        self.tensors = {k: v for k, v in hdr.items() if k != "__metadata__"}

    def close(self):
        self._mm.close()
        self._f.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def has(self, name: str) -> bool:
        return name in self.tensors

    def _entry(self, name: str) -> dict:
        t = self.tensors.get(name)
        if t is None:
            raise QtError(f"{self.path}: no tensor '{name}'")
        return t

    def numel(self, name: str) -> int:
        return int(np.prod(self._entry(name)["shape"], dtype=np.int64))

    def uncompressed_nbytes(self, name: str) -> int:
        t = self._entry(name)
        if "uncompressed_nbytes" in t:
            return int(t["uncompressed_nbytes"])
        a, b = t["data_offsets"]
        return int(b - a)

    def read_raw(self, name: str) -> np.ndarray:
        """safetensors.rs:465-505: the payload bytes, decompressed, a kblock
        layout permuted back to row-major."""
        t = self._entry(name)
        a, b = t["data_offsets"]
        if self._base + b > len(self._mm) or a > b:
            raise QtError(f"'{name}': data_offsets [{a}, {b}) outside the file")
        comp = t.get("compression")
        if comp:
            raise QtError(f"'{name}': '{comp}'-compressed payload; this build has no {comp} decoder "
                          "(rewrite the container uncompressed)")
        raw = np.frombuffer(self._mm, np.uint8, b - a, self._base + a).copy()
        if t.get("layout") == "kblock":
            o = int(t["shape"][0]) if t.get("shape") else 0
            raw = from_kblock(raw, o, int(t["layout_gs_bytes"]))
        return raw

    def read_f32(self, name: str) -> np.ndarray:
        t = self._entry(name)
        raw = self.read_raw(name)
        dt = t["dtype"]
        if dt == "BF16":
            return (raw.view(np.uint16).astype(np.uint32) << 16).view(np.float32)
        if dt not in _DTYPE:
            raise QtError(f"'{name}': dtype {dt} is not a float tensor")
        return raw.view(_DTYPE[dt]).astype(np.float32)

    def detect(self, name: str, o: int, i: int) -> QtInfo:
        """QtInfo::detect (qt.rs:89-160): from the uncompressed payload size and
        the scale count."""
        sname = name + ".qs"
        if not self.has(name) or not self.has(sname):
            return QtInfo(FMT_F32, o, i, 0, 0)
        nb = self.uncompressed_nbytes(name)
        ns = self.numel(sname)
        ng64 = (i + 63) // 64
        if ng64 >= 2 and nb == o * ng64 * 16 and ns == o * ng64 * 2:
            fmt = FMT_I2G64
        elif nb == o * i:
            fmt = FMT_I8
        elif nb == o * ((i + 1) // 2):
            fmt = FMT_I4
        elif nb == o * ((i + 3) // 4):
            fmt = FMT_I2
        elif nb == o * ng64 * 24 and ns == o * ng64:
            fmt = FMT_I3G64
        else:
            return QtInfo(FMT_UNKNOWN, o, i, 0, 0)
        gs = 0
        if fmt == FMT_I4:
            gs = detect_group_size(o, i, ns)
            if gs:
                fmt = FMT_I4G
        count = {FMT_I4G: o * ((i + gs - 1) // gs) if gs else 0, FMT_I3G64: o * ng64,
                 FMT_I2G64: o * ng64 * 2}.get(fmt, o)
        return QtInfo(fmt, o, i, gs, count)

    def read_qt(self, name: str, o: int, i: int):
        """(payload bytes, scales, info) of a weight this lane can compute."""
        info = self.detect(name, o, i)
        if info.fmt not in LANE_FORMATS:
            raise QtError(f"'{name}' [{o}x{i}]: container format {info.fmt} is not computed by the HIP lane "
                          "(int8/int4 per row and grouped int4 only)")
        if info.fmt == FMT_I4G and info.gs not in LANE_GROUP_SIZES:
            raise QtError(f"'{name}': grouped int4 with gs={info.gs} (supported: {LANE_GROUP_SIZES})")
        sc = self.read_f32(name + ".qs")
        if sc.size != info.scale_count:
            raise QtError(f"'{name}.qs': {sc.size} scales, expected {info.scale_count}")
        return self.read_raw(name), sc, info


def write_qt(path: str, blobs) -> None:
    """Writes the same container (pack.rs:358-395, uncompressed): blobs are
    (name, dtype, shape, bytes[, (layout_tag, layout_gs_bytes)])."""
    header, chunks, cur = {}, [], 0
    for bl in blobs:
        name, dtype, shape, data = bl[:4]
        data = np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        e = {"dtype": dtype, "shape": [int(v) for v in shape], "data_offsets": [cur, cur + data.size]}
        if len(bl) > 4 and bl[4]:
            e["layout"], e["layout_gs_bytes"] = bl[4][0], int(bl[4][1])
        header[name] = e
        chunks.append(data.tobytes())
        cur += data.size
    hdr = json.dumps(header).encode("utf-8")
    if os.path.isdir(path):
        path = os.path.join(path, "model.safetensors")
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hdr)))
        f.write(hdr)
        for c in chunks:
            f.write(c)


def upload_expert(device: int, qf: QtFile, gate: str, up: str, down: str, hidden: int, inter: int):
    """A resident GpuExpert from three container weights (gate/up [inter x
    hidden], down [hidden x inter]), each in its detected format."""
    from . import hip
    done = []
    try:
        for name, (o, i) in ((gate, (inter, hidden)), (up, (inter, hidden)), (down, (hidden, inter))):
            q, sc, info = qf.read_qt(name, o, i)
            done.append(hip._upload(device, q, sc, info.fmt, i, o, info.gs))
    except Exception:
        for t in done:
            hip.lib.coli_hip_tensor_free(t)
        raise
    return hip.GpuExpert(done[0], done[1], done[2], hidden, inter)


__all__ = ["QtFile", "QtInfo", "QtError", "detect_group_size", "to_kblock", "from_kblock", "write_qt",
           "upload_expert"]
