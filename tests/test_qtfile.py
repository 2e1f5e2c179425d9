"""The QT container loader bridge (peregrine_amd/qtfile.py) against the
reference's own container tests (peregrine-core/src/qt.rs:175-350) and the
kblock permutation's definition (peregrine-core/src/pack.rs:316-353)."""
import json
import struct

import numpy as np
import pytest

from peregrine_amd import qt, qtfile as Q


def test_group_size_probe_reference_cases():
    # qt.rs:176-185
    assert Q.detect_group_size(2, 32, 4) == 16
    assert Q.detect_group_size(2, 32, 2) == 0
    assert Q.detect_group_size(2, 64, 4) == 32
    assert Q.detect_group_size(4, 8, 100) == 0


def _zeros(n):
    return np.zeros(n, np.uint8)


def test_detect_formats(tmp_path):
    # qt.rs:197-232: O=2, I=32
    o, i = 2, 32
    Q.write_qt(str(tmp_path / "model.safetensors"), [
        ("w4", "U8", [o, i // 2], _zeros(32)), ("w4.qs", "F32", [o], _zeros(o * 4)),
        ("wg", "U8", [o, i // 2], _zeros(32)), ("wg.qs", "F32", [o * 2], _zeros(o * 2 * 4)),
        ("w8", "U8", [o, i], _zeros(64)), ("w8.qs", "F32", [o], _zeros(o * 4)),
        ("wf", "F32", [o, i], _zeros(o * i * 4)),
    ])
    with Q.QtFile(str(tmp_path / "model.safetensors")) as f:
        assert f.detect("w4", o, i).fmt == Q.FMT_I4
        g = f.detect("wg", o, i)
        assert g.fmt == Q.FMT_I4G and g.gs == 16 and g.scale_count == 4
        assert f.detect("w8", o, i).fmt == Q.FMT_I8
        assert f.detect("wf", o, i).fmt == Q.FMT_F32
        assert f.detect("absent", o, i).fmt == Q.FMT_F32


def test_int2_and_int2_g64_told_apart_by_scales(tmp_path):
    # qt.rs:234-274: same payload bytes, different scale cardinality
    o, i = 4, 128
    ng = (i + 63) // 64
    pay = o * (i // 4)
    assert pay == o * ng * 16
    Q.write_qt(str(tmp_path / "model.safetensors"), [
        ("wr", "U8", [o, i // 4], _zeros(pay)), ("wr.qs", "F32", [o], _zeros(o * 4)),
        ("wg", "U8", [o, i // 4], _zeros(pay)), ("wg.qs", "F32", [o * ng * 2], _zeros(o * ng * 2 * 4)),
    ])
    with Q.QtFile(str(tmp_path)) as f:
        assert f.detect("wr", o, i).fmt == Q.FMT_I2
        assert f.detect("wg", o, i).fmt == Q.FMT_I2G64


def test_int2_g64_ragged_width(tmp_path):
    # qt.rs:276-304
    o, i = 3, 100
    ng = (i + 63) // 64
    Q.write_qt(str(tmp_path / "model.safetensors"), [
        ("w", "U8", [o, ng * 16], _zeros(o * ng * 16)), ("w.qs", "F32", [o * ng * 2], _zeros(o * ng * 2 * 4)),
    ])
    with Q.QtFile(str(tmp_path)) as f:
        assert f.detect("w", o, i).fmt == Q.FMT_I2G64


def test_unrecognized_payload_size_is_not_guessed(tmp_path):
    # qt.rs:335-350
    o, i = 2, 32
    Q.write_qt(str(tmp_path / "model.safetensors"), [
        ("w", "U8", [o, 7], _zeros(o * 7)), ("w.qs", "F32", [o], _zeros(o * 4)),
    ])
    with Q.QtFile(str(tmp_path)) as f:
        assert f.detect("w", o, i).fmt == Q.FMT_UNKNOWN
        with pytest.raises(Q.QtError):
            f.read_qt("w", o, i)


def test_compressed_payload_detected_by_uncompressed_size_and_refused(tmp_path):
    # qt.rs:306-333: detection uses uncompressed_nbytes; this build has no zstd
    o, i = 4, 64
    path = tmp_path / "model.safetensors"
    Q.write_qt(str(path), [("w4", "U8", [o, i // 2], _zeros(20)), ("w4.qs", "F32", [o], _zeros(o * 4))])
    raw = path.read_bytes()
    (hlen,) = struct.unpack("<Q", raw[:8])
    hdr = json.loads(raw[8:8 + hlen])
    hdr["w4"]["compression"] = "zstd"
    hdr["w4"]["uncompressed_nbytes"] = o * (i // 2)
    new = json.dumps(hdr).encode()
    path.write_bytes(struct.pack("<Q", len(new)) + new + raw[8 + hlen:])
    with Q.QtFile(str(path)) as f:
        assert f.detect("w4", o, i).fmt == Q.FMT_I4
        with pytest.raises(Q.QtError, match="zstd"):
            f.read_raw("w4")


def test_kblock_permutation_matches_definition():
    rng = np.random.default_rng(5)
    o, g, gsb = 5, 7, 3
    b = rng.integers(0, 256, o * g * gsb, dtype=np.uint8)
    t = Q.to_kblock(b, o, gsb)
    ref = np.zeros_like(b)
    for row in range(o):              # pack.rs:321-335, the loop itself
        for gg in range(g):
            ref[(gg * o + row) * gsb:(gg * o + row + 1) * gsb] = b[(row * g + gg) * gsb:(row * g + gg + 1) * gsb]
    assert np.array_equal(t, ref)
    assert np.array_equal(Q.from_kblock(t, o, gsb), b)
    with pytest.raises(Q.QtError):
        Q.to_kblock(b[:-1], o, gsb)


def test_read_qt_kblock_grouped_int4_round_trip(tmp_path):
    rng = np.random.default_rng(6)
    o, i, gs = 6, 128, 32
    w = rng.standard_normal((o, i)).astype(np.float32)
    q, sc = qt.quant_i4_grouped(w, gs)
    tiled = Q.to_kblock(q, o, gs // 2)
    Q.write_qt(str(tmp_path / "model.safetensors"), [
        ("e.w", "U8", [o, i // 2], tiled, ("kblock", gs // 2)), ("e.w.qs", "F32", [sc.size], sc),
    ])
    with Q.QtFile(str(tmp_path)) as f:
        q2, sc2, info = f.read_qt("e.w", o, i)
    assert info.fmt == Q.FMT_I4G and info.gs == gs
    assert np.array_equal(q2, np.asarray(q).reshape(-1)) and np.array_equal(sc2, np.asarray(sc).reshape(-1))


def test_read_qt_refuses_formats_the_lane_does_not_compute(tmp_path):
    o, i = 2, 32
    Q.write_qt(str(tmp_path / "model.safetensors"), [
        ("wg", "U8", [o, i // 2], _zeros(32)), ("wg.qs", "F32", [o * 2], _zeros(16)),   # gs 16
        ("wf", "F32", [o, i], _zeros(o * i * 4)),
    ])
    with Q.QtFile(str(tmp_path)) as f:
        with pytest.raises(Q.QtError, match="gs=16"):
            f.read_qt("wg", o, i)
        with pytest.raises(Q.QtError, match="format 0"):
            f.read_qt("wf", o, i)
