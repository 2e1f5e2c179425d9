"""exp as the reference evaluates it. Rust's f32::exp (math.rs:108-111,
router.rs:52-170) is glibc's expf on Linux; the oracle calls glibc's expf and
the kernels call expf_glibc (peregrine_amd/csrc/expf_glibc.h), a restatement
of the published method glibc implements. These CPU tests pin the
restatement against the host's glibc over every f32 input, and measure what
the previous construction (exp in double, rounded once) would have changed."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from peregrine_amd import qt

HERE = os.path.dirname(os.path.abspath(__file__))
_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]
_libm.exp.restype = ctypes.c_double
_libm.exp.argtypes = [ctypes.c_double]


def _host_has_fma():
    try:
        return " fma " in open("/proc/cpuinfo").read().replace("\n", " ")
    except OSError:
        return False


@pytest.fixture(scope="module")
def sweep_bin(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("expf") / "expf_sweep")
    flags = ["-O2", "-std=c++17", "-ffp-contract=off", "-pthread"] + (["-mfma"] if _host_has_fma() else [])
    subprocess.run(["g++", *flags, os.path.join(HERE, "native", "expf_sweep.cpp"), "-o", out, "-lm"], check=True)
    return out


@pytest.mark.skipif(not _host_has_fma(), reason="glibc selects its FMA build of expf only on FMA CPUs")
def test_expf_glibc_equals_libm_on_every_f32(sweep_bin):
    """All 2^32 bit patterns (NaN payloads aside): zero differences."""
    r = subprocess.run([sweep_bin, "1", str(min(os.cpu_count() or 1, 8))], check=True, capture_output=True,
                       text=True, timeout=600)
    checked, bad = (int(v) for v in r.stdout.split()[1::2])
    assert checked == 1 << 32 and bad == 0, r.stdout + r.stderr


def test_double_rounded_exp_differs_from_glibc():
    """The construction used before, exp in double rounded once to f32,
    differs from glibc's expf on a measurable share of inputs (170,648 of the
    2^32 patterns on the glibc this was first measured on; 131 of this fixed
    sample of 200,000 in [-20, 20], where SiLU's and the router's arguments
    lie). The exact count depends on the glibc build, so only its presence
    and its rarity are asserted."""
    xs = np.random.default_rng(0).uniform(-20, 20, 200000).astype(np.float32)
    dbl = np.array([_libm.exp(float(v)) for v in xs], np.float64).astype(np.float32)
    gl = np.array([_libm.expf(float(v)) for v in xs], np.float32)
    n = int(np.sum(dbl.view(np.uint32) != gl.view(np.uint32)))
    assert 0 < n <= 0.01 * len(xs), n


def test_oracle_silu_is_glibc_expf(orc):
    xs = np.random.default_rng(1).uniform(-30, 30, 20000).astype(np.float32)
    for v in xs:
        ref = np.float32(v / np.float32(np.float32(1.0) + np.float32(_libm.expf(float(-v)))))
        assert ref.tobytes() == orc.silu(v).tobytes(), v


def _h_codes(g, u, exp_f32):
    den = np.float32(1.0) + exp_f32(-g)
    h = (g / den * u).astype(np.float32)
    return h


def test_h_requant_codes_under_both_exps(orc):
    """On the committed golden layer (every token through every expert), the
    SwiGLU h of glibc expf equals the oracle's h bit for bit, and the int8
    codes of h (per-32 and per-row) under the double-rounded exp: counted."""
    from tests.test_golden import GOLD, golden_layer_tensors
    f = np.load(os.path.join(GOLD, "moe_layer_small.npz"))
    experts = golden_layer_tensors(f, orc)
    x = f["x"]
    glibc = np.vectorize(lambda v: np.float32(_libm.expf(float(v))), otypes=[np.float32])
    dbl = np.vectorize(lambda v: np.float32(_libm.exp(float(v))), otypes=[np.float32])
    flips = {0: 0, 32: 0}
    for ga in (0, 32):
        xq, sx = orc.quant_rows(x, ga)
        for gate, up, down in experts:
            g = orc.linear(xq, sx, ga, gate)
            u = orc.linear(xq, sx, ga, up)
            h_gl = _h_codes(g, u, glibc)
            _, h_orc = orc.expert_swiglu(x, gate, up, down, ga, want_h=True)
            assert h_gl.tobytes() == h_orc.tobytes()
            h_db = _h_codes(g, u, dbl)
            qa, _ = orc.quant_rows(h_gl, ga)
            qb, _ = orc.quant_rows(h_db, ga)
            flips[ga] += int(np.sum(qa != qb))
    assert flips == {0: 0, 32: 0}, flips
