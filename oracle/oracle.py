"""ctypes front-end of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` — as the checker, never as the thing
measured or shipped. The product package ``peregrine_amd`` does not import it.

Each wrapper names the C function it calls; the C file cites the peregrine
source it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build() -> None:
    """Compile oracle/liboracle.so with the Makefile beside this file."""
    subprocess.run(["make", "-s", "-C", _HERE, "-B", "liboracle.so"], check=True)


def _load() -> C.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    return C.CDLL(_LIB_PATH)


_lib = _load()

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")


class _OrcTensor(C.Structure):
    _fields_ = [("q", C.c_void_p), ("scale", C.c_void_p), ("fmt", C.c_int), ("I", C.c_int),
                ("O", C.c_int), ("gs", C.c_int)]


class _OrcExpert(C.Structure):
    _fields_ = [("gate", _OrcTensor), ("up", _OrcTensor), ("down", _OrcTensor)]


def _sig(name, res, *args):
    fn = getattr(_lib, name)
    fn.restype = res
    fn.argtypes = list(args)
    return fn


_qrow = _sig("orc_qrow_i8", C.c_float, _f32p, C.c_int, _i8p)
_quant_rows = _sig("orc_quant_rows", None, _f32p, C.c_int, C.c_int, C.c_int, _i8p, _f32p)
_dot88 = _sig("orc_dot_i8i8", C.c_int32, _i8p, _i8p, C.c_int)
_dot48 = _sig("orc_dot_i4i8", C.c_int32, _u8p, _i8p, C.c_int)
_dot48g = _sig("orc_dot_i4i8_grouped", C.c_float, _u8p, _i8p, _f32p, C.c_int, C.c_int)
_dot48v = _sig("orc_dot_i4i8_avx2", C.c_int32, _u8p, _i8p, C.c_int)
_have_avx2 = _sig("orc_have_avx2", C.c_int)
_linear = _sig("orc_linear", None, _f32p, _i8p, _f32p, C.c_int, C.POINTER(_OrcTensor), C.c_int)
_block_dots = _sig("orc_block_dots", None, _i32p, _i8p, C.POINTER(_OrcTensor), C.c_int)
_matmul_f32 = _sig("orc_matmul_f32", None, _f32p, _f32p, _f32p, C.c_int, C.c_int, C.c_int)
_silu = _sig("orc_silu", C.c_float, C.c_float)
_silu_mul = _sig("orc_silu_mul", None, _f32p, _f32p, C.c_int)
_swiglu = _sig("orc_expert_swiglu", None, _f32p, _f32p, C.c_int, C.POINTER(_OrcTensor),
               C.POINTER(_OrcTensor), C.POINTER(_OrcTensor), C.c_int, C.c_void_p)
_route_sig = _sig("orc_route_sigmoid", C.c_int, _f32p, _f32p, C.c_int, C.c_int, C.c_int, C.c_int,
                  C.c_float, C.c_float, _i32p, _f32p, _i32p)
_neg_tail = _sig("orc_negligible_tail", C.c_int, _f32p, C.c_int, C.c_float)
_route_smx = _sig("orc_route_softmax_topk", None, _f32p, C.c_int, C.c_int, C.c_int, _i32p, _f32p)
_union = _sig("orc_batch_union", C.c_int, _i32p, C.c_void_p, C.c_int, C.c_int, C.c_int, _i32p)
_table = _sig("orc_expert_table", C.c_int, _i32p, C.c_int, C.c_int, C.c_int, _i32p, _i32p, _i32p,
              _i32p, _i32p)
_rl_build = _sig("orc_reduce_layout_build", C.c_int, _i32p, C.c_int, C.c_int, _i32p, _i32p)
_greduce = _sig("orc_grouped_reduce", None, _f32p, _f32p, _i32p, _i32p, _f32p, C.c_int, C.c_int)
_moe = _sig("orc_moe_forward", C.c_int, _f32p, _f32p, C.c_int, C.c_int, _i32p, _f32p, C.c_int,
            C.POINTER(_OrcExpert), C.c_int, C.c_int, C.c_void_p, C.c_int, C.c_int, C.c_int)


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


class Tensor:
    """A QT weight as the oracle sees it (peregrine-core/src/qt.rs:14-45).

    ``q`` is the row-major byte payload ([O][ceil(I/2)] for int4, [O][I] for
    int8), ``scale`` holds O per-row or O*ceil(I/gs) grouped f32 scales.
    """

    def __init__(self, q, scale, fmt, I, O, gs=0):
        self.fmt, self.I, self.O, self.gs = int(fmt), int(I), int(O), int(gs)
        self.q = _c(q, np.int8 if fmt in (1, 8) else np.uint8).reshape(-1)
        self.scale = _c(scale, np.float32).reshape(-1)
        self._s = _OrcTensor(self.q.ctypes.data, self.scale.ctypes.data, self.fmt, self.I, self.O, self.gs)

    @property
    def ref(self):
        return C.byref(self._s)


def qrow_i8(x):
    x = _c(x, np.float32)
    q = np.zeros(x.shape[-1], np.int8)
    s = _qrow(x, x.size, q)
    return q, np.float32(s)


def quant_rows(x, ga=0):
    """orc_quant_rows: int8 rows plus [rows] (ga=0) or [rows][ceil(n/ga)] scales."""
    x = _c(x, np.float32)
    rows, n = x.shape
    q = np.zeros((rows, n), np.int8)
    nb = 1 if ga <= 0 else -(-n // ga)
    sx = np.zeros((rows, nb), np.float32)
    _quant_rows(x, rows, n, ga, q, sx)
    return q, sx


def dot_i8i8(w, x):
    return int(_dot88(_c(w, np.int8), _c(x, np.int8), len(x)))


def dot_i4i8(w4, x, n=None):
    x = _c(x, np.int8)
    return int(_dot48(_c(w4, np.uint8), x, len(x) if n is None else n))


def dot_i4i8_avx2(w4, x, n=None):
    x = _c(x, np.int8)
    return int(_dot48v(_c(w4, np.uint8), x, len(x) if n is None else n))


def dot_i4i8_grouped(w4, x, scales, gs):
    x = _c(x, np.int8)
    return np.float32(_dot48g(_c(w4, np.uint8), x, _c(scales, np.float32), len(x), gs))


def have_avx2() -> bool:
    return bool(_have_avx2())


def linear(xq, sx, ga, t: Tensor):
    xq = _c(xq, np.int8)
    S = xq.shape[0]
    y = np.zeros((S, t.O), np.float32)
    _linear(y, xq, _c(sx, np.float32), ga, t.ref, S)
    return y


def block_dots(xq, t: Tensor):
    """int32 dots per (row, output, 32-block): shape [S, O, ceil(I/32)]."""
    xq = _c(xq, np.int8)
    S = xq.shape[0]
    nb = -(-t.I // 32)
    d = np.zeros((S, t.O, nb), np.int32)
    _block_dots(d, xq, t.ref, S)
    return d


def matmul_f32(x, w, d_n, o_n):
    x = _c(x, np.float32)
    s_n = x.size // d_n
    y = np.zeros((s_n, o_n), np.float32)
    _matmul_f32(y, x, _c(w, np.float32), s_n, d_n, o_n)
    return y


def silu(v):
    return np.float32(_silu(float(v)))


def silu_mul(g, u):
    g = _c(g, np.float32).copy()
    _silu_mul(g, _c(u, np.float32), g.size)
    return g


def expert_swiglu(x, gate: Tensor, up: Tensor, down: Tensor, ga=0, want_h=False):
    x = _c(x, np.float32)
    S = x.shape[0]
    y = np.zeros((S, down.O), np.float32)
    h = np.zeros((S, gate.O), np.float32) if want_h else None
    _swiglu(y, x, S, gate.ref, up.ref, down.ref, ga, h.ctypes.data if want_h else None)
    return (y, h) if want_h else y


def route_sigmoid(logits, bias, k, norm_topk=True, routed_scale=1.0, min_share=0.0):
    logits = _c(logits, np.float32)
    s_n, e_n = logits.shape
    idx = np.zeros((s_n, k), np.int32)
    w = np.zeros((s_n, k), np.float32)
    keff = np.zeros(s_n, np.int32)
    _route_sig(logits, _c(bias, np.float32), s_n, e_n, k, int(norm_topk), routed_scale, min_share, idx, w, keff)
    return idx, w, keff


def negligible_tail(w, kept, min_share):
    return int(_neg_tail(_c(w, np.float32), kept, min_share))


def route_softmax_topk(logits, k):
    logits = _c(logits, np.float32)
    s_n, e_n = logits.shape
    idx = np.zeros((s_n, k), np.int32)
    w = np.zeros((s_n, k), np.float32)
    _route_smx(logits, s_n, e_n, k, idx, w)
    return idx, w


def batch_union(idx, e_n, keff=None):
    idx = _c(idx, np.int32)
    s_n, k = idx.shape
    out = np.zeros(e_n, np.int32)
    ke = _c(keff, np.int32) if keff is not None else None
    n = _union(idx, ke.ctypes.data if ke is not None else None, s_n, k, e_n, out)
    return out[:n]


def expert_table(idx, e_n):
    """orc_expert_table -> dict(uexp, off, row_tok, row_kk, tok_rows)."""
    idx = _c(idx, np.int32)
    s_n, k = idx.shape
    R = s_n * k
    uexp = np.zeros(e_n, np.int32)
    off = np.zeros(e_n + 1, np.int32)
    row_tok = np.zeros(R, np.int32)
    row_kk = np.zeros(R, np.int32)
    tok_rows = np.zeros((s_n, k), np.int32)
    n_u = _table(idx, s_n, k, e_n, uexp, off, row_tok, row_kk, tok_rows)
    nr = int(off[n_u])
    return dict(n_u=n_u, uexp=uexp[:n_u], off=off[:n_u + 1], row_tok=row_tok[:nr], row_kk=row_kk[:nr],
                tok_rows=tok_rows)


def reduce_layout_build(dst, s_n):
    """ReduceLayout::build restated; None when a dst is out of range."""
    dst = _c(dst, np.int32)
    row_ptr = np.zeros(s_n + 1, np.int32)
    row_idx = np.zeros(max(dst.size, 1), np.int32)
    if not _rl_build(dst, dst.size, s_n, row_ptr, row_idx):
        return None
    return row_ptr, row_idx[:dst.size]


def grouped_reduce(y, row_ptr, row_idx, rw, s_n):
    y = _c(y, np.float32)
    D = y.shape[1]
    out = np.zeros((s_n, D), np.float32)
    _greduce(out, y, _c(row_ptr, np.int32), _c(row_idx, np.int32), _c(rw, np.float32), s_n, D)
    return out


def moe_forward(x, idx, w, experts, ga=0, subset=None, nthreads=1, simd=False):
    """orc_moe_forward: experts is a list of (gate, up, down) Tensor triples."""
    x = _c(x, np.float32)
    idx = _c(idx, np.int32)
    w = _c(w, np.float32)
    s_n, D = x.shape
    k = idx.shape[1]
    arr = (_OrcExpert * len(experts))()
    for i, (g, u, d) in enumerate(experts):
        arr[i] = _OrcExpert(g._s, u._s, d._s)
    out = np.zeros((s_n, D), np.float32)
    sub = _c(subset, np.int32) if subset is not None else None
    _moe(out, x, s_n, D, idx, w, k, arr, len(experts), ga, sub.ctypes.data if sub is not None else None,
         0 if sub is None else sub.size, nthreads, int(simd))
    return out
