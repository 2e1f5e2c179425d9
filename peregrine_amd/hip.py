"""Host-side mirror of peregrine's GPU-lane API over libperegrine_hip.so.

Same names, argument meaning and error behaviour as the Rust crate this lane
replaces (crates/peregrine-cuda/src/lib.rs): ``init``, ``shutdown``,
``mem_info``, ``GpuExpert.upload_int4``, ``expert_group``,
``expert_group_tiled``, ``ReduceLayout.build``, ``expert_group_reduce``,
``group_stats``, ``graph_cache_stats``, ``capture``/``Graph``. Failures raise
``HipError`` where the Rust API returns ``Err(Error::Format(..))``.

Additions (no reference counterpart): ``GpuExpert.upload_grouped`` for grouped
int4/int8 QT tensors, ``ExpertSet`` + ``moe_forward_dev`` for a whole routed
MoE layer with activations resident in HBM, and instrumentation helpers.
"""
from __future__ import annotations

import ctypes as C
import enum
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import qt
from ._lib import lib


class HipError(RuntimeError):
    """Error::Format of the reference crate."""


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


def _ipt(a: np.ndarray):
    return a.ctypes.data_as(C.POINTER(C.c_int))


# ---------------------------------------------------------------- devices (lib.rs:160-254)

def device_count() -> int:
    return int(lib.coli_hip_device_count())


def probe_device_count() -> int:
    return int(lib.coli_hip_probe_device_count())


def is_available() -> bool:
    return probe_device_count() > 0


def status() -> str:
    return "HIP backend linked (peregrine_amd/csrc, gfx950)"


def init(devices: Sequence[int]) -> int:
    arr = (C.c_int * len(devices))(*devices)
    return int(lib.coli_hip_init(arr, len(devices)))


def shutdown() -> None:
    lib.coli_hip_shutdown()


def mem_info(device: int):
    free, total = C.c_size_t(0), C.c_size_t(0)
    if lib.coli_hip_mem_info(device, C.byref(free), C.byref(total)) != 1:
        raise HipError(f"hip mem_info(device={device}) failed")
    return free.value, total.value


def pipe_sync(device: int = 0) -> None:
    if lib.coli_hip_pipe_sync(device) != 1:
        raise HipError("hip stream synchronize failed")


# ---------------------------------------------------------------- resident experts (lib.rs:256-414)

def _upload(device, q, scales, fmt, i, o, gs=0):
    t = C.c_void_p(None)
    q = np.ascontiguousarray(q)
    s = _f32(scales)
    if fmt in (qt.FMT_I4, qt.FMT_I8):
        ok = lib.coli_hip_tensor_upload(C.byref(t), _ptr(q), _ptr(s), fmt, i, o, device)
    else:
        ok = lib.coli_hip_tensor_upload_grouped(C.byref(t), _ptr(q), _ptr(s), fmt, i, o, gs, device)
    if ok != 1 or not t.value:
        lib.coli_hip_tensor_free(t)
        raise HipError(f"hip tensor_upload failed (fmt={fmt}, i={i}, o={o}, gs={gs})")
    return t


class GpuExpert:
    """One expert's gate/up/down resident in HBM; frees them when dropped."""

    def __init__(self, gate, up, down, hidden: int, inter: int):
        self.gate, self.up, self.down = gate, up, down
        self.hidden, self.inter = hidden, inter

    @staticmethod
    def upload(device, gate, up, down, hidden, inter):
        """f32 experts (fmt 0) are not resident on this lane: the IDOT kernels
        consume quantised weights only. Quantise first (qt.quant_i4_*)."""
        raise HipError("gpu expert upload: f32 weights are not supported by the HIP lane; upload quantised QT tensors")

    @staticmethod
    def upload_int4(device, gate, up, down, hidden, inter):
        """Per-row int4 (fmt 2): each argument is (packed_nibbles, row_scales)."""
        def ok(t, o, i):
            return np.asarray(t[0]).size == o * ((i + 1) // 2) and np.asarray(t[1]).size == o
        if not (ok(gate, inter, hidden) and ok(up, inter, hidden) and ok(down, hidden, inter)):
            raise HipError("gpu int4 expert upload: byte/scale length mismatch")
        return GpuExpert._upload3(device, gate, up, down, hidden, inter, qt.FMT_I4, 0)

    @staticmethod
    def upload_grouped(device, gate, up, down, hidden, inter, fmt=qt.FMT_I4G, gs=32):
        """Grouped QT (fmt 4 int4 or 8 int8) with scales sc[o*ng+g]; also fmt 1/2."""
        return GpuExpert._upload3(device, gate, up, down, hidden, inter, fmt, gs)

    @staticmethod
    def _upload3(device, gate, up, down, hidden, inter, fmt, gs):
        done = []
        try:
            for (q, s), (i, o) in ((gate, (hidden, inter)), (up, (hidden, inter)), (down, (inter, hidden))):
                done.append(_upload(device, q, s, fmt, i, o, gs))
        except HipError:
            for t in done:
                lib.coli_hip_tensor_free(t)
            raise
        return GpuExpert(done[0], done[1], done[2], hidden, inter)

    def bytes(self) -> int:
        return sum(int(lib.coli_hip_tensor_bytes(t)) for t in (self.gate, self.up, self.down))

    def close(self):
        for name in ("gate", "up", "down"):
            t = getattr(self, name, None)
            if t is not None:
                lib.coli_hip_tensor_free(t)
                setattr(self, name, None)

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _handles(experts):
    n = len(experts)
    g = (C.c_void_p * n)(*[e.gate for e in experts])
    u = (C.c_void_p * n)(*[e.up for e in experts])
    d = (C.c_void_p * n)(*[e.down for e in experts])
    return g, u, d


def _check(experts, rows, x, hidden, what):
    if len(experts) != len(rows):
        raise HipError(f"{what}: experts/rows length mismatch")
    if any(r < 0 for r in rows):
        raise HipError(f"{what}: negative row count")
    total = int(sum(rows))
    if np.asarray(x).size != total * hidden:
        raise HipError(f"{what}: x length != sum(rows)*hidden")
    return total


def expert_group(experts, rows, x, hidden):
    """lib.rs:420: y[sum(rows), hidden] for VRAM-resident experts."""
    y, _ = _dispatch(experts, rows, x, hidden, want_arm=False)
    return y


class GroupArm(enum.Enum):
    """Which kernel arm ran (lib.rs:437-477). The matrix-core arm takes the
    reference's Int4Tc code (0), the GEMV arm its PackedW4 code (2)."""
    Int4Tc = 0
    W4A16 = 1
    PackedW4 = 2
    Generic = 3

    @staticmethod
    def from_c(v: int) -> "GroupArm":
        return {0: GroupArm.Int4Tc, 1: GroupArm.W4A16, 2: GroupArm.PackedW4}.get(v, GroupArm.Generic)


def expert_group_tiled(experts, rows, x, hidden, tile=None):
    return _dispatch(experts, rows, x, hidden, want_arm=True, tile=tile)


def _dispatch(experts, rows, x, hidden, want_arm, tile=None):
    total = _check(experts, rows, x, hidden, "expert_group")
    xr = _f32(x)
    y = np.zeros((total, hidden), np.float32)
    rw = _i32(rows)
    g, u, d = _handles(experts)
    if not want_arm:
        ok = lib.coli_hip_expert_group(g, u, d, _ipt(rw), len(experts), _ptr(y), _ptr(xr))
        arm = None
    else:
        tm, tn, tk = tile if tile else (0, 0, 0)
        a = C.c_int(-1)
        ok = lib.coli_hip_expert_group_tiled(g, u, d, _ipt(rw), len(experts), _ptr(y), _ptr(xr), tm, tn, tk,
                                             C.byref(a))
        arm = GroupArm.from_c(a.value)
    if ok != 1:
        raise HipError("hip expert_group failed")
    return y, arm


@dataclass
class ReduceLayout:
    """CSR the fused reduce accumulates through (lib.rs:562-604)."""
    row_ptr: np.ndarray
    row_idx: np.ndarray

    @staticmethod
    def build(dst, s_n: int) -> Optional["ReduceLayout"]:
        """Counting sort of y-row k into output row dst[k], ascending k; None
        if any dst is out of range."""
        dst = np.asarray(dst, dtype=np.int64)
        if np.any(dst < 0) or np.any(dst >= s_n):
            return None
        counts = np.zeros(s_n + 1, np.int32)
        np.add.at(counts, dst + 1, 1)
        row_ptr = np.cumsum(counts).astype(np.int32)
        fill = row_ptr[:-1].copy()
        row_idx = np.zeros(dst.size, np.int32)
        for k, s in enumerate(dst):
            row_idx[fill[s]] = k
            fill[s] += 1
        return ReduceLayout(row_ptr, row_idx)


def expert_group_reduce(experts, rows, x, hidden, layout: ReduceLayout, rw, s_n: int):
    """lib.rs:620: expert_group with the gate-weighted reduce fused on device."""
    total = _check(experts, rows, x, hidden, "expert_group_reduce")
    rw = _f32(rw)
    if rw.size != total or layout.row_idx.size != total:
        raise HipError("expert_group_reduce: weights/row_idx length != sum(rows)")
    if s_n == 0 or layout.row_ptr.size != s_n + 1:
        raise HipError("expert_group_reduce: row_ptr length != s_n + 1")
    if layout.row_ptr[-1] != total or layout.row_ptr[0] != 0:
        raise HipError("expert_group_reduce: row_ptr does not span [0, sum(rows)]")
    if np.any(layout.row_idx < 0) or np.any(layout.row_idx >= total):
        raise HipError("expert_group_reduce: row_idx out of range")
    out = np.zeros((s_n, hidden), np.float32)
    rp, ri, rws = _i32(layout.row_ptr), _i32(layout.row_idx), _i32(rows)
    g, u, d = _handles(experts)
    ok = lib.coli_hip_expert_group_reduce(g, u, d, _ipt(rws), len(experts), _ipt(rp), _ipt(ri), _ptr(rw), s_n,
                                          _ptr(out), _ptr(_f32(x)))
    if ok != 1:
        raise HipError("hip expert_group_reduce failed")
    return out


# ---------------------------------------------------------------- stats (lib.rs:151, 686-737)

@dataclass
class GroupStats:
    calls: int = 0
    experts: int = 0
    rows: int = 0
    h2d_ms: float = 0.0
    kernel_ms: float = 0.0
    d2h_ms: float = 0.0


def group_stats() -> GroupStats:
    v = [C.c_uint64(0) for _ in range(3)] + [C.c_double(0) for _ in range(3)]
    lib.coli_hip_group_stats(*[C.byref(a) for a in v])
    return GroupStats(*[a.value for a in v])


@dataclass
class GraphCacheStats:
    captures: int = 0
    replays: int = 0
    invalidations: int = 0
    uncacheable: int = 0


def graph_cache_stats() -> GraphCacheStats:
    v = [C.c_uint64(0) for _ in range(4)]
    lib.coli_hip_graph_cache_stats(*[C.byref(a) for a in v])
    return GraphCacheStats(*[a.value for a in v])


class Graph:
    """A captured + instantiated HIP graph of a device's stream (lib.rs:744-798)."""

    def __init__(self, ptr):
        self.ptr = ptr

    def launch(self):
        if lib.coli_hip_graph_launch(self.ptr) != 1:
            raise HipError("hip graph launch failed")

    def __del__(self):
        try:
            lib.coli_hip_graph_free(self.ptr)
        except Exception:
            pass


def capture(device: int, body) -> Graph:
    """Capture the ops `body` issues on the device stream; the capture is
    always ended, even when body raises."""
    if lib.coli_hip_graph_begin(device) != 1:
        raise HipError("hip graph begin failed")
    err = None
    try:
        body()
    except Exception as e:  # surfaced after the capture is closed
        err = e
    p = C.c_void_p(None)
    ended = lib.coli_hip_graph_end(device, C.byref(p))
    g = Graph(p) if ended == 1 and p.value else None
    if err is not None:
        raise err
    if g is None:
        raise HipError("hip graph end/instantiate failed")
    return g


# ---------------------------------------------------------------- device-resident layer (new)

def set_act_group(ga: int) -> None:
    if lib.coli_hip_set_act_group(ga) != 1:
        raise HipError("act group must be 0 or 32")


def set_arm(arm: int) -> None:
    if lib.coli_hip_set_arm(arm) != 1:
        raise HipError("unknown arm")


def set_fused_route(mode: int) -> None:
    """One-token router inside the gate/up GEMV: -1 automatic, 0 never, 1 whenever eligible."""
    if lib.coli_hip_set_fused_route(mode) != 1:
        raise HipError("coli_hip_set_fused_route failed")


def set_gemv_split(target_wgs: int) -> None:
    """Split-K decode GEMV: workgroups a GEMV launch aims for (0: never
    split, -1: the default)."""
    if lib.coli_hip_set_gemv_split(target_wgs) != 1:
        raise HipError("coli_hip_set_gemv_split failed")


def set_fused_combine(mode: int) -> None:
    """One token on the GEMV arm, down projection and combine in one launch:
    -1 automatic (k <= 2), 0 never, 1 whenever eligible (k <= 8, K <= 1536)."""
    if lib.coli_hip_set_fused_combine(mode) != 1:
        raise HipError("coli_hip_set_fused_combine failed")


ARM_AUTO, ARM_MFMA, ARM_GEMV = -1, 0, 2


class ExpertSet:
    """A fixed expert table on one device: expert id -> GpuExpert."""

    def __init__(self, experts: Sequence[GpuExpert]):
        self.experts = list(experts)
        g, u, d = _handles(self.experts)
        p = C.c_void_p(None)
        if lib.coli_hip_expert_set_create(C.byref(p), g, u, d, len(self.experts)) != 1:
            raise HipError("hip expert_set_create failed")
        self.ptr = p

    def close(self):
        if getattr(self, "ptr", None):
            lib.coli_hip_expert_set_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def route_softmax_topk_dev(device, logits_ptr, S, E, k, ids_ptr, w_ptr):
    if lib.coli_hip_route_softmax_topk_dev(device, C.c_void_p(logits_ptr), S, E, k, C.c_void_p(ids_ptr),
                                           C.c_void_p(w_ptr)) != 1:
        raise HipError("hip route_softmax_topk failed")


def route_sigmoid_topk_dev(device, logits_ptr, bias_ptr, S, E, k, ids_ptr, w_ptr, keff_ptr=0, norm_topk=True,
                           routed_scale=1.0, min_share=0.0):
    """router.rs:52-170 on the device (async): sigmoid scores, top-k over
    score + bias (bias_ptr 0: none), weights = sigmoid, tail drop, renorm,
    routed_scale; keff_ptr (optional) receives the kept counts."""
    if lib.coli_hip_route_sigmoid_topk_dev(device, C.c_void_p(logits_ptr), C.c_void_p(bias_ptr or None), S, E, k,
                                           int(norm_topk), float(routed_scale), float(min_share),
                                           C.c_void_p(ids_ptr), C.c_void_p(w_ptr),
                                           C.c_void_p(keff_ptr or None)) != 1:
        raise HipError("hip route_sigmoid_topk failed")


def moe_forward_dev(eset: ExpertSet, x_ptr, S, ids_ptr, w_ptr, k, out_ptr, act_group=0, arm=ARM_AUTO):
    """Async: enqueue one routed MoE layer on the device stream."""
    if lib.coli_hip_moe_forward_dev(eset.ptr, C.c_void_p(x_ptr), S, C.c_void_p(ids_ptr), C.c_void_p(w_ptr), k,
                                    C.c_void_p(out_ptr), act_group, arm) != 1:
        raise HipError("hip moe_forward failed")


def moe_forward_dev_noalloc(eset: ExpertSet, x_ptr, S, ids_ptr, w_ptr, k, out_ptr, act_group=0, arm=ARM_AUTO):
    """As moe_forward_dev, with no device allocation: scratch is the device's
    fixed array (refused above its size)."""
    if lib.coli_hip_moe_forward_dev_noalloc(eset.ptr, C.c_void_p(x_ptr), S, C.c_void_p(ids_ptr),
                                            C.c_void_p(w_ptr), k, C.c_void_p(out_ptr), act_group, arm) != 1:
        raise HipError("hip moe_forward (no allocation) failed")


def moe_forward_logits_dev(eset: ExpertSet, x_ptr, S, logits_ptr, k, ids_ptr, w_ptr, out_ptr, act_group=0,
                           arm=ARM_AUTO):
    """Async: route logits[S][E] (writing ids/w) and run the layer, router fused."""
    if lib.coli_hip_moe_forward_logits_dev(eset.ptr, C.c_void_p(x_ptr), S, C.c_void_p(logits_ptr), k,
                                           C.c_void_p(ids_ptr), C.c_void_p(w_ptr), C.c_void_p(out_ptr), act_group,
                                           arm) != 1:
        raise HipError("hip moe_forward_logits failed")


def stream_handle(device: int = 0) -> int:
    return int(lib.coli_hip_stream(device) or 0)


def set_profile(on: bool) -> None:
    lib.coli_hip_set_profile(1 if on else 0)


KERNELS = ("table", "quant_x", "gateup", "quant_h", "down", "combine")


def kernel_stats():
    out = {}
    for i, name in enumerate(KERNELS):
        n, ms = C.c_uint64(0), C.c_double(0)
        lib.coli_hip_kernel_stats(i, C.byref(n), C.byref(ms))
        out[name] = (n.value, ms.value)
    return out


def reset_stats() -> None:
    lib.coli_hip_reset_stats()


def set_debug_dots(gateup_ptr: int = 0, down_ptr: int = 0) -> None:
    lib.coli_hip_set_debug_dots(C.c_void_p(gateup_ptr or None), C.c_void_p(down_ptr or None))


def set_spin_limit(polls: int) -> None:
    """Test hook: polls before a GEMV bounded wait gives up (0: the default)."""
    if lib.coli_hip_set_spin_limit(polls) != 1:
        raise HipError("spin limit must be >= 0")


def last_table(device, E, R):
    hdr = np.zeros(4, np.int32)
    uexp = np.zeros(E, np.int32)
    off = np.zeros(E + 1, np.int32)
    row_tok = np.zeros(R, np.int32)
    tok_rows = np.zeros(R, np.int32)
    if lib.coli_hip_last_table(device, _ipt(hdr), _ipt(uexp), _ipt(off), _ipt(row_tok), _ipt(tok_rows), E, R) != 1:
        raise HipError("hip last_table failed")
    n_u = int(hdr[2])
    return dict(rows=int(hdr[0]), tiles=int(hdr[1]), n_u=n_u, uexp=uexp[:n_u], off=off[:n_u + 1],
                row_tok=row_tok[:int(hdr[0])], tok_rows=tok_rows)


# ---------------------------------------------------------------- device memory (pipe_* primitives)

class DeviceBuffer:
    """Raw device allocation through coli_hip_pipe_alloc (no torch involved)."""

    def __init__(self, nbytes: int, device: int = 0):
        self.device, self.nbytes = device, int(nbytes)
        self.ptr = int(lib.coli_hip_pipe_alloc(device, max(self.nbytes, 1)) or 0)
        if not self.ptr:
            raise HipError(f"hip pipe_alloc({nbytes}) failed")

    @staticmethod
    def from_array(arr: np.ndarray, device: int = 0) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        b = DeviceBuffer(arr.nbytes, device)
        b.upload(arr)
        return b

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise HipError("upload larger than the buffer")
        if lib.coli_hip_pipe_upload(self.device, C.c_void_p(self.ptr), _ptr(arr), arr.nbytes) != 1:
            raise HipError("hip pipe_upload failed")

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype)
        if out.nbytes > self.nbytes:
            raise HipError("download larger than the buffer")
        if lib.coli_hip_pipe_download(self.device, C.c_void_p(self.ptr), _ptr(out), out.nbytes) != 1:
            raise HipError("hip pipe_download failed")
        return out

    def fill(self, n: int, kind: int, a: float = 0.0, b: float = 1.0, seed: int = 0) -> None:
        if lib.coli_hip_synth_fill(self.device, C.c_void_p(self.ptr), n, kind, a, b, seed & ((1 << 64) - 1)) != 1:
            raise HipError("hip synth_fill failed")

    def free(self) -> None:
        if self.ptr:
            lib.coli_hip_pipe_free(self.device, C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def upload_tensor_dev(device, w_ptr, sc_ptr, fmt, i, o, gs):
    """Resident tensor from QT bytes/scales already in device memory."""
    t = C.c_void_p(None)
    if lib.coli_hip_tensor_upload_dev(C.byref(t), C.c_void_p(w_ptr), C.c_void_p(sc_ptr), fmt, i, o, gs, device) != 1:
        raise HipError(f"hip tensor_upload_dev failed (fmt={fmt}, i={i}, o={o}, gs={gs})")
    return t


def event_record(device: int, slot: int) -> None:
    if lib.coli_hip_event_record(device, slot) != 1:
        raise HipError("hip event_record failed")


def event_elapsed(device: int, a: int, b: int) -> float:
    ms = float(lib.coli_hip_event_elapsed(device, a, b))
    if ms < 0:
        raise HipError("hip event_elapsed failed")
    return ms
