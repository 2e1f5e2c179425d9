"""Benchmark of the MI355X MoE expert lane on BASELINE.json's configurations.

A step is one routed MoE layer (config 5: four resident layers back to back)
over one batch of synthetic tokens: device router (softmax top-k) ->
expert-offset table -> int8 activation quant -> fused gate/up + SwiGLU (+ h
quant) -> down -> weighted combine. Inputs (tokens, router logits, resident
experts) are in HBM before timing starts; every step uses its own tokens and
router logits, so the experts a step reads change from step to step.

    python bench.py                      # config 5 (the largest single-GPU one), int4
    python bench.py --config 2           # decode, batch 1 (headline = that config)
    python bench.py --config 5 --wfmt int8

The JSON line's headline is the chosen config. Unless --no-detail, it also
carries the decode config 2 (HBM fraction) and the prefill config 4 (int8
MFMA fraction) under detail.workloads, each with its own roofline.

Kernel durations come from HIP events that the kernels' own dispatch packets
record (hipExtLaunchKernelGGL) in a second, profiled pass over the same steps:
kernel execution alone, as rocprofv3's kernel trace measures it.
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, published (no sparsity)

# The five benchmark configurations, numbered 1..5
CONFIGS = {
    1: dict(name="cfg1_single_expert_1tok", E=1, D=5120, I=1536, S=1, k=1, route="one", layers=1),
    2: dict(name="cfg2_decode_moe_layer_b1_160x_int4", E=160, D=5120, I=1536, S=1, k=8, route="normal", layers=1),
    3: dict(name="cfg3_batched_decode_64tok_zipf", E=160, D=5120, I=1536, S=64, k=8, route="zipf", layers=1),
    4: dict(name="cfg4_prefill_2048tok_zipf", E=160, D=5120, I=1536, S=2048, k=8, route="zipf", layers=1),
    5: dict(name="cfg5_large_layer_512tok_256x", E=256, D=6144, I=2048, S=512, k=8, route="normal", layers=4),
}
DEFAULT_STEPS = {1: 200, 2: 200, 3: 100, 4: 20, 5: 20}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", type=int, default=5, choices=sorted(CONFIGS))
    ap.add_argument("--wfmt", choices=("int4", "int8"), default="int4")
    ap.add_argument("--act-group", type=int, default=32, choices=(0, 32),
                    help="activation scale per 32-block (BASELINE, default) or per row (reference)")
    ap.add_argument("--arm", choices=("auto", "gemv", "mfma"), default="auto")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--no-detail", action="store_true", help="only the chosen config (no config 2 / 4 lines)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-pcie", action="store_true",
                    help="skip the host-buffer (PCIe-inclusive) timing, e.g. under a profiler")
    ap.add_argument("--cpu-seconds", type=float, default=8.0,
                    help="CPU work per thread setting of the baseline (single thread, then all cores)")
    ap.add_argument("--experts", type=int, default=None, help="override the resident expert count (experiments)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device-to-device copy kernel 5 times (scales rocprofv3 "
                         "FETCH_SIZE/WRITE_SIZE to bytes)")
    return ap.parse_args()


def algorithmic(cfg, wfmt, distinct):
    """Bytes (weights + scales of each distinct expert touched, once) and int
    ops for one layer; the per-expert figure is D*I*(3 matrices)."""
    D, I = cfg["D"], cfg["I"]
    wb = 0.5 if wfmt == "int4" else 1.0
    per_mat = D * I * wb + D * I / 32 * 4
    gateup_bytes = distinct * 2 * per_mat
    layer_bytes = distinct * 3 * per_mat
    rows = cfg["S"] * cfg["k"]
    gateup_ops = 2 * 2 * rows * D * I
    layer_ops = 3 * 2 * rows * D * I
    return gateup_bytes, layer_bytes, gateup_ops, layer_ops


def build_experts(hip, cfg, wfmt, seed):
    """Resident experts with device-generated QT bytes (uniform nibbles =
    int4 values uniform in [-8, 7]; int8 uniform bytes) and lognormal(ln 0.01,
    0.5) scales per 32 weights. One staging buffer is reused."""
    from peregrine_amd import qt
    D, I, E, L = cfg["D"], cfg["I"], cfg["E"], cfg["layers"]
    fmt = qt.FMT_I4G if wfmt == "int4" else qt.FMT_I8G
    wbytes = D * I // 2 if wfmt == "int4" else D * I
    nsc = D * I // 32
    raw_w = hip.DeviceBuffer(wbytes)
    raw_s = hip.DeviceBuffer(nsc * 4)
    layers = []
    for layer in range(L):
        experts = []
        for e in range(E):
            mats = []
            for m, (o, i) in enumerate(((I, D), (I, D), (D, I))):
                s = seed * 1_000_003 + (layer * 4096 + e) * 3 + m
                raw_w.fill(wbytes, 0, seed=s * 2)
                raw_s.fill(nsc, 2, float(np.log(0.01)), 0.5, seed=s * 2 + 1)
                mats.append(hip.upload_tensor_dev(0, raw_w.ptr, raw_s.ptr, fmt, i, o, 32))
            experts.append(hip.GpuExpert(mats[0], mats[1], mats[2], D, I))
        layers.append((hip.ExpertSet(experts), experts))
    raw_w.free()
    raw_s.free()
    hip.pipe_sync(0)
    return layers


def pcie_inclusive(hip, cfg, experts, x_step, ids, w, ga, seconds=0.5):
    """The reference's host-buffer entry point (coli_hip_expert_group_reduce,
    lib.rs:620) on one step's routing: x rows and the layer output cross
    PCIe on every call, which blocks. Timed eagerly and with the automatic
    graph cache (COLI_HIP_GRAPH=1). Reported beside the device-resident rate,
    never as the benchmark value."""
    S, D, k = cfg["S"], cfg["D"], cfg["k"]
    ids = ids.reshape(S, k)
    w = w.reshape(S, k)
    order, rows, xr, dst, rw = [], [], [], [], []
    for e in dict.fromkeys(ids.reshape(-1).tolist()):   # batch-union order
        for t in range(S):
            for j in range(k):
                if ids[t, j] == e:
                    xr.append(x_step[t])
                    dst.append(t)
                    rw.append(w[t, j])
        order.append(e)
        rows.append(int(np.sum(ids == e)))
    xr = np.stack(xr).astype(np.float32)
    rw = np.array(rw, np.float32)
    layout = hip.ReduceLayout.build(np.array(dst), S)
    sel = [experts[e] for e in order]
    hip.set_act_group(ga)
    out = {}
    # The call as a native caller makes it: every argument built once, then
    # the C entry point called in a loop through ctypes (a few microseconds of
    # call overhead; no per-call NumPy conversion or checks).
    import ctypes
    from peregrine_amd._lib import lib
    ref = hip.expert_group_reduce(sel, rows, xr, D, layout, rw, S)
    res = np.zeros((S, D), np.float32)
    rws, rp, ri = (np.ascontiguousarray(a, np.int32) for a in (rows, layout.row_ptr, layout.row_idx))
    g, u, d = hip._handles(sel)
    ip = ctypes.POINTER(ctypes.c_int)
    args = (g, u, d, rws.ctypes.data_as(ip), len(sel), rp.ctypes.data_as(ip), ri.ctypes.data_as(ip),
            ctypes.c_void_p(rw.ctypes.data), S, ctypes.c_void_p(res.ctypes.data), ctypes.c_void_p(xr.ctypes.data))
    call = lib.coli_hip_expert_group_reduce
    for mode in ("eager", "graph_cache"):
        os.environ["COLI_HIP_GRAPH"] = "1" if mode == "graph_cache" else "0"
        st0 = hip.graph_cache_stats()
        try:
            for _ in range(3):
                assert call(*args) == 1
            n, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < seconds:
                for _ in range(50):
                    call(*args)
                n += 50
            dt = (time.perf_counter() - t0) / n
            same = bool(np.array_equal(res, ref))
        finally:
            os.environ.pop("COLI_HIP_GRAPH", None)
        out[mode] = {"tokens_per_s": round(S / dt, 1), "ms_per_call": round(dt * 1e3, 4), "calls": n,
                     "equals_python_mirror_call": same}
        if mode == "graph_cache":   # the cache keeps replaying only where replay probed faster than eager
            st1 = hip.graph_cache_stats()
            out[mode]["replayed_calls"] = st1.replays - st0.replays
            out[mode]["eager_calls"] = st1.uncacheable - st0.uncacheable
    out["entry_point"] = ("coli_hip_expert_group_reduce (host x in, host out; blocking), called through ctypes "
                          "with prebuilt arguments")
    return out


def make_logits(cfg, n_steps, seed):
    from peregrine_amd import synth
    rng = np.random.default_rng(seed)
    S, E = cfg["S"], cfg["E"]
    out = np.empty((n_steps, S, E), np.float32)
    for i in range(n_steps):
        if cfg["route"] == "zipf":
            out[i] = synth.zipf_logits(rng, S, E)
        else:
            out[i] = synth.normal_logits(rng, S, E)
    return out


def cpu_info():
    model = platform.processor() or "unknown"
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return model, os.cpu_count() or 1


def cpu_threads():
    """All cores this process may use: the affinity set, capped by the
    OMP_NUM_THREADS-style share the GPU box gives one GPU."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(n, 1)


def cpu_baseline(cfg, wfmt, ga, seconds):
    """The oracle's AVX2 restatement of the reference CPU path (dot_i4i8_avx2,
    idot.rs:214-239; the expert is Mlp::swiglu, mlp.rs:21-26, the combine the
    moe_forward scatter, mlp.rs:111-119) over a bounded sample of the
    workload's tokens, single-threaded and on all cores (threads over the
    routed experts, as par_map in mlp.rs:96-104). The sample's expert slots
    alias 16 distinct host experts of the configuration's shape (host memory
    and set-up time); each expert is still streamed from DRAM per use."""
    from oracle import oracle as orc
    from peregrine_amd import qt, synth
    D, I, E, k = cfg["D"], cfg["I"], cfg["E"], cfg["k"]
    rng = np.random.default_rng(99)
    fmt = qt.FMT_I4G if wfmt == "int4" else qt.FMT_I8G
    n_dist = min(E, 16)
    dist = []
    for _ in range(n_dist):
        trip = synth.make_expert(rng, D, I, fmt, 32)
        shp = ((I, D), (I, D), (D, I))
        dist.append(tuple(orc.Tensor(t[0], t[1], fmt, i, o, 32) for t, (o, i) in zip(trip, shp)))
    experts = [dist[e % n_dist] for e in range(E)]
    S = min(cfg["S"], 16)
    model, nproc = cpu_info()
    res = {}
    for label, threads in (("single", 1), ("all", cpu_threads())):
        n, t0 = 0, time.perf_counter()
        while True:
            x = rng.standard_normal((S, D)).astype(np.float32)
            logits = synth.zipf_logits(rng, S, E) if cfg["route"] == "zipf" else synth.normal_logits(rng, S, E)
            idx, w = orc.route_softmax_topk(logits, k)
            orc.moe_forward(x, idx, w, experts, ga, nthreads=threads, simd=orc.have_avx2())
            n += S
            el = time.perf_counter() - t0
            if el >= seconds:
                break
        res[label] = (n / el, threads, n)
    return dict(value=round(res["all"][0], 3), unit="tokens/s", cores=res["all"][1], kind="port",
                single_thread_value=round(res["single"][0], 3), nproc=nproc, cpu_model=model,
                sample=f"{res['single'][2]} tokens single-threaded and {res['all'][2]} on {res['all'][1]} threads, "
                       f"in batches of {S} tokens of {cfg['name']} (top-{k} of {E} expert slots aliasing "
                       f"{n_dist} distinct experts, D={D}, I={I}, {wfmt} gs=32, act group {ga}); AVX2 "
                       f"restatement of dot_i4i8_avx2, threads over routed experts")


METRIC = "MoE-layer tokens/s + HBM GB/s % peak (decode) / int8 MFMA % peak (prefill)"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_pmc.md")


def calibrate_copy():
    """A copy kernel of known size for scaling the PMC byte counters."""
    import torch
    n = 256 << 20
    a = torch.ones(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(5):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"calibration": "copy", "bytes_read": n, "bytes_written": n, "launches": 5}))


def measured_traffic(workload):
    """HBM bytes per launch of the dominant (gate/up) kernel, from the committed
    rocprofv3 --pmc summary (FETCH_SIZE and WRITE_SIZE per dispatch, scaled by
    the copy-kernel calibration); None when that workload was not profiled."""
    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    col = None
    for ln in lines:
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if "traffic B" in cells:   # the table's header names the column
            col = cells.index("traffic B")
            continue
        if col is None or len(cells) <= col or cells[0] != workload or "<" not in cells[1]:
            continue
        targs = [t.strip() for t in cells[1].split("<", 1)[1].rstrip(">").split(",")]
        if len(targs) >= 3 and targs[2] == "true":   # the gate/up instantiation
            try:
                return int(float(cells[col]))
            except ValueError:
                return None
    return None


def run_workload(hip, cfg, wfmt, ga, arm, steps, warmup, use_graph=True, layers=None, pcie=False):
    """Times `steps` steps of one workload (after `warmup` eager ones), then
    a profiled pass over the same steps for per-kernel durations. Returns
    (summary dict, layers) so a later workload of the same shape can reuse
    the resident experts."""
    S, D, E, k, L = cfg["S"], cfg["D"], cfg["E"], cfg["k"], cfg["layers"]
    t_build = time.perf_counter()
    if layers is None:
        layers = build_experts(hip, cfg, wfmt, seed=cfg.get("seed", 1))
    n_all = warmup + steps
    bx = hip.DeviceBuffer(n_all * S * D * 4)
    bx.fill(n_all * S * D, 1, 0.0, 1.0, seed=7)
    # router logits per step and layer: every layer is routed from its own
    logits = make_logits(cfg, n_all * L, seed=11)
    if cfg["route"] == "one":
        logits[:] = 0.0
    bl = hip.DeviceBuffer.from_array(logits)
    n_sel = n_all * L * S * k
    bids = hip.DeviceBuffer(n_sel * 4)
    bw = hip.DeviceBuffer(n_sel * 4)
    bh = [hip.DeviceBuffer(S * D * 4) for _ in range(2)]
    hip.pipe_sync(0)
    t_build = time.perf_counter() - t_build

    def step(i):
        cur = bx.ptr + i * S * D * 4
        for layer in range(L):
            j = i * L + layer
            ip, wp = bids.ptr + j * S * k * 4, bw.ptr + j * S * k * 4
            out = bh[layer & 1].ptr
            # device router (softmax top-k) fused with the layer's activation quantisation
            hip.moe_forward_logits_dev(layers[layer][0], cur, S, bl.ptr + j * S * E * 4, k, ip, wp, out, ga, arm)
            cur = out

    # eager warm-up passes reserve all scratch (a graph must not allocate)
    for i in range(warmup):
        step(i)
    hip.pipe_sync(0)
    graph = None
    if use_graph:
        graph = hip.capture(0, lambda: [step(warmup + i) for i in range(steps)])
        graph.launch()   # warm the graph once (same steps as the timed replay)

    hip.pipe_sync(0)
    hip.event_record(0, 0)
    t0 = time.perf_counter()
    if use_graph:
        graph.launch()
    else:
        for i in range(steps):
            step(warmup + i)
    hip.event_record(0, 1)
    hip.pipe_sync(0)
    wall = time.perf_counter() - t0
    gpu_ms = hip.event_elapsed(0, 0, 1)
    ms_per_step = wall * 1e3 / steps
    del graph

    # distinct experts each layer of a step touches (for algorithmic bytes)
    ids_all = bids.download(np.int32, (n_all * L, S * k))
    ids = ids_all[warmup * L:]
    distinct = float(np.mean([len(np.unique(r)) for r in ids]))

    # profiled pass: per-kernel execution times from the dispatch packets
    hip.reset_stats()
    hip.set_profile(True)
    for i in range(steps):
        step(warmup + i)
    hip.pipe_sync(0)
    hip.set_profile(False)
    ks = hip.kernel_stats()

    gu_bytes, layer_bytes, gu_ops, layer_ops = algorithmic(cfg, wfmt, distinct)
    n_gu, ms_gu = ks["gateup"]
    gu_ms = ms_gu / max(n_gu, 1)
    n_dn, ms_dn = ks["down"]
    dn_ms = ms_dn / max(n_dn, 1)
    layer_ms = ms_per_step / L
    prefill = cfg["S"] >= 1024
    if prefill:
        achieved = gu_ops / (gu_ms * 1e-3) / 1e12
        roof = dict(bound="mfma", achieved=round(achieved, 2), peak=INT8_PEAK_TOPS, unit="TFLOP/s",
                    frac=round(achieved / INT8_PEAK_TOPS, 4))
        layer_frac = layer_ops / (layer_ms * 1e-3) / 1e12 / INT8_PEAK_TOPS
    else:
        achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
        roof = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4))
        layer_frac = layer_bytes / (layer_ms * 1e-3) / 1e9 / HBM_PEAK_GBS
    wl_name = cfg["name"] + ("_int8" if wfmt == "int8" else "")
    roof["traffic"] = measured_traffic(wl_name)
    roof["kernel"] = "gate/up (fused SwiGLU + h quant)"
    roof["kernel_avg_us"] = round(gu_ms * 1e3, 2)
    roof["layer_frac"] = round(layer_frac, 4)
    summary = {
        "workload": wl_name,
        "value": round(S * L * steps / wall, 2),
        "unit": "tokens/s",
        "value_unit": "MoE-layer tokens/s (tokens x layers per second)",
        "stack_tokens_per_s": round(S * steps / wall, 2),
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "gpu_event_ms_per_step": round(gpu_ms / steps, 4),
        "roofline": roof,
        "layer_GBps": round(layer_bytes / (layer_ms * 1e-3) / 1e9, 1),
        "layer_TOPS": round(layer_ops / (layer_ms * 1e-3) / 1e12, 2),
        "distinct_experts_per_step": distinct,
        "kernel_avg_us": {name: round(ms / max(n, 1) * 1e3, 2) for name, (n, ms) in ks.items() if n},
        "gateup_GBps": round(gu_bytes / (gu_ms * 1e-3) / 1e9, 1),
        "down_GBps": round((layer_bytes - gu_bytes) / (dn_ms * 1e-3) / 1e9, 1) if n_dn else None,
        "gateup_TOPS": round(gu_ops / (gu_ms * 1e-3) / 1e12, 2),
        "down_TOPS": round((layer_ops - gu_ops) / (dn_ms * 1e-3) / 1e12, 2) if n_dn else None,
        "setup_s": round(t_build, 1),
    }
    if pcie and S <= 64 and L == 1:
        x0 = bx.download(np.float32, ((warmup + 1) * S, D))[warmup * S:]
        summary["pcie_inclusive"] = pcie_inclusive(hip, cfg, layers[0][1], x0, ids[0],
                                                   bw.download(np.float32, (n_all * L, S * k))[warmup * L], ga)
    for b in (bx, bl, bids, bw, *bh):
        b.free()
    return summary, layers


def main():
    args = parse()
    if args.calibrate_copy:
        calibrate_copy()
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; --gpus must be 1 "
                                   "(no collectives or sharding in scope)"}))
        sys.exit(2)
    cfg = dict(CONFIGS[args.config])
    if args.experts:
        cfg["E"] = args.experts
        cfg["name"] += f"_E{args.experts}"
    cfg["seed"] = args.config
    steps = args.steps if args.steps is not None else DEFAULT_STEPS[args.config]
    warmup = args.warmup if args.warmup is not None else max(2, steps // 10)
    from peregrine_amd import hip

    assert hip.init([0]) == 1, "coli_hip_init failed"
    arm = {"auto": -1, "gemv": hip.ARM_GEMV, "mfma": hip.ARM_MFMA}[args.arm]
    ga = args.act_group
    # The decode (HBM) and prefill (MFMA) halves of the metric first, on the
    # 160-expert layer (config 4 reuses config 2's resident experts), then
    # the headline configuration.
    wl = {}
    if not args.no_detail:
        # every BASELINE configuration gets a driver-timed line with its own
        # roofline: configs 1-4 int4, then config 5 with the other weight
        # format than the headline's (configs 2-4 share one resident layer)
        shared = None
        for cid, wf in ((1, "int4"), (2, "int4"), (3, "int4"), (4, "int4"),
                        (5, "int8" if args.wfmt == "int4" else "int4")):
            if (cid, wf) == (args.config, args.wfmt):
                continue
            c2 = dict(CONFIGS[cid])
            c2["seed"] = cid if cid in (1, 5) else 2
            st = DEFAULT_STEPS[cid]
            s, lay = run_workload(hip, c2, wf, ga, -1, st, max(2, st // 10),
                                  layers=shared if cid in (2, 3, 4) else None, pcie=not args.no_pcie)
            if cid in (2, 3, 4):
                shared = lay
            del lay
            wl[s["workload"]] = s
            print(f"[bench] {s['workload']}: {s['value']} tokens/s, {s['ms_per_step']} ms/step, "
                  f"roofline frac {s['roofline']['frac']}", file=sys.stderr, flush=True)
        del shared
    head, layers = run_workload(hip, cfg, args.wfmt, ga, arm, steps, warmup, use_graph=not args.no_graph,
                                pcie=not args.no_pcie)
    del layers
    line = {
        "metric": METRIC,
        "value": head["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": head["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint4" if args.wfmt == "int4" else "int8xint8",
        "data": "synthetic (seeded, device-generated weights; random-init experts)",
        "config": {
            "workload": head["workload"], "experts": cfg["E"], "hidden": cfg["D"], "moe_intermediate": cfg["I"],
            "tokens": cfg["S"], "top_k": cfg["k"], "layers": cfg["layers"],
            "weights": f"{args.wfmt} QT, f32 scale per 32", "act_group": ga, "arm": args.arm,
            "graph": not args.no_graph, "parallelism": "none (1 GPU)",
            "routing": "device softmax top-k per layer, from that layer's own router logits",
            "value_unit": "MoE-layer tokens/s = tokens x layers per second",
            "stack_tokens_per_s": head["stack_tokens_per_s"],
        },
        "roofline": head["roofline"],
        "detail": {k: v for k, v in head.items() if k not in ("value", "unit", "steps", "warmup", "ms_per_step",
                                                             "roofline", "workload")},
    }
    if wl:
        line["detail"]["workloads"] = wl
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.wfmt, ga, args.cpu_seconds)
        if args.config != 2 and not args.no_detail:   # BASELINE's plan: also the decode layer (config 2)
            c2 = dict(CONFIGS[2])
            line["detail"]["cpu_baseline_cfg2"] = cpu_baseline(c2, "int4", ga, args.cpu_seconds / 2)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
