"""Benchmark of the MI355X MoE expert lane on BASELINE.json's configurations.

A step is one routed MoE layer over one batch of synthetic tokens: device
router (softmax top-k) -> expert-offset table -> int8 activation quant ->
fused gate/up + SwiGLU (+ h quant) -> down -> weighted combine. Inputs
(tokens, router logits, 160+ resident experts) are in HBM before timing
starts; every step uses its own tokens and router logits, so the experts a
step reads change from step to step.

    python bench.py                      # config 2 (decode, batch 1), 1 GPU
    python bench.py --config 4           # prefill, 2048 tokens
    python bench.py --config 5 --wfmt int8

Prints one JSON line (the driver's contract). Per-kernel durations come from
HIP events recorded on the library's device stream in a second, profiled
pass over the same steps.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, published
INT8_PEAK_TOPS = 5000.0        # MI355X dense int8 MFMA, published (no sparsity)

# BASELINE.json configs, numbered 1..5 as in BASELINE.md
CONFIGS = {
    1: dict(name="cfg1_single_expert_1tok", E=1, D=5120, I=1536, S=1, k=1, route="one", layers=1),
    2: dict(name="cfg2_decode_moe_layer_b1_160x_int4", E=160, D=5120, I=1536, S=1, k=8, route="normal", layers=1),
    3: dict(name="cfg3_batched_decode_64tok_zipf", E=160, D=5120, I=1536, S=64, k=8, route="zipf", layers=1),
    4: dict(name="cfg4_prefill_2048tok_zipf", E=160, D=5120, I=1536, S=2048, k=8, route="zipf", layers=1),
    5: dict(name="cfg5_large_layer_512tok_256x", E=256, D=6144, I=2048, S=512, k=8, route="normal", layers=4),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--config", type=int, default=2, choices=sorted(CONFIGS))
    ap.add_argument("--wfmt", choices=("int4", "int8"), default="int4")
    ap.add_argument("--act-group", type=int, default=32, choices=(0, 32),
                    help="activation scale per 32-block (BASELINE, default) or per row (reference)")
    ap.add_argument("--arm", choices=("auto", "gemv", "mfma"), default="auto")
    ap.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-pcie", action="store_true",
                    help="skip the host-buffer (PCIe-inclusive) timing, e.g. under a profiler")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
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


def pcie_inclusive(hip, cfg, experts, bx, step_ids, step_w, step, ga, seconds=0.5):
    """The reference's host-buffer entry point (coli_hip_expert_group_reduce,
    lib.rs:620) on one step's routing: x rows and the layer output cross
    PCIe on every call, which blocks. Reported beside the device-resident
    rate, never as the benchmark value."""
    S, D, k = cfg["S"], cfg["D"], cfg["k"]
    x = bx.download(np.float32, ((step + 1) * S, D))[step * S:]
    ids = step_ids.reshape(S, k)
    w = step_w.reshape(S, k)
    order, rows, xr, dst, rw = [], [], [], [], []
    for e in dict.fromkeys(ids.reshape(-1).tolist()):   # batch-union order
        toks = [t for t in range(S) for j in range(k) if ids[t, j] == e]
        slots = [j for t in range(S) for j in range(k) if ids[t, j] == e]
        order.append(e)
        rows.append(len(toks))
        for t, j in zip(toks, slots):
            xr.append(x[t])
            dst.append(t)
            rw.append(w[t, j])
    xr = np.stack(xr).astype(np.float32)
    layout = hip.ReduceLayout.build(np.array(dst), S)
    sel = [experts[e] for e in order]
    hip.set_act_group(ga)
    for _ in range(3):
        hip.expert_group_reduce(sel, rows, xr, D, layout, np.array(rw, np.float32), S)
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        hip.expert_group_reduce(sel, rows, xr, D, layout, np.array(rw, np.float32), S)
        n += 1
    dt = (time.perf_counter() - t0) / n
    return {"tokens_per_s": round(S / dt, 1), "ms_per_call": round(dt * 1e3, 4), "calls": n,
            "entry_point": "coli_hip_expert_group_reduce (host x in, host out; blocking)"}


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


def cpu_baseline(cfg, wfmt, ga, seconds):
    """The oracle's AVX2 restatement of the reference CPU path (dot_i4i8_avx2,
    idot.rs:214-239) over one layer: tokens one at a time, experts in parallel
    over threads (par_map, mlp.rs:96-104). Timed on this host for a bounded
    sample of tokens."""
    from oracle import oracle as orc
    from peregrine_amd import qt, synth
    D, I = cfg["D"], cfg["I"]
    E = min(cfg["E"], 16)
    k = min(cfg["k"], E)
    rng = np.random.default_rng(99)
    fmt = qt.FMT_I4G if wfmt == "int4" else qt.FMT_I8G
    experts = []
    for _ in range(E):
        trip = synth.make_expert(rng, D, I, fmt, 32)
        shp = ((I, D), (I, D), (D, I))
        experts.append(tuple(orc.Tensor(t[0], t[1], fmt, i, o, 32) for t, (o, i) in zip(trip, shp)))
    threads = min(os.cpu_count() or 1, 16, max(k, 1))
    n, t0 = 0, time.perf_counter()
    while True:
        x = rng.standard_normal((1, D)).astype(np.float32)
        idx, w = orc.route_softmax_topk(synth.normal_logits(rng, 1, E), k)
        orc.moe_forward(x, idx, w, experts, ga, nthreads=threads, simd=orc.have_avx2())
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds or n >= 2000:
            break
    return dict(value=round(n / el, 3), unit="tokens/s", cores=threads, kind="port",
                sample=f"{n} single-token MoE-layer forwards (top-{k} of {E} experts, D={D}, I={I}, "
                       f"{wfmt} gs=32, act group {ga}), AVX2 int4 dot, {threads} threads over experts")


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
    for ln in lines:
        cells = [c.strip() for c in ln.strip().strip("|").split("|")]
        if len(cells) < 3 or cells[0] != workload or "<" not in cells[1]:
            continue
        targs = [t.strip() for t in cells[1].split("<", 1)[1].rstrip(">").split(",")]
        if len(targs) >= 3 and targs[2] == "true":   # the gate/up instantiation
            try:
                return int(float(cells[-1]))
            except ValueError:
                return None
    return None


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
    if args.wfmt == "int8":
        cfg["name"] += "_int8"
    steps = args.steps if args.steps is not None else {1: 200, 2: 200, 3: 100, 4: 20, 5: 10}[args.config]
    warmup = args.warmup if args.warmup is not None else max(2, steps // 10)
    from peregrine_amd import hip

    assert hip.init([0]) == 1, "coli_hip_init failed"
    S, D, E, k, L = cfg["S"], cfg["D"], cfg["E"], cfg["k"], cfg["layers"]
    arm = {"auto": -1, "gemv": hip.ARM_GEMV, "mfma": hip.ARM_MFMA}[args.arm]
    ga = args.act_group
    t_build = time.perf_counter()
    layers = build_experts(hip, cfg, args.wfmt, seed=args.config)
    n_all = warmup + steps
    # inputs for every step resident in HBM
    bx = hip.DeviceBuffer(n_all * S * D * 4)
    bx.fill(n_all * S * D, 1, 0.0, 1.0, seed=7)
    logits = make_logits(cfg, n_all, seed=11)
    if cfg["route"] == "one":
        logits[:] = 0.0
    bl = hip.DeviceBuffer.from_array(logits)
    bids = hip.DeviceBuffer(n_all * S * k * 4)
    bw = hip.DeviceBuffer(n_all * S * k * 4)
    bh = [hip.DeviceBuffer(S * D * 4) for _ in range(2)]
    hip.pipe_sync(0)
    t_build = time.perf_counter() - t_build

    def step(i):
        xp = bx.ptr + i * S * D * 4
        ip, wp = bids.ptr + i * S * k * 4, bw.ptr + i * S * k * 4
        cur = xp
        for layer in range(L):
            out = bh[layer & 1].ptr
            if layer == 0:   # router fused with the first layer's activation quantisation
                hip.moe_forward_logits_dev(layers[0][0], cur, S, bl.ptr + i * S * E * 4, k, ip, wp, out, ga, arm)
            else:            # later resident layers reuse the step's routing
                hip.moe_forward_dev(layers[layer][0], cur, S, ip, wp, k, out, ga, arm)
            cur = out

    # one eager pass reserves all scratch (a graph must not allocate)
    for i in range(warmup):
        step(i)
    hip.pipe_sync(0)

    use_graph = not args.no_graph
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

    # distinct experts each step touches (for algorithmic bytes)
    ids = bids.download(np.int32, (n_all, S * k))[warmup:]
    distinct = float(np.mean([len(np.unique(r)) for r in ids]))

    # profiled pass: per-kernel durations from HIP events on the device stream
    hip.reset_stats()
    hip.set_profile(True)
    for i in range(steps):
        step(warmup + i)
    hip.pipe_sync(0)
    hip.set_profile(False)
    ks = hip.kernel_stats()

    # The profiled pass brackets every kernel with events on the device
    # stream, so each duration also holds one event's own processing. That
    # cost is measured here, in the same run: pairs of events with nothing
    # between them, queued behind a long fill so they run back to back as the
    # profiled kernels do (no waiting on the host in between).
    backlog = hip.DeviceBuffer(256 << 20)
    over = []
    for _ in range(4):
        backlog.fill(256 << 20, 0, 0.0, 0.0, 3)
        for p in range(7):
            hip.event_record(0, 2 + 2 * p)
            hip.event_record(0, 3 + 2 * p)
        over += [hip.event_elapsed(0, 2 + 2 * p, 3 + 2 * p) for p in range(7)]
    ev_over_ms = float(np.median(over))
    del backlog

    gu_bytes, layer_bytes, gu_ops, layer_ops = algorithmic(cfg, args.wfmt, distinct)
    n_gu, ms_gu = ks["gateup"]
    gu_raw_ms = ms_gu / max(n_gu, 1)
    gu_ms = max(gu_raw_ms - ev_over_ms, 1e-6)
    n_dn, ms_dn = ks["down"]
    dn_ms = max(ms_dn / max(n_dn, 1) - ev_over_ms, 1e-6)
    prefill = args.config == 4
    if prefill:
        achieved = gu_ops / (gu_ms * 1e-3) / 1e12
        roof = dict(bound="mfma", achieved=round(achieved, 2), peak=INT8_PEAK_TOPS, unit="TFLOP/s",
                    frac=round(achieved / INT8_PEAK_TOPS, 4), traffic=measured_traffic(cfg["name"]))
    else:
        achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
        roof = dict(bound="hbm", achieved=round(achieved, 1), peak=HBM_PEAK_GBS, unit="GB/s",
                    frac=round(achieved / HBM_PEAK_GBS, 4), traffic=measured_traffic(cfg["name"]))
    value = S * L * steps / wall
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xint4" if args.wfmt == "int4" else "int8xint8",
        "data": "synthetic (seeded, device-generated weights; random-init experts)",
        "config": {
            "workload": cfg["name"], "experts": E, "hidden": D, "moe_intermediate": cfg["I"], "tokens": S,
            "top_k": k, "layers": L, "weights": f"{args.wfmt} QT, f32 scale per 32", "act_group": ga,
            "arm": args.arm, "graph": use_graph, "parallelism": "none (1 GPU)",
        },
        "roofline": roof,
        "detail": {
            "gpu_event_ms_per_step": round(gpu_ms / steps, 4),
            "layer_GBps": round(layer_bytes * L / (ms_per_step * 1e-3) / 1e9, 1),
            "layer_TOPS": round(layer_ops * L / (ms_per_step * 1e-3) / 1e12, 2),
            "distinct_experts_per_step": distinct,
            "kernel_avg_us": {name: round((ms / max(n, 1) - ev_over_ms) * 1e3, 2) for name, (n, ms) in ks.items() if n},
            "event_bracket_overhead_us": round(ev_over_ms * 1e3, 2),
            "gateup_event_us_raw": round(gu_raw_ms * 1e3, 2),
            "gateup_GBps": round(gu_bytes / (gu_ms * 1e-3) / 1e9, 1),
            "down_GBps": round((layer_bytes - gu_bytes) / (dn_ms * 1e-3) / 1e9, 1) if n_dn else None,
            "gateup_TOPS": round(gu_ops / (gu_ms * 1e-3) / 1e12, 2),
            "down_TOPS": round((layer_ops - gu_ops) / (dn_ms * 1e-3) / 1e12, 2) if n_dn else None,
            "setup_s": round(t_build, 1),
        },
    }
    if S <= 64 and L == 1 and not args.no_pcie:
        line["detail"]["pcie_inclusive"] = pcie_inclusive(hip, cfg, layers[0][1], bx, ids[0],
                                                          bw.download(np.float32, (n_all, S * k))[warmup], warmup, ga)
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(cfg, args.wfmt, ga, args.cpu_seconds)
    else:
        line["cpu_baseline"] = None
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
