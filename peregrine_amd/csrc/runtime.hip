// runtime.hip — the C ABI of libperegrine_hip.so: device contexts, resident
// tensors, per-device scratch, the expert-group dispatch and the
// device-resident MoE layer. Replaces cuda/backend_cuda.cu's host side
// (contexts :484-592, tensors :747-810, expert_group_impl :1035-1243).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <atomic>
#include <chrono>
#include <mutex>
#include <vector>

#include "../../include/peregrine_hip.h"
#include "common.h"

using namespace phip;

// Scratch of coli_hip_moe_forward_dev_noalloc: a fixed array in every
// device's code object, mapped at init (hipGetSymbolAddress per device).
// Host code uses only the per-device address kept in Ctx::fixed_scratch,
// never this name.
static __device__ __align__(256) uint8_t scratch[COLI_HIP_FIXED_SCRATCH_BYTES];
// Per-tile arrival counters of the down GEMV's tail combine: zero at load,
// and each dispatch leaves them zero again (the tile's last workgroup resets
// its counter), so no clearing launch is needed. One stream per device uses
// them; host code uses the address kept in Ctx::tail_ctr.
static __device__ int tail_ctr[GEMV_TAIL_TILES];
// Per-unit arrival counters of the split-K GEMV, kept zero between
// dispatches the same way (the unit's finishing workgroup resets its own).
static __device__ int split_ctr[GEMV_SPLIT_UNITS];

namespace {
struct Slab;
}

struct ColiHipTensor {
    int fmt, I, O, gs, device;
    MatGeom g;
    uint8_t *w;            // tiled weights; the scales follow in the same arena block
    float *sc;
    size_t w_bytes, sc_bytes;
    Slab *slab;            // arena slab holding w and sc
    size_t blk_off, blk_bytes;
};

struct ColiHipGraph {
    hipGraph_t graph;
    hipGraphExec_t exec;
    int device;
    unsigned gen;   // the device's scratch generation at capture: the graph holds those buffers' addresses
};

struct ColiHipExpertSet {
    int device, count;
    MatGeom gg, gd;          // gate/up geometry, down geometry
    ExpertDesc *desc_dev;    // [count]
};

namespace {

struct Buf {
    void *p = nullptr;
    size_t cap = 0;
    void *d = nullptr;   // pinned buffers: the device's address of the mapped host memory
};

constexpr int GRAPH_CACHE = 16;   // cached expert-group graphs per device
constexpr int N_EVENTS = 2 * (COLI_HIP_K_COUNT + 4);   // (start, stop) per kernel slot of a dispatch

// One launch shape of the expert-group graph cache: its key, its graph and
// the scratch generation it was captured under, its last use (least recently
// used is evicted), and whether replaying it pays. A new shape is captured,
// then its next calls alternate replay and eager launch (GRAPH_PROBES of
// each, timed on the host clock around enqueue and synchronise); the faster
// one is kept. A shape where eager wins keeps no graph and runs eagerly.
enum SlotState { SLOT_PROBE = 0, SLOT_GRAPH = 1, SLOT_EAGER = 2 };
constexpr int GRAPH_PROBES = 3;
struct GraphSlot {
    bool live = false;
    uint64_t key = 0;
    ColiHipGraph *g = nullptr;
    unsigned gen = 0;
    uint64_t used = 0;
    int state = SLOT_PROBE;
    int n_graph = 0, n_eager = 0;
    double t_graph = 0, t_eager = 0;   // fastest probe of each, seconds
};

struct Ctx {
    int device = -1;
    hipStream_t stream = nullptr;
    size_t tensor_count = 0, tensor_bytes = 0;
    unsigned gen = 0;   // bumped on every scratch reallocation
    Buf xq, sx, h, hq, sh, y, meta, tbl, rdesc, part_d, part_f;
    Buf pin_x, pin_y, pin_meta;
    hipEvent_t ev[N_EVENTS] = {};
    hipEvent_t phase_ev[4] = {};   // expert_group phases under profiling: H2D | kernels | D2H
    hipEvent_t user_ev[16] = {};
    // Host-visible word a GEMV sets when one of its bounded waits gives up
    // (mapped pinned memory: the host reads it after a stream synchronise).
    int *wait_flag = nullptr, *wait_flag_dev = nullptr;
    GraphSlot graphs[GRAPH_CACHE];
    uint64_t graph_clock = 0;
    // device address of this device's copy of the fixed scratch array (the
    // no-allocation entry point), looked up at init with the device current
    uint8_t *fixed_scratch = nullptr;
    int *tail_ctr = nullptr;   // this device's copy of tail_ctr[]
    int *split_ctr = nullptr;  // this device's copy of split_ctr[]
    // last device-resident table (for coli_hip_last_table)
    TableOut tbl_view{};
    int tbl_E = 0, tbl_R = 0;
};

Ctx g_ctx[COLI_HIP_MAX_DEVICES];
int g_nctx = 0;
std::mutex g_stats_mu;
uint64_t g_calls = 0, g_experts = 0, g_rows = 0;
double g_h2d_ms = 0, g_d2h_ms = 0;   // expert_group phases, under profiling
uint64_t g_k_launches[COLI_HIP_K_COUNT] = {};
double g_k_ms[COLI_HIP_K_COUNT] = {};
uint64_t g_graph_captures = 0, g_graph_replays = 0, g_graph_invalidations = 0, g_graph_uncacheable = 0;
int g_act_group = -1;   // -1: read COLI_HIP_ACT_GROUP on first use
int g_arm = -2;         // -2: read COLI_HIP_ARM on first use
int g_profile = -1;
int g_spin_limit = GEMV_SPIN_LIMIT;
int32_t *g_dbg_gu = nullptr, *g_dbg_dn = nullptr;
thread_local int g_cur_dev = -1;
}  // namespace
thread_local phip::LaunchTiming phip::g_launch_timing;
namespace {

int hip_ok(hipError_t e, const char *what) {
    if (e == hipSuccess) return 1;
    std::fprintf(stderr, "[HIP] %s: %s\n", what, hipGetErrorString(e));
    return 0;
}

int fail(const char *what) {
    std::fprintf(stderr, "[HIP] %s\n", what);
    return 0;
}

// ---------------------------------------------------------------------------
// Resident-tensor arena. Expert tensors are sub-allocated from large slabs
// (512 MB, or one slab per larger tensor) instead of one small hipMalloc per
// weight and scale buffer: a streaming kernel then reads a few large mappings
// rather than hundreds of small ones, and a tensor's weights and scales sit in
// one block. First fit over each slab's free ranges, coalesced on release; a
// slab returns to the device when its last block is released.
// ---------------------------------------------------------------------------
size_t round_up(size_t v, size_t m) { return (v + m - 1) / m * m; }

struct Slab {
    int device;
    uint8_t *base;
    size_t size, used;
    std::map<size_t, size_t> free_ranges;   // offset -> length
};

constexpr size_t SLAB_BYTES = (size_t)512 << 20;
constexpr size_t ARENA_ALIGN = 4096;
std::mutex g_arena_mu;
std::vector<Slab *> g_slabs;

bool slab_take(Slab *s, size_t bytes, size_t *off) {
    for (auto it = s->free_ranges.begin(); it != s->free_ranges.end(); ++it) {
        if (it->second < bytes) continue;
        *off = it->first;
        const size_t rest = it->second - bytes;
        s->free_ranges.erase(it);
        if (rest) s->free_ranges[*off + bytes] = rest;
        s->used += bytes;
        return true;
    }
    return false;
}

// Caller has selected the device.
Slab *arena_alloc(int device, size_t bytes, size_t *off) {
    bytes = round_up(bytes, ARENA_ALIGN);
    std::lock_guard<std::mutex> lock(g_arena_mu);
    for (Slab *s : g_slabs)
        if (s->device == device && slab_take(s, bytes, off)) return s;
    Slab *s = new Slab{device, nullptr, std::max(SLAB_BYTES, round_up(bytes, (size_t)2 << 20)), 0, {}};
    if (!hip_ok(hipMalloc(&s->base, s->size), "tensor arena slab")) {
        delete s;
        return nullptr;
    }
    s->free_ranges[0] = s->size;
    g_slabs.push_back(s);
    slab_take(s, bytes, off);
    return s;
}

void arena_release(Slab *s, size_t off, size_t bytes) {
    bytes = round_up(bytes, ARENA_ALIGN);
    std::lock_guard<std::mutex> lock(g_arena_mu);
    auto it = s->free_ranges.emplace(off, bytes).first;
    if (it != s->free_ranges.begin()) {   // merge with the range before
        auto prev = std::prev(it);
        if (prev->first + prev->second == off) {
            prev->second += it->second;
            s->free_ranges.erase(it);
            it = prev;
        }
    }
    auto next = std::next(it);
    if (next != s->free_ranges.end() && it->first + it->second == next->first) {
        it->second += next->second;
        s->free_ranges.erase(next);
    }
    s->used -= bytes;
    if (s->used == 0) {
        int cur = -1;
        if (hipGetDevice(&cur) == hipSuccess && cur != s->device) (void)hipSetDevice(s->device);
        hipFree(s->base);
        if (cur >= 0 && cur != s->device) (void)hipSetDevice(cur);
        g_slabs.erase(std::find(g_slabs.begin(), g_slabs.end(), s));
        delete s;
    }
}

int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    return v && *v ? std::atoi(v) : dflt;
}

int act_group() {
    if (g_act_group < 0) g_act_group = env_int("COLI_HIP_ACT_GROUP", 0) == 32 ? 32 : 0;
    return g_act_group;
}

// Fused one-token router: -1 automatic, 0 never, 1 whenever eligible.
// COLI_HIP_FUSED_ROUTE=0 (1) in the environment sets 0 (1) at first use.
std::atomic<int> g_fused_route{-2};
int fused_route_mode() {
    int m = g_fused_route.load();
    if (m == -2) {
        const char *e = getenv("COLI_HIP_FUSED_ROUTE");
        m = e && e[0] == '0' ? 0 : (e && e[0] == '1' ? 1 : -1);
        g_fused_route.store(m);
    }
    return m;
}

// One-token down GEMV + combine in one launch: -1 automatic (k <= 2; with
// more slots every weight block in flight at once streams slower than the
// separate down GEMV's rounds: config 2, k = 8, 34.2 vs 32.5 us per layer;
// config 1, k = 1, 15.2 vs 18.2 us), 0 never, 1 whenever eligible.
// COLI_HIP_FUSED_COMBINE=0 (1) in the environment sets 0 (1) at first use.
std::atomic<int> g_fused_combine{-2};
// Automatic mode leaves a split-K down projection (with its tail combine) in
// place of the fused kernel.
bool fused_combine_on(int k, bool down_split) {
    int m = g_fused_combine.load();
    if (m == -2) {
        const char *e = getenv("COLI_HIP_FUSED_COMBINE");
        m = e && e[0] == '0' ? 0 : (e && e[0] == '1' ? 1 : -1);
        g_fused_combine.store(m);
    }
    return m == 1 || (m == -1 && k <= 2 && !down_split);
}

// Split-K decode GEMV: the number of workgroups a GEMV launch aims for
// (0: never split). COLI_HIP_GEMV_SPLIT in the environment sets it at first
// use; coli_hip_set_gemv_split overrides it. Off by default: measured on
// configs 1 and 2 the cross-workgroup hand-off (write-through pairs, the
// device-scope counter, coherent reloads) costs more than the extra CUs
// gain (config 1 gate/up 10.5 -> 11.4-14.4 us, down 5.4 -> 12.5-13.4 us;
// config 2 gate/up 19.4 -> 33 us at five splits).
constexpr int GEMV_SPLIT_DEFAULT = 0;
std::atomic<int> g_gemv_split{-2};
int gemv_split_target() {
    int m = g_gemv_split.load();
    if (m == -2) {
        m = env_int("COLI_HIP_GEMV_SPLIT", GEMV_SPLIT_DEFAULT);
        g_gemv_split.store(m);
    }
    return m < 0 ? GEMV_SPLIT_DEFAULT : m;
}

// COLI_HIP_TAIL_COMBINE=0 keeps the separate combine launch after a
// one-token down GEMV (A/B measurement); default on.
bool tail_combine_on() {
    static const bool on = !(getenv("COLI_HIP_TAIL_COMBINE") && getenv("COLI_HIP_TAIL_COMBINE")[0] == '0');
    return on;
}

int forced_arm() {
    if (g_arm == -2) {
        const char *v = std::getenv("COLI_HIP_ARM");
        g_arm = -1;
        if (v && !std::strcmp(v, "gemv")) g_arm = COLI_HIP_ARM_GEMV;
        if (v && !std::strcmp(v, "mfma")) g_arm = COLI_HIP_ARM_MFMA;
    }
    return g_arm;
}

int profiling() {
    if (g_profile < 0) g_profile = env_int("COLI_HIP_PROFILE", 0) ? 1 : 0;
    return g_profile;
}

Ctx *find_ctx(int device) {
    for (int i = 0; i < g_nctx; i++)
        if (g_ctx[i].device == device) return &g_ctx[i];
    return nullptr;
}

int select_ctx(Ctx *c) {
    if (!c) return 0;
    if (g_cur_dev == c->device) return 1;
    if (!hip_ok(hipSetDevice(c->device), "select device")) return 0;
    g_cur_dev = c->device;
    return 1;
}

// After the device's stream has synchronised: fails (0) if a GEMV bounded
// wait gave up since the last check, and clears the flag.
int check_waits(Ctx *c) {
    if (!c->wait_flag || !*(volatile int *)c->wait_flag) return 1;
    *(volatile int *)c->wait_flag = 0;
    // clear the tail combine's tile counters too (the stream is idle here),
    // so a faulty dispatch cannot leave later ones a stale count
    if (c->tail_ctr) {
        hipMemsetAsync(c->tail_ctr, 0, GEMV_TAIL_TILES * sizeof(int), c->stream);
        if (c->split_ctr) hipMemsetAsync(c->split_ctr, 0, GEMV_SPLIT_UNITS * sizeof(int), c->stream);
        hipStreamSynchronize(c->stream);
    }
    return fail("GEMV: a bounded wait between the streaming and chain waves gave up; the output of the "
                "dispatches since the last check is not valid");
}

// Grow-only device scratch. A reallocation bumps the generation so anything
// holding baked addresses (captured graphs) knows it is stale.
// Scratch must not move while a capture is recording addresses into it.
static int capturing(Ctx *c) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(c->stream, &st) == hipSuccess && st != hipStreamCaptureStatusNone;
}

int reserve(Ctx *c, Buf &b, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (b.cap >= bytes) return 1;
    if (capturing(c)) return fail("scratch would grow during graph capture: run the same call eagerly first");
    if (b.p) hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    c->gen++;
    if (!hip_ok(hipMalloc(&b.p, bytes), "scratch allocation")) return 0;
    b.cap = bytes;
    return 1;
}

int reserve_pinned(Ctx *c, Buf &b, size_t bytes) {
    if (bytes == 0) bytes = 256;
    if (b.cap >= bytes) return 1;
    if (capturing(c)) return fail("staging would grow during graph capture: run the same call eagerly first");
    if (b.p) hipHostFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    c->gen++;
    // mapped and coherent: kernels read and write it across PCIe directly
    if (!hip_ok(hipHostMalloc(&b.p, bytes, hipHostMallocMapped | hipHostMallocCoherent), "pinned staging allocation"))
        return 0;
    if (!hip_ok(hipHostGetDevicePointer(&b.d, b.p, 0), "pinned staging mapping")) {
        hipHostFree(b.p);
        b = Buf{};
        return 0;
    }
    b.cap = bytes;
    return 1;
}

void graph_destroy(ColiHipGraph *g) {
    if (!g) return;
    if (g->exec) hipGraphExecDestroy(g->exec);
    if (g->graph) hipGraphDestroy(g->graph);
    std::free(g);
}

// Drops every cached expert-group graph of a device.
void graph_cache_clear(Ctx *c) {
    for (GraphSlot &sl : c->graphs) {
        graph_destroy(sl.g);
        sl = GraphSlot{};
    }
}

void free_ctx(Ctx *c) {
    graph_cache_clear(c);
    Buf *dev[] = {&c->xq, &c->sx, &c->h, &c->hq, &c->sh, &c->y, &c->meta, &c->tbl, &c->rdesc};
    for (Buf *b : dev) {
        if (b->p) hipFree(b->p);
        *b = Buf{};
    }
    Buf *pin[] = {&c->pin_x, &c->pin_y, &c->pin_meta};
    for (Buf *b : pin) {
        if (b->p) hipHostFree(b->p);
        *b = Buf{};
    }
    for (auto &e : c->ev)
        if (e) {
            hipEventDestroy(e);
            e = nullptr;
        }
    for (auto &e : c->user_ev)
        if (e) {
            hipEventDestroy(e);
            e = nullptr;
        }
    for (auto &e : c->phase_ev)
        if (e) {
            hipEventDestroy(e);
            e = nullptr;
        }
    if (c->wait_flag) hipHostFree(c->wait_flag);
    c->wait_flag = c->wait_flag_dev = nullptr;
    if (c->stream) hipStreamDestroy(c->stream);
    c->stream = nullptr;
}


// Every context of this process, released (device selected for each).
void release_all() {
    for (int i = 0; i < g_nctx; i++)
        if (select_ctx(&g_ctx[i])) free_ctx(&g_ctx[i]);
    g_nctx = 0;
    g_cur_dev = -1;
}

// Builds one device context: its stream, the host-visible GEMV wait flag and
// the address of its copy of the fixed scratch array; reports the device.
int open_ctx(Ctx *c) {
    g_cur_dev = -1;
    if (!select_ctx(c)) return 0;
    hipDeviceProp_t prop{};
    if (!hip_ok(hipGetDeviceProperties(&prop, c->device), "init: device properties") ||
        !hip_ok(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking), "init: stream") ||
        !hip_ok(hipHostMalloc((void **)&c->wait_flag, sizeof(int), hipHostMallocMapped | hipHostMallocCoherent),
                "init: wait flag") ||
        !hip_ok(hipHostGetDevicePointer((void **)&c->wait_flag_dev, c->wait_flag, 0), "init: wait flag mapping") ||
        !hip_ok(hipGetSymbolAddress((void **)&c->fixed_scratch, HIP_SYMBOL(scratch)), "init: fixed scratch") ||
        !hip_ok(hipGetSymbolAddress((void **)&c->tail_ctr, HIP_SYMBOL(tail_ctr)), "init: tail counters") ||
        !hip_ok(hipGetSymbolAddress((void **)&c->split_ctr, HIP_SYMBOL(split_ctr)), "init: split counters"))
        return 0;
    *c->wait_flag = 0;
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, c->device) != hipSuccess) lds = 0;
    set_lds_limit(lds);
    std::fprintf(stderr, "[HIP] device %d: %s (%s), %.1f GB HBM, %d CUs, %d KB LDS per workgroup\n", c->device,
                 prop.name, prop.gcnArchName, prop.totalGlobalMem / 1e9, prop.multiProcessorCount, lds / 1024);
    return 1;
}

int make_geom(int fmt, int I, int O, int gs, MatGeom *g) {
    const bool grouped = fmt == COLI_HIP_FMT_I4G || fmt == COLI_HIP_FMT_I8G;
    if (I < 1 || O < 1) return fail("tensor shape must be positive");
    if (!(fmt == COLI_HIP_FMT_I8 || fmt == COLI_HIP_FMT_I4 || grouped)) {
        std::fprintf(stderr, "[HIP] weight format %d is not supported (1, 2, 4, 8)\n", fmt);
        return 0;
    }
    if (grouped && gs != 32 && gs != 64 && gs != 128 && gs != 256) {
        std::fprintf(stderr, "[HIP] group size %d is not supported (32, 64, 128, 256)\n", gs);
        return 0;
    }
    g->K = I;
    g->Kp = (int)round_up((size_t)I, 32);
    g->nb = g->Kp / 32;
    g->O = O;
    g->Op = (int)round_up((size_t)O, 64);
    g->w4 = (fmt == COLI_HIP_FMT_I4 || fmt == COLI_HIP_FMT_I4G) ? 1 : 0;
    g->per_row = grouped ? 0 : 1;
    g->gpb = grouped ? gs / 32 : g->nb;
    g->ng = grouped ? (g->nb + g->gpb - 1) / g->gpb : 1;
    g->gshift = grouped ? __builtin_ctz((unsigned)g->gpb) : 30;
    return 1;
}

size_t raw_weight_bytes(int fmt, int I, int O) {
    const bool w4 = fmt == COLI_HIP_FMT_I4 || fmt == COLI_HIP_FMT_I4G;
    return (size_t)O * (w4 ? (size_t)(I + 1) / 2 : (size_t)I);
}

size_t raw_scale_count(const MatGeom &g) { return (size_t)g.O * g.ng; }

void tensor_release(ColiHipTensor *t) {
    if (!t) return;
    if (t->slab) arena_release(t->slab, t->blk_off, t->blk_bytes);
    std::free(t);
}

// Repack raw QT bytes/scales (device pointers) into t's tiled layout; blocks.
int repack_into(Ctx *c, ColiHipTensor *t, const void *raw_w, const float *raw_sc) {
    launch_repack((const uint8_t *)raw_w, raw_sc, t->fmt, t->I, t->O, t->gs, t->w, t->sc, t->g, c->stream);
    return hip_ok(hipGetLastError(), "weight repack launch") &&
           hip_ok(hipStreamSynchronize(c->stream), "weight repack");
}

// Copy host raw weights to a temporary device buffer, then repack.
int repack_from_host(Ctx *c, ColiHipTensor *t, const void *w, const float *scales) {
    const size_t wb = raw_weight_bytes(t->fmt, t->I, t->O), sb = raw_scale_count(t->g) * sizeof(float);
    void *tmp = nullptr;
    if (!hip_ok(hipMalloc(&tmp, round_up(wb, 256) + sb), "upload staging")) return 0;
    int ok = hip_ok(hipMemcpy(tmp, w, wb, hipMemcpyHostToDevice), "tensor upload") &&
             hip_ok(hipMemcpy((uint8_t *)tmp + round_up(wb, 256), scales, sb, hipMemcpyHostToDevice), "scale upload") &&
             repack_into(c, t, tmp, (const float *)((uint8_t *)tmp + round_up(wb, 256)));
    hipFree(tmp);
    return ok;
}

int upload_impl(ColiHipTensor **tensor, const void *weights, const float *scales, int fmt, int I, int O, int gs,
                int device, bool from_device) {
    Ctx *c = find_ctx(device);
    if (!tensor || !weights || !scales || !select_ctx(c)) return 0;
    MatGeom g{};
    if (!make_geom(fmt, I, O, gs, &g)) return 0;
    const int gs_eff = g.per_row ? 0 : gs;
    if (*tensor) {
        const ColiHipTensor *t = *tensor;
        return t->fmt == fmt && t->I == I && t->O == O && t->device == device && t->gs == gs_eff;
    }
    ColiHipTensor *t = (ColiHipTensor *)std::calloc(1, sizeof(ColiHipTensor));
    if (!t) return 0;
    t->fmt = fmt;
    t->I = I;
    t->O = O;
    t->gs = gs_eff;
    t->device = device;
    t->g = g;
    t->w_bytes = (size_t)g.Op * g.nb * (g.w4 ? 16 : 32);
    t->sc_bytes = (size_t)g.Op * g.ng * sizeof(float);
    t->blk_bytes = round_up(t->w_bytes, 256) + t->sc_bytes;
    t->slab = arena_alloc(device, t->blk_bytes, &t->blk_off);
    if (!t->slab) {
        tensor_release(t);
        return 0;
    }
    t->w = t->slab->base + t->blk_off;
    t->sc = (float *)(t->w + round_up(t->w_bytes, 256));
    const int ok = from_device ? repack_into(c, t, weights, scales) : repack_from_host(c, t, weights, scales);
    if (!ok) {
        tensor_release(t);
        return 0;
    }
    c->tensor_count++;
    c->tensor_bytes += t->w_bytes + t->sc_bytes;
    *tensor = t;
    return 1;
}

int epi_act(int ga) { return ga == 32 ? ACT_B32 : ACT_ROW; }

// Validate a gate/up/down triple list; fills the two geometries.
int check_group(ColiHipTensor *const *gates, ColiHipTensor *const *ups, ColiHipTensor *const *downs, int count,
                int *device, MatGeom *gg, MatGeom *gd) {
    if (!gates || !ups || !downs || count < 1) return 0;
    const ColiHipTensor *g0 = gates[0], *d0 = downs[0];
    if (!g0 || !d0) return 0;
    const int D = g0->I, I = g0->O;
    for (int c = 0; c < count; c++) {
        const ColiHipTensor *g = gates[c], *u = ups[c], *d = downs[c];
        if (!g || !u || !d) return 0;
        if (g->device != g0->device || u->device != g0->device || d->device != g0->device) return 0;
        if (g->I != D || u->I != D || g->O != I || u->O != I || d->I != I || d->O != D) return 0;
        if (g->fmt != g0->fmt || u->fmt != g0->fmt || g->gs != g0->gs || u->gs != g0->gs)
            return fail("expert group: gate/up formats differ within the call");
        if (d->fmt != d0->fmt || d->gs != d0->gs) return fail("expert group: down formats differ within the call");
    }
    *device = g0->device;
    *gg = g0->g;
    *gd = d0->g;
    return 1;
}

void note_group(int count, int total) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_calls++;
    g_experts += (uint64_t)count;
    g_rows += (uint64_t)total;
}

// Kernel durations under profiling: mark(w) arms an event pair that the
// launches of slot w record inside their dispatch packets (launch_k); mark(-1)
// disarms. finish() waits and accumulates the slots that launched anything.
struct Prof {
    Ctx *c;
    bool on;
    int n = 0;
    int which[N_EVENTS / 2];
    bool used[N_EVENTS / 2];
    explicit Prof(Ctx *ctx) : c(ctx), on(profiling() != 0) {
        if (!on) return;
        for (auto &e : c->ev)
            if (!e && hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) on = false;
    }
    ~Prof() { g_launch_timing = LaunchTiming{}; }
    void close_slot() {   // records whether the armed slot launched anything, then disarms
        if (n > 0 && g_launch_timing.stop) used[n - 1] = g_launch_timing.used;
        g_launch_timing = LaunchTiming{};
    }
    void mark(int w) {   // the launches that follow belong to kernel slot w (w = -1: none)
        if (!on) return;
        close_slot();
        if (w < 0 || n >= N_EVENTS / 2) return;
        which[n] = w;
        used[n] = false;
        g_launch_timing = LaunchTiming{c->ev[2 * n], c->ev[2 * n + 1], false};
        n++;
    }
    void finish() {
        if (!on) return;
        close_slot();
        if (n == 0 || hipStreamSynchronize(c->stream) != hipSuccess) return;
        std::lock_guard<std::mutex> lock(g_stats_mu);
        for (int i = 0; i < n; i++) {
            float ms = 0;
            if (!used[i] || hipEventElapsedTime(&ms, c->ev[2 * i], c->ev[2 * i + 1]) != hipSuccess) continue;
            g_k_launches[which[i]]++;
            g_k_ms[which[i]] += ms;
        }
    }
};

struct Scratch {
    int8_t *xq;
    float *sx, *h;
    int8_t *hq;
    float *sh, *y;
    int xs, sxs, hs, hqs, shs, ys;
};

// Reserve per-row scratch for `rows_x` activation rows and `R` expert rows.
int reserve_rows(Ctx *c, const MatGeom &gg, const MatGeom &gd, int rows_x, int R, int ga, Scratch *s) {
    s->xs = gg.Kp;
    s->sxs = ga == 32 ? gg.nb : 1;
    s->hs = gd.Kp;   // h row: I padded to 32 (= down's K layout)
    s->hqs = gd.Kp;
    s->shs = ga == 32 ? gd.nb : 1;
    s->ys = gd.O;
    if (!reserve(c, c->xq, (size_t)rows_x * s->xs) || !reserve(c, c->sx, (size_t)rows_x * s->sxs * 4) ||
        !reserve(c, c->h, (size_t)R * s->hs * 4) || !reserve(c, c->hq, (size_t)R * s->hqs) ||
        !reserve(c, c->sh, (size_t)R * s->shs * 4) || !reserve(c, c->y, (size_t)R * s->ys * 4))
        return 0;
    s->xq = (int8_t *)c->xq.p;
    s->sx = (float *)c->sx.p;
    s->h = (float *)c->h.p;
    s->hq = (int8_t *)c->hq.p;
    s->sh = (float *)c->sh.p;
    s->y = (float *)c->y.p;
    return 1;
}

// The same per-row scratch as reserve_rows, laid out from `base` (256-byte
// aligned pieces). With base == nullptr only the size is computed.
int carve_rows(const MatGeom &gg, const MatGeom &gd, int rows_x, int R, int ga, uint8_t *base, size_t *bytes,
               Scratch *s) {
    s->xs = gg.Kp;
    s->sxs = ga == 32 ? gg.nb : 1;
    s->hs = gd.Kp;
    s->hqs = gd.Kp;
    s->shs = ga == 32 ? gd.nb : 1;
    s->ys = gd.O;
    const size_t sz[6] = {(size_t)rows_x * s->xs, (size_t)rows_x * s->sxs * 4, (size_t)R * s->hs * 4,
                          (size_t)R * s->hqs, (size_t)R * s->shs * 4, (size_t)R * s->ys * 4};
    size_t off = 0, at[6];
    for (int i = 0; i < 6; i++) {
        at[i] = off;
        off += round_up(std::max(sz[i], (size_t)1), 256);
    }
    *bytes = off;
    if (base) {
        s->xq = (int8_t *)(base + at[0]);
        s->sx = (float *)(base + at[1]);
        s->h = (float *)(base + at[2]);
        s->hq = (int8_t *)(base + at[3]);
        s->sh = (float *)(base + at[4]);
        s->y = (float *)(base + at[5]);
    }
    return 1;
}

// Optional pieces of a dispatch beyond the expert matmuls.
struct DispatchOpts {
    bool x_quantized = false;   // xq/sx already written (fused router + quant)
    bool act_zero = false;      // every row reads activation row 0 (one token)
    int n_rows_fixed = -1;      // row count known on the host
    RouteArgs route{};          // one token: router + quant fused into the gate/up GEMV
    int w_reuse = 0;                    // about two or more M tiles per expert: weights stay cacheable
    const float *combine_w = nullptr;   // one token: down + combine in one launch, weights [k]
    float *combine_out = nullptr;       //   and the layer output [D]
    const float *tail_w = nullptr;      // one token: the down GEMV's last workgroup per tile combines
    float *tail_out = nullptr;
    int *tail_ctr = nullptr;    // host-buffer calls: the activation quantisation also stages this metadata
    const void *meta_src = nullptr;
    void *meta_dst = nullptr;
    int meta_n16 = 0;
    hipEvent_t after_quant = nullptr;   // recorded after the activation quantisation (profiling)
    // split-K GEMV plans of the gate/up and down launches (split 0: unsplit)
    // and their partial buffers (shared: the launches run one after the other)
    GemvSplit split_gu, split_dn;
    int32_t *part_d = nullptr;
    float *part_f = nullptr;
    int *split_ctr = nullptr;
};

// Plans the split-K GEMV launches of a dispatch with up to `rows` rows and
// reserves their partial buffers (before any graph capture). The fused
// router prologue and the per-block dot dump run only in the unsplit kernel.
int plan_split(Ctx *c, const MatGeom &gg, const MatGeom &gd, int rows, int act, bool route_fused,
               DispatchOpts *opt) {
    const int target = gemv_split_target();
    opt->split_gu = route_fused || g_dbg_gu ? GemvSplit{} : plan_gemv_split(gg, true, rows, act, target);
    opt->split_dn = g_dbg_dn ? GemvSplit{} : plan_gemv_split(gd, false, rows, act, target);
    const size_t bd = std::max(opt->split_gu.part_d_bytes, opt->split_dn.part_d_bytes);
    const size_t bf = std::max(opt->split_gu.part_f_bytes, opt->split_dn.part_f_bytes);
    if (!bd) return 1;
    if (!reserve(c, c->part_d, bd) || (bf && !reserve(c, c->part_f, bf))) return 0;
    opt->part_d = (int32_t *)c->part_d.p;
    opt->part_f = (float *)c->part_f.p;
    opt->split_ctr = c->split_ctr;
    return 1;
}

void apply_split(DotArgs &d, const GemvSplit &p, const DispatchOpts &opt) {
    d.split = p.split;
    d.split_kb = p.kb;
    d.split_nw = p.nw;
    d.part_d = opt.part_d;
    d.part_f = opt.part_f;
    d.split_ctr = opt.split_ctr;
}

// The kernel sequence of one dispatch: quantise x (device memory, or mapped
// host memory for the host-buffer calls), gate/up (+SwiGLU), [quantise h],
// down.
void run_experts(Ctx *c, Prof &prof, const ExpertDesc *desc, const RowPlan &plan, const MatGeom &gg,
                 const MatGeom &gd, const float *x_dev, int rows_x, bool x_identity, int R_bound, int T_bound,
                 int ga, int arm, const Scratch &s, const DispatchOpts &opt = DispatchOpts()) {
    const int act = epi_act(ga);
    if (!opt.x_quantized) {
        QuantArgs qa{x_dev, gg.K, rows_x, gg.K, gg.Kp, s.xq, s.xs, s.sx, s.sxs, act,
                     (const uint4 *)opt.meta_src, (uint4 *)opt.meta_dst, opt.meta_n16};
        prof.mark(COLI_HIP_K_QUANT_X);
        launch_quant_rows(qa, c->stream);
        if (opt.after_quant) hipEventRecord(opt.after_quant, c->stream);
    }

    DotArgs da{};
    da.desc = desc;
    da.plan = plan;
    da.xq = s.xq;
    da.x_stride = s.xs;
    da.sx = s.sx;
    da.sx_stride = s.sxs;
    da.out = s.h;
    da.out_stride = s.hs;
    da.hq = act == ACT_B32 ? s.hq : nullptr;
    da.hq_stride = s.hqs;
    da.sh = s.sh;
    da.sh_stride = s.shs;
    da.dots = g_dbg_gu;
    da.act_identity = x_identity ? 1 : 0;
    da.act_zero = opt.act_zero ? 1 : 0;
    da.n_rows_fixed = opt.n_rows_fixed;
    da.route = opt.route;
    da.w_reuse = opt.w_reuse;
    da.spin_limit = g_spin_limit;
    da.wait_failed = c->wait_flag_dev;
    prof.mark(COLI_HIP_K_GATEUP);
    if (arm == COLI_HIP_ARM_GEMV && !opt.route.logits) apply_split(da, opt.split_gu, opt);
    if (arm == COLI_HIP_ARM_GEMV)
        launch_gemv_gateup(da, gg, act, R_bound, c->stream);
    else
        launch_mfma_gateup(da, gg, act, T_bound, c->stream);

    if (act == ACT_ROW) {
        QuantArgs qh{s.h, s.hs, R_bound, gd.K, gd.Kp, s.hq, s.hqs, s.sh, s.shs, ACT_ROW};
        prof.mark(COLI_HIP_K_QUANT_H);
        launch_quant_rows(qh, c->stream);
    }

    DotArgs dd = da;
    dd.xq = s.hq;
    dd.x_stride = s.hqs;
    dd.sx = s.sh;
    dd.sx_stride = s.shs;
    dd.out = s.y;
    dd.out_stride = s.ys;
    dd.hq = nullptr;
    dd.sh = nullptr;
    dd.dots = g_dbg_dn;
    dd.act_identity = 1;
    dd.act_zero = 0;
    dd.route = RouteArgs{};
    dd.tail_out = opt.tail_out;
    dd.tail_w = opt.tail_w;
    dd.tail_ctr = opt.tail_ctr;
    apply_split(dd, arm == COLI_HIP_ARM_GEMV ? opt.split_dn : GemvSplit{}, opt);
    prof.mark(COLI_HIP_K_DOWN);
    if (arm == COLI_HIP_ARM_GEMV && opt.combine_out) {
        launch_gemv_down_combine(dd, gd, act, opt.n_rows_fixed, opt.combine_w, opt.combine_out, c->stream);
    } else if (arm == COLI_HIP_ARM_GEMV) {
        launch_gemv_down(dd, gd, act, R_bound, c->stream);
    } else {
        launch_mfma_down(dd, gd, act, T_bound, c->stream);
    }
}

struct ReduceSpec {
    const int *row_ptr, *row_idx;
    const float *rw;
    int s_n;
    float *out;
};

// ---------------------------------------------------------------------------
// Expert-group graph cache (COLI_HIP_GRAPH=1, or COLI_CUDA_GRAPH=1 as the
// reference's knob). A decode loop calls expert_group with the same launch
// shape (arm, expert count, widths, rows per expert) over and over while the
// contents change: which experts (their descriptors) and the activations.
// The shape becomes one captured graph; the contents ride in through the
// pinned staging buffers that the graph's own H2D copies read, so one graph
// serves every later call of that shape (backend_cuda.cu:666-745, 1104-1166).
// A slot keeps the full shape, not only its hash, so two shapes never share
// a graph. A graph captured before a scratch reallocation is dropped at
// lookup (its baked addresses are stale); a failed capture drops them all.
// ---------------------------------------------------------------------------
bool graph_cache_enabled() {
    // COLI_CUDA_GRAPH, the reference's knob, is read as an alias so that the
    // unchanged Rust caller's environment keeps its meaning
    const char *v = std::getenv("COLI_HIP_GRAPH");
    if (!v || !*v) v = std::getenv("COLI_CUDA_GRAPH");
    return v && std::atoi(v) != 0;
}

// COLI_HIP_GRAPH_ADAPT=0: replay every cached shape, never decline one.
bool graph_adapt() {
    const char *v = std::getenv("COLI_HIP_GRAPH_ADAPT");
    return !(v && v[0] == '0');
}

// A call's launch shape: fixed fields, then rows per expert (at most 256).
// Built on the stack per call; a slot copies it only when a graph is stored.
constexpr int SHAPE_FIELDS = 12, SHAPE_MAX = SHAPE_FIELDS + 256;
struct ShapeKey {
    int n = 0;
    int v[SHAPE_MAX];
    uint64_t hash = 0;
};

void shape_key(ShapeKey *k, const int (&fields)[SHAPE_FIELDS], const int *rows, int count) {
    k->n = SHAPE_FIELDS + count;
    std::memcpy(k->v, fields, sizeof(fields));
    std::memcpy(k->v + SHAPE_FIELDS, rows, (size_t)count * sizeof(int));
    uint64_t h = 0xcbf29ce484222325ull;   // FNV-1a, 64-bit
    for (int i = 0; i < k->n; i++)
        for (int b = 0; b < 4; b++) {
            h ^= (uint64_t)((uint32_t)k->v[i] >> (8 * b)) & 0xff;
            h *= 0x100000001b3ull;
        }
    k->hash = h;
}

std::vector<int> g_slot_shape[COLI_HIP_MAX_DEVICES][GRAPH_CACHE];

bool slot_shape_is(const std::vector<int> &s, const ShapeKey &key) {
    return (int)s.size() == key.n && std::memcmp(s.data(), key.v, (size_t)key.n * sizeof(int)) == 0;
}

void drop_slot(GraphSlot &sl) {   // a graph whose baked scratch addresses are stale
    graph_destroy(sl.g);
    sl = GraphSlot{};
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_graph_invalidations++;
}

// The shape's slot, or null. A slot whose graph was captured before a scratch
// reallocation is dropped here (its baked addresses are stale), so the shape
// is captured and probed again.
GraphSlot *slot_lookup(Ctx *c, const ShapeKey &key) {
    const int ci = (int)(c - g_ctx);
    for (int i = 0; i < GRAPH_CACHE; i++) {
        GraphSlot &sl = c->graphs[i];
        if (!sl.live || sl.key != key.hash || !slot_shape_is(g_slot_shape[ci][i], key)) continue;
        if (sl.g && sl.gen != c->gen) {
            drop_slot(sl);
            return nullptr;
        }
        sl.used = ++c->graph_clock;
        return &sl;
    }
    return nullptr;
}

GraphSlot *graph_store(Ctx *c, const ShapeKey &key, ColiHipGraph *g) {
    const int ci = (int)(c - g_ctx);
    // graphs captured before a scratch reallocation can never replay: free
    // them (and their exec resources) before choosing an LRU victim
    for (int i = 0; i < GRAPH_CACHE; i++)
        if (c->graphs[i].g && c->graphs[i].gen != c->gen) drop_slot(c->graphs[i]);
    int victim = 0;
    for (int i = 0; i < GRAPH_CACHE; i++) {
        if (!c->graphs[i].live) {
            victim = i;
            break;
        }
        if (c->graphs[i].used < c->graphs[victim].used) victim = i;
    }
    GraphSlot &sl = c->graphs[victim];
    graph_destroy(sl.g);
    sl = GraphSlot{};
    sl.live = true;
    sl.key = key.hash;
    sl.g = g;
    sl.gen = c->gen;
    sl.used = ++c->graph_clock;
    sl.state = graph_adapt() ? SLOT_PROBE : SLOT_GRAPH;
    g_slot_shape[ci][victim].assign(key.v, key.v + key.n);
    return &sl;
}

// A probe's host time; once both ways have GRAPH_PROBES samples the faster
// fastest sample wins (ties to the graph).
void slot_probe(GraphSlot *sl, bool graph, double secs) {
    if (graph) {
        sl->t_graph = sl->n_graph++ ? std::min(sl->t_graph, secs) : secs;
    } else {
        sl->t_eager = sl->n_eager++ ? std::min(sl->t_eager, secs) : secs;
    }
    if (sl->n_graph < GRAPH_PROBES || sl->n_eager < GRAPH_PROBES) return;
    if (sl->t_graph <= sl->t_eager) {
        sl->state = SLOT_GRAPH;
    } else {
        sl->state = SLOT_EAGER;
        graph_destroy(sl->g);
        sl->g = nullptr;
    }
}

int expert_group_impl(ColiHipTensor *const *gates, ColiHipTensor *const *ups, ColiHipTensor *const *downs,
                      const int *rows, int count, float *y, const float *x, const ReduceSpec *red, int *arm_out) {
    if (!rows || !x || count < 1) return 0;
    if (!red && !y) return 0;
    if (red && (!red->row_ptr || !red->row_idx || !red->rw || !red->out || red->s_n < 1)) return 0;
    if (count > 256) return fail("expert group: more than 256 experts in one call");
    int device = -1;
    MatGeom gg{}, gd{};
    if (!check_group(gates, ups, downs, count, &device, &gg, &gd)) return 0;
    int total = 0, max_rows = 0;
    for (int c = 0; c < count; c++) {
        if (rows[c] < 1) return 0;
        total += rows[c];
        max_rows = std::max(max_rows, rows[c]);
    }
    if (red) {
        if (red->row_ptr[0] != 0 || red->row_ptr[red->s_n] != total) return fail("reduce: row_ptr does not span rows");
        for (int s = 0; s < red->s_n; s++)
            if (red->row_ptr[s + 1] < red->row_ptr[s]) return fail("reduce: row_ptr not ascending");
        for (int j = 0; j < total; j++)
            if (red->row_idx[j] < 0 || red->row_idx[j] >= total) return fail("reduce: row_idx out of range");
    }
    Ctx *c = find_ctx(device);
    if (!select_ctx(c)) return 0;
    const int D = gg.K, ga = act_group();
    int arm = forced_arm();
    if (arm < 0) arm = max_rows <= 1 ? COLI_HIP_ARM_GEMV : COLI_HIP_ARM_MFMA;
    if (arm_out) *arm_out = arm;

    // host-built plan: descriptors in call order, rows consecutive
    int T = 0;
    for (int i = 0; i < count; i++) T += (rows[i] + MT_ROWS - 1) / MT_ROWS;
    const int s_n = red ? red->s_n : 0;
    const size_t n_int = (size_t)total /*row_exp*/ + 4 * (size_t)T + 2 + (red ? (size_t)(s_n + 1) + total : 0);
    const size_t desc_b = round_up((size_t)count * sizeof(ExpertDesc), 16);
    // (a whole number of 16-byte words: the quantisation kernel stages it)
    const size_t meta_b = round_up(desc_b + n_int * 4 + (red ? (size_t)total * 4 : 0), 16);
    const size_t xb = (size_t)total * D * 4;
    const size_t ob = red ? (size_t)s_n * D * 4 : xb;
    // every reservation happens here, before any capture (scratch must not
    // move while a graph records its addresses)
    Scratch s{};
    if (!reserve_rows(c, gg, gd, total, total, ga, &s) || !reserve(c, c->meta, meta_b) ||
        !reserve_pinned(c, c->pin_meta, meta_b) || !reserve_pinned(c, c->pin_x, xb) ||
        !reserve_pinned(c, c->pin_y, ob))
        return 0;

    // stage the call's contents: descriptors, row plan, reduce layout, x
    uint8_t *hm = (uint8_t *)c->pin_meta.p;
    ExpertDesc *hd = (ExpertDesc *)hm;
    for (int i = 0; i < count; i++) {
        hd[i].w[0] = gates[i]->w;
        hd[i].w[1] = ups[i]->w;
        hd[i].w[2] = downs[i]->w;
        hd[i].sc[0] = gates[i]->sc;
        hd[i].sc[1] = ups[i]->sc;
        hd[i].sc[2] = downs[i]->sc;
    }
    int *hi = (int *)(hm + desc_b);
    int *row_exp = hi, *mt_exp = row_exp + total, *mt_row0 = mt_exp + T, *mt_rend = mt_row0 + T;
    int *mt_first = mt_rend + T;
    int *counts = mt_first + T;
    int *rp = counts + 2, *ri = rp + (red ? s_n + 1 : 0);
    float *rwv = (float *)(ri + (red ? total : 0));
    for (int i = 0, r = 0, t = 0; i < count; i++) {
        for (int q = 0; q < rows[i]; q++) row_exp[r + q] = i;
        const int t0 = t;
        for (int q = 0; q < rows[i]; q += MT_ROWS, t++) {
            mt_exp[t] = i;
            mt_row0[t] = r + q;
            mt_rend[t] = r + rows[i];
            mt_first[t] = t0;
        }
        r += rows[i];
    }
    counts[0] = total;
    counts[1] = T;
    if (red) {
        std::memcpy(rp, red->row_ptr, (size_t)(s_n + 1) * 4);
        std::memcpy(ri, red->row_idx, (size_t)total * 4);
        std::memcpy(rwv, red->rw, (size_t)total * 4);
    }
    std::memcpy(c->pin_x.p, x, xb);

    uint8_t *dm = (uint8_t *)c->meta.p;
    int *di = (int *)(dm + desc_b);
    RowPlan plan{};
    plan.row_exp = di;
    plan.row_act = di;   // unused: activation rows are the call's rows
    plan.mt_exp = di + total;
    plan.mt_row0 = di + total + T;
    plan.mt_rend = di + total + 2 * T;
    plan.mt_first = di + total + 3 * T;
    plan.counts = di + total + 4 * T;
    // No copy engine in the call: the staging buffers are mapped host
    // memory. The activation quantisation reads x across PCIe and also stages
    // the metadata into device memory (every later kernel reads it there); the
    // last kernel (the combine, else the down projection) writes the result
    // across PCIe. Config 2's call (8 rows, one token out): 89 -> 62.5 us
    // eager, 79 -> 68.7 us from a cached graph (profiled, the copies alone had
    // taken 22 us in and 48 us out).
    DispatchOpts opt;
    if (arm == COLI_HIP_ARM_GEMV && !plan_split(c, gg, gd, total, epi_act(ga), false, &opt)) return 0;
    opt.w_reuse = total >= 2 * MT_ROWS * count;   // about two or more M tiles per expert
    opt.meta_src = c->pin_meta.d;
    opt.meta_dst = dm;
    opt.meta_n16 = (int)(meta_b / 16);
    const float *x_dev = (const float *)c->pin_x.d;
    Scratch so = s;
    if (!red) so.y = (float *)c->pin_y.d;   // [total][D], the y buffer's own layout

    // The whole call as stream work. The same sequence runs eagerly or is
    // captured once per shape. Under profiling, h2d = the quantisation kernel
    // that reads x across PCIe, d2h = the combine that writes the output
    // across PCIe (0 without a reduce: the down projection writes it, and its
    // time is kernel time).
    const bool profile = profiling() != 0;
    auto enqueue = [&](Prof &prof, bool phases) -> int {
        if (phases) hipEventRecord(c->phase_ev[0], c->stream);
        opt.after_quant = phases ? c->phase_ev[1] : nullptr;
        prof.mark(-1);
        run_experts(c, prof, (const ExpertDesc *)dm, plan, gg, gd, x_dev, total, true, total, T, ga, arm, so, opt);
        prof.mark(-1);
        if (phases) hipEventRecord(c->phase_ev[2], c->stream);
        if (red) {
            const int *drp = plan.counts + 2, *dri = drp + s_n + 1;
            const float *drw = (const float *)(dri + total);
            prof.mark(COLI_HIP_K_COMBINE);
            launch_combine((float *)c->pin_y.d, s.y, drp, dri, drw, s_n, D, s.ys, c->stream);
            prof.mark(-1);
        }
        if (phases) hipEventRecord(c->phase_ev[3], c->stream);
        return hip_ok(hipGetLastError(), "expert group launch");
    };
    auto finish = [&]() -> int {
        if (!check_waits(c)) return 0;
        std::memcpy(red ? red->out : y, c->pin_y.p, ob);
        note_group(count, total);
        return 1;
    };

    const bool graphs_on = graph_cache_enabled();
    if (graphs_on && !profile && !g_dbg_gu && !g_dbg_dn) {
        const ColiHipTensor *g0 = gates[0], *d0 = downs[0];
        ShapeKey key;
        shape_key(&key, {arm, count, D, gg.O, s_n, ga, g0->fmt, g0->gs, d0->fmt, d0->gs, g_spin_limit, gemv_split_target()},
                  rows, count);
        GraphSlot *sl = slot_lookup(c, key);
        if (!sl) {
            Prof off(c);
            off.on = false;
            int ok = hip_ok(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "graph begin capture");
            ok = ok && enqueue(off, false);
            hipGraph_t graph = nullptr;
            const hipError_t end = hipStreamEndCapture(c->stream, &graph);   // always ends a begun capture
            hipGraphExec_t exec = nullptr;
            ok = ok && hip_ok(end, "graph end capture") &&
                 hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "graph instantiate");
            ColiHipGraph *g = nullptr;
            if (ok) g = (ColiHipGraph *)std::calloc(1, sizeof(ColiHipGraph));
            if (!g) {
                // a failed capture: nothing recorded near it is trusted again
                if (exec) hipGraphExecDestroy(exec);
                if (graph) hipGraphDestroy(graph);
                graph_cache_clear(c);
                (void)hipGetLastError();
                return fail("expert group: graph capture failed; the device's graph cache was cleared");
            }
            g->graph = graph;
            g->exec = exec;
            g->device = device;
            g->gen = c->gen;
            sl = graph_store(c, key, g);
            {
                std::lock_guard<std::mutex> lock(g_stats_mu);
                g_graph_captures++;
            }
            if (!hip_ok(hipGraphLaunch(g->exec, c->stream), "expert group graph launch") ||
                !hip_ok(hipStreamSynchronize(c->stream), "expert group graph synchronize"))
                return 0;
            return finish();
        }
        // replay unless this shape runs eagerly (it lost its probes), or it
        // is being probed and the eager side is behind
        const bool replay = sl->state == SLOT_GRAPH || (sl->state == SLOT_PROBE && sl->n_graph <= sl->n_eager);
        const auto t0 = std::chrono::steady_clock::now();
        if (replay) {
            if (!hip_ok(hipGraphLaunch(sl->g->exec, c->stream), "expert group graph launch") ||
                !hip_ok(hipStreamSynchronize(c->stream), "expert group graph synchronize"))
                return 0;
        } else {
            Prof off(c);
            off.on = false;
            if (!enqueue(off, false) || !hip_ok(hipStreamSynchronize(c->stream), "expert group synchronize")) return 0;
        }
        if (sl->state == SLOT_PROBE)
            slot_probe(sl, replay, std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count());
        {
            std::lock_guard<std::mutex> lock(g_stats_mu);
            if (replay) g_graph_replays++;
            else g_graph_uncacheable++;   // ran eagerly with the cache on
        }
        return finish();
    }
    if (graphs_on) {
        std::lock_guard<std::mutex> lock(g_stats_mu);
        g_graph_uncacheable++;
    }

    Prof prof(c);
    bool phases = profile;
    for (auto &e : c->phase_ev)
        if (phases && !e && hipEventCreateWithFlags(&e, hipEventDisableSystemFence) != hipSuccess) phases = false;
    if (!enqueue(prof, phases) || !hip_ok(hipStreamSynchronize(c->stream), "expert group synchronize")) return 0;
    prof.finish();
    if (phases) {
        float h2d = 0, d2h = 0;
        hipEventElapsedTime(&h2d, c->phase_ev[0], c->phase_ev[1]);
        hipEventElapsedTime(&d2h, c->phase_ev[2], c->phase_ev[3]);
        std::lock_guard<std::mutex> lock(g_stats_mu);
        g_h2d_ms += h2d;
        g_d2h_ms += d2h;
    }
    return finish();
}

}  // namespace

// ============================================================================
// C ABI
// ============================================================================
extern "C" {

// The ordinal list is checked as a whole before anything is built: every
// entry must name a visible device and none may repeat (0 otherwise, and the
// contexts of an earlier init stay as they were). Then the earlier contexts
// are released and one is built per ordinal, in list order; if building one
// fails, every context built so far is released again.
int coli_hip_init(const int *devices, int count) {
    if (!devices || count < 1 || count > COLI_HIP_MAX_DEVICES) return 0;
    int visible = 0;
    if (!hip_ok(hipGetDeviceCount(&visible), "init: counting HIP devices")) return 0;
    for (int i = 0; i < count; i++) {
        if (devices[i] < 0 || devices[i] >= visible) {
            std::fprintf(stderr, "[HIP] init: ordinal %d names no device (%d visible)\n", devices[i], visible);
            return 0;
        }
        for (int j = 0; j < i; j++)
            if (devices[j] == devices[i]) {
                std::fprintf(stderr, "[HIP] init: ordinal %d appears twice in the list\n", devices[i]);
                return 0;
            }
    }
    release_all();
    for (int i = 0; i < count; i++) {
        Ctx *c = &g_ctx[i];
        *c = Ctx{};
        c->device = devices[i];
        if (!open_ctx(c)) {
            free_ctx(c);
            release_all();
            return 0;
        }
        g_nctx = i + 1;
    }
    return 1;
}

void coli_hip_shutdown(void) { release_all(); }

int coli_hip_device_count(void) { return g_nctx; }

int coli_hip_probe_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n < 0) {
        (void)hipGetLastError();
        return 0;
    }
    return n;
}

int coli_hip_device_at(int index) { return index >= 0 && index < g_nctx ? g_ctx[index].device : -1; }

int coli_hip_mem_info(int device, size_t *free_bytes, size_t *total_bytes) {
    Ctx *c = find_ctx(device);
    if (!free_bytes || !total_bytes || !select_ctx(c)) return 0;
    return hip_ok(hipMemGetInfo(free_bytes, total_bytes), "memory info");
}

void coli_hip_stats(int device, size_t *tensor_count, size_t *tensor_bytes) {
    size_t n = 0, b = 0;
    for (int i = 0; i < g_nctx; i++)
        if (device < 0 || g_ctx[i].device == device) {
            n += g_ctx[i].tensor_count;
            b += g_ctx[i].tensor_bytes;
        }
    if (tensor_count) *tensor_count = n;
    if (tensor_bytes) *tensor_bytes = b;
}

void coli_hip_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows, double *h2d_ms, double *kernel_ms,
                          double *d2h_ms) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    if (calls) *calls = g_calls;
    if (experts) *experts = g_experts;
    if (rows) *rows = g_rows;
    if (h2d_ms) *h2d_ms = g_h2d_ms;
    if (kernel_ms) {
        double k = 0;
        for (int i = 0; i < COLI_HIP_K_COUNT; i++) k += g_k_ms[i];
        *kernel_ms = k;
    }
    if (d2h_ms) *d2h_ms = g_d2h_ms;
}

int coli_hip_tensor_upload(ColiHipTensor **tensor, const void *weights, const float *scales, int fmt, int I, int O,
                           int device) {
    if (fmt != COLI_HIP_FMT_I8 && fmt != COLI_HIP_FMT_I4)
        return fail("tensor_upload takes per-row formats 1 and 2; use tensor_upload_grouped");
    return upload_impl(tensor, weights, scales, fmt, I, O, 0, device, false);
}

int coli_hip_tensor_upload_grouped(ColiHipTensor **tensor, const void *weights, const float *scales, int fmt, int I,
                                   int O, int gs, int device) {
    return upload_impl(tensor, weights, scales, fmt, I, O, gs, device, false);
}

int coli_hip_tensor_upload_dev(ColiHipTensor **tensor, const void *weights_dev, const float *scales_dev, int fmt,
                               int I, int O, int gs, int device) {
    return upload_impl(tensor, weights_dev, scales_dev, fmt, I, O, gs, device, true);
}

void coli_hip_tensor_free(ColiHipTensor *t) {
    if (!t) return;
    Ctx *c = find_ctx(t->device);
    if (c) {
        select_ctx(c);
        c->tensor_count--;
        c->tensor_bytes -= t->w_bytes + t->sc_bytes;
    }
    tensor_release(t);
}

size_t coli_hip_tensor_bytes(const ColiHipTensor *t) { return t ? t->w_bytes + t->sc_bytes : 0; }

int coli_hip_tensor_device(const ColiHipTensor *t) { return t ? t->device : -1; }

int coli_hip_tensor_update(ColiHipTensor *t, const void *weights, const float *scales) {
    if (!t || !weights || !scales) return 0;
    Ctx *c = find_ctx(t->device);
    if (!select_ctx(c)) return 0;
    return repack_from_host(c, t, weights, scales);
}

int coli_hip_expert_group(ColiHipTensor *const *gates, ColiHipTensor *const *ups, ColiHipTensor *const *downs,
                          const int *rows, int count, float *y, const float *x) {
    return expert_group_impl(gates, ups, downs, rows, count, y, x, nullptr, nullptr);
}

int coli_hip_expert_group_tiled(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                ColiHipTensor *const *downs, const int *rows, int count, float *y, const float *x,
                                int tile_m, int tile_n, int tile_k, int *arm_out) {
    (void)tile_m;
    (void)tile_n;
    (void)tile_k;
    return expert_group_impl(gates, ups, downs, rows, count, y, x, nullptr, arm_out);
}

int coli_hip_expert_group_reduce(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                 ColiHipTensor *const *downs, const int *rows, int count, const int *row_ptr,
                                 const int *row_idx, const float *rw, int s_n, float *out, const float *x) {
    ReduceSpec red{row_ptr, row_idx, rw, s_n, out};
    return expert_group_impl(gates, ups, downs, rows, count, nullptr, x, &red, nullptr);
}

int coli_hip_graph_begin(int device) {
    Ctx *c = find_ctx(device);
    if (!select_ctx(c)) return 0;
    return hip_ok(hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal), "graph begin capture");
}

int coli_hip_graph_end(int device, ColiHipGraph **out) {
    Ctx *c = find_ctx(device);
    if (!out || !select_ctx(c)) return 0;
    hipGraph_t graph = nullptr;
    if (!hip_ok(hipStreamEndCapture(c->stream, &graph), "graph end capture")) return 0;
    hipGraphExec_t exec = nullptr;
    if (!hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "graph instantiate")) {
        hipGraphDestroy(graph);
        return 0;
    }
    ColiHipGraph *g = (ColiHipGraph *)std::calloc(1, sizeof(ColiHipGraph));
    if (!g) {
        hipGraphExecDestroy(exec);
        hipGraphDestroy(graph);
        return 0;
    }
    g->graph = graph;
    g->exec = exec;
    g->device = device;
    g->gen = c->gen;
    *out = g;
    return 1;
}

int coli_hip_graph_launch(ColiHipGraph *g) {
    if (!g) return 0;
    Ctx *c = find_ctx(g->device);
    if (!select_ctx(c)) return 0;
    if (c->gen != g->gen) return fail("graph launch: scratch was reallocated after the capture; capture the graph again");
    if (!hip_ok(hipGraphLaunch(g->exec, c->stream), "graph launch")) return 0;
    return hip_ok(hipStreamSynchronize(c->stream), "graph synchronize") && check_waits(c);
}

void coli_hip_graph_free(ColiHipGraph *g) { graph_destroy(g); }

void coli_hip_graph_cache_stats(uint64_t *captures, uint64_t *replays, uint64_t *invalidations,
                                uint64_t *uncacheable) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    if (captures) *captures = g_graph_captures;
    if (replays) *replays = g_graph_replays;
    if (invalidations) *invalidations = g_graph_invalidations;
    if (uncacheable) *uncacheable = g_graph_uncacheable;
}

int coli_hip_pipe_sync(int device) {
    Ctx *c = find_ctx(device);
    if (!select_ctx(c)) return 0;
    return hip_ok(hipStreamSynchronize(c->stream), "stream synchronize") && check_waits(c);
}

void *coli_hip_pipe_alloc(int device, size_t bytes) {
    Ctx *c = find_ctx(device);
    void *p = nullptr;
    if (!select_ctx(c) || bytes == 0) return nullptr;
    if (!hip_ok(hipMalloc(&p, bytes), "pipe allocation")) return nullptr;
    return p;
}

void coli_hip_pipe_free(int device, void *p) {
    Ctx *c = find_ctx(device);
    if (!p || !select_ctx(c)) return;
    hipStreamSynchronize(c->stream);
    hipFree(p);
}

int coli_hip_pipe_upload(int device, void *dst, const void *src, size_t bytes) {
    Ctx *c = find_ctx(device);
    if (!dst || !src || !select_ctx(c)) return 0;
    return hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, c->stream), "pipe upload") &&
           hip_ok(hipStreamSynchronize(c->stream), "pipe upload sync");
}

int coli_hip_pipe_download(int device, const void *src, void *dst, size_t bytes) {
    Ctx *c = find_ctx(device);
    if (!dst || !src || !select_ctx(c)) return 0;
    return hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, c->stream), "pipe download") &&
           hip_ok(hipStreamSynchronize(c->stream), "pipe download sync");
}

int coli_hip_event_record(int device, int slot) {
    Ctx *c = find_ctx(device);
    if (slot < 0 || slot >= 16 || !select_ctx(c)) return 0;
    // device-stream timing only: no system-scope fence (as the profiler's events)
    if (!c->user_ev[slot] &&
        !hip_ok(hipEventCreateWithFlags(&c->user_ev[slot], hipEventDisableSystemFence), "event create"))
        return 0;
    return hip_ok(hipEventRecord(c->user_ev[slot], c->stream), "event record");
}

float coli_hip_event_elapsed(int device, int a, int b) {
    Ctx *c = find_ctx(device);
    if (a < 0 || a >= 16 || b < 0 || b >= 16 || !select_ctx(c) || !c->user_ev[a] || !c->user_ev[b]) return -1.0f;
    if (!hip_ok(hipEventSynchronize(c->user_ev[b]), "event sync")) return -1.0f;
    float ms = -1.0f;
    if (!hip_ok(hipEventElapsedTime(&ms, c->user_ev[a], c->user_ev[b]), "event elapsed")) return -1.0f;
    return ms;
}

int coli_hip_synth_fill(int device, void *dst, size_t n, int kind, float a, float b, uint64_t seed) {
    Ctx *c = find_ctx(device);
    if (!dst || kind < 0 || kind > 2 || !select_ctx(c)) return 0;
    launch_synth_fill(dst, n, kind, a, b, seed, c->stream);
    return hip_ok(hipGetLastError(), "synthetic fill");
}

int coli_hip_set_act_group(int ga) {
    if (ga != 0 && ga != 32) return fail("act group must be 0 (per row) or 32");
    g_act_group = ga;
    return 1;
}

int coli_hip_get_act_group(void) { return act_group(); }

int coli_hip_set_arm(int arm) {
    if (arm != -1 && arm != COLI_HIP_ARM_GEMV && arm != COLI_HIP_ARM_MFMA) return fail("unknown arm");
    g_arm = arm;
    return 1;
}

int coli_hip_set_fused_combine(int mode) {
    if (mode < -1 || mode > 1) return fail("fused combine mode must be -1, 0 or 1");
    g_fused_combine.store(mode);
    return 1;
}

int coli_hip_set_gemv_split(int target_wgs) {
    if (target_wgs < -1) return fail("GEMV split target must be -1 (default), 0 (off) or a workgroup count");
    g_gemv_split.store(target_wgs < 0 ? GEMV_SPLIT_DEFAULT : target_wgs);
    return 1;
}

int coli_hip_set_fused_route(int mode) {
    if (mode < -1 || mode > 1) return fail("fused route mode must be -1, 0 or 1");
    g_fused_route.store(mode);
    return 1;
}

int coli_hip_set_profile(int on) {
    g_profile = on ? 1 : 0;
    return 1;
}

void coli_hip_kernel_stats(int which, uint64_t *launches, double *total_ms) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    const bool ok = which >= 0 && which < COLI_HIP_K_COUNT;
    if (launches) *launches = ok ? g_k_launches[which] : 0;
    if (total_ms) *total_ms = ok ? g_k_ms[which] : 0.0;
}

void coli_hip_reset_stats(void) {
    std::lock_guard<std::mutex> lock(g_stats_mu);
    g_calls = g_experts = g_rows = 0;
    g_h2d_ms = g_d2h_ms = 0;
    for (int i = 0; i < COLI_HIP_K_COUNT; i++) {
        g_k_launches[i] = 0;
        g_k_ms[i] = 0;
    }
}

int coli_hip_set_spin_limit(int polls) {
    if (polls < 0) return fail("spin limit must be >= 0");
    g_spin_limit = polls ? polls : GEMV_SPIN_LIMIT;
    return 1;
}

int coli_hip_set_debug_dots(int32_t *gateup_dev, int32_t *down_dev) {
    g_dbg_gu = gateup_dev;
    g_dbg_dn = down_dev;
    return 1;
}

int coli_hip_expert_set_create(ColiHipExpertSet **set, ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                               ColiHipTensor *const *downs, int count) {
    if (!set) return 0;
    int device = -1;
    MatGeom gg{}, gd{};
    if (!check_group(gates, ups, downs, count, &device, &gg, &gd)) return 0;
    Ctx *c = find_ctx(device);
    if (!select_ctx(c)) return 0;
    std::vector<ExpertDesc> hd((size_t)count);
    for (int i = 0; i < count; i++) {
        hd[i].w[0] = gates[i]->w;
        hd[i].w[1] = ups[i]->w;
        hd[i].w[2] = downs[i]->w;
        hd[i].sc[0] = gates[i]->sc;
        hd[i].sc[1] = ups[i]->sc;
        hd[i].sc[2] = downs[i]->sc;
    }
    ColiHipExpertSet *s = (ColiHipExpertSet *)std::calloc(1, sizeof(ColiHipExpertSet));
    if (!s) return 0;
    s->device = device;
    s->count = count;
    s->gg = gg;
    s->gd = gd;
    if (!hip_ok(hipMalloc(&s->desc_dev, sizeof(ExpertDesc) * count), "expert set allocation") ||
        !hip_ok(hipMemcpy(s->desc_dev, hd.data(), sizeof(ExpertDesc) * count, hipMemcpyHostToDevice),
                "expert set upload")) {
        if (s->desc_dev) hipFree(s->desc_dev);
        std::free(s);
        return 0;
    }
    *set = s;
    return 1;
}

void coli_hip_expert_set_free(ColiHipExpertSet *s) {
    if (!s) return;
    Ctx *c = find_ctx(s->device);
    if (c) select_ctx(c);
    if (s->desc_dev) hipFree(s->desc_dev);
    std::free(s);
}

int coli_hip_route_sigmoid_topk_dev(int device, const float *logits_dev, const float *bias_dev, int S, int E, int k,
                                    int norm_topk, float routed_scale, float min_share, int *ids_dev, float *w_dev,
                                    int *keff_dev) {
    Ctx *c = find_ctx(device);
    if (!logits_dev || !ids_dev || !w_dev || S < 1 || E < 1 || E > 1024 || k < 1 || k > 16 || k > E ||
        !select_ctx(c))
        return 0;
    launch_route_sigmoid(logits_dev, bias_dev, S, E, k, norm_topk, routed_scale, min_share, ids_dev, w_dev, keff_dev,
                         c->stream);
    return hip_ok(hipGetLastError(), "sigmoid router launch");
}

int coli_hip_route_softmax_topk_dev(int device, const float *logits_dev, int S, int E, int k, int *ids_dev,
                                    float *w_dev) {
    Ctx *c = find_ctx(device);
    if (!logits_dev || !ids_dev || !w_dev || S < 1 || E < 1 || E > 1024 || k < 1 || k > 16 || k > E || !select_ctx(c))
        return 0;
    launch_route_softmax(logits_dev, S, E, k, ids_dev, w_dev, c->stream);
    return hip_ok(hipGetLastError(), "router launch");
}

}  // extern "C"

namespace {

int moe_forward_impl(const ColiHipExpertSet *set, const float *x_dev, int S, const float *logits_dev, int *ids_dev,
                     float *w_dev, int k, float *out_dev, int ga, int arm, bool fixed_scratch = false) {
    if (!set || !x_dev || !ids_dev || !w_dev || !out_dev || S < 1 || k < 1) return 0;
    if (k > 16) return fail("moe_forward: k > 16 is not supported");
    if (set->count > 512) return fail("moe_forward: more than 512 experts");
    if (logits_dev && k > set->count) return fail("moe_forward: k > experts");
    if (ga != 0 && ga != 32) return fail("moe_forward: act group must be 0 or 32");
    Ctx *c = find_ctx(set->device);
    if (!select_ctx(c)) return 0;
    const int E = set->count, R = S * k;
    const int tmax = (R + MT_ROWS - 1) / MT_ROWS + std::min(E, R);
    if (arm < 0) arm = forced_arm();
    if (arm < 0) arm = S == 1 ? COLI_HIP_ARM_GEMV : COLI_HIP_ARM_MFMA;
    const MatGeom &gg = set->gg, &gd = set->gd;

    // table layout in one buffer
    const size_t n_int =
        4 + (size_t)E + (E + 1) + 3 * (size_t)R + 2 * (size_t)R + 4 * (size_t)tmax + table_work_ints(S, k, E);
    Scratch s{};
    int *p = nullptr;
    if (fixed_scratch) {
        // the whole dispatch's scratch carved out of the device's fixed array:
        // nothing is allocated, so sizes beyond it are refused
        if (!c->fixed_scratch) return fail("moe_forward (no allocation): the fixed scratch array is not mapped");
        size_t need = 0;
        if (!carve_rows(gg, gd, S, R, ga, nullptr, &need, &s)) return 0;
        const size_t tbl_off = need;
        need += round_up(n_int * 4, 256);
        if (need > COLI_HIP_FIXED_SCRATCH_BYTES) {
            std::fprintf(stderr,
                         "[HIP] moe_forward (no allocation): this call needs %zu bytes of scratch, more than the "
                         "fixed %d MiB\n",
                         need, COLI_HIP_FIXED_SCRATCH_BYTES >> 20);
            return 0;
        }
        carve_rows(gg, gd, S, R, ga, c->fixed_scratch, &need, &s);
        p = (int *)(c->fixed_scratch + tbl_off);
    } else {
        if (!reserve_rows(c, gg, gd, S, R, ga, &s) || !reserve(c, c->tbl, n_int * 4)) return 0;
        p = (int *)c->tbl.p;
    }
    TableOut t{};
    t.hdr = p;
    p += 4;
    t.uexp = p;
    p += E;
    t.off = p;
    p += E + 1;
    t.row_tok = p;
    p += R;
    t.row_kk = p;
    p += R;
    t.row_exp = p;
    p += R;
    t.tok_rows = p;
    p += R;
    t.tok_kk = p;
    p += R;
    t.mt_exp = p;
    p += tmax;
    t.mt_row0 = p;
    p += tmax;
    t.mt_rend = p;
    p += tmax;
    t.mt_first = p;
    p += tmax;
    int *tbl_work = p;
    c->tbl_view = t;
    c->tbl_E = E;
    c->tbl_R = R;

    Prof prof(c);
    if (fixed_scratch) prof.on = false;   // profiling creates events: not on the no-allocation path
    DispatchOpts opt;
    opt.w_reuse = R >= 2 * MT_ROWS * E;   // about two or more M tiles per expert
    const int act = epi_act(ga);
    // one token routes to k distinct experts in top-k order, which is also
    // batch-union order: row r is (token 0, slot r) and no table is needed
    // Ids from the router are always in range and distinct per token; ids
    // from the caller may not be (out-of-range ids are skipped, repeats keep
    // slot order), so those always go through the table.
    const bool one_token = S == 1 && arm == COLI_HIP_ARM_GEMV && logits_dev;
    ExpertDesc *rdesc = nullptr;
    if (one_token && logits_dev) {
        if (!reserve(c, c->rdesc, (size_t)k * sizeof(ExpertDesc))) return 0;
        rdesc = (ExpertDesc *)c->rdesc.p;
    }
    // fused router: worth it once the gate/up grid covers the chip (the
    // prologue costs every workgroup ~2 us; with few workgroups the separate
    // router launch, spread over many, is shorter)
    // split-K GEMV (not on the no-allocation path: its partials would need
    // more fixed scratch); a split gate/up has the router launched apart
    const int gu_wgs = k * ((gg.O + 31) / 32), fmode = fused_route_mode();
    const bool gemv_split = arm == COLI_HIP_ARM_GEMV && !fixed_scratch &&
                            plan_gemv_split(gg, true, R, act, gemv_split_target()).split > 1;
    if (logits_dev && one_token && E <= ROUTE_MAX_E && (fmode == 1 || (fmode == -1 && gu_wgs >= 256 && !gemv_split))) {
        // the gate/up GEMV routes and quantises the token itself
        opt.route = RouteArgs{logits_dev, E, k, ids_dev, w_dev, rdesc, x_dev, gg.K, gg.Kp, act};
        opt.x_quantized = true;
    } else if (logits_dev) {
        QuantArgs qa{x_dev, gg.K, S, gg.K, gg.Kp, s.xq, s.xs, s.sx, s.sxs, act};
        prof.mark(COLI_HIP_K_QUANT_X);
        launch_route_quant(logits_dev, S, E, k, ids_dev, w_dev, qa, set->desc_dev, rdesc, c->stream);
        opt.x_quantized = true;
    }
    // one token: the down GEMV also applies the router weights (one launch
    // fewer) when the k activation rows fit its LDS
    if (arm == COLI_HIP_ARM_GEMV && !fixed_scratch && !plan_split(c, gg, gd, R, act, opt.route.logits, &opt)) return 0;
    const bool fuse_dc = one_token && fused_combine_on(k, opt.split_dn.split > 1) && !g_dbg_dn &&
                         gemv_down_combine_ok(gd, k);
    if (fuse_dc) {
        opt.combine_w = w_dev;
        opt.combine_out = out_dev;
    }
    // otherwise, one token: the down GEMV's tail does the combine
    const bool tail_c = one_token && !fuse_dc && tail_combine_on() && !g_dbg_dn && k <= GEMV_TAIL_MAXK &&
                        (gd.O + 63) / 64 <= GEMV_TAIL_TILES;
    if (tail_c) {
        opt.tail_w = w_dev;
        opt.tail_out = out_dev;
        opt.tail_ctr = c->tail_ctr;
    }
    RowPlan plan{};
    if (one_token) {
        c->tbl_view.hdr = nullptr;
        plan.row_desc = rdesc;
        plan.row_exp = ids_dev;
        plan.row_act = ids_dev;   // unused (act_zero)
        plan.counts = ids_dev;    // unused (n_rows_fixed)
        opt.act_zero = true;
        opt.n_rows_fixed = k;
    } else {
        prof.mark(COLI_HIP_K_TABLE);
        launch_build_table(ids_dev, S, k, E, t, tmax, tbl_work, c->stream);
        plan.row_exp = t.row_exp;
        plan.row_act = t.row_tok;
        plan.mt_exp = t.mt_exp;
        plan.mt_row0 = t.mt_row0;
        plan.mt_rend = t.mt_rend;
        plan.mt_first = t.mt_first;
        plan.counts = t.hdr;
    }
    run_experts(c, prof, set->desc_dev, plan, gg, gd, x_dev, S, false, R, tmax, ga, arm, s, opt);
    prof.mark(COLI_HIP_K_COMBINE);
    if (fuse_dc || tail_c) {
        // combined by the down GEMV
    } else if (one_token) {   // rows 0..k-1 of token 0, in top-k order
        launch_combine_tok(out_dev, s.y, nullptr, nullptr, w_dev, 1, k, gd.O, s.ys, c->stream);
    }
    else
        launch_combine_tok(out_dev, s.y, t.tok_rows, t.tok_kk, w_dev, S, k, gd.O, s.ys, c->stream);
    prof.mark(-1);
    if (!hip_ok(hipGetLastError(), "moe forward launch")) return 0;
    prof.finish();
    note_group(E, R);
    return 1;
}

}  // namespace

extern "C" {

int coli_hip_moe_forward_dev(const ColiHipExpertSet *set, const float *x_dev, int S, const int *ids_dev,
                             const float *w_dev, int k, float *out_dev, int ga, int arm) {
    return moe_forward_impl(set, x_dev, S, nullptr, (int *)ids_dev, (float *)w_dev, k, out_dev, ga, arm);
}

int coli_hip_moe_forward_dev_noalloc(const ColiHipExpertSet *set, const float *x_dev, int S, const int *ids_dev,
                                     const float *w_dev, int k, float *out_dev, int ga, int arm) {
    return moe_forward_impl(set, x_dev, S, nullptr, (int *)ids_dev, (float *)w_dev, k, out_dev, ga, arm, true);
}

int coli_hip_moe_forward_logits_dev(const ColiHipExpertSet *set, const float *x_dev, int S, const float *logits_dev,
                                    int k, int *ids_dev, float *w_dev, float *out_dev, int ga, int arm) {
    if (!logits_dev) return 0;
    return moe_forward_impl(set, x_dev, S, logits_dev, ids_dev, w_dev, k, out_dev, ga, arm);
}

void *coli_hip_stream(int device) {
    Ctx *c = find_ctx(device);
    return c ? (void *)c->stream : nullptr;
}

int coli_hip_last_table(int device, int *hdr, int *uexp, int *off, int *row_tok, int *tok_rows, int e_cap,
                        int r_cap) {
    Ctx *c = find_ctx(device);
    if (!select_ctx(c) || !c->tbl_view.hdr) return fail("last_table: the last dispatch built no table");
    const TableOut &t = c->tbl_view;
    if (!hip_ok(hipStreamSynchronize(c->stream), "table sync")) return 0;
    const int E = std::min(c->tbl_E, e_cap), R = std::min(c->tbl_R, r_cap);
    int ok = 1;
    if (hdr) ok &= hip_ok(hipMemcpy(hdr, t.hdr, 16, hipMemcpyDeviceToHost), "table copy");
    if (uexp) ok &= hip_ok(hipMemcpy(uexp, t.uexp, (size_t)E * 4, hipMemcpyDeviceToHost), "table copy");
    if (off) ok &= hip_ok(hipMemcpy(off, t.off, (size_t)(E + 1) * 4, hipMemcpyDeviceToHost), "table copy");
    if (row_tok) ok &= hip_ok(hipMemcpy(row_tok, t.row_tok, (size_t)R * 4, hipMemcpyDeviceToHost), "table copy");
    if (tok_rows) ok &= hip_ok(hipMemcpy(tok_rows, t.tok_rows, (size_t)R * 4, hipMemcpyDeviceToHost), "table copy");
    return ok;
}

}  // extern "C"
