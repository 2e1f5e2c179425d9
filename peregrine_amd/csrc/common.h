// common.h — shared device helpers and launch structures of libperegrine_hip.
//
// Arithmetic contract (identical to oracle/oracle.c, which restates
// peregrine-kernels): every per-block integer dot is exact; every fp32
// epilogue is evaluated in the same order with the same roundings. The whole
// library is compiled with -ffp-contract=off so a*b+c never silently fuses.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "expf_glibc.h"

namespace phip {

// Dynamic LDS above 64 KB needs an explicit opt-in, per kernel and per
// device. `opted` is the caller's per-kernel table, indexed by device.
constexpr int LDS_OPT_DEVICES = 64;
inline void lds_opt_in(const void *kern, size_t lds, size_t (&opted)[LDS_OPT_DEVICES]) {
    if (lds <= 64 * 1024) return;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= LDS_OPT_DEVICES) return;
    if (lds > opted[dev] &&
        hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess)
        opted[dev] = lds;
}

// ---- activation scale granularity ("act group") ----
// ACT_ROW: one scale per row (qrow_i8, peregrine-kernels/src/quant.rs:14-33).
// ACT_B32: one scale per 32-element block (BASELINE extension).
enum ActMode { ACT_ROW = 0, ACT_B32 = 1 };

// ---- epilogue kinds (how int32 block dots become f32) ----
//  EPI_ROW   per-row weight scale: D = sum of all block dots (exact int),
//            y = ((f32)D * sc) * sx                   (matmul.rs:61-87)
//  EPI_GRP   grouped weight scale, row act scale:
//            acc = acc + sw[g]*(f32)d_g ; y = acc*sx   (matmul.rs:93-106)
//  EPI_B32   32-block act scale (any weight grouping):
//            acc = fmaf(sw(b)*sx[b], (f32)d_b, acc)   (BASELINE extension)
enum Epi { EPI_ROW = 0, EPI_GRP = 1, EPI_B32 = 2 };

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 128-/64-bit streaming loads (weights are read once per dispatch).
__device__ __forceinline__ uint4 ldg_stream4(const void *p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg_stream2(const void *p) {
    const u32x2 v = __builtin_nontemporal_load((const u32x2 *)p);
    return make_uint2(v.x, v.y);
}

// The same through global-address-space pointers: global (not flat) loads,
// which count only against vmcnt, so LDS waits never wait on them.
typedef const __attribute__((address_space(1))) uint8_t GU8;
typedef const __attribute__((address_space(1))) float GF32;
__device__ __forceinline__ uint4 ldg_stream4g(GU8 *p) {
    const u32x4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ldg_stream2g(GU8 *p) {
    const u32x2 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) u32x2 *)p);
    return make_uint2(v.x, v.y);
}

constexpr int TILE_O = 32;     // rows of a weight tile in the device layout
constexpr int BLK = 32;        // K elements per block (one MFMA K step)
constexpr int MT_ROWS = 32;    // rows of one M tile of the grouped GEMM

// One expert's three resident tensors as the kernels see them.
// Weights are tiled [Op/32][nb][32][BB] (BB = 16 bytes int4, 32 bytes int8);
// scales are tiled [Op/32][ng][32] f32. One tile is the contiguous stream a
// GEMV half-wave reads; Op is padded to 64 so tiles come in pairs.
struct ExpertDesc {
    const uint8_t *w[3];   // gate, up, down
    const float *sc[3];
};

// Per-matrix geometry shared by every expert of a call.
struct MatGeom {
    int K, Kp, nb;         // inputs, inputs padded to 32, blocks
    int O, Op;             // outputs, outputs padded to 64
    int gpb, ng;           // blocks per weight group, groups (per-row: gpb = nb, ng = 1)
    int gshift;            // log2(gpb) for grouped weights; 30 for per-row (every block maps to group 0)
    int w4;                // 1: int4 weights, 0: int8
    int per_row;           // weight scale per row
};

// Row bookkeeping of one MoE dispatch (device arrays).
struct RowPlan {
    const int *row_exp;    // [R] descriptor index of row r
    const int *row_act;    // [R] activation row of row r
    const int *mt_exp;     // [T] M-tile -> descriptor index
    const int *mt_row0;    // [T] first row of the tile
    const int *mt_rend;    // [T] one past the last row of that expert
    const int *mt_first;   // [T] the first M tile of that expert (its tiles are consecutive)
    const int *counts;     // [2] {R, T} as built on the device (or host)
    const ExpertDesc *row_desc;  // optional [R]: row r's descriptor, written by the router
};

// ---- device helpers ----

// Address-space hints: pointers read from descriptor tables are generic; cast
// them so loads are emitted as global (not flat) memory operations.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T *gptr(const T *p) {
    return (const __attribute__((address_space(1))) T *)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(1))) T *gptr_w(T *p) {
    return (__attribute__((address_space(1))) T *)p;
}

// Buffer-resource loads: a uniform descriptor (base, byte range) in SGPRs, a
// 32-bit per-lane offset and a uniform 32-bit offset. No 64-bit address math
// per load, and reads past the range return zero instead of faulting.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000);
}
// Weight streams are read once per pass: the loads carry the non-temporal
// hint (cache-policy bit 1), which on gfx950 doubles the rate of a streaming
// read against plain loads that allocate in the caches.
constexpr int BUF_NT = 2;
// Cache-policy bit SC1 (device scope on gfx942/gfx950): the same encoding the
// compiler gives agent-scope atomic loads and stores, i.e. coherent across
// the XCDs' L2s, but as plain operations the compiler may batch.
constexpr int BUF_SC1 = 16;
__device__ __forceinline__ uint4 bload16(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, BUF_NT);
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ float bloadf(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, BUF_NT));
}

// Read-only views in the constant address space: uniform loads through them
// become scalar loads (reads only).
typedef const __attribute__((address_space(4))) int CInt;
typedef const __attribute__((address_space(4))) float CFloat;

// Index of the wavefront in its workgroup, known to the compiler as uniform.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Weight group of block b and whether b closes its group.
__device__ __forceinline__ int grp_of(int b, int gshift) { return gshift >= 30 ? 0 : b >> gshift; }
__device__ __forceinline__ bool grp_end(int b, int gshift, int nb) {
    return b + 1 == nb || (gshift < 30 && ((b + 1) & ((1 << gshift) - 1)) == 0);
}

// siluf(x) * u — peregrine-model/src/math.rs:108-118 (division correctly
// rounded; exp with glibc expf's results, as Rust's f32::exp on Linux).
__device__ __forceinline__ float silu_mul(float g, float u) {
    float den = __fadd_rn(1.0f, expf_glibc(-g));
    return __fmul_rn(__fdiv_rn(g, den), u);
}

// Byte position of element k inside its 8-element group in the device
// activation layout: even elements first, then odd (0,2,4,6,1,3,5,7). This is
// the order the int4 unpack below produces from QT nibble pairs.
__device__ __forceinline__ int perm8(int k) { return (k & ~7) | ((k & 1) << 2) | ((k & 7) >> 1); }

// int4 QT dword (two's-complement nibbles after the upload XOR) -> two dwords
// of int8 values scaled by 16: even elements and odd elements.
__device__ __forceinline__ int i4_even16(uint32_t w) { return (int)((w << 4) & 0xF0F0F0F0u); }
__device__ __forceinline__ int i4_odd16(uint32_t w) { return (int)(w & 0xF0F0F0F0u); }

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// 32-block dot, int4 weights: 16 bytes of weights against 8 dwords of the
// permuted activation block. Returns 16 * the exact dot.
__device__ __forceinline__ int dot_blk_w4(uint4 w, const int *x) {
    int acc = 0;
    acc = sdot4(i4_even16(w.x), x[0], acc);
    acc = sdot4(i4_odd16(w.x), x[1], acc);
    acc = sdot4(i4_even16(w.y), x[2], acc);
    acc = sdot4(i4_odd16(w.y), x[3], acc);
    acc = sdot4(i4_even16(w.z), x[4], acc);
    acc = sdot4(i4_odd16(w.z), x[5], acc);
    acc = sdot4(i4_even16(w.w), x[6], acc);
    acc = sdot4(i4_odd16(w.w), x[7], acc);
    return acc;
}

// 32-block dot, int8 weights already in the permuted order. Exact dot.
__device__ __forceinline__ int dot_blk_w8(uint4 a, uint4 b, const int *x) {
    int acc = 0;
    acc = sdot4((int)a.x, x[0], acc);
    acc = sdot4((int)a.y, x[1], acc);
    acc = sdot4((int)a.z, x[2], acc);
    acc = sdot4((int)a.w, x[3], acc);
    acc = sdot4((int)b.x, x[4], acc);
    acc = sdot4((int)b.y, x[5], acc);
    acc = sdot4((int)b.z, x[6], acc);
    acc = sdot4((int)b.w, x[7], acc);
    return acc;
}

template <typename T>
__device__ __forceinline__ T warp_max(T v, int width) {
    for (int off = width >> 1; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, width));
    return v;
}

}  // namespace phip

// ---- host-side launchers (defined in the kernel translation units) ----
namespace phip {
// Kernel timing under profiling: the runtime arms a (start, stop) event pair
// for a kernel slot; the slot's first launch records `start` and every launch
// records `stop` inside its own dispatch packet (hipExtLaunchKernelGGL), so
// the elapsed time is the kernels' execution alone, as a profiler's kernel
// trace measures it, with no marker packets between them.
struct LaunchTiming {
    hipEvent_t start = nullptr, stop = nullptr;
    bool used = false;
};
extern thread_local LaunchTiming g_launch_timing;
template <typename K, typename... Args>
inline void launch_k(K kern, dim3 grid, dim3 block, size_t lds, hipStream_t st, Args... args) {
    LaunchTiming &t = g_launch_timing;
    if (t.stop) {
        hipExtLaunchKernelGGL(kern, grid, block, (uint32_t)lds, st, t.used ? nullptr : t.start, t.stop, 0u, args...);
        t.used = true;
    } else {
        hipLaunchKernelGGL(kern, grid, block, lds, st, args...);
    }
}

struct QuantArgs {
    const float *x; int x_stride; int rows; int K; int Kp;
    int8_t *q; int q_stride; float *s; int s_stride; int mode;
    // optional: the workgroups also copy n16 16-byte words src -> dst (a
    // host-buffer call's metadata, staged from mapped host memory)
    const uint4 *copy_src; uint4 *copy_dst; int copy_n16;
};
void launch_quant_rows(const QuantArgs &a, hipStream_t st);

void launch_repack(const uint8_t *raw, const float *raw_sc, int fmt, int I, int O, int gs, uint8_t *w, float *sc,
                   const MatGeom &g, hipStream_t st);

// One-token decode: the gate/up GEMV routes the token and quantises its
// activation row itself (every workgroup redundantly, no grid-wide wait), so
// the expert weights start streaming without a separate router launch.
struct RouteArgs {
    const float *logits; int E; int k;          // logits [E]; greedy top-k, softmax weights
    int *ids; float *w; ExpertDesc *row_desc;   // [k] outputs, written by workgroup (0, 0)
    const float *x; int K; int Kp; int mode;    // activation row f32 [K] -> DotArgs.xq / .sx (mode: ACT_*)
};
constexpr int ROUTE_MAX_E = 256;   // 4 logits per lane

struct DotArgs {   // shared by the GEMV and MFMA arms
    const ExpertDesc *desc;
    RowPlan plan;
    const int8_t *xq; int x_stride; const float *sx; int sx_stride;   // activations
    float *out; int out_stride;                                         // h (gate/up) or y (down)
    int8_t *hq; int hq_stride; float *sh; int sh_stride;                // fused h quant (ACT_B32)
    int32_t *dots;                                                      // optional per-block dot dump
    int act_identity;                                                   // activation row = r (down proj)
    int act_zero;                                                       // activation row = 0 (one token)
    int n_rows_fixed;                                                   // >= 0: row count known on the host
    int spin_limit;                                                     // GEMV: polls before a bounded wait gives up
    int *wait_failed;                                                   // GEMV: host-visible word, set to 1 when one does
    int w_reuse;                                                        // MFMA arm: M tiles re-read each expert's weights
    RouteArgs route;                                                    // gate/up GEMV: logits != null -> fused router
    // down GEMV, one token (rows 0..n-1 in top-k order): the last workgroup
    // to finish an output tile also writes tail_out over that tile, the
    // router-weighted sum of the rows in row order (the combine's order);
    // tail_ctr holds one arrival counter per tile, zero between dispatches
    float *tail_out;
    const float *tail_w;
    int *tail_ctr;
    // split-K GEMV (split > 1): each (row, output tile) unit's K blocks are
    // spread over `split` workgroups of split_kb blocks each; they park their
    // exact block dots and f32 factors in part_d / part_f and count in on
    // split_ctr[unit] (zero between dispatches); the last to arrive runs the
    // unit's ascending f32 chain and its epilogue
    int split, split_kb, split_nw;
    int32_t *part_d;
    float *part_f;
    int *split_ctr;
};
// output tiles the tail counters cover (down GEMV tiles are 64 channels)
constexpr int GEMV_TAIL_TILES = 4096;
constexpr int GEMV_TAIL_MAXK = 16;
// split-K GEMV: arrival counters (units = rows x output tiles) and the most
// blocks one wave of the finishing workgroup holds for the chain
constexpr int GEMV_SPLIT_UNITS = 16384;
constexpr int GEMV_SPLIT_SEG = 24;
// Split-K plan of one GEMV launch: 0 = the unsplit kernel. Fills split /
// split_kb of a DotArgs and returns the partial-buffer bytes it needs.
struct GemvSplit {
    int split = 0, kb = 0, nw = 0, ch = 0;
    size_t part_d_bytes = 0, part_f_bytes = 0;
};
GemvSplit plan_gemv_split(const MatGeom &g, bool gateup, int rows, int act, int target_wgs);
// grid_rows / grid_tiles: host-side upper bounds; the kernels read the true
// counts from plan.counts and idle the excess workgroups.
void launch_gemv_gateup(const DotArgs &a, const MatGeom &g, int act, int grid_rows, hipStream_t st);
void launch_gemv_down(const DotArgs &a, const MatGeom &g, int act, int grid_rows, hipStream_t st);
void launch_mfma_gateup(const DotArgs &a, const MatGeom &g, int act, int grid_tiles, hipStream_t st);
void launch_mfma_down(const DotArgs &a, const MatGeom &g, int act, int grid_tiles, hipStream_t st);

void launch_combine(float *out, const float *y, const int *row_ptr, const int *row_idx, const float *rw,
                    int s_n, int D, int y_stride, hipStream_t st);
void launch_combine_tok(float *out, const float *y, const int *tok_rows, const int *tok_kk, const float *w, int s_n,
                        int k, int D, int y_stride, hipStream_t st);
void launch_route_softmax(const float *logits, int S, int E, int k, int *ids, float *w, hipStream_t st);
void launch_route_sigmoid(const float *logits, const float *bias, int S, int E, int k, int norm_topk,
                          float routed_scale, float min_share, int *ids, float *w, int *keff, hipStream_t st);
void launch_route_quant(const float *logits, int S, int E, int k, int *ids, float *w, const QuantArgs &a,
                        const ExpertDesc *desc, ExpertDesc *row_desc, hipStream_t st);
// Polls a GEMV's bounded wait makes before it gives up (the default; a test
// hook may lower it). 2^22 polls of >= 64 clocks each: ~0.1 s at 2.4 GHz.
constexpr int GEMV_SPIN_LIMIT = 1 << 22;
// LDS bytes one workgroup may use (device attribute), set at init.
void set_lds_limit(int bytes);
// one token: down GEMV + router-weighted combine in one launch (k rows in top-k order)
bool gemv_down_combine_ok(const MatGeom &g, int k);
void launch_gemv_down_combine(const DotArgs &a, const MatGeom &g, int act, int k, const float *w, float *out,
                              hipStream_t st);

struct TableOut {
    int *hdr;          // [4]: R, T, n_u, flags
    int *uexp, *off;   // [E], [E+1]
    int *row_tok, *row_kk, *row_exp;  // [R]
    int *tok_rows, *tok_kk;           // [S*k]: each token's rows in union order (-1 pads), their top-k slot
    int *mt_exp, *mt_row0, *mt_rend, *mt_first;  // [Tmax]
};
void launch_synth_fill(void *dst, size_t n, int kind, float a, float b, uint64_t seed, hipStream_t st);
// work: table_work_ints(S, k, E) ints of device scratch, fully rewritten by every call
size_t table_work_ints(int S, int k, int E);
void launch_build_table(const int *ids, int S, int k, int E, const TableOut &t, int tmax, int *work,
                        hipStream_t st);
}  // namespace phip
