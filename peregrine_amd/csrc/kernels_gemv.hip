// kernels_gemv.hip — the decode arm: one token row against one expert's
// weights, one output channel per lane.
//
// Layout of a workgroup (NW wavefronts):
//   gate/up: 32 output channels; lanes 0-31 run the gate rows, lanes 32-63 the
//            up rows of the same channels, so SwiGLU is a cross-lane read.
//   down:    64 output channels, one per lane.
//   K (the 32-blocks of the input) is cut into NW segments, one per wave, so
//   a workgroup streams its weight rows with NW waves in flight.
//
// Exact order: each wave turns its blocks into per-block f32 terms held in
// registers; the accumulator then walks the waves in segment order through
// LDS (wave 0's blocks first), so every output sees the same left-to-right
// f32 chain as oracle/oracle.c (peregrine-kernels/src/idot.rs:82-88). Integer
// dots are exact whatever the split.
//
// Memory: every weight byte is read once with 128-bit coalesced loads (64
// lanes x 16 B = one 1 KB tile row per block); the activation block (32 B) is
// the same for every lane.
#include <cstdlib>

#include "common.h"

namespace phip {

template <bool W4>
struct WBlk;
template <>
struct WBlk<true> {
    uint4 a;
};
template <>
struct WBlk<false> {
    uint4 a, b;
};

template <bool W4>
__device__ __forceinline__ WBlk<W4> load_wblk(const uint8_t *p) {
    WBlk<W4> r;
    r.a = ldg_stream4(p);
    if constexpr (!W4) r.b = ldg_stream4(p + 16);
    return r;
}

template <bool W4>
__device__ __forceinline__ int dot_wblk(const WBlk<W4> &w, const int *x) {
    if constexpr (W4)
        return dot_blk_w4(w.a, x);
    else
        return dot_blk_w8(w.a, w.b, x);
}

// Workgroup of NW streaming waves plus one chain wave over one tile (32 gate
// + 32 up channels, or 64 down channels) of one row. K is walked in rounds of
// NW*CH blocks; in round c streaming wave w owns the CH consecutive blocks
// c*NW*CH + w*CH + [0, CH). Streaming waves keep two chunks of weights in
// flight (unconditional loads, so the wait counts are exact), turn each block
// into its epilogue inputs — the integer dot (int16 for int4 weights, whose
// 32-block dots fit in 16 bits; int32 for int8) and an f32 factor (c = sw*sx[b]
// for 32-block activation scales, sw for grouped weights) — and park them in
// an LDS ring of RING rounds. The chain wave walks each finished round in
// ascending block order with the oracle's exact f32 chain while later rounds
// stream; a streaming wave waits only when it is RING rounds ahead of the
// chain. Per-row weight scales only sum integers. All waits are bounded.
template <bool W4>
struct DStore;
template <>
struct DStore<true> {
    typedef short T;
};
template <>
struct DStore<false> {
    typedef int T;
};

constexpr int GEMV_CH = 4;            // blocks per chunk (per streaming wave per round)
constexpr int GEMV_RING = 2;          // rounds of epilogue inputs held in LDS
constexpr int GEMV_SPIN_LIMIT = 1 << 22;

__device__ __forceinline__ void spin_until_geq(int *ctr, int target) {
    for (int spin = 0; spin < GEMV_SPIN_LIMIT; ++spin) {
        if (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
        __builtin_amdgcn_s_sleep(1);
    }
}

template <bool W4, int EPI, bool GATEUP, int NW, bool BUF>
__global__ __launch_bounds__((NW + 1) * 64) void gemv_kernel(DotArgs a, MatGeom g, const int8_t *__restrict__ xq,
                                                             const float *__restrict__ sxv) {
    constexpr int BB = W4 ? 16 : 32;
    constexpr int CH = GEMV_CH;
    constexpr int RB = NW * CH;                  // blocks per round
    constexpr int SLOT = RB * 64;                // entries per ring slot
    typedef typename DStore<W4>::T DT;
    extern __shared__ float lds_f[];   // [RING][RB][64] f32 factors, [RING][RB][64] dots, activation row
    __shared__ int produced[GEMV_RING];          // per slot: streaming waves done (cumulative)
    __shared__ int consumed;                     // rounds the chain wave has finished

    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const bool chainer = wave == NW;
    const int r = blockIdx.y;
#ifdef PHIP_GEMV_TRACE
    long long tr[6] = {0, 0, 0, 0, 0, 0};
    const bool tracing = a.trace != nullptr && chainer;
#else
    long long tr[6];
    constexpr bool tracing = false;
#endif
    if (tracing) tr[0] = trace_stamp();
    const int nrows = a.n_rows_fixed >= 0 ? a.n_rows_fixed : a.plan.counts[0];
    if (r >= nrows) return;  // uniform: fewer rows than the grid bound

    // the router may have copied this row's descriptor already (one load
    // instead of row -> expert id -> descriptor)
    const ExpertDesc *dsc = a.plan.row_desc ? &a.plan.row_desc[r] : &a.desc[a.plan.row_exp[r]];
    const int arow = a.act_identity ? r : (a.act_zero ? 0 : a.plan.row_act[r]);
    const int mat = GATEUP ? (lane >> 5) : 2;
    const int o = GATEUP ? (int)blockIdx.x * 32 + (lane & 31) : (int)blockIdx.x * 64 + lane;
    const int t = GATEUP ? (int)blockIdx.x >> 1 : (int)blockIdx.x;   // 64-row weight tile (uniform)
    const int ol = o & 63;
    // Weights of this row tile: [nb][64][BB]; scales [ng][64]. BUF: one buffer
    // descriptor spans the gate and up tiles (the host checked they lie within
    // 2 GB of each other), the up lanes carry the distance in their 32-bit
    // offset. Otherwise 64-bit global addresses.
    const uint32_t wtile = (uint32_t)g.nb * TILE_O * BB, stile = (uint32_t)g.ng * TILE_O * 4;
    const int m0 = GATEUP ? 0 : 2;
    const uint8_t *wt0 = dsc->w[m0] + (size_t)t * wtile;
    const uint8_t *wt1 = GATEUP ? dsc->w[1] + (size_t)t * wtile : wt0;
    const uint8_t *st0 = (const uint8_t *)dsc->sc[m0] + (size_t)t * stile;
    const uint8_t *st1 = GATEUP ? (const uint8_t *)dsc->sc[1] + (size_t)t * stile : st0;
    const uint8_t *wlo = wt0 < wt1 ? wt0 : wt1, *slo = st0 < st1 ? st0 : st1;
    const uint8_t *wmine = mat == 1 ? wt1 : wt0, *smine = mat == 1 ? st1 : st0;
    const __amdgpu_buffer_rsrc_t rw =
        make_rsrc(wlo, (uint32_t)((wt0 < wt1 ? wt1 - wt0 : wt0 - wt1) + wtile));
    const __amdgpu_buffer_rsrc_t rs =
        make_rsrc(slo, (uint32_t)((st0 < st1 ? st1 - st0 : st0 - st1) + stile));
    const int lw = (int)(wmine - wlo) + ol * BB, ls = (int)(smine - slo) + ol * 4;   // per-lane offsets
    const auto *wg64 = gptr(wmine + ol * BB);                                        // !BUF path
    const auto *sg64 = gptr((const float *)(smine + ol * 4));
    const auto *sbase = gptr(dsc->sc[mat] + (size_t)t * g.ng * TILE_O + ol);
    const int8_t *xg = xq + (size_t)arow * a.x_stride;
    const float *sx = sxv + (size_t)arow * a.sx_stride;
    DT *lds_d = (DT *)(lds_f + (size_t)GEMV_RING * SLOT);
    int *lds_x = (int *)(lds_d + (size_t)GEMV_RING * SLOT);   // the activation row, Kp bytes

    const int nb = g.nb;
    const int nrounds = (nb + RB - 1) / RB;
    WBlk<W4> w0[CH], w1[CH], w2[CH];
    float s0[CH], s1[CH], s2[CH];
    auto load_chunk = [&](int c, WBlk<W4> (&wv)[CH], float (&sv)[CH]) {
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int b = min(c * RB + wave * CH + j, nb - 1);
            const int sw_off = b * TILE_O * BB, sg = grp_of(b, g.gshift);
            if constexpr (BUF) {
                wv[j].a = bload16(rw, lw, sw_off);
                if constexpr (!W4) wv[j].b = bload16(rw, lw + 16, sw_off);
                if constexpr (EPI != EPI_ROW) sv[j] = bloadf(rs, ls, sg * TILE_O * 4);
            } else {
                wv[j] = load_wblk<W4>((const uint8_t *)(wg64 + (size_t)sw_off));
                if constexpr (EPI != EPI_ROW) sv[j] = sg64[(size_t)sg * TILE_O];
            }
        }
    };
    auto compute_chunk = [&](int c, const WBlk<W4> (&wv)[CH], const float (&sv)[CH]) {
        // the ring slot of round c is free once the chain finished round c - RING
        if (c >= GEMV_RING) spin_until_geq(&consumed, c - GEMV_RING + 1);
        const int slot = (c % GEMV_RING) * SLOT;
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int bi = wave * CH + j;      // block within the round
            const int b = c * RB + bi;
            if (b < nb) {
                const int4 *xb = (const int4 *)(lds_x + b * (BLK / 4));
                const int4 xa = xb[0], xc = xb[1];
                const int xv[8] = {xa.x, xa.y, xa.z, xa.w, xc.x, xc.y, xc.z, xc.w};
                const int d16 = dot_wblk<W4>(wv[j], xv);
                const int d = W4 ? (d16 >> 4) : d16;   // exact block dot
                if constexpr (EPI != EPI_ROW) {
                    // W4 scale tables hold sw/16; x16 is exact
                    const float sw = W4 ? __fmul_rn(sv[j], 16.0f) : sv[j];
                    lds_f[slot + bi * 64 + lane] = EPI == EPI_B32 ? __fmul_rn(sw, sx[b]) : sw;
                }
                lds_d[slot + bi * 64 + lane] = (DT)d;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0)
            __hip_atomic_fetch_add(&produced[c % GEMV_RING], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    };

    if (threadIdx.x < GEMV_RING) produced[threadIdx.x] = 0;
    if (threadIdx.x == 0) consumed = 0;
    if (!chainer) {
        load_chunk(0, w0, s0);
        load_chunk(min(1, nrounds - 1), w1, s1);
    }
    {   // stage the activation row in LDS while the first weights are in flight
        const int nwd = g.Kp / 4;
        for (int i = threadIdx.x; i < nwd; i += (NW + 1) * 64) lds_x[i] = ((const int *)xg)[i];
    }
    __syncthreads();
    if (tracing) tr[1] = trace_stamp();

    float facc = 0.0f;   // chain accumulator (chain wave)
    int gsum = 0;        // EPI_GRP: open group's integer sum
    int isum = 0;        // EPI_ROW: exact integer sum
    if (!chainer) {
        // three buffers rotate through a runtime loop; every load is
        // unconditional (clamped to the last block), so the wait counts stay
        // exact and no address is precomputed for all rounds
#pragma unroll 1
        for (int c = 0; c < nrounds; c += 3) {
            load_chunk(min(c + 2, nrounds - 1), w2, s2);
            compute_chunk(c, w0, s0);
            load_chunk(min(c + 3, nrounds - 1), w0, s0);
            if (c + 1 < nrounds) compute_chunk(c + 1, w1, s1);
            load_chunk(min(c + 4, nrounds - 1), w1, s1);
            if (c + 2 < nrounds) compute_chunk(c + 2, w2, s2);
        }
    } else {
#pragma unroll 1
        for (int c = 0; c < nrounds; ++c) {
            spin_until_geq(&produced[c % GEMV_RING], NW * (c / GEMV_RING + 1));
            const int slot = (c % GEMV_RING) * SLOT;
            const int lo = c * RB, hi = min(nb, lo + RB);
            for (int b8 = lo; b8 < hi; b8 += 16) {
                int dd[16];
                float ff[16];
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    const int bi = min(b8 + q, hi - 1) - lo;
                    dd[q] = (int)lds_d[slot + bi * 64 + lane];
                    ff[q] = EPI == EPI_ROW ? 0.0f : lds_f[slot + bi * 64 + lane];
                }
#pragma unroll
                for (int q = 0; q < 16; ++q) {
                    if (b8 + q < hi) {
                        const int b = b8 + q;
                        const int d = dd[q];
                        if (a.dots && o < g.O)
                            a.dots[(((size_t)r * (GATEUP ? 2 : 1) + (GATEUP ? mat : 0)) * g.O + o) * g.nb + b] = d;
                        if constexpr (EPI == EPI_ROW) {
                            isum += d;
                        } else if constexpr (EPI == EPI_B32) {
                            facc = __fmaf_rn(ff[q], (float)d, facc);
                        } else {
                            gsum += d;
                            if (grp_end(b, g.gshift, g.nb)) {
                                facc = __fadd_rn(facc, __fmul_rn((float)gsum, ff[q]));
                                gsum = 0;
                            }
                        }
                    }
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_store(&consumed, c + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }
    if (tracing) tr[2] = tr[3] = tr[4] = trace_stamp();

    if (!chainer) return;
    float v;
    if constexpr (EPI == EPI_ROW) {
        const float sc = W4 ? __fmul_rn(sbase[0], 16.0f) : sbase[0];
        v = __fmul_rn(__fmul_rn((float)isum, sc), sx[0]);
    } else if constexpr (EPI == EPI_GRP) {
        v = __fmul_rn(facc, sx[0]);
    } else {
        v = facc;
    }
    if constexpr (GATEUP) {
        const float u = __shfl(v, (lane & 31) + 32);
        if (lane < 32) {
            const float h = silu_mul(v, u);
            a.out[(size_t)r * a.out_stride + o] = h;
            if (EPI == EPI_B32 && a.hq) {
                const float m = warp_max(fabsf(h), 32);
                float sc = __fdiv_rn(m, 127.0f);
                if (sc < 1e-12f) sc = 1e-12f;
                const float inv = __fdiv_rn(1.0f, sc);
                a.hq[(size_t)r * a.hq_stride + perm8(o)] = (int8_t)(int)rintf(__fmul_rn(h, inv));
                if ((lane & 31) == 0) a.sh[(size_t)r * a.sh_stride + (o >> 5)] = sc;
            }
        }
    } else {
        if (o < g.O) a.out[(size_t)r * a.out_stride + o] = v;
    }
    if (tracing) {
        tr[5] = trace_stamp();
        if (lane == 0) {
            long long *dst = a.trace + ((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 8;
            for (int i = 0; i < 6; ++i) dst[i] = tr[i];
            dst[6] = (long long)__smid();
        }
    }
}

static int g_lds_limit = 64 * 1024;
void set_lds_limit(int bytes) { g_lds_limit = bytes > 0 ? bytes : 64 * 1024; }

// gate/up: 7 streaming waves + 1 chain wave (512 threads); down: 3 + 1.
template <bool W4, int EPI, bool GATEUP, bool BUF>
static void launch_gemv_b(const DotArgs &a, const MatGeom &g, int grid_rows, hipStream_t st) {
    constexpr int NW = GATEUP ? 7 : 3;
    const int per_block = 64 * (4 + (W4 ? 2 : 4));
    const size_t lds = (size_t)GEMV_RING * NW * GEMV_CH * per_block + (size_t)g.Kp;
    auto kern = gemv_kernel<W4, EPI, GATEUP, NW, BUF>;
    static size_t attr_set = 64 * 1024;   // dynamic LDS above 64 KB needs an explicit opt-in
    if (lds > attr_set &&
        hipFuncSetAttribute((const void *)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess)
        attr_set = lds;
    dim3 grid(GATEUP ? (unsigned)((g.O + 31) / 32) : (unsigned)((g.O + 63) / 64), (unsigned)grid_rows);
    hipLaunchKernelGGL(kern, grid, dim3((NW + 1) * 64), lds, st, a, g, a.xq, a.sx);
}

template <bool W4, int EPI, bool GATEUP>
static void launch_gemv_t(const DotArgs &a, const MatGeom &g, int grid_rows, hipStream_t st) {
    if constexpr (GATEUP) {
        if (!a.buf_ok) {
            launch_gemv_b<W4, EPI, GATEUP, false>(a, g, grid_rows, st);
            return;
        }
    }
    launch_gemv_b<W4, EPI, GATEUP, true>(a, g, grid_rows, st);
}

template <bool GATEUP>
static void launch_gemv_any(const DotArgs &a, const MatGeom &g, int act, int grid_rows, hipStream_t st) {
    if (grid_rows <= 0) return;
    const int epi = act == ACT_B32 ? EPI_B32 : (g.per_row ? EPI_ROW : EPI_GRP);
    if (g.w4) {
        if (epi == EPI_ROW) launch_gemv_t<true, EPI_ROW, GATEUP>(a, g, grid_rows, st);
        else if (epi == EPI_GRP) launch_gemv_t<true, EPI_GRP, GATEUP>(a, g, grid_rows, st);
        else launch_gemv_t<true, EPI_B32, GATEUP>(a, g, grid_rows, st);
    } else {
        if (epi == EPI_ROW) launch_gemv_t<false, EPI_ROW, GATEUP>(a, g, grid_rows, st);
        else if (epi == EPI_GRP) launch_gemv_t<false, EPI_GRP, GATEUP>(a, g, grid_rows, st);
        else launch_gemv_t<false, EPI_B32, GATEUP>(a, g, grid_rows, st);
    }
}

void launch_gemv_gateup(const DotArgs &a, const MatGeom &g, int act, int grid_rows, hipStream_t st) {
    launch_gemv_any<true>(a, g, act, grid_rows, st);
}
void launch_gemv_down(const DotArgs &a, const MatGeom &g, int act, int grid_rows, hipStream_t st) {
    launch_gemv_any<false>(a, g, act, grid_rows, st);
}

}  // namespace phip
