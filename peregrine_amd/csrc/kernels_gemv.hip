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

// NW waves, MAXT = most blocks one wave holds per pass (multiple of CH).
template <bool W4, int EPI, bool GATEUP, int NW, int MAXT>
__global__ __launch_bounds__(NW * 64) void gemv_kernel(DotArgs a, MatGeom g, const int8_t *__restrict__ xq,
                                                       const float *__restrict__ sxv, int seg, int passes) {
    constexpr int CH = 8;
    constexpr int NCH = MAXT / CH;
    constexpr int BB = W4 ? 16 : 32;
    __shared__ float relay[64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int r = blockIdx.y;
    if (r >= a.plan.counts[0]) return;  // uniform: fewer rows than the grid bound

    const int e = a.plan.row_exp[r];
    const int arow = a.act_identity ? r : a.plan.row_act[r];
    const int mat = GATEUP ? (lane >> 5) : 2;
    const int o = GATEUP ? (int)blockIdx.x * 32 + (lane & 31) : (int)blockIdx.x * 64 + lane;
    const int t = o >> 6, ol = o & 63;
    const uint8_t *wbase = a.desc[e].w[mat] + ((size_t)t * g.nb * TILE_O + ol) * BB;
    const float *sbase = a.desc[e].sc[mat] + (size_t)t * g.ng * TILE_O + ol;
    const int8_t *x = xq + (size_t)arow * a.x_stride;
    const float *sx = sxv + (size_t)arow * a.sx_stride;

    // EPI_ROW: exact int sum; EPI_GRP / EPI_B32: f32 chain.
    float facc = 0.0f;
    int iacc = 0;

    for (int p = 0; p < passes; ++p) {
        const int segi = p * NW + wave;
        const int b0 = segi * seg;
        int nmy = g.nb - b0;
        nmy = nmy < 0 ? 0 : (nmy > seg ? seg : nmy);

        float tc[MAXT], tf[MAXT];   // EPI_B32: (c, f); EPI_GRP: tf = term, tc = 1 if a term ends here
        int isum = 0, gsum = 0;

        WBlk<W4> wb[2][CH];
        float sb[2][CH];
        auto load_chunk = [&](int c, int buf) {
#pragma unroll
            for (int j = 0; j < CH; ++j) {
                int i = c * CH + j;
                int b = b0 + (i < nmy ? i : nmy - 1);
                wb[buf][j] = load_wblk<W4>(wbase + (size_t)b * TILE_O * BB);
                sb[buf][j] = sbase[(size_t)(b / g.gpb) * TILE_O];
            }
        };
        if (nmy > 0) load_chunk(0, 0);
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            if (c * CH < nmy) {
                if (c + 1 < NCH && (c + 1) * CH < nmy) load_chunk(c + 1, (c + 1) & 1);
#pragma unroll
                for (int j = 0; j < CH; ++j) {
                    const int i = c * CH + j;
                    if (i < nmy) {
                        const int b = b0 + i;
                        const int *xb = (const int *)(x + (size_t)b * BLK);
                        int xv[8];
#pragma unroll
                        for (int q = 0; q < 8; ++q) xv[q] = xb[q];
                        const int d = dot_wblk<W4>(wb[c & 1][j], xv);
                        if (a.dots && o < g.O)
                            a.dots[(((size_t)r * (GATEUP ? 2 : 1) + (GATEUP ? mat : 0)) * g.O + o) * g.nb + b] =
                                W4 ? (d >> 4) : d;
                        if constexpr (EPI == EPI_ROW) {
                            isum += d;
                        } else if constexpr (EPI == EPI_GRP) {
                            gsum += d;
                            const bool end = ((b + 1) % g.gpb == 0) || (b + 1 == g.nb);
                            tf[i] = end ? __fmul_rn((float)gsum, sb[c & 1][j]) : 0.0f;
                            tc[i] = end ? 1.0f : 0.0f;
                            if (end) gsum = 0;
                        } else {
                            tc[i] = __fmul_rn(sb[c & 1][j], sx[b]);
                            tf[i] = (float)d;
                        }
                    }
                }
            }
        }
        // relay the accumulator through the waves in segment order
        for (int step = 0; step < NW; ++step) {
            if (wave == step) {
                if (p > 0 || step > 0) {
                    if constexpr (EPI == EPI_ROW)
                        iacc = __float_as_int(relay[lane]);
                    else
                        facc = relay[lane];
                }
                if constexpr (EPI == EPI_ROW) {
                    iacc += isum;
                } else {
#pragma unroll
                    for (int i = 0; i < MAXT; ++i) {
                        if (i < nmy) {
                            if constexpr (EPI == EPI_GRP) {
                                if (tc[i] != 0.0f) facc = __fadd_rn(facc, tf[i]);
                            } else {
                                facc = __fmaf_rn(tc[i], tf[i], facc);
                            }
                        }
                    }
                }
                if constexpr (EPI == EPI_ROW)
                    relay[lane] = __int_as_float(iacc);
                else
                    relay[lane] = facc;
            }
            __syncthreads();
        }
    }

    if (wave != NW - 1) return;
    float v;
    if constexpr (EPI == EPI_ROW) {
        const int D = W4 ? (iacc >> 4) : iacc;
        const float sc = W4 ? __fmul_rn(sbase[0], 16.0f) : sbase[0];
        v = __fmul_rn(__fmul_rn((float)D, sc), sx[0]);
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
                float s = __fdiv_rn(m, 127.0f);
                if (s < 1e-12f) s = 1e-12f;
                const float inv = __fdiv_rn(1.0f, s);
                a.hq[(size_t)r * a.hq_stride + perm8(o)] = (int8_t)(int)rintf(__fmul_rn(h, inv));
                if ((lane & 31) == 0) a.sh[(size_t)r * a.sh_stride + (o >> 5)] = s;
            }
        }
    } else {
        if (o < g.O) a.out[(size_t)r * a.out_stride + o] = v;
    }
}

template <bool W4, int EPI, bool GATEUP>
static void launch_gemv_t(const DotArgs &a, const MatGeom &g, int grid_rows, hipStream_t st) {
    // cut K into per-wave segments aligned to weight groups
    const int align = (EPI == EPI_GRP) ? g.gpb : 1;
    if (g.nb > 64) {
        constexpr int NW = 8, MAXT = 24;
        int seg = (g.nb + NW - 1) / NW;
        seg = (seg + align - 1) / align * align;
        if (seg > MAXT) seg = MAXT / align * align;
        const int nseg = (g.nb + seg - 1) / seg, passes = (nseg + NW - 1) / NW;
        dim3 grid(GATEUP ? (unsigned)((g.O + 31) / 32) : (unsigned)((g.O + 63) / 64), (unsigned)grid_rows);
        hipLaunchKernelGGL((gemv_kernel<W4, EPI, GATEUP, NW, MAXT>), grid, dim3(NW * 64), 0, st, a, g, a.xq, a.sx,
                           seg, passes);
    } else {
        constexpr int NW = 4, MAXT = 16;
        int seg = (g.nb + NW - 1) / NW;
        seg = (seg + align - 1) / align * align;
        if (seg > MAXT) seg = MAXT / align * align;
        const int nseg = (g.nb + seg - 1) / seg, passes = (nseg + NW - 1) / NW;
        dim3 grid(GATEUP ? (unsigned)((g.O + 31) / 32) : (unsigned)((g.O + 63) / 64), (unsigned)grid_rows);
        hipLaunchKernelGGL((gemv_kernel<W4, EPI, GATEUP, NW, MAXT>), grid, dim3(NW * 64), 0, st, a, g, a.xq, a.sx,
                           seg, passes);
    }
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
