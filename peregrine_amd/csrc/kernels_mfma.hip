// kernels_mfma.hip — the batched arm: per-expert grouped GEMM on the int8
// matrix cores (v_mfma_i32_32x32x32_i8, gfx950).
//
// Work unit: one 32-row M-tile of one expert (from the expert-offset table)
// times a slab of output channels. One MFMA consumes exactly one 32-element
// K block, so each block's int32 dot leaves the matrix core whole and the f32
// epilogue runs block by block in ascending order — the same chain as
// oracle/oracle.c, element for element. With a per-row weight scale (or a
// group spanning several blocks) the int32 dots accumulate inside the MFMA
// and the f32 step runs once per group.
//
// Operand mapping (A = activations, rows = tokens; B = weights, columns =
// output channels): lane l supplies row/column (l % 32) and the K half
// (l / 32); A and B use the same K slots, so the integer dot is the exact
// sum whatever order the hardware walks K in. Accumulator register r of
// lane l holds row 8*(r/4) + 4*(l/32) + r%4, column l % 32.
//
// int4 weights are unpacked in registers: 8 bytes (16 nibbles) per lane per
// block -> 16 int8 values scaled by 16 (the scale tables carry the 1/16).
#include <cstdlib>

#include "common.h"
#include "mfma_map.h"

namespace phip {

static_assert(mmap::TILE_O == TILE_O && mmap::BLK == BLK && mmap::MT_ROWS == MT_ROWS, "mfma_map.h geometry");

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

template <bool W4>
__device__ __forceinline__ v4i load_b(GU8 *p) {
    v4i r;
    if constexpr (W4) {
        const uint2 w = ldg_stream2g(p);
        r[0] = i4_even16(w.x);
        r[1] = i4_odd16(w.x);
        r[2] = i4_even16(w.y);
        r[3] = i4_odd16(w.y);
    } else {
        const uint4 w = ldg_stream4g(p);
        r[0] = (int)w.x;
        r[1] = (int)w.y;
        r[2] = (int)w.z;
        r[3] = (int)w.w;
    }
    return r;
}

__device__ __forceinline__ int acc_row(int reg, int lane) { return 8 * (reg >> 2) + 4 * (lane >> 5) + (reg & 3); }

// The per-32 activation scales of a tile's 32 rows into LDS, [nb][32]: eight
// threads per row read consecutive blocks, four loads in flight per thread
// (rows past the expert's end repeat its last row).
__device__ __forceinline__ void load_tile_sx(const DotArgs &a, int r0, int rend, int nb, float *sxl) {
    const int i = threadIdx.x >> 3, b0 = threadIdx.x & 7;
    int rr = r0 + i;
    if (rr >= rend) rr = rend - 1;
    const float *src = a.sx + (size_t)(a.act_identity ? rr : a.plan.row_act[rr]) * a.sx_stride;
    for (int bb = b0; bb < nb; bb += 32) {
        float v[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = bb + 8 * q < nb ? src[bb + 8 * q] : 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (bb + 8 * q < nb) sxl[(bb + 8 * q) * 32 + i] = v[q];
    }
}

// NSUB column subtiles of 32 per wave. GATEUP: subtile 0 = gate, 1 = up (same
// channels). Down: NSUB adjacent 32-channel subtiles.
template <bool W4, int EPI, bool GATEUP, int NSUB, int PD>
__global__ __launch_bounds__(256) void mfma_kernel(DotArgs a, MatGeom g, const int8_t *__restrict__ xq,
                                                   const float *__restrict__ sxv) {
    constexpr int BB = W4 ? 16 : 32;
    extern __shared__ float sxl[];   // EPI_B32: [nb][32] activation scales of this tile's rows

    const int lane = threadIdx.x & 63, wave = wave_id();
    const int tile = blockIdx.y;
    if (tile >= a.plan.counts[1]) return;
    const int e = a.plan.mt_exp[tile], r0 = a.plan.mt_row0[tile], rend = a.plan.mt_rend[tile];
    const int j = lane & 31, hh = lane >> 5;
    const int n0 = GATEUP ? ((int)blockIdx.x * 4 + wave) * 32 : ((int)blockIdx.x * 4 + wave) * 32 * NSUB;

    // activation row of this lane's A slot (rows past the expert's end repeat
    // its last row; their results are never stored)
    int ra = r0 + j;
    if (ra >= rend) ra = rend - 1;
    const int arow_a = a.act_identity ? ra : a.plan.row_act[ra];
    GU8 *xa = (GU8 *)gptr(xq + (size_t)arow_a * a.x_stride + hh * 16);

    if constexpr (EPI == EPI_B32) {
        load_tile_sx(a, r0, rend, g.nb, sxl);
        __syncthreads();
    }

    GU8 *wp[NSUB];
    GF32 *sp[NSUB];
    int oc[NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
        const int mat = GATEUP ? s : 2;
        int o = GATEUP ? n0 + j : n0 + s * 32 + j;
        oc[s] = o;
        if (o >= g.Op) o = g.Op - 1;
        wp[s] = gptr(a.desc[e].w[mat] + ((size_t)(o / TILE_O) * g.nb * TILE_O + (o % TILE_O)) * BB + hh * (BB / 2));
        sp[s] = gptr(a.desc[e].sc[mat] + (size_t)(o / TILE_O) * g.ng * TILE_O + (o % TILE_O));
    }

    float acc[NSUB][16];
    v16i iacc[NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[s][i] = 0.0f;
        iacc[s] = v16i{};
    }

    // Software pipeline, PD blocks ahead: PD + 1 operand slots rotate through
    // a loop unrolled by PD + 1. Loads are unconditional (clamped to the last
    // block) so the wait counts stay exact; the weight scales travel with
    // their block instead of being fetched when the epilogue needs them.
    const int nrow = rend - r0;   // rows of this tile (1..32)
    auto load_blk = [&](int b, v4i &A, v4i (&B)[NSUB], float (&S)[NSUB]) {
        const int bc = b < g.nb ? b : g.nb - 1;
        A = *(const __attribute__((address_space(1))) v4i *)(xa + (size_t)bc * BLK);
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            B[s] = load_b<W4>(wp[s] + (size_t)bc * TILE_O * BB);
            if constexpr (EPI != EPI_ROW) S[s] = sp[s][(size_t)grp_of(bc, g.gshift) * TILE_O];
        }
    };
    // Each block: the MFMAs (integer dots), then the f32 epilogue. The loop
    // issues block b+1's MFMAs before block b's epilogue, so the matrix cores
    // run under the VALU epilogue. A block that opens a weight group starts
    // its MFMA accumulation from zero; the int32 result of a block that
    // closes one is the group's exact dot.
    auto mma_blk = [&](int b, const v4i &A, const v4i (&B)[NSUB], v16i (&D)[NSUB]) {
        const bool opens = EPI == EPI_B32 || (EPI == EPI_GRP && (b == 0 || grp_end(b - 1, g.gshift, g.nb))) ||
                           (EPI == EPI_ROW && b == 0);
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            const v16i cin = opens ? v16i{} : iacc[s];
            D[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B[s], cin, 0, 0, 0);
            if (EPI != EPI_B32) iacc[s] = D[s];
            if (a.dots) {
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int row = r0 + acc_row(i, lane);
                    const int val = D[s][i] - cin[i];
                    if (row < rend && oc[s] < g.O)
                        a.dots[(((size_t)row * (GATEUP ? 2 : 1) + (GATEUP ? s : 0)) * g.O + oc[s]) * g.nb + b] =
                            W4 ? (val >> 4) : val;
                }
            }
        }
    };
    auto epi_blk = [&](int b, const v16i (&D)[NSUB], const float (&S)[NSUB]) {
        if constexpr (EPI == EPI_ROW) return;   // integer sum to the end
        if (EPI == EPI_GRP && !grp_end(b, g.gshift, g.nb)) return;
        if constexpr (EPI == EPI_B32) {
            const float4 *sx4 = (const float4 *)(sxl + b * 32 + 4 * hh);
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                if (8 * gq >= nrow) break;   // uniform: rows past the tile's end
                const float4 sq = sx4[2 * gq];
                const float sxr[4] = {sq.x, sq.y, sq.z, sq.w};
#pragma unroll
                for (int s = 0; s < NSUB; ++s) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int i = 4 * gq + t;
                        acc[s][i] = __fmaf_rn(__fmul_rn(S[s], sxr[t]), (float)D[s][i], acc[s][i]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                if (8 * gq >= nrow) break;
#pragma unroll
                for (int s = 0; s < NSUB; ++s) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int i = 4 * gq + t;
                        acc[s][i] = __fadd_rn(acc[s][i], __fmul_rn((float)D[s][i], S[s]));
                    }
                }
            }
        }
    };
    // PD + 1 operand slots and two MFMA-result buffers rotate through a loop
    // unrolled by a multiple of both, so every index is a compile-time constant:
    // iteration u refills the slot block u-1 has released with block u + PD,
    // issues block u's MFMAs, then runs block u-1's epilogue.
    constexpr int NS = PD + 1, NU = NS % 2 ? 2 * NS : NS;   // unroll: a multiple of both rotations
    v4i Ar[NS];
    v4i Br[NS][NSUB];
    float Sr[NS][NSUB];
    v16i Dr[2][NSUB];
#pragma unroll
    for (int u = 0; u < PD; ++u) load_blk(u, Ar[u], Br[u], Sr[u]);
#pragma unroll 1
    for (int b = 0; b < g.nb; b += NU) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int cur = u % NS, prev = (u + NS - 1) % NS;
            float Sp[NSUB];   // block u-1's scales: its slot is refilled first
#pragma unroll
            for (int s = 0; s < NSUB; ++s) Sp[s] = Sr[prev][s];
            load_blk(b + u + PD, Ar[prev], Br[prev], Sr[prev]);
            if (b + u < g.nb) mma_blk(b + u, Ar[cur], Br[cur], Dr[u & 1]);
            if (b + u > 0 && b + u - 1 < g.nb) epi_blk(b + u - 1, Dr[(u + 1) & 1], Sp);
        }
    }
    if (g.nb % NU == 0) {   // the last block's epilogue did not run inside the loop
        epi_blk(g.nb - 1, Dr[(NU - 1) & 1], Sr[(NU - 1) % NS]);
    }

    // per-row activation scale (EPI_ROW / EPI_GRP) of each accumulator row
    float v[NSUB][16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float sxr = 1.0f;
        if constexpr (EPI != EPI_B32) {
            int rr = r0 + acc_row(i, lane);
            if (rr >= rend) rr = rend - 1;
            const int ar = a.act_identity ? rr : a.plan.row_act[rr];
            sxr = sxv[(size_t)ar * a.sx_stride];
        }
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            if constexpr (EPI == EPI_ROW) {
                const int D = W4 ? (iacc[s][i] >> 4) : iacc[s][i];
                const float sc = W4 ? __fmul_rn(sp[s][0], 16.0f) : sp[s][0];
                v[s][i] = __fmul_rn(__fmul_rn((float)D, sc), sxr);
            } else if constexpr (EPI == EPI_GRP) {
                v[s][i] = __fmul_rn(acc[s][i], sxr);
            } else {
                v[s][i] = acc[s][i];
            }
        }
    }

    if constexpr (GATEUP) {
        const int o = oc[0];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = r0 + acc_row(i, lane);
            const float h = silu_mul(v[0][i], v[1][i]);
            const bool ok = row < rend && o < ((g.O + 31) & ~31);
            // with the h quantisation fused, only hq / sh are read downstream
            if (ok && !(EPI == EPI_B32 && a.hq)) a.out[(size_t)row * a.out_stride + o] = h;
            if (EPI == EPI_B32 && a.hq) {
                // one h row's 32 channels live in the 32 lanes of this half-wave
                const float m = warp_max(fabsf(h), 32);
                float sc = __fdiv_rn(m, 127.0f);
                if (sc < 1e-12f) sc = 1e-12f;
                const float inv = __fdiv_rn(1.0f, sc);
                if (ok) {
                    a.hq[(size_t)row * a.hq_stride + perm8(o)] = (int8_t)(int)rintf(__fmul_rn(h, inv));
                    if (j == 0) a.sh[(size_t)row * a.sh_stride + (o >> 5)] = sc;
                }
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            const int o = oc[s];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = r0 + acc_row(i, lane);
                if (row < rend && o < g.O) a.out[(size_t)row * a.out_stride + o] = v[s][i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// LDS-staged variant (the default MFMA kernel). Operands travel from HBM
// straight into shared LDS stages with the LDS-DMA loads, PD blocks ahead, so
// the bytes in flight cost no registers. The copies are issued from inline
// assembly (the compiler would otherwise wait for every copy before any LDS
// read); the loop issues no other vector-memory operation, so "older than the
// last OPS*PD" is exactly the block about to be used. Stage layout and the
// per-block barrier: see DmaStage below.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void lds_dma16(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma16_nt(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(g), "s"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma4(const void *g, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(g), "s"(lds) : "memory");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One stage (a block in flight), shared by the workgroup's four waves:
// [A: 32 activation rows x 32 B] then, per wave, [weights of its two
// subtiles][their scales]. Each wave copies a quarter of A (8 rows) and its
// own weights and scales: the same copy count for every wave, so one constant
// wait count holds, and one barrier per block makes the quarters of A visible
// to all. Per-32 activation scales for the whole tile sit after the stages,
// loaded once.
template <bool W4>
struct DmaStage {
    static constexpr int A = 0;
    static constexpr int WAVE0 = 1024;
    static constexpr int SW = W4 ? 1024 : 2048;   // within a wave's part: weights, then scales
    static constexpr int WAVE_BYTES = SW + 256;
    static constexpr int BYTES = WAVE0 + 4 * WAVE_BYTES;
};

// Dispatches with int8 weights run this kernel (int4 ones run
// mfma_sa_kernel below). An int4 instantiation caps the down projection at
// 128 VGPRs (four waves per SIMD); int8 ones are left uncapped (capped, the
// int8 down projection spills eight registers: config 5 735 vs 630 us).
template <bool W4, int EPI, bool GATEUP, int NSUB, int PD, bool WNT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GATEUP || !W4 ? 1 : 4))) void mfma_dma_kernel(DotArgs a, MatGeom g) {
    static_assert(NSUB == 2, "a wave's weight copy covers two 32-column subtiles");
    typedef DmaStage<W4> ST;
    constexpr int NSTG = PD + 2;   // stage b-2 is refilled once every wave is past block b-1's barrier
    constexpr int OPS = 1 + (W4 ? 1 : 2) + (EPI != EPI_ROW ? 1 : 0);   // copies per block and wave
    constexpr int BB = W4 ? 16 : 32;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_u8[];   // [NSTG][ST::BYTES], then sxl

    const int lane = threadIdx.x & 63, wave = wave_id();
    const int tile = blockIdx.y;
    if (tile >= a.plan.counts[1]) return;
    const int e = a.plan.mt_exp[tile], r0 = a.plan.mt_row0[tile], rend = a.plan.mt_rend[tile];
    const int j = lane & 31, hh = lane >> 5;
    const int n0 = mmap::dma_n0(GATEUP, (int)blockIdx.x, wave);
    const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_u8);
    float *sxl = (float *)(lds_u8 + (size_t)NSTG * ST::BYTES);   // EPI_B32: [nb][32] activation scales

    // copy sources of this lane: a dword of A (row 8*wave + lane/8), its
    // weights (subtile lane/32, column lane%32) and their scales; rows past
    // the expert's end repeat its last row (never stored)
    const int ra = mmap::a_row(r0, rend, wave, lane);
    const uint8_t *src_a = (const uint8_t *)a.xq +
                           (size_t)(a.act_identity ? ra : a.plan.row_act[ra]) * a.x_stride + mmap::a_col(lane);
    const int oc_l = mmap::dma_ch(GATEUP, n0, lane, g.Op);
    const int mat_l = mmap::dma_mat(GATEUP, lane);
    const uint8_t *src_w = nullptr;
    if constexpr (W4) src_w = a.desc[e].w[mat_l] + mmap::dma_w4(oc_l, g.nb);
    const float *src_s = a.desc[e].sc[mat_l] + mmap::dma_s(oc_l, g.ng);
    const uint8_t *src_w8[2] = {nullptr, nullptr};
    if constexpr (!W4) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
            src_w8[q] = a.desc[e].w[GATEUP ? q : 2] + mmap::dma_w8(mmap::dma_ch8(GATEUP, n0, lane, q, g.Op), g.nb, lane);
    }
    auto copy_blk = [&](int b) {
        const int bc = b < g.nb ? b : g.nb - 1;
        const uint32_t st = lds_addr + (uint32_t)((b % NSTG) * ST::BYTES);
        const uint32_t wv = st + ST::WAVE0 + wave * ST::WAVE_BYTES;
        lds_dma4(src_a + (size_t)bc * BLK, st + ST::A + wave * 256);
        // weights read once per dispatch stream past the caches (WNT); weights
        // that several M tiles of an expert re-read are left cacheable
        auto wcopy = [&](const void *src, uint32_t dst) {
            if constexpr (WNT) lds_dma16_nt(src, dst);
            else lds_dma16(src, dst);
        };
        if constexpr (W4) {
            wcopy(src_w + (size_t)bc * TILE_O * BB, wv);
        } else {
            wcopy(src_w8[0] + (size_t)bc * TILE_O * BB, wv);
            wcopy(src_w8[1] + (size_t)bc * TILE_O * BB, wv + 1024);
        }
        if constexpr (EPI != EPI_ROW) lds_dma4(src_s + (size_t)grp_of(bc, g.gshift) * TILE_O, wv + ST::SW);
    };

    // the tile's activation scales ([nb][32] in LDS) by LDS-DMA, all issued
    // at once: one copy per wave covers two blocks of the 32 rows. Nothing
    // waits on them before block 0's wait, which covers them (a wave's loads
    // complete in order). Rows past the tile's end repeat its last row.
    if constexpr (EPI == EPI_B32) {
        const int rx = mmap::sx_row(r0, rend, lane);
        const float *srcx = a.sx + (size_t)(a.act_identity ? rx : a.plan.row_act[rx]) * a.sx_stride;
        const uint32_t sx_lds = lds_addr + (uint32_t)(NSTG * ST::BYTES);
        for (int i = wave; i < (g.nb + 1) >> 1; i += 4)
            lds_dma4(srcx + mmap::sx_blk(i, lane, g.nb), sx_lds + (uint32_t)(i * 256));
    }
#pragma unroll
    for (int u = 0; u < PD; ++u)
        if (u < g.nb) copy_blk(u);

    int oc[NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) oc[s] = GATEUP ? n0 + j : n0 + s * 32 + j;
    float acc[NSUB][16];
    v16i iacc[NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[s][i] = 0.0f;
        iacc[s] = v16i{};
    }
    const int nrow = rend - r0;

    auto read_ops = [&](int b, v4i &A, v4i (&B)[NSUB], float (&S)[NSUB]) {
        const uint8_t *st = lds_u8 + (b % NSTG) * ST::BYTES;
        const uint8_t *wv = st + ST::WAVE0 + wave * ST::WAVE_BYTES;
        A = *(const v4i *)(st + ST::A + j * 32 + hh * 16);
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            if constexpr (W4) {
                const uint2 w = *(const uint2 *)(wv + (s * 32 + j) * 16 + hh * 8);
                B[s][0] = i4_even16(w.x);
                B[s][1] = i4_odd16(w.x);
                B[s][2] = i4_even16(w.y);
                B[s][3] = i4_odd16(w.y);
            } else {
                B[s] = *(const v4i *)(wv + s * 1024 + j * 32 + hh * 16);
            }
            if constexpr (EPI != EPI_ROW) S[s] = *(const float *)(wv + ST::SW + (s * 32 + j) * 4);
        }
    };
    auto mma_blk = [&](int b, const v4i &A, const v4i (&B)[NSUB], v16i (&D)[NSUB]) {
        const bool opens = EPI == EPI_B32 || (EPI == EPI_GRP && (b == 0 || grp_end(b - 1, g.gshift, g.nb))) ||
                           (EPI == EPI_ROW && b == 0);
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            const v16i cin = opens ? v16i{} : iacc[s];
            D[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B[s], cin, 0, 0, 0);
            if (EPI != EPI_B32) iacc[s] = D[s];
        }
    };
    auto epi_blk = [&](int b, const v16i (&D)[NSUB], const float (&S)[NSUB]) {
        if constexpr (EPI == EPI_ROW) return;
        if (EPI == EPI_GRP && !grp_end(b, g.gshift, g.nb)) return;
        if constexpr (EPI == EPI_B32) {
            const float4 *sx4 = (const float4 *)(sxl + b * 32 + 4 * hh);
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                if (8 * gq >= nrow) break;   // uniform: rows past the tile's end
                const float4 sq = sx4[2 * gq];
                const float sxr[4] = {sq.x, sq.y, sq.z, sq.w};
#pragma unroll
                for (int s = 0; s < NSUB; ++s) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int i = 4 * gq + t;
                        acc[s][i] = __fmaf_rn(__fmul_rn(S[s], sxr[t]), (float)D[s][i], acc[s][i]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                if (8 * gq >= nrow) break;
#pragma unroll
                for (int s = 0; s < NSUB; ++s) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int i = 4 * gq + t;
                        acc[s][i] = __fadd_rn(acc[s][i], __fmul_rn((float)D[s][i], S[s]));
                    }
                }
            }
        }
    };

    v16i Dr[2][NSUB];
    float Sr[2][NSUB];
#pragma unroll 1
    for (int b = 0; b < g.nb; b += 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int bb = b + u;
            if (bb < g.nb) {   // uniform
                if (bb + PD < g.nb) {
                    copy_blk(bb + PD);
                    wait_vm<OPS * PD>();   // this wave's copies of block bb have landed
                } else {
                    wait_vm<0>();          // the last blocks: nothing copied past the end
                }
                // every wave's quarter of A (and, on the first pass, its
                // share of the activation scales) is in LDS once all waves are here
                asm volatile("s_barrier" ::: "memory");
                v4i A;
                v4i B[NSUB];
                read_ops(bb, A, B, Sr[u]);
                mma_blk(bb, A, B, Dr[u]);
            }
            if (bb > 0 && bb - 1 < g.nb) epi_blk(bb - 1, Dr[u ^ 1], Sr[u ^ 1]);
        }
    }
    if (g.nb % 2 == 0) epi_blk(g.nb - 1, Dr[1], Sr[1]);   // the last block's epilogue did not run in the loop

    // per-row activation scale (EPI_ROW / EPI_GRP) of each accumulator row
    float v[NSUB][16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float sxr = 1.0f;
        if constexpr (EPI != EPI_B32) {
            int rr = r0 + acc_row(i, lane);
            if (rr >= rend) rr = rend - 1;
            const int ar = a.act_identity ? rr : a.plan.row_act[rr];
            sxr = a.sx[(size_t)ar * a.sx_stride];
        }
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            if constexpr (EPI == EPI_ROW) {
                const int D = W4 ? (iacc[s][i] >> 4) : iacc[s][i];
                int o = oc[s];
                if (o >= g.Op) o = g.Op - 1;
                const int mat = GATEUP ? s : 2;
                const float *sp = a.desc[e].sc[mat] + (size_t)(o / TILE_O) * g.ng * TILE_O + (o % TILE_O);
                const float sc = W4 ? __fmul_rn(sp[0], 16.0f) : sp[0];
                v[s][i] = __fmul_rn(__fmul_rn((float)D, sc), sxr);
            } else if constexpr (EPI == EPI_GRP) {
                v[s][i] = __fmul_rn(acc[s][i], sxr);
            } else {
                v[s][i] = acc[s][i];
            }
        }
    }

    if constexpr (GATEUP) {
        const int o = oc[0];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = r0 + acc_row(i, lane);
            const float h = silu_mul(v[0][i], v[1][i]);
            const bool ok = row < rend && o < ((g.O + 31) & ~31);
            // with the h quantisation fused, only hq / sh are read downstream
            if (ok && !(EPI == EPI_B32 && a.hq)) a.out[(size_t)row * a.out_stride + o] = h;
            if (EPI == EPI_B32 && a.hq) {
                const float m = warp_max(fabsf(h), 32);
                float sc = __fdiv_rn(m, 127.0f);
                if (sc < 1e-12f) sc = 1e-12f;
                const float inv = __fdiv_rn(1.0f, sc);
                if (ok) {
                    a.hq[(size_t)row * a.hq_stride + perm8(o)] = (int8_t)(int)rintf(__fmul_rn(h, inv));
                    if (j == 0) a.sh[(size_t)row * a.sh_stride + (o >> 5)] = sc;
                }
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            const int o = oc[s];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = r0 + acc_row(i, lane);
                if (row < rend && o < g.O) a.out[(size_t)row * a.out_stride + o] = v[s][i];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Scalar-address staged variant. The same stages and per-block barrier as
// mfma_dma_kernel, with two changes that take the per-block address work off
// the VALU (which the exact f32 epilogue already keeps busy):
//  * every LDS-DMA copy uses the scalar-base form: a uniform 64-bit base in
//    SGPRs, advanced per block by scalar adds, plus a fixed 32-bit per-lane
//    offset. For that, each copy reads one tensor: wave w copies subtiles 2w
//    and 2w+1 of the stage (gate/up: waves 0-1 the gate tiles of channel
//    groups 0-3, waves 2-3 the up tiles; down: its own two subtiles);
//  * the block loop is unrolled over the stages, so every LDS offset is an
//    instruction immediate.
// Stage: [A: 32 rows x 32 B][8 weight subtiles x 32 x BB][8 x 32 f32 scales].
// ---------------------------------------------------------------------------
__device__ __forceinline__ void lds_dma16_s(uint32_t voff, const void *base, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma16_s_nt(uint32_t voff, const void *base, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(voff), "s"(base), "s"(lds) : "memory");
}
__device__ __forceinline__ void lds_dma4_s(uint32_t voff, const void *base, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds) : "memory");
}
__device__ __forceinline__ const uint8_t *uniform_ptr(const void *p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (const uint8_t *)(uintptr_t)(((uint64_t)hi << 32) | lo);
}

template <bool W4>
struct SaStage {
    static constexpr int SUB = 32 * (W4 ? 16 : 32);   // one 32-column subtile of one block
    static constexpr int A = 0;
    static constexpr int W = 1024;
    static constexpr int S = W + 8 * SUB;
    static constexpr int BYTES = S + 8 * 128;
};

template <bool W4, int EPI, bool GATEUP, int PD, bool WNT, bool XO = false>
__global__ __launch_bounds__(256) void mfma_sa_kernel(DotArgs a, MatGeom g) {
    constexpr int NSUB = 2;
    typedef SaStage<W4> ST;
    constexpr int NSTG = PD + 2;   // stage b-2 is refilled once every wave is past block b-1's barrier
    constexpr int NU = NSTG % 2 ? 2 * NSTG : NSTG;   // unroll: stages and the two result buffers rotate
    constexpr int OPS = 1 + (W4 ? 1 : 2) + (EPI != EPI_ROW ? 1 : 0);   // copies per block and wave
    constexpr int BB = W4 ? 16 : 32;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds_u8[];   // [NSTG][ST::BYTES], then sxl

    const int lane = threadIdx.x & 63, wave = wave_id();
    // XO (dispatches that re-read each expert's weights over several M
    // tiles): workgroup L runs on XCD L mod 8, and each XCD takes a
    // contiguous run of the items in (expert, group of XO_G tiles, slab,
    // tile) order. The tiles of a group read each weight slab through one L2
    // back to back, and the group's activation rows (XO_G x 32 rows) stay in
    // that L2 across the slabs. An expert whose tiles are [ts, ts + nt) owns
    // items [NS * ts, NS * (ts + nt)).
    int tile = blockIdx.y, slab = blockIdx.x;
    if constexpr (XO) {
        const int T = a.plan.counts[1], NS = (int)gridDim.x;
        const int item = mmap::xo_item(slab + NS * (int)blockIdx.y, NS * T);
        if (item < 0) return;
        const int q = item / NS;                 // a tile of the item's expert
        const int ts = a.plan.mt_first[q];
        const int nt = (a.plan.mt_rend[q] - a.plan.mt_row0[ts] + MT_ROWS - 1) / MT_ROWS;
        mmap::xo_place(item, NS, ts, nt, &slab, &tile);
    }
    if (tile >= a.plan.counts[1]) return;
    const int e = a.plan.mt_exp[tile], r0 = a.plan.mt_row0[tile], rend = a.plan.mt_rend[tile];
    const int j = lane & 31, hh = lane >> 5;
    const int n0 = mmap::dma_n0(GATEUP, slab, wave);
    const uint32_t lds_addr = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds_u8);
    float *sxl = (float *)(lds_u8 + (size_t)NSTG * ST::BYTES);   // EPI_B32: [nb][32] activation scales
    auto act_row = [&](int r) { return a.act_identity ? r : a.plan.row_act[r]; };

    // ---- copy sources: uniform bases + per-lane offsets ----
    // A: a dword of row 8*wave + lane/8 (rows past the expert's end repeat
    // its last row; never stored)
    const uint32_t voff_a = (uint32_t)act_row(mmap::a_row(r0, rend, wave, lane)) * (uint32_t)a.x_stride + mmap::a_col(lane);
    const uint8_t *base_a = uniform_ptr(a.xq);
    // weights and their scales: this wave's two subtiles 2w, 2w+1 (one
    // tensor), lane half hh -> subtile 2w + hh; tiles past the tensor clamp
    // to its last tile (never stored)
    const int mat = mmap::sa_mat(GATEUP, wave);
    const int ntile = g.Op / TILE_O;
    const uint8_t *base_w = uniform_ptr(a.desc[e].w[mat]);
    const uint8_t *base_s = uniform_ptr(a.desc[e].sc[mat]);
    uint32_t voff_w;
    if constexpr (W4) voff_w = mmap::sa_voff_w4(GATEUP, slab, wave, lane, ntile, g.nb);
    else voff_w = mmap::sa_voff_w8(lane);   // int8: one subtile per copy
    uint32_t tile_w8[2] = {0, 0};
    if constexpr (!W4) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
            tile_w8[q] = __builtin_amdgcn_readfirstlane(mmap::sa_tile8(GATEUP, slab, wave, q, ntile, g.nb));
    }
    const uint32_t voff_s = mmap::sa_voff_s(GATEUP, slab, wave, lane, ntile, g.ng);

    auto copy_blk = [&](int b, int stg) {
        const uint32_t st = lds_addr + (uint32_t)(stg * ST::BYTES);
        lds_dma4_s(voff_a, base_a + (size_t)b * BLK, st + ST::A + wave * 256);
        const uint8_t *wb = base_w + (size_t)b * ST::SUB;
        if constexpr (W4) {
            if constexpr (WNT) lds_dma16_s_nt(voff_w, wb, st + ST::W + wave * 2 * ST::SUB);
            else lds_dma16_s(voff_w, wb, st + ST::W + wave * 2 * ST::SUB);
        } else {
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                if constexpr (WNT) lds_dma16_s_nt(voff_w, wb + tile_w8[q], st + ST::W + (wave * 2 + q) * ST::SUB);
                else lds_dma16_s(voff_w, wb + tile_w8[q], st + ST::W + (wave * 2 + q) * ST::SUB);
            }
        }
        if constexpr (EPI != EPI_ROW)
            lds_dma4_s(voff_s, base_s + (size_t)grp_of(b, g.gshift) * 128, st + ST::S + wave * 256);
    };

    // the tile's activation scales ([nb][32] in LDS), all issued at once:
    // one copy per wave covers two blocks of the 32 rows; block 0's wait
    // covers them (a wave's loads complete in order)
    if constexpr (EPI == EPI_B32) {
        const float *srcx = a.sx + (size_t)act_row(mmap::sx_row(r0, rend, lane)) * a.sx_stride;
        const uint32_t sx_lds = lds_addr + (uint32_t)(NSTG * ST::BYTES);
        for (int i = wave; i < (g.nb + 1) >> 1; i += 4)
            lds_dma4(srcx + mmap::sx_blk(i, lane, g.nb), sx_lds + (uint32_t)(i * 256));
    }
#pragma unroll
    for (int u = 0; u < PD; ++u)
        if (u < g.nb) copy_blk(u, u);

    int oc[NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) oc[s] = GATEUP ? n0 + j : n0 + s * 32 + j;
    // this wave's subtiles in the stage: gate/up -> gate group w and up group
    // w; down -> subtiles 2w, 2w+1
    const int sub0 = GATEUP ? wave : 2 * wave, sub1 = GATEUP ? 4 + wave : 2 * wave + 1;
    const uint32_t rd_w0 = ST::W + sub0 * ST::SUB + j * BB + hh * (BB / 2);
    const uint32_t rd_w1 = ST::W + sub1 * ST::SUB + j * BB + hh * (BB / 2);
    const uint32_t rd_s0 = ST::S + sub0 * 128 + j * 4, rd_s1 = ST::S + sub1 * 128 + j * 4;
    const uint32_t rd_a = ST::A + j * 32 + hh * 16;
    float acc[NSUB][16];
    v16i iacc[NSUB];
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[s][i] = 0.0f;
        iacc[s] = v16i{};
    }
    const int nrow = rend - r0;

    auto read_ops = [&](int stg, v4i &A, v4i (&B)[NSUB], float (&S)[NSUB]) {
        const uint8_t *st = lds_u8 + stg * ST::BYTES;
        A = *(const v4i *)(st + rd_a);
        const uint32_t rw[2] = {rd_w0, rd_w1}, rs[2] = {rd_s0, rd_s1};
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            if constexpr (W4) {
                const uint2 w = *(const uint2 *)(st + rw[s]);
                B[s][0] = i4_even16(w.x);
                B[s][1] = i4_odd16(w.x);
                B[s][2] = i4_even16(w.y);
                B[s][3] = i4_odd16(w.y);
            } else {
                B[s] = *(const v4i *)(st + rw[s]);
            }
            if constexpr (EPI != EPI_ROW) S[s] = *(const float *)(st + rs[s]);
        }
    };
    auto mma_blk = [&](int b, const v4i &A, const v4i (&B)[NSUB], v16i (&D)[NSUB]) {
        const bool opens = EPI == EPI_B32 || (EPI == EPI_GRP && (b == 0 || grp_end(b - 1, g.gshift, g.nb))) ||
                           (EPI == EPI_ROW && b == 0);
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            const v16i cin = opens ? v16i{} : iacc[s];
            D[s] = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B[s], cin, 0, 0, 0);
            if (EPI != EPI_B32) iacc[s] = D[s];
        }
    };
    auto epi_blk = [&](int b, const v16i (&D)[NSUB], const float (&S)[NSUB]) {
        if constexpr (EPI == EPI_ROW) return;
        if (EPI == EPI_GRP && !grp_end(b, g.gshift, g.nb)) return;
        if constexpr (EPI == EPI_B32) {
            const float4 *sx4 = (const float4 *)(sxl + b * 32 + 4 * hh);
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                if (8 * gq >= nrow) break;   // uniform: rows past the tile's end
                const float4 sq = sx4[2 * gq];
                const float sxr[4] = {sq.x, sq.y, sq.z, sq.w};
#pragma unroll
                for (int s = 0; s < NSUB; ++s) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int i = 4 * gq + t;
                        acc[s][i] = __fmaf_rn(__fmul_rn(S[s], sxr[t]), (float)D[s][i], acc[s][i]);
                    }
                }
            }
        } else {
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                if (8 * gq >= nrow) break;
#pragma unroll
                for (int s = 0; s < NSUB; ++s) {
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        const int i = 4 * gq + t;
                        acc[s][i] = __fadd_rn(acc[s][i], __fmul_rn((float)D[s][i], S[s]));
                    }
                }
            }
        }
    };

    v16i Dr[2][NSUB];
    float Sr[2][NSUB];
#pragma unroll 1
    for (int b0 = 0; b0 < g.nb; b0 += NU) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int bb = b0 + u;   // stage u % NSTG: b0 is a multiple of NSTG
            if (bb < g.nb) {   // uniform
                if (bb + PD < g.nb) {
                    copy_blk(bb + PD, (u + PD) % NSTG);
                    wait_vm<OPS * PD>();   // this wave's copies of block bb have landed
                } else {
                    wait_vm<0>();          // the last blocks: nothing copied past the end
                }
                asm volatile("s_barrier" ::: "memory");
                v4i A;
                v4i B[NSUB];
                read_ops(u % NSTG, A, B, Sr[u & 1]);
                mma_blk(bb, A, B, Dr[u & 1]);
            }
            if (bb > 0 && bb - 1 < g.nb) epi_blk(bb - 1, Dr[(u + 1) & 1], Sr[(u + 1) & 1]);
        }
    }
    if (g.nb % NU == 0) epi_blk(g.nb - 1, Dr[1], Sr[1]);   // the last block's epilogue did not run in the loop

    // per-row activation scale (EPI_ROW / EPI_GRP) of each accumulator row
    float v[NSUB][16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float sxr = 1.0f;
        if constexpr (EPI != EPI_B32) {
            int rr = r0 + acc_row(i, lane);
            if (rr >= rend) rr = rend - 1;
            sxr = a.sx[(size_t)act_row(rr) * a.sx_stride];
        }
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            if constexpr (EPI == EPI_ROW) {
                const int D = W4 ? (iacc[s][i] >> 4) : iacc[s][i];
                int o = oc[s];
                if (o >= g.Op) o = g.Op - 1;
                const int m = GATEUP ? s : 2;
                const float *sp = a.desc[e].sc[m] + (size_t)(o / TILE_O) * g.ng * TILE_O + (o % TILE_O);
                const float sc = W4 ? __fmul_rn(sp[0], 16.0f) : sp[0];
                v[s][i] = __fmul_rn(__fmul_rn((float)D, sc), sxr);
            } else if constexpr (EPI == EPI_GRP) {
                v[s][i] = __fmul_rn(acc[s][i], sxr);
            } else {
                v[s][i] = acc[s][i];
            }
        }
    }

    if constexpr (GATEUP) {
        const int o = oc[0];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = r0 + acc_row(i, lane);
            const float h = silu_mul(v[0][i], v[1][i]);
            const bool ok = row < rend && o < ((g.O + 31) & ~31);
            // with the h quantisation fused, only hq / sh are read downstream
            if (ok && !(EPI == EPI_B32 && a.hq)) a.out[(size_t)row * a.out_stride + o] = h;
            if (EPI == EPI_B32 && a.hq) {
                const float m = warp_max(fabsf(h), 32);
                float sc = __fdiv_rn(m, 127.0f);
                if (sc < 1e-12f) sc = 1e-12f;
                const float inv = __fdiv_rn(1.0f, sc);
                if (ok) {
                    a.hq[(size_t)row * a.hq_stride + perm8(o)] = (int8_t)(int)rintf(__fmul_rn(h, inv));
                    if (j == 0) a.sh[(size_t)row * a.sh_stride + (o >> 5)] = sc;
                }
            }
        }
    } else {
#pragma unroll
        for (int s = 0; s < NSUB; ++s) {
            const int o = oc[s];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = r0 + acc_row(i, lane);
                if (row < rend && o < g.O) a.out[(size_t)row * a.out_stride + o] = v[s][i];
            }
        }
    }
}

template <bool W4, int EPI, int PD>
static size_t mfma_sa_lds(const MatGeom &g) {
    return (size_t)(PD + 2) * SaStage<W4>::BYTES + (EPI == EPI_B32 ? (size_t)(g.nb + 1) / 2 * 2 * 32 * sizeof(float) : 0);
}

template <bool W4, int EPI, bool GATEUP, int PD, bool WNT, bool XO = false>
static void launch_mfma_sa_h(const DotArgs &a, const MatGeom &g, int grid_tiles, hipStream_t st) {
    dim3 grid((unsigned)mmap::slab_count(GATEUP, g.O), (unsigned)grid_tiles);
    const size_t lds = mfma_sa_lds<W4, EPI, PD>(g);
    auto kern = mfma_sa_kernel<W4, EPI, GATEUP, PD, WNT, XO>;
    static size_t opted[LDS_OPT_DEVICES];
    lds_opt_in((const void *)kern, lds, opted);
    launch_k(kern, grid, dim3(256), lds, st, a, g);
}

template <bool W4, int EPI, bool GATEUP, int PD>
static void launch_mfma_p(const DotArgs &a, const MatGeom &g, int grid_tiles, hipStream_t st) {
    constexpr int NSUB = 2;
    const int ch_per_wg = GATEUP ? 4 * 32 : 4 * 32 * NSUB;
    const int span = GATEUP ? ((g.O + 31) & ~31) : g.O;
    dim3 grid((unsigned)((span + ch_per_wg - 1) / ch_per_wg), (unsigned)grid_tiles);
    const size_t lds = EPI == EPI_B32 ? (size_t)g.nb * 32 * sizeof(float) : 0;
    launch_k((mfma_kernel<W4, EPI, GATEUP, NSUB, PD>), grid, dim3(256), lds, st, a, g, a.xq, a.sx);
}

// stages plus (per-32 activation scales) the tile's scales
template <bool W4, int EPI, int PD>
static size_t mfma_dma_lds(const MatGeom &g) {
    // EPI_B32: the scales are copied two blocks at a time, so an odd nb rounds up
    return (size_t)(PD + 2) * DmaStage<W4>::BYTES + (EPI == EPI_B32 ? (size_t)(g.nb + 1) / 2 * 2 * 32 * sizeof(float) : 0);
}
// Blocks in flight: three, when the stages and the tile's activation scales
// fit three workgroups per CU (160 KB / 3); else two, if that fits three per
// CU; else six with two per CU (80 KB). Measured: occupancy wins over depth
// (configs 3, 4 and every down projection at three; config 5's int4 gate/up,
// K = 6144, 806 us at two blocks and three per CU against 868 us at six and
// two per CU).
constexpr int DMA_PD_SHALLOW = 3, DMA_PD_NARROW = 2, DMA_PD_DEEP_W4 = 6, DMA_PD_W8 = 3;

template <bool W4, int EPI, bool GATEUP, int PD, bool WNT>
static void launch_mfma_dma_h(const DotArgs &a, const MatGeom &g, int grid_tiles, hipStream_t st) {
    constexpr int NSUB = 2;
    dim3 grid((unsigned)mmap::slab_count(GATEUP, g.O), (unsigned)grid_tiles);
    const size_t lds = mfma_dma_lds<W4, EPI, PD>(g);
    auto kern = mfma_dma_kernel<W4, EPI, GATEUP, NSUB, PD, WNT>;
    static size_t opted[LDS_OPT_DEVICES];
    lds_opt_in((const void *)kern, lds, opted);
    launch_k(kern, grid, dim3(256), lds, st, a, g);
}

// Weights are copied non-temporally unless the dispatch re-reads them (about
// two or more M tiles per expert on average). Measured: config 4 (102 rows
// per expert) 1.85 -> 1.72 ms cacheable; configs 3 and 5 (3 and 16 rows)
// 4-7% slower cacheable.
template <bool W4, int EPI, bool GATEUP, int PD>
static void launch_mfma_dma(const DotArgs &a, const MatGeom &g, int grid_tiles, hipStream_t st) {
    // int4 weights: the scalar-address kernel. Gate/up: config 4 1203 ->
    // 1060 us, config 5 780 -> 766 us, config 3 209 -> 201 us. Down (without
    // a VGPR cap; capped at 128 its unrolled loop spills): config 3 106 ->
    // 99 us, config 4 509 -> 501 us. int8 weights keep mfma_dma_kernel
    // (config 5 int8 gate/up 1186 vs 1214 us).
    if constexpr (W4) {
        // weight-reuse dispatches in the XCD-aware expert-major order: config 4
        // gate/up fetch 3.69 -> 2.60 GB, down 1.50 -> 1.01 GB, step 1.5% faster
        if (a.w_reuse) launch_mfma_sa_h<W4, EPI, GATEUP, PD, false, true>(a, g, grid_tiles, st);
        else launch_mfma_sa_h<W4, EPI, GATEUP, PD, true>(a, g, grid_tiles, st);
    } else {
        if (a.w_reuse) launch_mfma_dma_h<W4, EPI, GATEUP, PD, false>(a, g, grid_tiles, st);
        else launch_mfma_dma_h<W4, EPI, GATEUP, PD, true>(a, g, grid_tiles, st);
    }
}

// COLI_HIP_MFMA_DMA: -1 (default) the LDS-staged kernel wherever its stages
// fit (two workgroups per CU), 0 / 1 force one kernel (A/B measurement). The
// register-prefetch kernel also serves the per-block dot dump.
static int mfma_mode() {
    static const int m = getenv("COLI_HIP_MFMA_DMA") ? atoi(getenv("COLI_HIP_MFMA_DMA")) : -1;
    return m;
}

template <bool W4, int EPI, bool GATEUP>
static void launch_mfma_t(const DotArgs &a, const MatGeom &g, int grid_tiles, hipStream_t st) {
    const int m = mfma_mode();
    if (!a.dots && m != 0) {
        if (mfma_dma_lds<W4, EPI, DMA_PD_SHALLOW>(g) <= 160 * 1024 / 3) {
            launch_mfma_dma<W4, EPI, GATEUP, DMA_PD_SHALLOW>(a, g, grid_tiles, st);
            return;
        }
        if (mfma_dma_lds<W4, EPI, DMA_PD_NARROW>(g) <= 160 * 1024 / 3) {
            launch_mfma_dma<W4, EPI, GATEUP, DMA_PD_NARROW>(a, g, grid_tiles, st);
            return;
        }
        constexpr int PD = W4 ? DMA_PD_DEEP_W4 : DMA_PD_W8;
        if (mfma_dma_lds<W4, EPI, PD>(g) <= 80 * 1024) {
            launch_mfma_dma<W4, EPI, GATEUP, PD>(a, g, grid_tiles, st);
            return;
        }
    }
    launch_mfma_p<W4, EPI, GATEUP, 2>(a, g, grid_tiles, st);   // two blocks ahead: deeper costs occupancy
}

template <bool GATEUP>
static void launch_mfma_any(const DotArgs &a, const MatGeom &g, int act, int grid_tiles, hipStream_t st) {
    if (grid_tiles <= 0) return;
    const int epi = act == ACT_B32 ? EPI_B32 : (g.per_row ? EPI_ROW : EPI_GRP);
    if (g.w4) {
        if (epi == EPI_ROW) launch_mfma_t<true, EPI_ROW, GATEUP>(a, g, grid_tiles, st);
        else if (epi == EPI_GRP) launch_mfma_t<true, EPI_GRP, GATEUP>(a, g, grid_tiles, st);
        else launch_mfma_t<true, EPI_B32, GATEUP>(a, g, grid_tiles, st);
    } else {
        if (epi == EPI_ROW) launch_mfma_t<false, EPI_ROW, GATEUP>(a, g, grid_tiles, st);
        else if (epi == EPI_GRP) launch_mfma_t<false, EPI_GRP, GATEUP>(a, g, grid_tiles, st);
        else launch_mfma_t<false, EPI_B32, GATEUP>(a, g, grid_tiles, st);
    }
}

void launch_mfma_gateup(const DotArgs &a, const MatGeom &g, int act, int grid_tiles, hipStream_t st) {
    launch_mfma_any<true>(a, g, act, grid_tiles, st);
}
void launch_mfma_down(const DotArgs &a, const MatGeom &g, int act, int grid_tiles, hipStream_t st) {
    launch_mfma_any<false>(a, g, act, grid_tiles, st);
}

}  // namespace phip
