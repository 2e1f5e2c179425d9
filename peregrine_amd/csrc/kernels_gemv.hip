// kernels_gemv.hip — the decode arm: one token row against one expert's
// weights, one output channel per lane.
//
// A workgroup covers one row and one output tile: 32 gate + 32 up channels
// (lanes 0-31 gate, 32-63 up, so SwiGLU is a cross-lane read) or 64 down
// channels. Each half-wave streams one 32-row weight tile, a contiguous
// [nb][32][BB] region no other workgroup reads, with 64-bit non-temporal
// 128-bit loads (16 B per lane; 512 B per half-wave per block).
//
// Exact order: every output must see the same left-to-right f32 chain over
// the 32-blocks as oracle/oracle.c (peregrine-kernels/src/idot.rs:82-88).
// Streaming waves turn blocks into (integer dot, f32 factor) pairs in an LDS
// ring; one chain wave applies them in ascending block order. Integer dots
// are exact whatever the split.
#include <algorithm>
#include <cstdlib>

#include "common.h"
#include "route.h"

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

template <bool W4>
struct DStore;
template <>
struct DStore<true> {
    typedef short T;   // an int4 x int8 32-block dot fits in 16 bits
};
template <>
struct DStore<false> {
    typedef int T;
};

constexpr int GEMV_RING = 2;          // rounds of epilogue inputs held in LDS


// dynamic LDS of the ring: [RING][NW*CH][64] f32 factors + the same count of dots
template <bool W4, int NW, int CH>
__host__ __device__ constexpr size_t gemv_ring_bytes() {
    return ((size_t)GEMV_RING * NW * CH * 64 * (4 + (W4 ? 2 : 4)) + 15) / 16 * 16;
}

// Waits until *ctr >= target for at most `limit` polls. On giving up (the
// ring would be read or overwritten out of order, so the dispatch's output is
// not valid) one lane stores 1 to the host-visible word `failed` and the wave
// carries on, so every wave still reaches the end of the kernel; the host
// reads the word after the stream synchronises and fails the call.
__device__ __forceinline__ void spin_until_geq(int *ctr, int target, int limit, int *failed) {
    for (int spin = 0;; ++spin) {
        if (__hip_atomic_load(ctr, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= target) return;
        if (spin >= limit) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if ((threadIdx.x & 63) == 0) __hip_atomic_store(failed, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// The chain wave of a down-GEMV workgroup, after its y stores: counts the
// workgroup in for its output tile; the workgroup that completes the tile's
// count (every row done) sums the tile's rows, out[o] = (((0 + w0*y0) +
// w1*y1) + ...) in row order, rounded multiply then rounded add, as
// combine_tok_kernel does for one token, and resets the counter for the next
// dispatch.
// Visibility across the XCDs' L2s without a whole-cache write-back and
// invalidate (an agent-scope fence per workgroup costs ~18 us at config 2):
// the y stores and the last workgroup's y loads are agent-scope atomics
// (write-through / coherent reads of just those lines), the stores have
// completed (vmcnt 0) before the count is incremented, the count is an
// agent-scope read-modify-write, and the loads issue only after it returns.
// This rests on the code gfx942/gfx950 get for agent-scope relaxed atomics
// (stores and loads with the SC1 cache policy: written through to, and read
// from, the device coherence point), not on a language-level release/acquire
// pair, whose whole-L2 write-back and invalidate is what the scheme avoids.
__device__ __forceinline__ void tail_combine(const DotArgs &a, int O, int nrows, int o, int tile) {
    const int lane = threadIdx.x & 63;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    int old = 0;
    if (lane == 0) old = __hip_atomic_fetch_add(&a.tail_ctr[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    old = __shfl(old, 0);
    if (old != nrows - 1) return;   // uniform
    asm volatile("" ::: "memory");
    const int oc = o < O ? o : O - 1;
    float yv[GEMV_TAIL_MAXK], wv[GEMV_TAIL_MAXK];
#pragma unroll
    for (int j = 0; j < GEMV_TAIL_MAXK; ++j) {   // every load issued before the sum
        const int jj = j < nrows ? j : 0;
        yv[j] = __hip_atomic_load(&a.out[(size_t)jj * a.out_stride + oc], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        wv[j] = a.tail_w[jj];
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < GEMV_TAIL_MAXK; ++j)
        if (j < nrows) acc = __fadd_rn(acc, __fmul_rn(wv[j], yv[j]));
    if (o < O) a.tail_out[o] = acc;
    if (lane == 0) __hip_atomic_store(&a.tail_ctr[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// NW streaming waves plus one chain wave. K is walked in rounds of NW*CH
// blocks; in round c streaming wave w owns blocks c*NW*CH + w*CH + [0, CH).
// A streaming wave issues its CH weight (and scale) loads for a round as one
// batch — unconditional, clamped to the last block, so the wait counts stay
// exact — turns each block into its integer dot and its f32 factor (sw*sx[b] for
// 32-block activation scales, sw for grouped weights) and parks them in an
// LDS ring of RING rounds. The chain wave walks each finished round in block
// order while later rounds stream; a streaming wave waits only when it is
// RING rounds ahead of the chain. Per-row weight scales only sum integers.
// All waits are bounded.
//
// ROUTE (gate/up, one token): the workgroup first routes the token (wave 0,
// greedy top-k over the logits) while the other waves copy the expert
// descriptor table into LDS and quantise the activation row into xq/sx. Every
// workgroup computes the same bytes, so the shared xq/sx buffers see only
// identical writes; each workgroup waits for its own stores before its scalar
// reads of them. Workgroup (0, 0) publishes ids / weights / row descriptors
// for the down projection and the combine.
template <bool W4, int EPI, bool GATEUP, int NW, int CH, bool ROUTE>
__global__ __launch_bounds__((NW + 1) * 64) void gemv_kernel(DotArgs a, MatGeom g, const int8_t *__restrict__ xq,
                                                             const float *__restrict__ sxv) {
    constexpr int BB = W4 ? 16 : 32;
    constexpr int RB = NW * CH;                  // blocks per round
    constexpr int SLOT = RB * 64;                // entries per ring slot
    typedef typename DStore<W4>::T DT;
    extern __shared__ float lds_f[];   // [RING][RB][64] f32 factors, then [RING][RB][64] dots
    __shared__ int produced[GEMV_RING];          // per slot: streaming waves done (cumulative)
    __shared__ int consumed;                     // rounds the chain wave has finished

    const int lane = threadIdx.x & 63;
    const int wave = wave_id();
    const bool chainer = wave == NW;
    const int r = blockIdx.y;
    const int nrows = a.n_rows_fixed >= 0 ? a.n_rows_fixed : a.plan.counts[0];
    if (r >= nrows) return;  // uniform: fewer rows than the grid bound

    const ExpertDesc *dsc;
    if constexpr (ROUTE) {
        static_assert(GATEUP, "the fused router runs in the gate/up GEMV");
        __shared__ int r_ids[16];
        __shared__ float r_max[NW + 1];
        const RouteArgs &ra = a.route;
        ExpertDesc *tdesc = (ExpertDesc *)((char *)lds_f + gemv_ring_bytes<W4, NW, CH>());
        // quantising waves: 1..NW except the one that shares wave 0's SIMD
        constexpr int QSKIP = 4;
        const int tq = (int)threadIdx.x - 64 - (wave > QSKIP ? 64 : 0), nq = (NW - 1) * 64;
        float rmax = 0.0f;
        uint64_t mykey = 0, first = 0;   // wave 0: the selection, kept for the weights
        int kept = 0;
        if (wave == 0) {
            __builtin_amdgcn_s_setprio(3);   // the selection is every wave's critical path: issue it first
            // a workgroup needs picks 0..r only; the publishing one needs all k
            const int k_sel = blockIdx.x == 0 && r == 0 ? ra.k : r + 1;
            route_select<ROUTE_MAX_E / 64>(ra.logits, ra.E, k_sel, mykey, kept, first);
            __builtin_amdgcn_s_setprio(0);
            if (lane < k_sel) r_ids[lane] = lane < kept ? route_key_index(mykey) : 0;
        } else if (wave != QSKIP) {
            const uint4 *src = (const uint4 *)a.desc;
            uint4 *dst = (uint4 *)tdesc;
            const int n16 = ra.E * (int)(sizeof(ExpertDesc) / 16);
            for (int i = tq; i < n16; i += nq) dst[i] = src[i];
            const int ngr = ra.Kp >> 3;   // 8-element groups; a 32-block is 4 consecutive lanes
            const bool vec = (ra.K & 7) == 0 && ((uintptr_t)ra.x & 15) == 0;
            for (int base = 0; base < ngr; base += nq) {
                const int gi = base + tq;
                float v[8];
                load_group8(ra.x, gi < ngr ? gi : ngr, ra.K, vec, v);   // past the row: zeros
                float m = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; j++) m = fmaxf(m, fabsf(v[j]));
                if (ra.mode == ACT_B32) {
                    m = quad_max(m);
                    uint2 pk;
                    const float sc = quant_group8(v, m, pk);
                    if (gi < ngr) {
                        *(uint2 *)(const_cast<int8_t *>(a.xq) + (size_t)gi * 8) = pk;
                        if ((gi & 3) == 0) const_cast<float *>(a.sx)[gi >> 2] = sc;
                    }
                } else {
                    rmax = fmaxf(rmax, m);
                }
            }
            if (ra.mode != ACT_B32) {
                rmax = warp_max(rmax, 64);
                if (lane == 0) r_max[wave] = rmax;
            }
        }
        if (ra.mode != ACT_B32) {   // one scale for the row: reduce, then quantise
            __syncthreads();
            if (wave != 0 && wave != QSKIP) {
                float m = 0.0f;
                for (int w2 = 1; w2 <= NW; w2++)
                    if (w2 != QSKIP) m = fmaxf(m, r_max[w2]);
                const int ngr = ra.Kp >> 3;
                const bool vec = (ra.K & 7) == 0 && ((uintptr_t)ra.x & 15) == 0;
                for (int gi = tq; gi < ngr; gi += nq) {
                    float v[8];
                    load_group8(ra.x, gi, ra.K, vec, v);
                    uint2 pk;
                    quant_group8(v, m, pk);
                    *(uint2 *)(const_cast<int8_t *>(a.xq) + (size_t)gi * 8) = pk;
                }
                if (tq == 0) {
                    float sc = __fdiv_rn(m, 127.0f);
                    if (sc < 1e-12f) sc = 1e-12f;
                    const_cast<float *>(a.sx)[0] = sc;
                }
            }
        }
        // the quantised row must be in L2 before any wave reads it as scalars
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (blockIdx.x == 0 && r == 0 && wave == 0)   // one workgroup publishes the routing
            route_weights(mykey, kept, first, ra.k, ra.ids, ra.w, tdesc, ra.row_desc);
        dsc = &tdesc[r_ids[r]];
    } else {
        // the router may have copied this row's descriptor already (one load
        // instead of row -> expert id -> descriptor)
        dsc = a.plan.row_desc ? &a.plan.row_desc[r] : &a.desc[a.plan.row_exp[r]];
    }
    const int arow = a.act_identity ? r : (a.act_zero ? 0 : a.plan.row_act[r]);
    const int half = lane >> 5, ol = lane & 31;
    const int o = GATEUP ? (int)blockIdx.x * 32 + ol : (int)blockIdx.x * 64 + lane;
    const int mat = GATEUP ? half : 2;
    // this half-wave's tile: gate or up tile x, or down tile 2x + half
    const int tile = GATEUP ? (int)blockIdx.x : 2 * (int)blockIdx.x + half;
    const auto *wp = gptr(dsc->w[mat] + ((size_t)tile * g.nb * TILE_O + ol) * BB);
    const auto *sp = gptr(dsc->sc[mat] + (size_t)tile * g.ng * TILE_O + ol);
    const int8_t *xg = xq + (size_t)arow * a.x_stride;
    const float *sx = sxv + (size_t)arow * a.sx_stride;
    // The activation row and its scales are the same for every lane: read
    // them as scalars (constant address space -> scalar loads into SGPRs that
    // v_dot4 takes directly), not through LDS.
    uintptr_t xa = (uintptr_t)xg, sa = (uintptr_t)sx;
    if constexpr (ROUTE) {
        // the compiler treats constant-space data as invariant: hide the
        // addresses until after the barrier that follows the quantising stores
        asm volatile("" : "+s"(xa), "+s"(sa));
    }
    const CInt *xs = (const CInt *)xa;
    const CFloat *sxs = (const CFloat *)sa;
    DT *lds_d = (DT *)(lds_f + (size_t)GEMV_RING * SLOT);

    const int nb = g.nb;
    const int nrounds = (nb + RB - 1) / RB;
    WBlk<W4> wA[CH];
    float sA[CH];
    int xr[CH][8];       // this wave's activation blocks for the round (uniform: SGPRs)
    float sxr[CH];
    auto load_round = [&](int c, WBlk<W4> (&wv)[CH], float (&sv)[CH]) {
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int b = min(c * RB + wave * CH + j, nb - 1);
            wv[j] = load_wblk<W4>((const uint8_t *)(wp + (size_t)b * (TILE_O * BB)));
            if constexpr (EPI != EPI_ROW)
                sv[j] = __builtin_nontemporal_load(&sp[(size_t)grp_of(b, g.gshift) * TILE_O]);
        }
        // the activations of the round, issued with the weights so their
        // latency hides under the weight loads
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int b = min(c * RB + wave * CH + j, nb - 1);
#pragma unroll
            for (int q = 0; q < 8; ++q) xr[j][q] = xs[b * (BLK / 4) + q];
            if constexpr (EPI == EPI_B32) sxr[j] = sxs[b];
        }
    };
    auto compute_round = [&](int c, const WBlk<W4> (&wv)[CH], const float (&sv)[CH]) {
        // the ring slot of round c is free once the chain finished round c - RING
        if (c >= GEMV_RING) spin_until_geq(&consumed, c - GEMV_RING + 1, a.spin_limit, a.wait_failed);
        const int slot = (c % GEMV_RING) * SLOT;
        // No per-block guard: blocks past nb (the last round's tail) read the
        // last block's activations and fill ring slots the chain never reads.
        // All reads and dots come first, then all ring writes: the ring and
        // the activation row share one LDS array, so interleaving them would
        // serialise every block on its own LDS round trips.
        int dv[CH];
        float fv[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int d16 = dot_wblk<W4>(wv[j], xr[j]);
            dv[j] = W4 ? (d16 >> 4) : d16;   // exact block dot
            if constexpr (EPI != EPI_ROW) {
                // W4 scale tables hold sw/16; x16 is exact
                const float sw = W4 ? __fmul_rn(sv[j], 16.0f) : sv[j];
                fv[j] = EPI == EPI_B32 ? __fmul_rn(sw, sxr[j]) : sw;
            }
        }
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int bi = wave * CH + j;   // block within the round
            if constexpr (EPI != EPI_ROW) lds_f[slot + bi * 64 + lane] = fv[j];
            lds_d[slot + bi * 64 + lane] = (DT)dv[j];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        if (lane == 0)
            __hip_atomic_fetch_add(&produced[c % GEMV_RING], 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    };

    if (threadIdx.x < GEMV_RING) produced[threadIdx.x] = 0;
    if (threadIdx.x == 0) consumed = 0;
    if (!chainer) load_round(0, wA, sA);
    __syncthreads();

    float facc = 0.0f;   // chain accumulator (chain wave)
    int gsum = 0;        // EPI_GRP: open group's integer sum
    int isum = 0;        // EPI_ROW: exact integer sum
    if (!chainer) {
#pragma unroll 1
        for (int c = 0; c < nrounds; ++c) {
            if (c > 0) load_round(c, wA, sA);
            compute_round(c, wA, sA);
        }
    } else {
#pragma unroll 1
        for (int c = 0; c < nrounds; ++c) {
            spin_until_geq(&produced[c % GEMV_RING], NW * (c / GEMV_RING + 1), a.spin_limit, a.wait_failed);
            const int slot = (c % GEMV_RING) * SLOT;
            const int lo = c * RB, n = min(nb, lo + RB) - lo;
            const float *fr = lds_f + slot + lane;   // block q of the round at [q * 64]
            const DT *dr = lds_d + slot + lane;
            auto apply = [&](int b, int d, float f) {
                if constexpr (EPI == EPI_ROW) {
                    isum += d;
                } else if constexpr (EPI == EPI_B32) {
                    facc = __fmaf_rn(f, (float)d, facc);
                } else {
                    gsum += d;
                    if (grp_end(b, g.gshift, g.nb)) {
                        facc = __fadd_rn(facc, __fmul_rn((float)gsum, f));
                        gsum = 0;
                    }
                }
            };
            if (a.dots) {   // debug: also record every block dot
                for (int q = 0; q < n; ++q) {
                    const int d = (int)dr[q * 64];
                    if (o < g.O)
                        a.dots[(((size_t)r * (GATEUP ? 2 : 1) + (GATEUP ? mat : 0)) * g.O + o) * g.nb + lo + q] = d;
                    apply(lo + q, d, EPI == EPI_ROW ? 0.0f : fr[q * 64]);
                }
            } else {
                int q = 0;
                for (; q + 16 <= n; q += 16) {
                    int dd[16];
                    float ff[16];
#pragma unroll
                    for (int j = 0; j < 16; ++j) {
                        dd[j] = (int)dr[(q + j) * 64];
                        ff[j] = EPI == EPI_ROW ? 0.0f : fr[(q + j) * 64];
                    }
#pragma unroll
                    for (int j = 0; j < 16; ++j) apply(lo + q + j, dd[j], ff[j]);
                }
                for (; q < n; ++q) apply(lo + q, (int)dr[q * 64], EPI == EPI_ROW ? 0.0f : fr[q * 64]);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            if (lane == 0) __hip_atomic_store(&consumed, c + 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
    }

    if (!chainer) return;
    float v;
    if constexpr (EPI == EPI_ROW) {
        const float sc = W4 ? __fmul_rn(sp[0], 16.0f) : sp[0];   // per-row scale
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
            if (!(EPI == EPI_B32 && a.hq)) a.out[(size_t)r * a.out_stride + o] = h;   // else only hq / sh are read
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
        if (!a.tail_out) {
            if (o < g.O) a.out[(size_t)r * a.out_stride + o] = v;
        } else {
            if (o < g.O) __hip_atomic_store(&a.out[(size_t)r * a.out_stride + o], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            tail_combine(a, g.O, nrows, o, (int)blockIdx.x);
        }
    }
}

// ---------------------------------------------------------------------------
// Split-K decode GEMV. A unit is one row and one output tile (32 gate + 32 up
// channels, or 64 down channels); its K blocks are spread over `split`
// workgroups of split_kb blocks, so a one-token layer runs on many more
// workgroups than it has tiles (config 1's gate/up has 48 tiles for 256 CUs).
//
// Streaming: wave w of workgroup s takes blocks s*kb + w*CH + [0, CH), issues
// its weight, scale and activation loads as one batch and turns each block
// into its exact integer dot and its f32 factor (sw*sx[b] for 32-block
// activation scales, sw for grouped weights), exactly as gemv_kernel's
// streaming waves do. It parks them in part_d / part_f (int4 dots fit 16
// bits, so two blocks share a dword) and the workgroup counts in on the
// unit's counter.
//
// The chain: the workgroup that completes the count loads the unit's pairs
// (wave w holds blocks [w*SEG, (w+1)*SEG)) and runs the one ascending f32
// chain of idot.rs:82-88 over them, wave after wave, handing the running
// value over through LDS; then the epilogue (SwiGLU and the h quantisation,
// or the y store and the one-token tail combine). The arithmetic is the
// unsplit kernel's, step for step, so the bits are too.
//
// Visibility across XCDs, the tail combine's scheme: the pairs are written
// with the device-scope cache policy (SC1, what agent-scope atomic stores
// compile to: written through the XCD's L2), every wave waits for its stores
// (vmcnt 0) before the workgroup barrier that precedes the agent-scope
// counter add, and the finishing workgroup reads the pairs with SC1 loads
// (coherent reads, as agent-scope atomic loads) issued after the add
// returned. As plain buffer operations rather than atomics they are issued
// as one batch: atomic loads were serialised one round trip each (config 1's
// split down projection took 19 us instead of 5). Nothing waits on another
// workgroup, so no dispatch order is assumed. The finisher resets the
// counter to 0 for the next dispatch.
// ---------------------------------------------------------------------------
template <bool W4, int EPI, bool GATEUP, int CH>
__global__ __launch_bounds__(1024) void gemv_split_kernel(DotArgs a, MatGeom g, const int8_t *__restrict__ xq,
                                                          const float *__restrict__ sxv) {
    static_assert(CH % 2 == 0, "int4 dots are parked in pairs of blocks");
    constexpr int BB = W4 ? 16 : 32;
    constexpr int SEGMAX = GEMV_SPLIT_SEG;
    __shared__ float hand_f[64];   // the chain's running value between waves
    __shared__ int hand_i[64];     // and its open integer sum (per-row / grouped weights)
    __shared__ int is_last;

    const int lane = threadIdx.x & 63, wave = wave_id(), nw = (int)blockDim.x >> 6;
    const int S = a.split, kb = a.split_kb, nb = g.nb;
    const int u = (int)blockIdx.x / S, s = (int)blockIdx.x - u * S, r = blockIdx.y;
    const int nrows = a.n_rows_fixed >= 0 ? a.n_rows_fixed : a.plan.counts[0];
    if (r >= nrows) return;   // uniform: fewer rows than the grid bound
    const int ntx = (int)gridDim.x / S;
    const size_t unit = (size_t)r * ntx + u;
    const int nbd = W4 ? (nb + 1) >> 1 : nb;   // dwords of parked dots per lane
    // this unit's parked pairs, [block][64 lanes] (int4 dots: [block pair][64]),
    // through buffer resources: offsets are lane*4 + block*256
    const auto rd = make_rsrc(a.part_d + unit * nbd * 64, (uint32_t)nbd * 256);
    const auto rf = make_rsrc(EPI == EPI_ROW ? (const void *)a.part_d : (const void *)(a.part_f + unit * nb * 64),
                              (uint32_t)nb * 256);
    const int lo4 = lane * 4;

    const ExpertDesc *dsc = a.plan.row_desc ? &a.plan.row_desc[r] : &a.desc[a.plan.row_exp[r]];
    const int arow = a.act_identity ? r : (a.act_zero ? 0 : a.plan.row_act[r]);
    const int half = lane >> 5, ol = lane & 31;
    const int o = GATEUP ? u * 32 + ol : u * 64 + lane;
    const int mat = GATEUP ? half : 2;
    const int tile = GATEUP ? u : 2 * u + half;
    const auto *wp = gptr(dsc->w[mat] + ((size_t)tile * nb * TILE_O + ol) * BB);
    const auto *sp = gptr(dsc->sc[mat] + (size_t)tile * g.ng * TILE_O + ol);
    const CInt *xs = (const CInt *)(xq + (size_t)arow * a.x_stride);
    const CFloat *sxs = (const CFloat *)(sxv + (size_t)arow * a.sx_stride);

    // ---- streaming: this wave's CH blocks ----
    const int bw = s * kb + wave * CH;
    if (bw < nb) {   // uniform
        WBlk<W4> wv[CH];
        float sv[CH];
        int xr[CH][8];
        float sxr[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int b = min(bw + j, nb - 1);
            wv[j] = load_wblk<W4>((const uint8_t *)(wp + (size_t)b * (TILE_O * BB)));
            if constexpr (EPI != EPI_ROW) sv[j] = __builtin_nontemporal_load(&sp[(size_t)grp_of(b, g.gshift) * TILE_O]);
        }
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int b = min(bw + j, nb - 1);
#pragma unroll
            for (int q = 0; q < 8; ++q) xr[j][q] = xs[b * (BLK / 4) + q];
            if constexpr (EPI == EPI_B32) sxr[j] = sxs[b];
        }
        int dv[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            const int d16 = dot_wblk<W4>(wv[j], xr[j]);
            dv[j] = W4 ? (d16 >> 4) : d16;   // exact block dot
            if constexpr (EPI != EPI_ROW) {
                const float sw = W4 ? __fmul_rn(sv[j], 16.0f) : sv[j];   // W4 scale tables hold sw/16
                const float f = EPI == EPI_B32 ? __fmul_rn(sw, sxr[j]) : sw;
                if (bw + j < nb) __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(f), rf, lo4 + (bw + j) * 256, 0, BUF_SC1);
            }
        }
        if constexpr (W4) {
#pragma unroll
            for (int j = 0; j < CH; j += 2) {
                const int pk = (int)(((uint32_t)dv[j] & 0xFFFFu) | ((uint32_t)dv[j + 1] << 16));
                if (bw + j < nb) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)pk, rd, lo4 + ((bw + j) >> 1) * 256, 0, BUF_SC1);
            }
        } else {
#pragma unroll
            for (int j = 0; j < CH; ++j)
                if (bw + j < nb) __builtin_amdgcn_raw_buffer_store_b32((uint32_t)dv[j], rd, lo4 + (bw + j) * 256, 0, BUF_SC1);
        }
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's pairs are written through
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(&a.split_ctr[unit], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        is_last = old == S - 1;
        if (old == S - 1) __hip_atomic_store(&a.split_ctr[unit], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!is_last) return;   // uniform over the workgroup
    asm volatile("" ::: "memory");

    // ---- the chain, in the workgroup that completed the count ----
    const int seg = (((nb + nw - 1) / nw) + 1) & ~1;   // even: int4 pairs never straddle waves
    const int c0 = wave * seg, n = max(0, min(nb, c0 + seg) - c0);
    int dd[SEGMAX];
    float ff[SEGMAX];
    if constexpr (W4) {
#pragma unroll
        for (int i = 0; i < SEGMAX; i += 2) {   // unconditional, clamped: one batch of loads
            const int bd = min((c0 + i) >> 1, nbd - 1);
            const int pk = (int)__builtin_amdgcn_raw_buffer_load_b32(rd, lo4 + bd * 256, 0, BUF_SC1);
            dd[i] = (int)(short)(pk & 0xFFFF);
            dd[i + 1] = pk >> 16;
        }
    } else {
#pragma unroll
        for (int i = 0; i < SEGMAX; ++i)
            dd[i] = (int)__builtin_amdgcn_raw_buffer_load_b32(rd, lo4 + min(c0 + i, nb - 1) * 256, 0, BUF_SC1);
    }
#pragma unroll
    for (int i = 0; i < SEGMAX; ++i)
        ff[i] = EPI == EPI_ROW ? 0.0f
                               : __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rf, lo4 + min(c0 + i, nb - 1) * 256, 0,
                                                                                      BUF_SC1));
    float facc = 0.0f;
    int isum = 0;   // EPI_ROW: exact integer sum; EPI_GRP: the open group's sum
    for (int w = 0; w < nw; ++w) {
        if (wave == w && (w == 0 || c0 < nb)) {
            if (w > 0) {
                facc = hand_f[lane];
                isum = hand_i[lane];
            }
#pragma unroll
            for (int i = 0; i < SEGMAX; ++i) {
                if (i >= n) break;   // uniform
                const int b = c0 + i;
                if constexpr (EPI == EPI_ROW) {
                    isum += dd[i];
                } else if constexpr (EPI == EPI_B32) {
                    facc = __fmaf_rn(ff[i], (float)dd[i], facc);
                } else {
                    isum += dd[i];
                    if (grp_end(b, g.gshift, nb)) {
                        facc = __fadd_rn(facc, __fmul_rn((float)isum, ff[i]));
                        isum = 0;
                    }
                }
            }
            hand_f[lane] = facc;
            hand_i[lane] = isum;
        }
        __syncthreads();
    }
    if (wave != 0) return;
    facc = hand_f[lane];
    isum = hand_i[lane];
    float v;
    if constexpr (EPI == EPI_ROW) {
        const float sc = W4 ? __fmul_rn(sp[0], 16.0f) : sp[0];   // per-row scale
        v = __fmul_rn(__fmul_rn((float)isum, sc), sxs[0]);
    } else if constexpr (EPI == EPI_GRP) {
        v = __fmul_rn(facc, sxs[0]);
    } else {
        v = facc;
    }
    if constexpr (GATEUP) {
        const float uu = __shfl(v, (lane & 31) + 32);
        if (lane < 32) {
            const float h = silu_mul(v, uu);
            if (!(EPI == EPI_B32 && a.hq)) a.out[(size_t)r * a.out_stride + o] = h;   // else only hq / sh are read
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
        if (!a.tail_out) {
            if (o < g.O) a.out[(size_t)r * a.out_stride + o] = v;
        } else {
            if (o < g.O) __hip_atomic_store(&a.out[(size_t)r * a.out_stride + o], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            tail_combine(a, g.O, nrows, o, u);
        }
    }
}

GemvSplit plan_gemv_split(const MatGeom &g, bool gateup, int rows, int act, int target_wgs) {
    GemvSplit p;
    const int ntx = gateup ? (g.O + 31) / 32 : (g.O + 63) / 64;
    const long units = (long)rows * ntx;
    if (target_wgs <= 0 || rows < 1 || units > GEMV_SPLIT_UNITS) return p;
    const int nb = g.nb;
    int S = (int)std::min<long>(std::max<long>(target_wgs / units, 1), nb);
    if (S <= 1) return p;
    int kb = (nb + S - 1) / S;
    const int ch = kb >= 16 ? 4 : 2;
    // the finishing workgroup holds at most SEG blocks per wave for the chain
    const int nw_chain = (nb + GEMV_SPLIT_SEG - 1) / GEMV_SPLIT_SEG;
    int nw = std::max((kb + ch - 1) / ch, nw_chain);
    if (nw > 16) return p;
    kb = nw * ch;
    S = (nb + kb - 1) / kb;
    if (S <= 1) return p;
    p.split = S;
    p.kb = kb;
    p.nw = nw;
    p.ch = ch;
    p.part_d_bytes = (size_t)units * (g.w4 ? (nb + 1) / 2 : nb) * 64 * 4;
    const int epi = act == ACT_B32 ? EPI_B32 : (g.per_row ? EPI_ROW : EPI_GRP);
    p.part_f_bytes = epi == EPI_ROW ? 0 : (size_t)units * nb * 64 * 4;
    return p;
}

// One token, down projection and combine in one launch. A workgroup owns 16
// channels (half a weight tile) for all k slots; wave w streams slot w. Lane
// l takes channel l % 16 and one quarter of K (blocks [qQ, qQ + Q), q = l / 16,
// Q = ceil(nb / 4)), every block of the wave in flight at once. The slots'
// activation rows and scales are staged in LDS by loads issued before the
// weight loads (a wave's loads return in order). Lanes 0-15 then run each
// channel's exact f32 chain in ascending block order, as the chain wave of
// gemv_kernel does, taking the other quarters' (dot, factor) pairs by
// cross-lane reads. The router-weighted sum runs in slot order,
// out = (((0 + w0*y0) + w1*y1) + ...), the combine's order for one token
// (its rows in top-k order), so the result equals the separate down and
// combine launches bit for bit.
constexpr int DC_MAXK = 8, DC_CH = 12, DC_XLD = 6;   // blocks per lane; 8-byte activation loads per thread
constexpr int DC_MAXNB = 4 * DC_CH;                   // K <= 1536

template <bool W4, int EPI>
__global__ __launch_bounds__(64 * DC_MAXK) void gemv_down_combine_kernel(DotArgs a, MatGeom g, int k,
                                                                         const float *wts, float *out) {
    constexpr int BB = W4 ? 16 : 32, CH = DC_CH;
    __shared__ __attribute__((aligned(16))) int8_t xl[DC_MAXK * DC_MAXNB * BLK];   // [k][nb * 32]
    __shared__ float sxl[DC_MAXK * DC_MAXNB];                                     // [k][nsx]
    __shared__ float comb[DC_MAXK * 16];
    const int nb = g.nb, Kp = nb * BLK, Q = (nb + 3) >> 2;
    const int nsx = EPI == EPI_B32 ? nb : 1;
    const int tid = threadIdx.x, nth = blockDim.x, lane = tid & 63, r = tid >> 6;
    const int qd = lane >> 4, ol = lane & 15;
    // activation rows and scales: a fixed number of loads per thread, issued
    // first (clamped; the extra ones repeat the last element)
    const int nx8 = k * Kp / 8, nsxt = k * nsx;
    uint2 xv[DC_XLD];
#pragma unroll
    for (int u = 0; u < DC_XLD; ++u) {
        const int i = min(tid + u * nth, nx8 - 1), rr = i / (Kp / 8), off = i - rr * (Kp / 8);
        xv[u] = *(const uint2 *)(a.xq + (size_t)rr * a.x_stride + (size_t)off * 8);
    }
    float sv0;
    {
        const int i = min(tid, nsxt - 1), rr = i / nsx;
        sv0 = a.sx[(size_t)rr * a.sx_stride + (i - rr * nsx)];
    }
    const ExpertDesc *dsc = a.plan.row_desc ? &a.plan.row_desc[r] : &a.desc[a.plan.row_exp[r]];
    const int sl = blockIdx.x, t = sl >> 1, row = (sl & 1) * 16 + ol;
    const auto *wp = gptr(dsc->w[2] + ((size_t)t * nb * TILE_O + row) * BB);
    const auto *sp = gptr(dsc->sc[2] + (size_t)t * g.ng * TILE_O + row);
    const int bbeg = qd * Q;
    WBlk<W4> wv[CH];
    float sw[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {   // unconditional, clamped: one batch of loads
        const int b = min(bbeg + j, nb - 1);
        wv[j] = load_wblk<W4>((const uint8_t *)(wp + (size_t)b * (TILE_O * BB)));
        if constexpr (EPI != EPI_ROW) sw[j] = __builtin_nontemporal_load(&sp[(size_t)grp_of(b, g.gshift) * TILE_O]);
    }
#pragma unroll
    for (int u = 0; u < DC_XLD; ++u) {
        const int i = tid + u * nth;
        if (i < nx8) *(uint2 *)(xl + (size_t)i * 8) = xv[u];   // rows are packed at nb * 32 bytes
    }
    if (tid < nsxt) sxl[tid] = sv0;
    __syncthreads();
    const int *xr = (const int *)(xl + (size_t)r * Kp);
    const float *sxr = sxl + (size_t)r * nsx;
    // this lane's exact block dots and f32 factors
    int dv[CH];
    float fv[CH];
#pragma unroll
    for (int j = 0; j < CH; ++j) {
        const int b = min(bbeg + j, nb - 1);
        int xb[8];
        const int4 q0 = *(const int4 *)(xr + b * (BLK / 4)), q1 = *(const int4 *)(xr + b * (BLK / 4) + 4);
        xb[0] = q0.x; xb[1] = q0.y; xb[2] = q0.z; xb[3] = q0.w;
        xb[4] = q1.x; xb[5] = q1.y; xb[6] = q1.z; xb[7] = q1.w;
        const int d16 = dot_wblk<W4>(wv[j], xb);
        dv[j] = W4 ? (d16 >> 4) : d16;
        if constexpr (EPI != EPI_ROW) {
            const float s = W4 ? __fmul_rn(sw[j], 16.0f) : sw[j];   // W4 scale tables hold sw/16
            fv[j] = EPI == EPI_B32 ? __fmul_rn(s, sxr[b]) : s;
        } else {
            fv[j] = 0.0f;
        }
    }
    float facc = 0.0f;
    int gsum = 0, isum = 0;
    auto apply = [&](int b, int d, float f) {
        if constexpr (EPI == EPI_ROW) {
            isum += d;
        } else if constexpr (EPI == EPI_B32) {
            facc = __fmaf_rn(f, (float)d, facc);
        } else {
            gsum += d;
            if (grp_end(b, g.gshift, nb)) {
                facc = __fadd_rn(facc, __fmul_rn((float)gsum, f));
                gsum = 0;
            }
        }
    };
    // quarters in order; every lane runs the chain, lanes 0-15 keep it
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        int dq[CH];
        float fq[CH];
#pragma unroll
        for (int j = 0; j < CH; ++j) {
            dq[j] = q == 0 ? dv[j] : __shfl(dv[j], ol + 16 * q);
            fq[j] = q == 0 ? fv[j] : __shfl(fv[j], ol + 16 * q);
        }
#pragma unroll
        for (int j = 0; j < CH; ++j)
            if (j < Q && q * Q + j < nb) apply(q * Q + j, dq[j], fq[j]);
    }
    float v;
    if constexpr (EPI == EPI_ROW) {
        const float sc = W4 ? __fmul_rn(sp[0], 16.0f) : sp[0];   // per-row scale
        v = __fmul_rn(__fmul_rn((float)isum, sc), sxr[0]);
    } else if constexpr (EPI == EPI_GRP) {
        v = __fmul_rn(facc, sxr[0]);
    } else {
        v = facc;
    }
    if (lane < 16) comb[r * 16 + ol] = v;
    __syncthreads();
    const int o = sl * 16 + tid;
    if (tid < 16 && o < g.O) {
        float acc = 0.0f;
        for (int rr = 0; rr < k; ++rr) acc = __fadd_rn(acc, __fmul_rn(wts[rr], comb[rr * 16 + tid]));
        out[o] = acc;
    }
}

// whether the fused down + combine covers this shape: k slots, K blocks, and
// every activation byte within the fixed per-thread loads (8 B each)
bool gemv_down_combine_ok(const MatGeom &g, int k) {
    return k >= 1 && k <= DC_MAXK && g.nb <= DC_MAXNB && g.nb * BLK / 8 <= DC_XLD * 64;
}

template <bool W4, int EPI>
static void launch_dc(const DotArgs &a, const MatGeom &g, int k, const float *w, float *out, hipStream_t st) {
    const dim3 grid((unsigned)((g.O + 15) / 16)), block((unsigned)(64 * k));
    launch_k((gemv_down_combine_kernel<W4, EPI>), grid, block, 0, st, a, g, k, w, out);
}

void launch_gemv_down_combine(const DotArgs &a, const MatGeom &g, int act, int k, const float *w, float *out,
                              hipStream_t st) {
    const int epi = act == ACT_B32 ? EPI_B32 : (g.per_row ? EPI_ROW : EPI_GRP);

    if (g.w4) {
        if (epi == EPI_ROW) launch_dc<true, EPI_ROW>(a, g, k, w, out, st);
        else if (epi == EPI_GRP) launch_dc<true, EPI_GRP>(a, g, k, w, out, st);
        else launch_dc<true, EPI_B32>(a, g, k, w, out, st);
    } else {
        if (epi == EPI_ROW) launch_dc<false, EPI_ROW>(a, g, k, w, out, st);
        else if (epi == EPI_GRP) launch_dc<false, EPI_GRP>(a, g, k, w, out, st);
        else launch_dc<false, EPI_B32>(a, g, k, w, out, st);
    }
}

static int g_lds_limit = 64 * 1024;
void set_lds_limit(int bytes) { g_lds_limit = bytes > 0 ? bytes : 64 * 1024; }

// int4 gate/up: 11 streaming waves + 1 chain wave (768 threads), 5 blocks per
// wave per round; int8 gate/up: 7 + 1 waves, 4 blocks; down: 3 + 1 waves, 8
// int4 (4 int8) blocks. Measured on config 2, the int4 gate/up as 11 x 5
// took 18.6 us against 19.3 us as 7 x 8 (about the same 55-56 blocks per
// round); 13 x 4 and 15 x 4 were slower.
template <bool W4, int EPI, bool GATEUP, int CH, bool ROUTE>
static void launch_gemv_c(const DotArgs &a, const MatGeom &g, int grid_rows, hipStream_t st) {
    constexpr int NW = GATEUP ? (W4 ? 11 : 7) : 3;
    // the fused router keeps the expert descriptor table after the ring
    const size_t lds = gemv_ring_bytes<W4, NW, CH>() + (ROUTE ? (size_t)a.route.E * sizeof(ExpertDesc) : 0);
    auto kern = gemv_kernel<W4, EPI, GATEUP, NW, CH, ROUTE>;
    static size_t opted[LDS_OPT_DEVICES];
    lds_opt_in((const void *)kern, lds, opted);
    dim3 grid(GATEUP ? (unsigned)((g.O + 31) / 32) : (unsigned)((g.O + 63) / 64), (unsigned)grid_rows);
    launch_k(kern, grid, dim3((NW + 1) * 64), lds, st, a, g, a.xq, a.sx);
}

template <bool W4, int EPI, bool GATEUP>
static void launch_gemv_t(const DotArgs &a, const MatGeom &g, int grid_rows, hipStream_t st) {
    if (a.split > 1) {
        const int ntx = GATEUP ? (g.O + 31) / 32 : (g.O + 63) / 64;
        const int ch = a.split_kb / a.split_nw;
        const dim3 grid((unsigned)(ntx * a.split), (unsigned)grid_rows), block((unsigned)(64 * a.split_nw));
        if (ch == 4) launch_k((gemv_split_kernel<W4, EPI, GATEUP, 4>), grid, block, 0, st, a, g, a.xq, a.sx);
        else launch_k((gemv_split_kernel<W4, EPI, GATEUP, 2>), grid, block, 0, st, a, g, a.xq, a.sx);
        return;
    }
    if constexpr (GATEUP) {
        if (a.route.logits) {
            launch_gemv_c<W4, EPI, GATEUP, W4 ? 5 : 4, true>(a, g, grid_rows, st);
            return;
        }
    }
    launch_gemv_c<W4, EPI, GATEUP, W4 ? (GATEUP ? 5 : 8) : 4, false>(a, g, grid_rows, st);
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
