// kernels_misc.hip — activation quantisation, weight repack at upload, the
// device router, the expert-offset table and the fixed-order combine.
#include <climits>

#include <algorithm>

#include "common.h"
#include "route.h"

namespace phip {

// ---------------------------------------------------------------------------
// Activation quantisation: qrow_i8 (peregrine-kernels/src/quant.rs:14-33) per
// row (ACT_ROW) or per 32-element block (ACT_B32). One 256-thread workgroup per
// row. Output bytes go to the permuted device layout (perm8) and the row is
// zero-padded to Kp, so padded weight columns contribute nothing. A host-
// buffer call's kernels also stage its metadata from mapped host memory
// (a.copy_*), spread over the grid.
// ---------------------------------------------------------------------------
__device__ __forceinline__ void quant_side_copy(const QuantArgs &a) {
    if (a.copy_n16 <= 0) return;
    const int nwg = (int)(gridDim.x * gridDim.y), wg = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    for (int i = wg * (int)blockDim.x + (int)threadIdx.x; i < a.copy_n16; i += nwg * (int)blockDim.x)
        a.copy_dst[i] = a.copy_src[i];
}

__global__ __launch_bounds__(1024) void quant_rows_kernel(QuantArgs a) {
    quant_side_copy(a);
    // ACT_ROW: one workgroup per row; every thread loads its elements in one
    // round, then a block reduction gives the row's amax.
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *x = a.x + (size_t)row * a.x_stride;
    int8_t *q = a.q + (size_t)row * a.q_stride;
    __shared__ float red[16];
    constexpr int PER = 8;
    float v[PER];
    float m = 0.0f;
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int k = tid + j * 1024;
        v[j] = k < a.K ? x[k] : 0.0f;
        m = fmaxf(m, fabsf(v[j]));
    }
    for (int k = tid + PER * 1024; k < a.K; k += 1024) m = fmaxf(m, fabsf(x[k]));
    m = warp_max(m, 64);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = red[0];
    for (int w = 1; w < 16; w++) m = fmaxf(m, red[w]);
    float s = __fdiv_rn(m, 127.0f);
    if (s < 1e-12f) s = 1e-12f;
    const float inv = __fdiv_rn(1.0f, s);
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int k = tid + j * 1024;
        if (k < a.Kp) q[perm8(k)] = (int8_t)(int)rintf(__fmul_rn(v[j], inv));
    }
    for (int k = tid + PER * 1024; k < a.Kp; k += 1024) {
        const float xv = k < a.K ? x[k] : 0.0f;
        q[perm8(k)] = (int8_t)(int)rintf(__fmul_rn(xv, inv));
    }
    if (tid == 0) a.s[(size_t)row * a.s_stride] = s;
}

__global__ __launch_bounds__(256) void quant_blocks_kernel(QuantArgs a) {
    quant_side_copy(a);
    // ACT_B32: 8 elements per thread, a workgroup covers 64 blocks of one row
    const int row = blockIdx.y, nbk = a.Kp / BLK;
    const int b_lo = blockIdx.x * 64, b_hi = min(nbk, b_lo + 64);
    quant_row_b32(a.x + (size_t)row * a.x_stride, a.K, a.Kp, a.q + (size_t)row * a.q_stride,
                  a.s + (size_t)row * a.s_stride, 4 * b_lo, 4 * b_hi, threadIdx.x, 256);
}

void launch_quant_rows(const QuantArgs &a, hipStream_t st) {
    if (a.rows <= 0) return;
    if (a.mode == ACT_ROW) {
        launch_k(quant_rows_kernel, dim3(a.rows), dim3(1024), 0, st, a);
    } else {
        const int nb = a.Kp / BLK;
        launch_k(quant_blocks_kernel, dim3((unsigned)((nb + 63) / 64), (unsigned)a.rows), dim3(256), 0, st,
                           a);
    }
}

// ---------------------------------------------------------------------------
// Upload repack: QT row-major bytes -> the tiled device layout.
//   int4: XOR 0x88 turns the biased nibbles (v+8) into two's-complement
//         nibbles (the conversion cuda/backend_cuda.cu:114-116 also makes);
//         the 16 bytes of each 32-block keep QT's nibble order.
//   int8: each 8-element group is permuted to perm8 order so it lines up with
//         the activation layout.
// Scales become [Op/32][ng][32]; int4 scales are stored divided by 16 because
// the unpacked int4 operands carry a factor 16 (exact: a power of two).
// ---------------------------------------------------------------------------
__global__ void repack_kernel(const uint8_t *raw, const float *raw_sc, int fmt, int I, int O, int gs, uint8_t *w,
                              float *sc, MatGeom g) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)g.Op * g.nb;
    if (idx >= total) return;
    const int o = (int)(idx / g.nb), b = (int)(idx % g.nb);
    const int t = o / TILE_O, ol = o % TILE_O;
    const bool grouped = (fmt == 4 || fmt == 8);
    if (g.w4) {
        const size_t rb = (size_t)(I + 1) / 2;
        uint8_t out[16];
        for (int j = 0; j < 16; j++) {
            const size_t bi = (size_t)b * 16 + j;
            uint8_t v = 0;
            if (o < O && bi < rb) {
                v = raw[(size_t)o * rb + bi] ^ 0x88;
                if (2 * bi + 1 >= (size_t)I) v &= 0x0F;  // element I of an odd row is padding
            }
            out[j] = v;
        }
        uint4 *dst = (uint4 *)(w + (((size_t)t * g.nb + b) * TILE_O + ol) * 16);
        *dst = *(const uint4 *)out;
    } else {
        uint8_t out[32];
        for (int j = 0; j < 32; j++) {
            const size_t k = (size_t)b * 32 + j;
            uint8_t v = 0;
            if (o < O && k < (size_t)I) v = raw[(size_t)o * I + k];
            out[(j & ~7) | ((j & 1) << 2) | ((j & 7) >> 1)] = v;
        }
        uint4 *dst = (uint4 *)(w + (((size_t)t * g.nb + b) * TILE_O + ol) * 32);
        dst[0] = *(const uint4 *)out;
        dst[1] = *(const uint4 *)(out + 16);
    }
    if (b < g.ng) {
        float v = 0.0f;
        if (o < O) v = grouped ? raw_sc[(size_t)o * g.ng + b] : raw_sc[o];
        if (g.w4) v = v * 0.0625f;
        sc[((size_t)t * g.ng + b) * TILE_O + ol] = v;
    }
    (void)gs;
}

void launch_repack(const uint8_t *raw, const float *raw_sc, int fmt, int I, int O, int gs, uint8_t *w, float *sc,
                   const MatGeom &g, hipStream_t st) {
    const size_t total = (size_t)g.Op * g.nb;
    launch_k(repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, raw, raw_sc, fmt, I,
                       O, gs, w, sc, g);
}

// ---------------------------------------------------------------------------
// Combine: grouped_reduce (cuda/backend_cuda.cu:151-160) — out[s,d] sums
// rw[k]*y[k,d] over its rows in a fixed order, rounded multiply then rounded
// add, no atomics. CSR form (row_ptr != null) or the device table's padded
// form (row_ptr == null: k slots per token, -1 terminates).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void combine_csr_kernel(float *out, const float *y, const int *row_ptr,
                                                          const int *row_idx, const float *rw, int D, int y_stride) {
    const int s = blockIdx.y;
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= D) return;
    float acc = 0.0f;
    for (int j = row_ptr[s]; j < row_ptr[s + 1]; j++) {
        const int r = row_idx[j];
        acc = __fadd_rn(acc, __fmul_rn(rw[r], y[(size_t)r * y_stride + d]));
    }
    out[(size_t)s * D + d] = acc;
}

// Device-table form: token s adds its rows tok_rows[s*k + j] (union order,
// -1 terminates) weighted by w[s*k + tok_kk[s*k + j]] — the reference scatter
// out[s] += w * y (mlp.rs:111-119) from a zero row.
// out[s] = sum over the token's rows in batch-union order of w * y[row]
// (mul then add, from 0). Four channels per thread; the token's row indices
// and weights are the same for the whole workgroup (scalar loads), and every
// y load is issued before the in-order sum.
__global__ __launch_bounds__(256) void combine_tok_kernel(float *out, const float *y, const int *tok_rows,
                                                          const int *tok_kk, const float *w, int k, int D,
                                                          int y_stride, int vec4) {
    const int s = blockIdx.y;
    const int d0 = (blockIdx.x * 256 + threadIdx.x) * 4;
    // The token's row list and weights: every index load is issued before
    // any is used (clamped, unconditional), then every weight load.
    int rr[16], kq[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        const int jj = min(j, k - 1);
        rr[j] = tok_rows ? tok_rows[(size_t)s * k + jj] : jj;
        kq[j] = tok_kk ? tok_kk[(size_t)s * k + jj] : jj;
    }
    int n = 0;   // rows up to the first -1
#pragma unroll
    for (int j = 0; j < 16; j++) n += (j < k && n == j && rr[j] >= 0) ? 1 : 0;
    float ww[16];
#pragma unroll
    for (int j = 0; j < 16; j++) ww[j] = w[(size_t)s * k + (j < n ? kq[j] : 0)];
    if (d0 >= D) return;
    if (vec4) {   // D and the row strides are multiples of 4
        float4 yv[16];
#pragma unroll
        for (int j = 0; j < 16; j++)   // past n: row 0, read and ignored (no waits between loads)
            if (j < k) {   // y is read once: non-temporal (config 4: 67 -> 60 us)
                typedef float f4v __attribute__((ext_vector_type(4)));
                const f4v t = __builtin_nontemporal_load((const f4v *)(y + (size_t)(j < n ? rr[j] : 0) * y_stride + d0));
                yv[j] = make_float4(t.x, t.y, t.z, t.w);
            }
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int j = 0; j < 16; j++) {
            if (j < n) {
                acc.x = __fadd_rn(acc.x, __fmul_rn(ww[j], yv[j].x));
                acc.y = __fadd_rn(acc.y, __fmul_rn(ww[j], yv[j].y));
                acc.z = __fadd_rn(acc.z, __fmul_rn(ww[j], yv[j].z));
                acc.w = __fadd_rn(acc.w, __fmul_rn(ww[j], yv[j].w));
            }
        }
        *(float4 *)(out + (size_t)s * D + d0) = acc;
    } else {
        for (int d = d0; d < min(D, d0 + 4); d++) {
            float acc = 0.0f;
            for (int j = 0; j < n; j++) acc = __fadd_rn(acc, __fmul_rn(ww[j], y[(size_t)rr[j] * y_stride + d]));
            out[(size_t)s * D + d] = acc;
        }
    }
}

void launch_combine(float *out, const float *y, const int *row_ptr, const int *row_idx, const float *rw, int s_n,
                    int D, int y_stride, hipStream_t st) {
    if (s_n <= 0) return;
    launch_k(combine_csr_kernel, dim3((unsigned)((D + 255) / 256), (unsigned)s_n), dim3(256), 0, st, out,
                       y, row_ptr, row_idx, rw, D, y_stride);
}

void launch_combine_tok(float *out, const float *y, const int *tok_rows, const int *tok_kk, const float *w, int s_n,
                        int k, int D, int y_stride, hipStream_t st) {
    if (s_n <= 0) return;
    const int vec4 = (D % 4 == 0 && y_stride % 4 == 0) ? 1 : 0;
    launch_k(combine_tok_kernel, dim3((unsigned)((D + 1023) / 1024), (unsigned)s_n), dim3(256), 0, st, out,
                       y, tok_rows, tok_kk, w, k, D, y_stride, vec4);
}

// ---------------------------------------------------------------------------
// The reference's own router (peregrine-model/src/router.rs:52-170, after
// the router matmul), one wavefront per token: sigmoid scores (exp evaluated
// as glibc expf), greedy top-k over score + bias with the same argmax rounds,
// weight = the winner's sigmoid; unfilled slots (0, 0); the negligible tail
// (router.rs:191-209) dropped when min_share > 0; optional renormalisation
// over all k slots (+1e-20, summed in slot order); times routed_scale.
template <int PER>
__global__ __launch_bounds__(64) void route_sigmoid_kernel(const float *logits, const float *bias, int E, int k,
                                                           int norm_topk, float routed_scale, float min_share,
                                                           int *ids_out, float *w_out, int *keff_out) {
    const int s = blockIdx.x, lane = threadIdx.x & 63;
    const float *l = logits + (size_t)s * E;
    float ve[PER], sg[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int e = lane + 64 * j;
        float c = -INFINITY, sig = 0.0f;
        if (e < E) {
            sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_glibc(-l[e])));
            c = __fadd_rn(sig, bias ? bias[e] : 0.0f);
        }
        sg[j] = sig;
        ve[j] = c > -INFINITY ? c : -INFINITY;   // NaN and -inf never qualify
    }
    float myw = 0.0f;
    int myid = 0, kept = 0;
    for (int kk = 0; kk < k; kk++) {
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (ve[j] > bv) {
                bv = ve[j];
                bi = lane + 64 * j;
            }
        wave_argmax(bv, bi);
        if (!(bv > -INFINITY)) break;   // uniform: nothing valid remains
        float cand = 0.0f;
#pragma unroll
        for (int j = 0; j < PER; j++)
            if (j == (bi >> 6)) cand = sg[j];
        const float wsel = __shfl(cand, bi & 63);   // the winner's sigmoid
        if (lane == kk) {
            myw = wsel;
            myid = bi;
        }
        if ((bi & 63) == lane) {
#pragma unroll
            for (int j = 0; j < PER; j++)
                if (j == (bi >> 6)) ve[j] = -INFINITY;
        }
        kept++;
    }
    // negligible tail: a trailing run of kept weights under min_share of the
    // kept sum, at most kept - 1 (every lane computes the same, uniformly)
    int drop = 0;
    if (min_share > 0.0f && kept > 1) {
        float sum = 0.0f;
        for (int i = 0; i < kept; i++) sum = __fadd_rn(sum, __shfl(myw, i));
        if (isfinite(sum) && sum > 0.0f) {
            while (drop < kept - 1) {
                const float wi = __shfl(myw, kept - 1 - drop);
                if (__fdiv_rn(wi, sum) >= min_share) break;
                drop++;
            }
        }
    }
    kept -= drop;
    if (lane >= kept) {
        myw = 0.0f;
        myid = 0;
    }
    if (norm_topk) {
        float sm = 0.0f;
        for (int i = 0; i < k; i++) sm = __fadd_rn(sm, __shfl(myw, i));
        sm = __fadd_rn(sm, 1e-20f);
        myw = __fdiv_rn(myw, sm);
    }
    myw = __fmul_rn(myw, routed_scale);
    if (lane < k) {
        ids_out[(size_t)s * k + lane] = myid;
        w_out[(size_t)s * k + lane] = myw;
    }
    if (lane == 0 && keff_out) keff_out[s] = kept;
}

void launch_route_sigmoid(const float *logits, const float *bias, int S, int E, int k, int norm_topk,
                          float routed_scale, float min_share, int *ids, float *w, int *keff, hipStream_t st) {
    if (S <= 0) return;
    const dim3 g((unsigned)S), b(64);
#define PHIP_ROUTE_SIG(P) \
    launch_k(route_sigmoid_kernel<P>, g, b, 0, st, logits, bias, E, k, norm_topk, routed_scale, min_share, \
                       ids, w, keff)
    if (E <= 64) PHIP_ROUTE_SIG(1);
    else if (E <= 128) PHIP_ROUTE_SIG(2);
    else if (E <= 256) PHIP_ROUTE_SIG(4);
    else if (E <= 512) PHIP_ROUTE_SIG(8);
    else PHIP_ROUTE_SIG(16);
#undef PHIP_ROUTE_SIG
}

template <int PER>
__global__ __launch_bounds__(64) void route_softmax_kernel(const float *logits, int E, int k, int *ids, float *w) {
    const int s = blockIdx.x;
    route_token<PER>(logits + (size_t)s * E, E, k, ids + (size_t)s * k, w + (size_t)s * k, nullptr, nullptr);
}

// Router fused with the activation quantisation of the same token. Grid
// (S, quant slabs): workgroup (s, 0) routes token s with its first wave; every
// workgroup quantises its slab of token s (ACT_B32: 8 blocks, one element per
// thread; ACT_ROW: one slab holds the whole row). Same arithmetic as
// quant_rows_kernel / quant_blocks_kernel.
template <int PER>
__global__ __launch_bounds__(256) void route_quant_kernel(const float *logits, int E, int k, int *ids, float *w,
                                                          QuantArgs a, const ExpertDesc *desc,
                                                          ExpertDesc *row_desc) {
    __shared__ float red[4];
    const int s = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = wave_id();
    if (blockIdx.y == 0 && wave == 0) {
        route_token<PER>(logits + (size_t)s * E, E, k, ids + (size_t)s * k, w + (size_t)s * k, desc,
                         row_desc ? row_desc + (size_t)s * k : nullptr);
    }
    const float *x = a.x + (size_t)s * a.x_stride;
    int8_t *q = a.q + (size_t)s * a.q_stride;
    if (a.mode == ACT_B32) {
        // this slab's 32-blocks, 8 elements per thread; in the routing
        // workgroup wave 0 routes while the other three quantise
        const int nbk = a.Kp / BLK;
        const int per = (nbk + (int)gridDim.y - 1) / (int)gridDim.y;
        const int b_lo = blockIdx.y * per, b_hi = min(nbk, b_lo + per);
        if (blockIdx.y == 0) {
            if (wave > 0) quant_row_b32(x, a.K, a.Kp, q, a.s + (size_t)s * a.s_stride, 4 * b_lo, 4 * b_hi, tid - 64, 192);
        } else {
            quant_row_b32(x, a.K, a.Kp, q, a.s + (size_t)s * a.s_stride, 4 * b_lo, 4 * b_hi, tid, 256);
        }
    } else {
        constexpr int PX = 32;   // K <= 8192 from registers, the rest re-read
        float v[PX];
        float m = 0.0f;
#pragma unroll
        for (int j = 0; j < PX; j++) {
            const int kx = tid + 256 * j;
            v[j] = kx < a.K ? x[kx] : 0.0f;
            m = fmaxf(m, fabsf(v[j]));
        }
        for (int kx = tid + 256 * PX; kx < a.K; kx += 256) m = fmaxf(m, fabsf(x[kx]));
        m = warp_max(m, 64);
        if (lane == 0) red[tid >> 6] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        float sc = __fdiv_rn(m, 127.0f);
        if (sc < 1e-12f) sc = 1e-12f;
        const float inv = __fdiv_rn(1.0f, sc);
#pragma unroll
        for (int j = 0; j < PX; j++) {
            const int kx = tid + 256 * j;
            if (kx < a.Kp) q[perm8(kx)] = (int8_t)(int)rintf(__fmul_rn(v[j], inv));
        }
        for (int kx = tid + 256 * PX; kx < a.Kp; kx += 256) {
            const float xv = kx < a.K ? x[kx] : 0.0f;
            q[perm8(kx)] = (int8_t)(int)rintf(__fmul_rn(xv, inv));
        }
        if (tid == 0) a.s[(size_t)s * a.s_stride] = sc;
    }
}

template <int PER>
static void route_quant_t(const float *logits, int S, int E, int k, int *ids, float *w, const QuantArgs &a,
                          const ExpertDesc *desc, ExpertDesc *row_desc, hipStream_t st) {
    // few tokens: spread a row over several workgroups (8 blocks each at one
    // token); many tokens: one workgroup per token
    const int nbk = a.Kp / BLK;
    const int slabs = a.mode == ACT_B32 ? std::max(1, std::min((nbk + 7) / 8, 256 / S)) : 1;
    launch_k(route_quant_kernel<PER>, dim3((unsigned)S, (unsigned)slabs), dim3(256), 0, st, logits, E, k,
                       ids, w, a, desc, row_desc);
}

void launch_route_quant(const float *logits, int S, int E, int k, int *ids, float *w, const QuantArgs &a,
                        const ExpertDesc *desc, ExpertDesc *row_desc, hipStream_t st) {
    if (S <= 0) return;
    if (E <= 64) route_quant_t<1>(logits, S, E, k, ids, w, a, desc, row_desc, st);
    else if (E <= 128) route_quant_t<2>(logits, S, E, k, ids, w, a, desc, row_desc, st);
    else if (E <= 256) route_quant_t<4>(logits, S, E, k, ids, w, a, desc, row_desc, st);
    else if (E <= 512) route_quant_t<8>(logits, S, E, k, ids, w, a, desc, row_desc, st);
    else route_quant_t<16>(logits, S, E, k, ids, w, a, desc, row_desc, st);
}

void launch_route_softmax(const float *logits, int S, int E, int k, int *ids, float *w, hipStream_t st) {
    if (S <= 0) return;
    const dim3 g((unsigned)S), b(64);
    if (E <= 64) launch_k(route_softmax_kernel<1>, g, b, 0, st, logits, E, k, ids, w);
    else if (E <= 128) launch_k(route_softmax_kernel<2>, g, b, 0, st, logits, E, k, ids, w);
    else if (E <= 256) launch_k(route_softmax_kernel<4>, g, b, 0, st, logits, E, k, ids, w);
    else if (E <= 512) launch_k(route_softmax_kernel<8>, g, b, 0, st, logits, E, k, ids, w);
    else launch_k(route_softmax_kernel<16>, g, b, 0, st, logits, E, k, ids, w);
}

// ---------------------------------------------------------------------------
// Expert-offset table, built on the device from router output, in the order
// peregrine's moe_forward uses (peregrine-model/src/mlp.rs:62-104):
//   experts in batch-union order (first seen over s ascending, kk ascending,
//   router.rs:420-445); an expert's rows in ascending (token, slot) order;
//   each token's contributions listed in union order, ties in slot order
//   (the order the scatter adds them).
// Also emits the 32-row M-tile list the MFMA arm walks. Three launches over
// chunks of whole tokens (at most 256 entries each): per-chunk counts, one
// scan over experts and chunks, per-chunk placement. Every step is a
// counting pass, so the result does not depend on thread timing.
// Limits: E <= 512, k <= 16.
// ---------------------------------------------------------------------------
// Inclusive scan across a wavefront: shifts of 1, 2, 4 and 8 lanes inside
// each row of 16 (DPP row_shr, zero fill), then the earlier rows' totals.
__device__ __forceinline__ int wave_inclusive_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
    const int r1 = __builtin_amdgcn_readlane(v, 15), r2 = __builtin_amdgcn_readlane(v, 31),
              r3 = __builtin_amdgcn_readlane(v, 47);
    const int row = (threadIdx.x & 63) >> 4;
    return v + (row >= 1 ? r1 : 0) + (row >= 2 ? r2 : 0) + (row >= 3 ? r3 : 0);
}

// Exclusive scan of one int per thread across a workgroup of up to 1024
// threads (wave scans, then a scan of the wave totals). Ends synchronised.
__device__ int block_exclusive_scan(int v, int *tmp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int inc = wave_inclusive_scan(v);
    __syncthreads();
    if (lane == 63) tmp[wave] = inc;
    __syncthreads();
    int wbase = 0;
    for (int w = 0; w < wave; w++) wbase += tmp[w];
    __syncthreads();
    return wbase + inc - v;
}

constexpr int TBL_MAXE = 512;
constexpr int TBL_CHUNK = 256;      // entries per chunk (whole tokens)
constexpr int TBL_TILE = 12288;     // (expert, chunk) counts one scan pass holds in LDS

// Per chunk g: cnt[g][e] = entries of expert e, first[g][e] = its first entry
// index (INT_MAX when none). Every (g, e) is written, so nothing needs clearing.
__global__ __launch_bounds__(TBL_CHUNK) void table_count_kernel(const int *ids, int N, int k, int E, int tpc,
                                                                int *firstg, int *cntg) {
    __shared__ int first[TBL_MAXE], cnt[TBL_MAXE];
    const int g = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < E; e += TBL_CHUNK) {
        first[e] = INT_MAX;
        cnt[e] = 0;
    }
    __syncthreads();
    const int i = g * tpc * k + tid;
    if (tid < tpc * k && i < N) {
        const int e = ids[i];
        if (e >= 0 && e < E) {
            atomicMin(&first[e], i);
            atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += TBL_CHUNK) {
        firstg[(size_t)g * E + e] = first[e];
        cntg[(size_t)g * E + e] = cnt[e];
    }
}

// Row offsets and M-tile offsets in union order, the M-tile list and the
// header, from the experts in union order (uex[0..n_u)) and their counts.
// base_out[e]: the expert's first row. ubuf: LDS for 2 * (n_u + 1) ints.
// Workgroup-wide; ends synchronised.
__device__ void table_offsets(int n_u, const int *uex, const int *cnt, int *base_out, const TableOut &t, int tmax,
                              int *scan_tmp, int *s_carry, int *ubuf) {
    const int tid = threadIdx.x, nth = blockDim.x;
    int *offs = ubuf, *mts = ubuf + n_u + 1;   // per union rank: first row, first M tile
    for (int u0 = 0; u0 < n_u; u0 += nth) {
        const int u = u0 + tid;
        const int c = u < n_u ? cnt[uex[u]] : 0;
        const int off = block_exclusive_scan(c, scan_tmp) + (u0 ? s_carry[0] : 0);
        const int mt = block_exclusive_scan((c + MT_ROWS - 1) / MT_ROWS, scan_tmp) + (u0 ? s_carry[1] : 0);
        if (u < n_u) {
            const int e = uex[u];
            base_out[e] = off;
            offs[u] = off;
            mts[u] = mt;
            t.uexp[u] = e;
            t.off[u] = off;
            if (u == n_u - 1) {
                offs[n_u] = off + c;
                mts[n_u] = mt + (c + MT_ROWS - 1) / MT_ROWS;
                t.off[n_u] = off + c;
                t.hdr[0] = off + c;
                t.hdr[1] = mt + (c + MT_ROWS - 1) / MT_ROWS;
                t.hdr[2] = n_u;
                t.hdr[3] = 0;
            }
        }
        __syncthreads();
        if (tid == nth - 1) {
            s_carry[0] = off + c;
            s_carry[1] = mt + (c + MT_ROWS - 1) / MT_ROWS;
        }
        __syncthreads();
    }
    if (n_u == 0) {
        if (tid == 0) {
            t.off[0] = 0;
            t.hdr[0] = t.hdr[1] = t.hdr[2] = t.hdr[3] = 0;
        }
        __syncthreads();
        return;
    }
    // the M-tile list, one tile per thread: its expert is the last union
    // rank whose first tile is at or before it (every present expert has one)
    const int T = min(mts[n_u], tmax);
    for (int q = tid; q < T; q += nth) {
        int lo = 0, hi = n_u - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (mts[mid] <= q) lo = mid;
            else hi = mid - 1;
        }
        t.mt_exp[q] = uex[lo];
        t.mt_row0[q] = offs[lo] + MT_ROWS * (q - mts[lo]);
        t.mt_rend[q] = offs[lo + 1];
        t.mt_first[q] = mts[lo];
    }
    __syncthreads();
}

// One workgroup: per expert, the first occurrence (min over chunks), the
// count, and in place of cnt[g][e] its exclusive prefix over chunks; then
// the union ranks (order of first occurrence), row offsets, M tiles and the
// header. ebase[e] = the expert's first row, erank[e] = its union rank.
__global__ __launch_bounds__(1024) void table_scan_kernel(int E, int G, const int *firstg, int *cntg, int *erank,
                                                          int *ebase, TableOut t, int tmax) {
    __shared__ int tile[TBL_TILE];
    __shared__ __attribute__((aligned(16))) int first[TBL_MAXE];
    __shared__ int cnt[TBL_MAXE], uex[TBL_MAXE];
    __shared__ int scan_tmp[32];
    __shared__ int s_carry[2], s_nu;
    const int tid = threadIdx.x, nth = blockDim.x;
    for (int e = tid; e < ((E + 3) & ~3); e += nth) {
        first[e] = INT_MAX;
        cnt[e] = 0;
    }
    if (tid == 0) s_nu = 0;
    __syncthreads();
    // passes over (chunk range, expert batch) tiles: load every count of the
    // tile at once (one memory latency per pass), then one thread per expert
    // walks its column of the tile; the running total stays in cnt[e]
    const int EB = min(E, nth), GW = max(1, TBL_TILE / EB);
    for (int g0 = 0; g0 < G; g0 += GW) {
        const int ng = min(GW, G - g0);
        for (int e0 = 0; e0 < E; e0 += EB) {
            const int ne = min(EB, E - e0);
            // all of a thread's loads first (at most TBL_TILE / nth each), then
            // the LDS work, so the loads overlap
            constexpr int PER = (TBL_TILE + 1023) / 1024;
            int cv[PER], fv[PER];
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int q = tid + j * nth;
                cv[j] = 0;
                fv[j] = INT_MAX;
                if (q < ne * ng) {
                    const int el = q % ne, gl = q / ne;   // consecutive threads: consecutive experts of one chunk
                    const size_t at = (size_t)(g0 + gl) * E + e0 + el;
                    cv[j] = cntg[at];
                    fv[j] = firstg[at];
                }
            }
#pragma unroll
            for (int j = 0; j < PER; j++) {
                const int q = tid + j * nth;
                if (q < ne * ng) {
                    tile[q] = cv[j];
                    if (fv[j] != INT_MAX) atomicMin(&first[e0 + q % ne], fv[j]);
                }
            }
            __syncthreads();
            if (tid < ne) {
                int run = cnt[e0 + tid];
#pragma unroll 8
                for (int gl = 0; gl < ng; gl++) {
                    const int c = tile[gl * ne + tid];
                    cntg[(size_t)(g0 + gl) * E + e0 + tid] = run;
                    run += c;
                }
                cnt[e0 + tid] = run;
            }
            __syncthreads();
        }
    }
    // union rank: experts present, ordered by first occurrence (distinct);
    // four first occurrences per LDS read, several reads in flight
    const int4 *f4 = (const int4 *)first;
    for (int e = tid; e < E; e += nth) {
        const int f = first[e];
        int r = -1;
        if (f != INT_MAX) {
            r = 0;
#pragma unroll 8
            for (int q = 0; q < (E + 3) >> 2; q++) {
                const int4 v = f4[q];
                r += (v.x < f) + (v.y < f) + (v.z < f) + (v.w < f);
            }
            uex[r] = e;
            atomicAdd(&s_nu, 1);
        }
        erank[e] = r;
    }
    __syncthreads();
    table_offsets(s_nu, uex, cnt, ebase, t, tmax, scan_tmp, s_carry, tile);   // the tile is free again
}

// Entry (tok, kk) of expert e (-1: invalid) at row r: its place among the
// token's rows, in union order with equal experts in slot order; invalid
// entries fill the tail in slot order. tid_e: the token's k expert ids.
__device__ __forceinline__ void table_token_slot(const int *tid_e, int tok, int kk, int k, int e, int r,
                                                 const int *rank, const TableOut &t) {
    const int ur = e >= 0 ? rank[e] : INT_MAX;
    int p = 0, nv = 0, inv_before = 0;
    for (int k2 = 0; k2 < k; k2++) {
        const int e2 = tid_e[k2];
        if (e2 >= 0) {
            nv++;
            const int r2 = rank[e2];
            p += r2 < ur || (r2 == ur && k2 < kk);
        } else if (k2 < kk) {
            inv_before++;
        }
    }
    const size_t at = (size_t)tok * k + (e >= 0 ? p : nv + inv_before);
    t.tok_rows[at] = r;
    t.tok_kk[at] = e >= 0 ? kk : 0;
}

// Per chunk g: an entry's row = its expert's first row + the expert's
// entries in earlier chunks + its earlier entries in this chunk (a popcount
// over the expert's entry mask); then its place among its token's rows.
__global__ __launch_bounds__(TBL_CHUNK) void table_place_kernel(const int *ids, int N, int k, int E, int tpc,
                                                                const int *pref, const int *erank,
                                                                const int *ebase, TableOut t) {
    constexpr int MW = TBL_CHUNK / 64;
    __shared__ int rank[TBL_MAXE], base[TBL_MAXE];
    __shared__ unsigned long long mask[TBL_MAXE * MW];
    __shared__ int sid[TBL_CHUNK];
    const int g = blockIdx.x, tid = threadIdx.x;
    for (int e = tid; e < E; e += TBL_CHUNK) {
        const int r = erank[e];
        rank[e] = r;
        base[e] = r >= 0 ? ebase[e] + pref[(size_t)g * E + e] : 0;   // absent experts: no base was written
#pragma unroll
        for (int w = 0; w < MW; w++) mask[e * MW + w] = 0ull;
    }
    const int i0 = g * tpc * k;
    const int n = min(N - i0, tpc * k);
    int e = -1;
    if (tid < n) {
        e = ids[i0 + tid];
        if (e < 0 || e >= E) e = -1;
        sid[tid] = e;
    }
    __syncthreads();
    if (e >= 0) atomicOr(&mask[e * MW + (tid >> 6)], 1ull << (tid & 63));
    __syncthreads();
    if (tid >= n) return;
    const int i = i0 + tid, tok = i / k, kk = i % k;
    int r = -1;
    if (e >= 0) {
        const unsigned long long *m = &mask[e * MW];
        int rk = __popcll(m[tid >> 6] & ((1ull << (tid & 63)) - 1ull));
        for (int w = 0; w < (tid >> 6); w++) rk += __popcll(m[w]);
        r = base[e] + rk;
        t.row_tok[r] = tok;
        t.row_kk[r] = kk;
        t.row_exp[r] = e;
    }
    table_token_slot(sid + (tid - kk), tok, kk, k, e, r, rank, t);   // chunks hold whole tokens
}

// Batches of at most TBL_SMALL entries in one launch, one entry per thread:
// union ranks from a scan over the first occurrences, an entry's rank among
// its expert's rows from a popcount over the expert's entry mask.
constexpr int TBL_SMALL = 512;
__global__ __launch_bounds__(TBL_SMALL) void table_small_kernel(const int *ids, int N, int k, int E, TableOut t,
                                                                int tmax) {
    constexpr int MW = TBL_SMALL / 64;
    __shared__ int sid[TBL_SMALL];
    __shared__ unsigned long long mask[TBL_MAXE * MW];
    __shared__ int first[TBL_MAXE], cnt[TBL_MAXE], uex[TBL_MAXE], rank[TBL_MAXE], base[TBL_MAXE];
    __shared__ int ubuf[2 * (TBL_MAXE + 1)];
    __shared__ int scan_tmp[32];
    __shared__ int s_carry[2], s_nu;
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += TBL_SMALL) {
        first[e] = INT_MAX;
        cnt[e] = 0;
        rank[e] = -1;
#pragma unroll
        for (int w = 0; w < MW; w++) mask[e * MW + w] = 0ull;
    }
    int e = -1;
    if (tid < N) {
        e = ids[tid];
        if (e < 0 || e >= E) e = -1;
        sid[tid] = e;
    }
    __syncthreads();
    if (e >= 0) {
        atomicMin(&first[e], tid);
        atomicAdd(&cnt[e], 1);
        atomicOr(&mask[e * MW + (tid >> 6)], 1ull << (tid & 63));
    }
    __syncthreads();
    const bool opens = e >= 0 && first[e] == tid;   // the expert's first entry
    const int u = block_exclusive_scan(opens, scan_tmp);
    if (opens) {
        rank[e] = u;
        uex[u] = e;
    }
    if (tid == TBL_SMALL - 1) s_nu = u + opens;
    __syncthreads();
    table_offsets(s_nu, uex, cnt, base, t, tmax, scan_tmp, s_carry, ubuf);
    if (tid >= N) return;
    const int tok = tid / k, kk = tid % k;
    int r = -1;
    if (e >= 0) {
        const unsigned long long *m = &mask[e * MW];
        int rk = __popcll(m[tid >> 6] & ((1ull << (tid & 63)) - 1ull));
        for (int w = 0; w < (tid >> 6); w++) rk += __popcll(m[w]);
        r = base[e] + rk;
        t.row_tok[r] = tok;
        t.row_kk[r] = kk;
        t.row_exp[r] = e;
    }
    table_token_slot(sid + (tid - kk), tok, kk, k, e, r, rank, t);
}

int table_chunks(int S, int k) {
    const int tpc = TBL_CHUNK / k;
    return (S + tpc - 1) / tpc;
}
size_t table_work_ints(int S, int k, int E) { return 2 * (size_t)table_chunks(S, k) * E + 2 * (size_t)E; }

void launch_build_table(const int *ids, int S, int k, int E, const TableOut &t, int tmax, int *work,
                        hipStream_t st) {
    const int tpc = TBL_CHUNK / k, G = table_chunks(S, k), N = S * k;
    if (N <= TBL_SMALL) {
        launch_k(table_small_kernel, dim3(1), dim3(TBL_SMALL), 0, st, ids, N, k, E, t, tmax);
        return;
    }
    int *firstg = work, *cntg = firstg + (size_t)G * E, *erank = cntg + (size_t)G * E, *ebase = erank + E;
    if (G > 0)
        launch_k(table_count_kernel, dim3(G), dim3(TBL_CHUNK), 0, st, ids, N, k, E, tpc, firstg, cntg);
    launch_k(table_scan_kernel, dim3(1), dim3(1024), 0, st, E, G, firstg, cntg, erank, ebase, t, tmax);
    if (G > 0)
        launch_k(table_place_kernel, dim3(G), dim3(TBL_CHUNK), 0, st, ids, N, k, E, tpc, cntg, erank, ebase,
                           t);
}

// ---------------------------------------------------------------------------
// Seeded synthetic fills for benchmarks and tests (not on the MoE path):
// element i draws from splitmix64(seed + i), so a buffer's contents depend
// only on (seed, index).
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__global__ void synth_fill_kernel(void *dst, size_t n, int kind, float a, float b, uint64_t seed) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;; i += stride) {
        if (kind == 0) {
            const size_t base = i * 8;
            if (base >= n) return;
            const uint64_t h = splitmix64(seed + i);
            uint8_t *d = (uint8_t *)dst;
            if (base + 8 <= n && (((uintptr_t)(d + base)) & 7) == 0) {
                *(uint64_t *)(d + base) = h;
            } else {
                for (int j = 0; j < 8 && base + j < n; j++) d[base + j] = (uint8_t)(h >> (8 * j));
            }
        } else {
            if (i >= n) return;
            const uint64_t h = splitmix64(seed + i);
            const double u1 = ((double)(h >> 11) + 1.0) * (1.0 / 9007199254740993.0);
            const double u2 = (double)(splitmix64(h) >> 11) * (1.0 / 9007199254740992.0);
            const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
            const double v = (double)a + (double)b * z;
            ((float *)dst)[i] = kind == 1 ? (float)v : (float)exp(v);
        }
    }
}

void launch_synth_fill(void *dst, size_t n, int kind, float a, float b, uint64_t seed, hipStream_t st) {
    if (n == 0) return;
    const size_t items = kind == 0 ? (n + 7) / 8 : n;
    size_t blocks = (items + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    launch_k(synth_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, n, kind, a, b, seed);
}

}  // namespace phip
