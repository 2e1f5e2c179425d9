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
// zero-padded to Kp, so padded weight columns contribute nothing.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void quant_rows_kernel(QuantArgs a) {
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
    // ACT_B32: each 32-lane half-wave owns one 32-block; one load per thread.
    const int row = blockIdx.y, tid = threadIdx.x;
    const int b = blockIdx.x * 8 + (tid >> 5), l32 = tid & 31;
    if (b * BLK >= a.Kp) return;
    const float *x = a.x + (size_t)row * a.x_stride;
    const int k = b * BLK + l32;
    const float v = k < a.K ? x[k] : 0.0f;
    const float m = warp_max(fabsf(v), 32);
    float s = __fdiv_rn(m, 127.0f);
    if (s < 1e-12f) s = 1e-12f;
    const float inv = __fdiv_rn(1.0f, s);
    a.q[(size_t)row * a.q_stride + perm8(k)] = (int8_t)(int)rintf(__fmul_rn(v, inv));
    if (l32 == 0) a.s[(size_t)row * a.s_stride + b] = s;
}

void launch_quant_rows(const QuantArgs &a, hipStream_t st) {
    if (a.rows <= 0) return;
    if (a.mode == ACT_ROW) {
        hipLaunchKernelGGL(quant_rows_kernel, dim3(a.rows), dim3(1024), 0, st, a);
    } else {
        const int nb = a.Kp / BLK;
        hipLaunchKernelGGL(quant_blocks_kernel, dim3((unsigned)((nb + 7) / 8), (unsigned)a.rows), dim3(256), 0, st,
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
    hipLaunchKernelGGL(repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, raw, raw_sc, fmt, I,
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

#ifdef PHIP_GEMV_TRACE
// debug timeline of the router/quant and combine kernels: [start, mid, end] per workgroup
__device__ long long *g_misc_trace;
void set_misc_trace(long long *p) { (void)hipMemcpyToSymbol(HIP_SYMBOL(g_misc_trace), &p, sizeof(p)); }
#define MISC_STAMP(slot, i) \
    do { if (g_misc_trace && threadIdx.x == 0) g_misc_trace[(slot) * 4 + (i)] = trace_stamp(); } while (0)
#else
#define MISC_STAMP(slot, i) do {} while (0)
#endif

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
    MISC_STAMP(1000 + blockIdx.x, 0);
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
            if (j < k) yv[j] = *(const float4 *)(y + (size_t)(j < n ? rr[j] : 0) * y_stride + d0);
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
        MISC_STAMP(1000 + blockIdx.x, 2);
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
    hipLaunchKernelGGL(combine_csr_kernel, dim3((unsigned)((D + 255) / 256), (unsigned)s_n), dim3(256), 0, st, out,
                       y, row_ptr, row_idx, rw, D, y_stride);
}

void launch_combine_tok(float *out, const float *y, const int *tok_rows, const int *tok_kk, const float *w, int s_n,
                        int k, int D, int y_stride, hipStream_t st) {
    if (s_n <= 0) return;
    const int vec4 = (D % 4 == 0 && y_stride % 4 == 0) ? 1 : 0;
    hipLaunchKernelGGL(combine_tok_kernel, dim3((unsigned)((D + 1023) / 1024), (unsigned)s_n), dim3(256), 0, st, out,
                       y, tok_rows, tok_kk, w, k, D, y_stride, vec4);
}

// ---------------------------------------------------------------------------
// The reference's own router (peregrine-model/src/router.rs:52-170, after
// the router matmul), one wavefront per token: sigmoid scores (exp evaluated
// as exp_cr), greedy top-k over score + bias with the same argmax rounds,
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
            sig = __fdiv_rn(1.0f, __fadd_rn(1.0f, exp_cr(-l[e])));
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
    hipLaunchKernelGGL(route_sigmoid_kernel<P>, g, b, 0, st, logits, bias, E, k, norm_topk, routed_scale, min_share, \
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
    MISC_STAMP(blockIdx.y, 0);
    if (blockIdx.y == 0 && wave == 0) {
        route_token<PER>(logits + (size_t)s * E, E, k, ids + (size_t)s * k, w + (size_t)s * k, desc,
                         row_desc ? row_desc + (size_t)s * k : nullptr);
        MISC_STAMP(blockIdx.y, 1);
    }
    const float *x = a.x + (size_t)s * a.x_stride;
    int8_t *q = a.q + (size_t)s * a.q_stride;
    if (a.mode == ACT_B32) {
        // this slab's 32-blocks; 8 lanes per block, 4 elements per lane, a
        // workgroup covers 32 blocks per step
        const int nbk = a.Kp / BLK;
        const int per = (nbk + (int)gridDim.y - 1) / (int)gridDim.y;
        const int b_lo = blockIdx.y * per, b_hi = min(nbk, b_lo + per);
        const int sub = lane & 7;
        for (int b = b_lo + wave * 8 + (lane >> 3); b - (wave * 8 + (lane >> 3)) < b_hi; b += 32) {
            const bool ok = b < b_hi;   // the same for the 8 lanes of a block
            float v[4];
            float m = 0.0f;
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const int kx = b * BLK + sub * 4 + t;
                v[t] = ok && kx < a.K ? x[kx] : 0.0f;
                m = fmaxf(m, fabsf(v[t]));
            }
            m = fmaxf(m, __shfl_xor(m, 1));
            m = fmaxf(m, __shfl_xor(m, 2));
            m = fmaxf(m, __shfl_xor(m, 4));
            float sc = __fdiv_rn(m, 127.0f);
            if (sc < 1e-12f) sc = 1e-12f;
            const float inv = __fdiv_rn(1.0f, sc);
            if (ok) {
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    const int kx = b * BLK + sub * 4 + t;
                    q[perm8(kx)] = (int8_t)(int)rintf(__fmul_rn(v[t], inv));
                }
                if (sub == 0) a.s[(size_t)s * a.s_stride + b] = sc;
            }
        }
        MISC_STAMP(blockIdx.y, 2);
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
    hipLaunchKernelGGL(route_quant_kernel<PER>, dim3((unsigned)S, (unsigned)slabs), dim3(256), 0, st, logits, E, k,
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
    if (E <= 64) hipLaunchKernelGGL(route_softmax_kernel<1>, g, b, 0, st, logits, E, k, ids, w);
    else if (E <= 128) hipLaunchKernelGGL(route_softmax_kernel<2>, g, b, 0, st, logits, E, k, ids, w);
    else if (E <= 256) hipLaunchKernelGGL(route_softmax_kernel<4>, g, b, 0, st, logits, E, k, ids, w);
    else if (E <= 512) hipLaunchKernelGGL(route_softmax_kernel<8>, g, b, 0, st, logits, E, k, ids, w);
    else hipLaunchKernelGGL(route_softmax_kernel<16>, g, b, 0, st, logits, E, k, ids, w);
}

// ---------------------------------------------------------------------------
// Expert-offset table, built on the device from router output, in the order
// peregrine's moe_forward uses (peregrine-model/src/mlp.rs:62-104):
//   experts in batch-union order (first seen over s ascending, kk ascending,
//   router.rs:420-445); an expert's rows in ascending token order; each token's
//   contributions listed in union order (the order the scatter adds them).
// Also emits the 32-row M-tile list the MFMA arm walks. One workgroup; every
// step is a counting pass, so the result does not depend on thread timing.
// The router ids are staged in LDS once; nothing written is read back.
// Limits: E <= 512, k <= 16 (ids beyond TBL_MAXN are read from global).
// ---------------------------------------------------------------------------
// Exclusive scan of one int per thread across a workgroup of up to 1024
// threads (wave scans, then a scan of the wave totals). Ends synchronised.
__device__ int block_exclusive_scan(int v, int *tmp) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    int inc = v;
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(inc, off);
        if (lane >= off) inc += o;
    }
    __syncthreads();
    if (lane == 63) tmp[wave] = inc;
    __syncthreads();
    int wbase = 0;
    for (int w = 0; w < wave; w++) wbase += tmp[w];
    (void)nw;
    __syncthreads();
    return wbase + inc - v;
}

constexpr int TBL_MAXE = 512;
constexpr int TBL_MAXN = 16384;

__global__ __launch_bounds__(1024) void build_table_kernel(const int *ids, int S, int k, int E, TableOut t,
                                                           int tmax) {
    __shared__ short sid[TBL_MAXN];
    __shared__ int first[TBL_MAXE], cnt[TBL_MAXE], rank[TBL_MAXE], fill[TBL_MAXE], uex[TBL_MAXE];
    __shared__ unsigned long long mask[TBL_MAXE * 4];   // [e][up to 4 words]: one pass's tokens
    __shared__ int scan_tmp[32];
    __shared__ int s_nu, s_carry[2];
    const int tid = threadIdx.x, nth = blockDim.x;
    const int N = S * k;
    const bool in_lds = N <= TBL_MAXN;
    auto id_at = [&](int i) -> int {
        const int e = in_lds ? (int)sid[i] : ids[i];
        return (e >= 0 && e < E) ? e : -1;
    };
    if (in_lds)
        for (int i = tid; i < N; i += nth) sid[i] = (short)max(-1, min(ids[i], 32767));
    for (int e = tid; e < E; e += nth) {
        first[e] = INT_MAX;
        cnt[e] = 0;
        mask[4 * e] = mask[4 * e + 1] = mask[4 * e + 2] = mask[4 * e + 3] = 0ull;
        rank[e] = -1;
    }
    __syncthreads();
    for (int i = tid; i < N; i += nth) {
        const int e = id_at(i);
        if (e >= 0) {
            atomicMin(&first[e], i);
            atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    // union rank = number of first occurrences before an expert's first
    // occurrence: flag first occurrences, then one block-wide scan over the
    // positions (each thread owns a contiguous run of them)
    {
        const int per = (N + nth - 1) / nth;
        const int lo = min(N, tid * per), hi = min(N, lo + per);
        int nf = 0;
        for (int i = lo; i < hi; i++) {
            const int e = id_at(i);
            nf += (e >= 0 && first[e] == i);
        }
        int base = block_exclusive_scan(nf, scan_tmp);
        for (int i = lo; i < hi; i++) {
            const int e = id_at(i);
            if (e >= 0 && first[e] == i) {
                rank[e] = base;
                uex[base] = e;
                base++;
            }
        }
        if (tid == nth - 1) s_nu = base;
    }
    __syncthreads();
    const int n_u = s_nu;
    // row offsets and M-tile offsets in union order (block scans over experts)
    for (int u0 = 0; u0 < n_u; u0 += nth) {
        const int u = u0 + tid;
        const int c = u < n_u ? cnt[uex[u]] : 0;
        const int off = block_exclusive_scan(c, scan_tmp) + (u0 ? s_carry[0] : 0);
        const int mt = block_exclusive_scan((c + MT_ROWS - 1) / MT_ROWS, scan_tmp) + (u0 ? s_carry[1] : 0);
        if (u < n_u) {
            const int e = uex[u];
            fill[e] = off;
            t.uexp[u] = e;
            t.off[u] = off;
            for (int j = 0; j < (c + MT_ROWS - 1) / MT_ROWS && mt + j < tmax; j++) {
                t.mt_exp[mt + j] = e;
                t.mt_row0[mt + j] = off + MT_ROWS * j;
                t.mt_rend[mt + j] = off + c;
            }
            if (u == n_u - 1) {
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
    if (n_u == 0 && tid == 0) {
        t.off[0] = 0;
        t.hdr[0] = t.hdr[1] = t.hdr[2] = t.hdr[3] = 0;
    }
    __syncthreads();
    // Stable placement, TPP tokens per pass (up to two (token, slot) entries
    // per thread): an entry's rank among its expert's rows in the pass =
    // earlier tokens of the pass with the same expert, a popcount over the
    // expert's per-pass token mask (TPP/64 words).
    constexpr int EPT = 2;
    const int TPP = min(256, (EPT * nth / k) & ~63);   // k <= 16 keeps this >= 64
    const int W = TPP >> 6;
    for (int c0 = 0; c0 < S; c0 += TPP) {
        int ev[EPT], tokv[EPT], rv[EPT];
        bool minev[EPT];
#pragma unroll
        for (int q = 0; q < EPT; q++) {
            const int slot = tid + q * nth;
            const int i = c0 * k + slot;
            minev[q] = slot < TPP * k && i < N;
            ev[q] = -1;
            tokv[q] = 0;
            if (minev[q]) {
                ev[q] = id_at(i);
                tokv[q] = i / k - c0;
                if (ev[q] >= 0) atomicOr(&mask[ev[q] * 4 + (tokv[q] >> 6)], 1ull << (tokv[q] & 63));
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < EPT; q++) {
            rv[q] = -1;
            if (minev[q] && ev[q] >= 0) {
                const int i = c0 * k + tid + q * nth, e = ev[q], tok = tokv[q];
                const unsigned long long *m = &mask[e * 4];
                int rk = __popcll(m[tok >> 6] & ((1ull << (tok & 63)) - 1ull));
                for (int w = 0; w < (tok >> 6); w++) rk += __popcll(m[w]);
                const int r = fill[e] + rk;
                t.row_tok[r] = i / k;
                t.row_kk[r] = i % k;
                t.row_exp[r] = e;
                rv[q] = r;
            }
        }
        __syncthreads();
        for (int e2 = tid; e2 < E; e2 += nth) {
            int n = 0;
            for (int w = 0; w < W; w++) {
                n += __popcll(mask[e2 * 4 + w]);
                mask[e2 * 4 + w] = 0ull;
            }
            fill[e2] += n;
        }
        // the token's rows in union (rank) order: an entry's slot is the
        // number of the token's valid entries with a lower union rank; the
        // invalid entries fill the tail in slot order
#pragma unroll
        for (int q = 0; q < EPT; q++) {
            if (!minev[q]) continue;
            const int i = c0 * k + tid + q * nth, e = ev[q];
            const int sx = i / k, kk = i % k;
            const int ur = e >= 0 ? rank[e] : INT_MAX;
            int p = 0, nv = 0, inv_before = 0;
            for (int k2 = 0; k2 < k; k2++) {
                const int e2 = id_at(sx * k + k2);
                if (e2 >= 0) {
                    nv++;
                    p += rank[e2] < ur;
                } else if (k2 < kk) {
                    inv_before++;
                }
            }
            const size_t at = (size_t)sx * k + (e >= 0 ? p : nv + inv_before);
            t.tok_rows[at] = e >= 0 ? rv[q] : -1;
            t.tok_kk[at] = e >= 0 ? kk : 0;
        }
        __syncthreads();
    }
}

void launch_build_table(const int *ids, int S, int k, int E, const TableOut &t, int tmax, hipStream_t st) {
    hipLaunchKernelGGL(build_table_kernel, dim3(1), dim3(1024), 0, st, ids, S, k, E, t, tmax);
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
    hipLaunchKernelGGL(synth_fill_kernel, dim3((unsigned)blocks), dim3(256), 0, st, dst, n, kind, a, b, seed);
}

}  // namespace phip
