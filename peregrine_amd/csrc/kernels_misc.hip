// kernels_misc.hip — activation quantisation, weight repack at upload, the
// device router, the expert-offset table and the fixed-order combine.
#include <climits>

#include "common.h"

namespace phip {

// ---------------------------------------------------------------------------
// Activation quantisation: qrow_i8 (peregrine-kernels/src/quant.rs:14-33) per
// row (ACT_ROW) or per 32-element block (ACT_B32). One 256-thread workgroup per
// row. Output bytes go to the permuted device layout (perm8) and the row is
// zero-padded to Kp, so padded weight columns contribute nothing.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void quant_rows_kernel(QuantArgs a) {
    const int row = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const float *x = a.x + (size_t)row * a.x_stride;
    int8_t *q = a.q + (size_t)row * a.q_stride;
    if (a.mode == ACT_ROW) {
        __shared__ float red[4];
        float m = 0.0f;
        for (int k = tid; k < a.K; k += 256) m = fmaxf(m, fabsf(x[k]));
        m = warp_max(m, 64);
        if (lane == 0) red[wave] = m;
        __syncthreads();
        m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        float s = __fdiv_rn(m, 127.0f);
        if (s < 1e-12f) s = 1e-12f;
        const float inv = __fdiv_rn(1.0f, s);
        for (int k = tid; k < a.Kp; k += 256) {
            float v = k < a.K ? rintf(__fmul_rn(x[k], inv)) : 0.0f;
            q[perm8(k)] = (int8_t)(int)v;
        }
        if (tid == 0) a.s[(size_t)row * a.s_stride] = s;
    } else {
        const int half = lane >> 5, l32 = lane & 31, nb = a.Kp / BLK;
        for (int b = wave * 2 + half; b < nb; b += 8) {
            const int k = b * BLK + l32;
            const float v = k < a.K ? x[k] : 0.0f;
            float m = warp_max(fabsf(v), 32);
            float s = __fdiv_rn(m, 127.0f);
            if (s < 1e-12f) s = 1e-12f;
            const float inv = __fdiv_rn(1.0f, s);
            q[perm8(k)] = (int8_t)(int)rintf(__fmul_rn(v, inv));
            if (l32 == 0) a.s[(size_t)row * a.s_stride + b] = s;
        }
    }
}

void launch_quant_rows(const QuantArgs &a, hipStream_t st) {
    if (a.rows <= 0) return;
    hipLaunchKernelGGL(quant_rows_kernel, dim3(a.rows), dim3(256), 0, st, a);
}

// ---------------------------------------------------------------------------
// Upload repack: QT row-major bytes -> the tiled device layout.
//   int4: XOR 0x88 turns the biased nibbles (v+8) into two's-complement
//         nibbles (the conversion cuda/backend_cuda.cu:114-116 also makes);
//         the 16 bytes of each 32-block keep QT's nibble order.
//   int8: each 8-element group is permuted to perm8 order so it lines up with
//         the activation layout.
// Scales become [Op/64][ng][64]; int4 scales are stored divided by 16 because
// the unpacked int4 operands carry a factor 16 (exact: a power of two).
// ---------------------------------------------------------------------------
__global__ void repack_kernel(const uint8_t *raw, const float *raw_sc, int fmt, int I, int O, int gs, uint8_t *w,
                              float *sc, MatGeom g) {
    const size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    const size_t total = (size_t)g.Op * g.nb;
    if (idx >= total) return;
    const int o = (int)(idx / g.nb), b = (int)(idx % g.nb);
    const int t = o >> 6, ol = o & 63;
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
__global__ __launch_bounds__(256) void combine_kernel(float *out, const float *y, const int *row_ptr,
                                                      const int *row_idx, const float *rw, int D, int y_stride,
                                                      int k) {
    const int s = blockIdx.y;
    const int d = blockIdx.x * 256 + threadIdx.x;
    if (d >= D) return;
    int lo, hi;
    if (row_ptr) {
        lo = row_ptr[s];
        hi = row_ptr[s + 1];
    } else {
        lo = s * k;
        hi = lo + k;
    }
    float acc = 0.0f;
    for (int j = lo; j < hi; j++) {
        const int r = row_idx[j];
        if (r < 0) break;
        acc = __fadd_rn(acc, __fmul_rn(rw[r], y[(size_t)r * y_stride + d]));
    }
    out[(size_t)s * D + d] = acc;
}

void launch_combine(float *out, const float *y, const int *row_ptr, const int *row_idx, const float *rw, int s_n,
                    int D, int y_stride, hipStream_t st) {
    if (s_n <= 0) return;
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((D + 255) / 256), (unsigned)s_n), dim3(256), 0, st, out, y,
                       row_ptr, row_idx, rw, D, y_stride, 0);
}

void launch_combine_padded(float *out, const float *y, const int *tok_rows, const float *rw, int s_n, int k, int D,
                           int y_stride, hipStream_t st) {
    if (s_n <= 0) return;
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((D + 255) / 256), (unsigned)s_n), dim3(256), 0, st, out, y,
                       (const int *)nullptr, tok_rows, rw, D, y_stride, k);
}

// ---------------------------------------------------------------------------
// Device router for the BASELINE configs: greedy top-k over the logits (strict
// >, ties to the lowest index — the loop of peregrine-model/src/router.rs:97-118)
// then w_j = exp(l_j - l_0) / sum_j exp(l_j - l_0) summed in selection order.
// One wavefront per token.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void route_softmax_kernel(const float *logits, int E, int k, int *ids, float *w) {
    const int s = blockIdx.x, lane = threadIdx.x;
    const float *l = logits + (size_t)s * E;
    int sel[16];
    int kept = k;
    for (int kk = 0; kk < k; kk++) {
        float bv = -INFINITY;
        int be = -1;
        for (int e = lane; e < E; e += 64) {
            bool taken = false;
            for (int j = 0; j < kk; j++) taken |= (sel[j] == e);
            const float v = l[e];
            if (!taken && v > bv) {
                bv = v;
                be = e;
            }
        }
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(bv, off);
            const int oe = __shfl_xor(be, off);
            if (oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be))) {
                bv = ov;
                be = oe;
            }
        }
        if (be < 0) {
            kept = kk;
            break;
        }
        sel[kk] = be;
    }
    if (lane == 0) {
        float ex[16];
        float z = 0.0f;
        for (int kk = 0; kk < kept; kk++) {
            ex[kk] = exp_cr(__fsub_rn(l[sel[kk]], l[sel[0]]));
            z = __fadd_rn(z, ex[kk]);
        }
        for (int kk = 0; kk < k; kk++) {
            ids[(size_t)s * k + kk] = kk < kept ? sel[kk] : 0;
            w[(size_t)s * k + kk] = kk < kept ? __fdiv_rn(ex[kk], z) : 0.0f;
        }
    }
}

void launch_route_softmax(const float *logits, int S, int E, int k, int *ids, float *w, hipStream_t st) {
    if (S <= 0) return;
    hipLaunchKernelGGL(route_softmax_kernel, dim3((unsigned)S), dim3(64), 0, st, logits, E, k, ids, w);
}

// ---------------------------------------------------------------------------
// Expert-offset table, built on the device from router output, in the order
// peregrine's moe_forward uses (peregrine-model/src/mlp.rs:62-104):
//   experts in batch-union order (first seen over s ascending, kk ascending,
//   router.rs:420-445); an expert's rows in ascending token order; each token's
//   contributions listed in union order (the order the scatter adds them).
// Also emits the 32-row M-tile list the MFMA arm walks. One workgroup; every
// step is a counting pass, so the result does not depend on thread timing.
// Limits: E <= 1024, k <= 16.
// ---------------------------------------------------------------------------
constexpr int TBL_MAXE = 1024;

__global__ __launch_bounds__(1024) void build_table_kernel(const int *ids, const float *wts, int S, int k, int E,
                                                           TableOut t, int tmax) {
    __shared__ int first[TBL_MAXE], cnt[TBL_MAXE], rank[TBL_MAXE], fill[TBL_MAXE], uex[TBL_MAXE];
    __shared__ unsigned long long mask[TBL_MAXE];
    __shared__ int s_nu;
    const int tid = threadIdx.x, nth = blockDim.x;
    const int N = S * k;
    for (int e = tid; e < E; e += nth) {
        first[e] = INT_MAX;
        cnt[e] = 0;
        mask[e] = 0ull;
    }
    if (tid == 0) s_nu = 0;
    __syncthreads();
    for (int i = tid; i < N; i += nth) {
        const int e = ids[i];
        if (e >= 0 && e < E) {
            atomicMin(&first[e], i);
            atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += nth) {
        int r = -1;
        if (cnt[e] > 0) {
            r = 0;
            for (int e2 = 0; e2 < E; e2++) r += (cnt[e2] > 0 && first[e2] < first[e]);
            atomicAdd(&s_nu, 1);
        }
        rank[e] = r;
    }
    __syncthreads();
    for (int e = tid; e < E; e += nth)
        if (rank[e] >= 0) uex[rank[e]] = e;
    __syncthreads();
    const int n_u = s_nu;
    for (int u = tid; u < n_u; u += nth) {
        int off = 0, mt = 0;
        for (int v = 0; v < u; v++) {
            const int c = cnt[uex[v]];
            off += c;
            mt += (c + 31) / 32;
        }
        const int e = uex[u], c = cnt[e];
        fill[e] = off;
        t.uexp[u] = e;
        t.off[u] = off;
        for (int j = 0; j < (c + 31) / 32 && mt + j < tmax; j++) {
            t.mt_exp[mt + j] = e;
            t.mt_row0[mt + j] = off + 32 * j;
            t.mt_rend[mt + j] = off + c;
        }
        if (u == n_u - 1) {
            t.off[n_u] = off + c;
            t.hdr[0] = off + c;
            t.hdr[1] = mt + (c + 31) / 32;
            t.hdr[2] = n_u;
            t.hdr[3] = 0;
        }
    }
    if (n_u == 0 && tid == 0) {
        t.off[0] = 0;
        t.hdr[0] = 0;
        t.hdr[1] = 0;
        t.hdr[2] = 0;
        t.hdr[3] = 0;
    }
    __syncthreads();
    // stable placement, 64 tokens per pass: rank within the pass = earlier
    // tokens of the pass that chose the same expert (a popcount of a bitmask)
    for (int c0 = 0; c0 < S; c0 += 64) {
        const int i = c0 * k + tid;
        const bool mine = tid < 64 * k && i < N;
        int e = -1, bit = 0;
        if (mine) {
            e = ids[i];
            bit = i / k - c0;
            if (e >= 0 && e < E) atomicOr(&mask[e], 1ull << bit);
            else e = -1;
        }
        __syncthreads();
        if (e >= 0) {
            const int r = fill[e] + __popcll(mask[e] & ((1ull << bit) - 1ull));
            t.row_tok[r] = i / k;
            t.row_kk[r] = i % k;
            t.row_exp[r] = e;
            t.rw_row[r] = wts[i];
            t.tok_rows[i] = r;
        } else if (mine) {
            t.tok_rows[i] = -1;
        }
        __syncthreads();
        for (int e2 = tid; e2 < E; e2 += nth) {
            fill[e2] += __popcll(mask[e2]);
            mask[e2] = 0ull;
        }
        __syncthreads();
    }
    // each token's rows, sorted by union rank (insertion sort, k <= 16)
    for (int s = tid; s < S; s += nth) {
        int rr[16], rk[16], j = 0;
        for (int kk = 0; kk < k; kk++) {
            const int r = t.tok_rows[(size_t)s * k + kk];
            if (r < 0) continue;
            rr[j] = r;
            rk[j] = rank[ids[(size_t)s * k + kk]];
            j++;
        }
        for (int a = 1; a < j; a++)
            for (int b = a; b > 0 && rk[b - 1] > rk[b]; b--) {
                int tmp = rk[b]; rk[b] = rk[b - 1]; rk[b - 1] = tmp;
                tmp = rr[b]; rr[b] = rr[b - 1]; rr[b - 1] = tmp;
            }
        for (int a = 0; a < k; a++) t.tok_rows[(size_t)s * k + a] = a < j ? rr[a] : -1;
    }
}

void launch_build_table(const int *ids, const float *w, int S, int k, int E, const TableOut &t, int tmax,
                        hipStream_t st) {
    hipLaunchKernelGGL(build_table_kernel, dim3(1), dim3(1024), 0, st, ids, w, S, k, E, t, tmax);
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
