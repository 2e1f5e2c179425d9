/*
 * oracle.c — CPU restatement of peregrine's IDOT MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path, never part of it.
 * Compiled with -ffp-contract=off so every `a*b + c` below rounds twice, as
 * the Rust reference does (rustc never contracts to FMA on its own).
 *
 * Citations are relative to the peregrine repository root.
 */
#include "oracle.h"

#include <immintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* exp as the reference evaluates it: Rust's f32::exp
 * (crates/peregrine-model/src/math.rs:108-111) calls libm expf, which on Linux
 * is glibc's. The oracle calls that same function. */
static float ref_expf(float x) { return expf(x); }

/* qrow_i8 — crates/peregrine-kernels/src/quant.rs:14-33. amax over |x|,
 * s = amax/127 floored at 1e-12, q = round_ties_even(x * (1/s)). Multiplying by
 * the reciprocal (not dividing by s) is what the reference does. */
float orc_qrow_i8(const float *x, int n, int8_t *q) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float s = amax / 127.0f;
    if (s < 1e-12f) s = 1e-12f;
    float inv = 1.0f / s;
    for (int i = 0; i < n; i++) q[i] = (int8_t)rintf(x[i] * inv);
    return s;
}

/* Row quantisation. ga == 0: one scale per row (the reference, matmul.rs:109-145
 * `*_from_f32`). ga > 0: the same rule applied to every ga-element slice
 * (BASELINE per-32-block extension; no reference). sx is [rows] or
 * [rows][ceil(n/ga)]. */
void orc_quant_rows(const float *x, int rows, int n, int ga, int8_t *q, float *sx) {
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * n;
        int8_t *qr = q + (size_t)r * n;
        if (ga <= 0) {
            sx[r] = orc_qrow_i8(xr, n, qr);
        } else {
            int nb = (n + ga - 1) / ga;
            for (int b = 0; b < nb; b++) {
                int s0 = b * ga, len = (s0 + ga <= n) ? ga : n - s0;
                sx[(size_t)r * nb + b] = orc_qrow_i8(xr + s0, len, qr + s0);
            }
        }
    }
}

/* dot_i8i8_scalar — crates/peregrine-kernels/src/idot.rs:14-20. */
int32_t orc_dot_i8i8(const int8_t *w, const int8_t *x, int n) {
    int32_t sum = 0;
    for (int i = 0; i < n; i++) sum += (int32_t)w[i] * (int32_t)x[i];
    return sum;
}

/* dot_i4i8_scalar — idot.rs:24-32: element i is the low nibble of byte i/2
 * (even i) or the high nibble (odd i), biased by -8. */
int32_t orc_dot_i4i8(const uint8_t *w4, const int8_t *x, int n) {
    int32_t sum = 0;
    for (int i = 0; i < n; i++) {
        uint8_t byte = w4[i >> 1];
        int32_t nib = (i & 1) == 0 ? (byte & 0x0F) : (byte >> 4);
        sum += (nib - 8) * (int32_t)x[i];
    }
    return sum;
}

/* dot_i4i8_grouped_scalar — idot.rs:78-90: acc += scales[g] * (f32)dot_g over
 * groups in ascending order, the last group possibly short. */
float orc_dot_i4i8_grouped(const uint8_t *w4, const int8_t *x, const float *scales, int n, int gs) {
    float acc = 0.0f;
    int g = 0;
    for (int start = 0; start < n; start += gs, g++) {
        int len = (gs < n - start) ? gs : n - start;
        int32_t d = orc_dot_i4i8(w4 + (start >> 1), x + start, len);
        acc += scales[g] * (float)d;
    }
    return acc;
}

/* dot_i4i8_avx2 — idot.rs:214-239 restated with the same intrinsic sequence
 * (nibble split, interleave, bias, maddubs sign trick, scalar tail). Used only
 * as the timed CPU baseline; equal to orc_dot_i4i8 bit-for-bit. */
__attribute__((target("avx2"))) static int32_t hsum256(__m256i v) {
    __m128i lo = _mm256_castsi256_si128(v);
    __m128i hi = _mm256_extracti128_si256(v, 1);
    __m128i s = _mm_add_epi32(lo, hi);
    s = _mm_hadd_epi32(s, s);
    s = _mm_hadd_epi32(s, s);
    return _mm_cvtsi128_si32(s);
}

__attribute__((target("avx2"))) int32_t orc_dot_i4i8_avx2(const uint8_t *w4, const int8_t *x, int n) {
    const __m128i m4 = _mm_set1_epi8(0x0F);
    const __m256i b8 = _mm256_set1_epi8(8);
    const __m256i ones = _mm256_set1_epi16(1);
    __m256i acc = _mm256_setzero_si256();
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        __m128i by = _mm_loadu_si128((const __m128i *)(w4 + (i >> 1)));
        __m128i lo = _mm_and_si128(by, m4);
        __m128i hi = _mm_and_si128(_mm_srli_epi16(by, 4), m4);
        __m128i n0 = _mm_unpacklo_epi8(lo, hi);
        __m128i n1 = _mm_unpackhi_epi8(lo, hi);
        __m256i wv = _mm256_sub_epi8(_mm256_set_m128i(n1, n0), b8);
        __m256i xv = _mm256_loadu_si256((const __m256i *)(x + i));
        __m256i p = _mm256_maddubs_epi16(_mm256_sign_epi8(wv, wv), _mm256_sign_epi8(xv, wv));
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(p, ones));
    }
    int32_t sum = hsum256(acc);
    if (i < n) sum += orc_dot_i4i8(w4 + (i >> 1), x + i, n - i);
    return sum;
}

int orc_have_avx2(void) { return __builtin_cpu_supports("avx2") ? 1 : 0; }

static size_t row_bytes(int fmt, int I) {
    if (fmt == 1 || fmt == 8) return (size_t)I;
    if (fmt == 2 || fmt == 4) return (size_t)(I + 1) / 2;
    return 0;
}

static int32_t dot_seg(const OrcTensor *w, const uint8_t *row, const int8_t *x, int start, int len, int simd) {
    if (w->fmt == 1 || w->fmt == 8) return orc_dot_i8i8((const int8_t *)row + start, x + start, len);
    if (simd) return orc_dot_i4i8_avx2(row + (start >> 1), x + start, len);
    return orc_dot_i4i8(row + (start >> 1), x + start, len);
}

/* One output element of the canonical quantised linear.
 *
 * ga == 0 (per-row activation scale sx[0]) restates the reference exactly:
 *   fmt 1/2: (f32)dot * scale[o] * sx, left to right   (matmul.rs:61-87)
 *   fmt 4:   grouped dot (acc += sc[g]*(f32)d_g), * sx  (matmul.rs:93-106)
 *   fmt 8:   the fmt-4 shape with int8 group dots      (new format)
 * ga == 32 (one activation scale per 32-block, sx[b]): no reference; defined as
 *   acc = fmaf(sw(b) * sx[b], (f32)d_b, acc) over 32-blocks b ascending,
 * where sw(b) is the scale of the weight group holding block b. */
static float linear_elem(const OrcTensor *w, int o, const int8_t *xs, const float *sxs, int ga, int simd) {
    const int I = w->I;
    const uint8_t *row = (const uint8_t *)w->q + (size_t)o * row_bytes(w->fmt, I);
    const int grouped = (w->fmt == 4 || w->fmt == 8);
    const int ng = grouped ? (I + w->gs - 1) / w->gs : 1;
    const float *sc = w->scale + (size_t)o * ng;
    if (ga <= 0) {
        if (!grouped) {
            int32_t d = dot_seg(w, row, xs, 0, I, simd);
            return (float)d * sc[0] * sxs[0];
        }
        float acc = 0.0f;
        int g = 0;
        for (int start = 0; start < I; start += w->gs, g++) {
            int len = (w->gs < I - start) ? w->gs : I - start;
            acc += sc[g] * (float)dot_seg(w, row, xs, start, len, simd);
        }
        return acc * sxs[0];
    }
    float acc = 0.0f;
    const int nb = (I + ga - 1) / ga;
    for (int b = 0; b < nb; b++) {
        int start = b * ga, len = (ga < I - start) ? ga : I - start;
        float sw = grouped ? sc[start / w->gs] : sc[0];
        float c = sw * sxs[b];
        acc = fmaf(c, (float)dot_seg(w, row, xs, start, len, simd), acc);
    }
    return acc;
}

static void linear_impl(float *y, const int8_t *xq, const float *sx, int ga, const OrcTensor *w, int S, int simd) {
    const int nbx = ga > 0 ? (w->I + ga - 1) / ga : 1;
    for (int s = 0; s < S; s++)
        for (int o = 0; o < w->O; o++)
            y[(size_t)s * w->O + o] =
                linear_elem(w, o, xq + (size_t)s * w->I, sx + (size_t)s * nbx, ga, simd);
}

void orc_linear(float *y, const int8_t *xq, const float *sx, int ga, const OrcTensor *w, int S) {
    linear_impl(y, xq, sx, ga, w, S, 0);
}

/* Per-32-block int32 dots d[(s*O + o)*nb + b] — the integer anchor the GPU
 * kernels must reproduce exactly (idot.rs:1-6: integer sums are order-free). */
void orc_block_dots(int32_t *d, const int8_t *xq, const OrcTensor *w, int S) {
    const int I = w->I, nb = (I + 31) / 32;
    for (int s = 0; s < S; s++)
        for (int o = 0; o < w->O; o++) {
            const uint8_t *row = (const uint8_t *)w->q + (size_t)o * row_bytes(w->fmt, I);
            for (int b = 0; b < nb; b++) {
                int start = 32 * b, len = (32 < I - start) ? 32 : I - start;
                d[((size_t)s * w->O + o) * nb + b] = dot_seg(w, row, xq + (size_t)s * I, start, len, 0);
            }
        }
}

/* matmul_f32 — crates/peregrine-kernels/src/matmul.rs:17-30. */
void orc_matmul_f32(float *y, const float *x, const float *w, int s_n, int d_n, int o_n) {
    for (int s = 0; s < s_n; s++)
        for (int o = 0; o < o_n; o++) {
            float acc = 0.0f;
            for (int d = 0; d < d_n; d++) acc += x[(size_t)s * d_n + d] * w[(size_t)o * d_n + d];
            y[(size_t)s * o_n + o] = acc;
        }
}

/* siluf / silu_mul — crates/peregrine-model/src/math.rs:108-118. */
float orc_silu(float x) { return x / (1.0f + ref_expf(-x)); }

void orc_silu_mul(float *g, const float *u, int n) {
    for (int i = 0; i < n; i++) g[i] = orc_silu(g[i]) * u[i];
}

/* Mlp::swiglu — crates/peregrine-model/src/mlp.rs:21-26 over QtWeight::apply_vec
 * (weight.rs:139-237): gate and up see the same quantised x; h = silu(g)*u is
 * re-quantised before down. */
static void expert_swiglu_impl(float *y, const float *x, int S, const OrcTensor *gate, const OrcTensor *up,
                               const OrcTensor *down, int ga, float *h_out, int simd) {
    const int D = gate->I, I = gate->O;
    const int nbd = ga > 0 ? (D + ga - 1) / ga : 1, nbi = ga > 0 ? (I + ga - 1) / ga : 1;
    int8_t *xq = malloc((size_t)S * (D > I ? D : I));
    float *sx = malloc(sizeof(float) * (size_t)S * (nbd > nbi ? nbd : nbi));
    float *g = malloc(sizeof(float) * (size_t)S * I);
    float *u = malloc(sizeof(float) * (size_t)S * I);
    orc_quant_rows(x, S, D, ga, xq, sx);
    linear_impl(g, xq, sx, ga, gate, S, simd);
    linear_impl(u, xq, sx, ga, up, S, simd);
    orc_silu_mul(g, u, S * I);
    if (h_out) memcpy(h_out, g, sizeof(float) * (size_t)S * I);
    orc_quant_rows(g, S, I, ga, xq, sx);
    linear_impl(y, xq, sx, ga, down, S, simd);
    free(xq);
    free(sx);
    free(g);
    free(u);
}

void orc_expert_swiglu(float *y, const float *x, int S, const OrcTensor *gate, const OrcTensor *up,
                       const OrcTensor *down, int ga, float *h_out) {
    expert_swiglu_impl(y, x, S, gate, up, down, ga, h_out, 0);
}

/* Greedy top-k by score, no replacement, ties to the lowest index (strict >),
 * exactly the selection loop of router.rs:97-118. Returns the kept count. */
static int greedy_topk(const float *score, int e_n, int k, int32_t *ib) {
    for (int kk = 0; kk < k; kk++) {
        int best = -1;
        float bv = -INFINITY;
        for (int e = 0; e < e_n; e++) {
            int taken = 0;
            for (int j = 0; j < kk; j++)
                if (ib[j] == e) { taken = 1; break; }
            if (taken) continue;
            if (score[e] > bv) { bv = score[e]; best = e; }
        }
        if (best < 0) return kk;
        ib[kk] = best;
    }
    return k;
}

/* negligible_tail — router.rs:191-209: how many trailing kept weights carry
 * less than min_share of the kept sum (scanned from the end, stopping at the
 * first one that does not; at most kept-1; none for a degenerate sum). */
int orc_negligible_tail(const float *w, int kept, float min_share) {
    if (min_share <= 0.0f || kept <= 1) return 0;
    float sum = 0.0f;
    for (int i = 0; i < kept; i++) sum += w[i];
    if (!isfinite(sum) || sum <= 0.0f) return 0;
    int drop = 0;
    while (drop < kept - 1) {
        const int i = kept - 1 - drop;
        if (w[i] / sum >= min_share) break;
        drop++;
    }
    return drop;
}

/* route — crates/peregrine-model/src/router.rs:52-170 (after the router
 * matmul): sigmoid scores, greedy top-k over score + bias (strict >, ties to
 * the lowest index, NaN never picked), weight = the sigmoid; unfilled slots
 * (0, 0); the negligible tail dropped (min_share > 0); optional renormalise
 * over all k slots with +1e-20; times routed_scale. sigmoid = 1/(1+exp(-x))
 * with exp evaluated as ref_expf. */
int orc_route_sigmoid(const float *logits, const float *bias, int s_n, int e_n, int k, int norm_topk,
                      float routed_scale, float min_share, int32_t *idx, float *w, int32_t *keff) {
    float *sig = malloc(sizeof(float) * e_n), *choice = malloc(sizeof(float) * e_n);
    for (int s = 0; s < s_n; s++) {
        for (int e = 0; e < e_n; e++) {
            sig[e] = 1.0f / (1.0f + ref_expf(-logits[(size_t)s * e_n + e]));
            choice[e] = sig[e] + bias[e];
        }
        int32_t *ib = idx + (size_t)s * k;
        float *wb = w + (size_t)s * k;
        int kept = greedy_topk(choice, e_n, k, ib);
        for (int kk = 0; kk < kept; kk++) wb[kk] = sig[ib[kk]];
        for (int kk = kept; kk < k; kk++) { ib[kk] = 0; wb[kk] = 0.0f; }
        const int drop = orc_negligible_tail(wb, kept, min_share);
        for (int kk = kept - drop; kk < kept; kk++) { ib[kk] = 0; wb[kk] = 0.0f; }
        kept -= drop;
        keff[s] = kept;
        if (norm_topk) {
            float sm = 0.0f;
            for (int kk = 0; kk < k; kk++) sm += wb[kk];
            sm += 1e-20f;
            for (int kk = 0; kk < k; kk++) wb[kk] /= sm;
        }
        for (int kk = 0; kk < k; kk++) wb[kk] *= routed_scale;
    }
    free(sig);
    free(choice);
    return 0;
}

/* BASELINE router ("softmax top-k with renormalised weights"; no reference
 * code): select the k largest logits with the same greedy loop, then
 * w_j = exp(l_j - l_0) / sum_j exp(l_j - l_0), where l_0 is the first (largest)
 * selection and the sum runs in selection order. That is softmax followed by
 * renormalisation over the kept set, evaluated over the k kept logits. */
void orc_route_softmax_topk(const float *logits, int s_n, int e_n, int k, int32_t *idx, float *w) {
    float *ex = malloc(sizeof(float) * k);
    for (int s = 0; s < s_n; s++) {
        const float *l = logits + (size_t)s * e_n;
        int32_t *ib = idx + (size_t)s * k;
        float *wb = w + (size_t)s * k;
        int kept = greedy_topk(l, e_n, k, ib);
        float z = 0.0f;
        for (int kk = 0; kk < kept; kk++) {
            ex[kk] = ref_expf(l[ib[kk]] - l[ib[0]]);
            z += ex[kk];
        }
        for (int kk = 0; kk < kept; kk++) wb[kk] = ex[kk] / z;
        for (int kk = kept; kk < k; kk++) { ib[kk] = 0; wb[kk] = 0.0f; }
    }
    free(ex);
}

/* batch_union — router.rs:420-445: distinct experts in first-seen order over
 * s ascending, kk < keff[s] ascending. Out-of-range ids are skipped, as
 * moe_forward's `slot_of` filter does (mlp.rs:75-82). Returns the count. */
int orc_batch_union(const int32_t *idx, const int32_t *keff, int s_n, int k, int e_n, int32_t *uniq) {
    char *seen = calloc((size_t)e_n, 1);
    int n = 0;
    for (int s = 0; s < s_n; s++) {
        int ke = keff ? keff[s] : k;
        for (int kk = 0; kk < ke; kk++) {
            int32_t e = idx[(size_t)s * k + kk];
            if (e < 0 || e >= e_n || seen[e]) continue;
            seen[e] = 1;
            uniq[n++] = e;
        }
    }
    free(seen);
    return n;
}

/* The expert-offset table the device builds from router output (new; its
 * order is fixed by the reference's moe_forward, mlp.rs:62-104):
 *   uexp[u]       u-th distinct expert in batch-union order
 *   off[u..u+1)   that expert's rows; off[n_u] = total rows
 *   row_tok/kk[r] token and top-k slot of row r; rows of one expert ascend in s
 *   tok_rows[s*k+j] the rows of token s ordered by union rank (= the order the
 *                 reference scatter adds them, mlp.rs:111-119); -1 pads.
 * Every (s, kk) with a valid id is one row (top-k ids are distinct per token).
 * Returns n_u. */
int orc_expert_table(const int32_t *idx, int s_n, int k, int e_n, int32_t *uexp, int32_t *off,
                     int32_t *row_tok, int32_t *row_kk, int32_t *tok_rows) {
    int32_t *rank = malloc(sizeof(int32_t) * e_n), *cnt = calloc((size_t)e_n, sizeof(int32_t));
    int32_t *fill = malloc(sizeof(int32_t) * e_n);
    for (int e = 0; e < e_n; e++) rank[e] = -1;
    int n_u = 0;
    for (int s = 0; s < s_n; s++)
        for (int kk = 0; kk < k; kk++) {
            int32_t e = idx[(size_t)s * k + kk];
            if (e < 0 || e >= e_n) continue;
            if (rank[e] < 0) { rank[e] = n_u; uexp[n_u++] = e; }
            cnt[e]++;
        }
    off[0] = 0;
    for (int u = 0; u < n_u; u++) {
        off[u + 1] = off[u] + cnt[uexp[u]];
        fill[uexp[u]] = off[u];
    }
    for (int s = 0; s < s_n; s++) {
        int j = 0;
        for (int kk = 0; kk < k; kk++) tok_rows[(size_t)s * k + kk] = -1;
        int32_t rows_s[256], ranks_s[256];
        for (int kk = 0; kk < k; kk++) {
            int32_t e = idx[(size_t)s * k + kk];
            if (e < 0 || e >= e_n) continue;
            int r = fill[e]++;
            row_tok[r] = s;
            row_kk[r] = kk;
            rows_s[j] = r;
            ranks_s[j] = rank[e];
            j++;
        }
        /* insertion sort of this token's rows by union rank */
        for (int a = 1; a < j; a++)
            for (int b = a; b > 0 && ranks_s[b - 1] > ranks_s[b]; b--) {
                int32_t t = ranks_s[b]; ranks_s[b] = ranks_s[b - 1]; ranks_s[b - 1] = t;
                t = rows_s[b]; rows_s[b] = rows_s[b - 1]; rows_s[b - 1] = t;
            }
        for (int a = 0; a < j; a++) tok_rows[(size_t)s * k + a] = rows_s[a];
    }
    free(rank);
    free(cnt);
    free(fill);
    return n_u;
}

/* ReduceLayout::build — crates/peregrine-cuda/src/lib.rs:583-603: counting sort
 * of y-row k into output row dst[k], ascending k within a row. Returns 0 when a
 * dst is out of range (the reference returns None), 1 otherwise. */
int orc_reduce_layout_build(const int32_t *dst, int n, int s_n, int32_t *row_ptr, int32_t *row_idx) {
    for (int k = 0; k < n; k++)
        if (dst[k] < 0 || dst[k] >= s_n) return 0;
    for (int s = 0; s <= s_n; s++) row_ptr[s] = 0;
    for (int k = 0; k < n; k++) row_ptr[dst[k] + 1]++;
    for (int s = 0; s < s_n; s++) row_ptr[s + 1] += row_ptr[s];
    int32_t *fill = malloc(sizeof(int32_t) * (s_n + 1));
    memcpy(fill, row_ptr, sizeof(int32_t) * (s_n + 1));
    for (int k = 0; k < n; k++) row_idx[fill[dst[k]]++] = k;
    free(fill);
    return 1;
}

/* grouped_reduce — cuda/backend_cuda.cu:151-160: out[s,d] = sum over
 * j in [row_ptr[s], row_ptr[s+1]) of rw[k]*y[k,d], k = row_idx[j], ascending j,
 * accumulating from 0 with a rounded multiply then a rounded add. */
void orc_grouped_reduce(float *out, const float *y, const int32_t *row_ptr, const int32_t *row_idx,
                        const float *rw, int s_n, int D) {
    for (int s = 0; s < s_n; s++)
        for (int d = 0; d < D; d++) {
            float acc = 0.0f;
            for (int j = row_ptr[s]; j < row_ptr[s + 1]; j++) {
                int k = row_idx[j];
                acc += rw[k] * y[(size_t)k * D + d];
            }
            out[(size_t)s * D + d] = acc;
        }
}

typedef struct {
    const float *x;
    int D, I, ga, simd, n_u, nthreads, tid;
    const OrcExpert *experts;
    const int32_t *uexp, *off, *row_tok;
    const char *want; /* per-row: compute it? */
    float *y;         /* [R][D] */
} MoeJob;

static void *moe_worker(void *arg) {
    MoeJob *j = (MoeJob *)arg;
    float *xg = malloc(sizeof(float) * (size_t)j->D * 1);
    size_t cap = 1;
    for (int u = j->tid; u < j->n_u; u += j->nthreads) {
        int r0 = j->off[u], r1 = j->off[u + 1], nr = 0;
        for (int r = r0; r < r1; r++) nr += j->want[r];
        if (!nr) continue;
        if ((size_t)nr > cap) {
            cap = (size_t)nr;
            xg = realloc(xg, sizeof(float) * (size_t)j->D * cap);
        }
        float *yg = malloc(sizeof(float) * (size_t)j->D * nr);
        int i = 0;
        for (int r = r0; r < r1; r++)
            if (j->want[r]) memcpy(xg + (size_t)i++ * j->D, j->x + (size_t)j->row_tok[r] * j->D, sizeof(float) * j->D);
        const OrcExpert *ex = &j->experts[j->uexp[u]];
        expert_swiglu_impl(yg, xg, nr, &ex->gate, &ex->up, &ex->down, j->ga, NULL, j->simd);
        i = 0;
        for (int r = r0; r < r1; r++)
            if (j->want[r]) memcpy(j->y + (size_t)r * j->D, yg + (size_t)i++ * j->D, sizeof(float) * j->D);
        free(yg);
    }
    free(xg);
    return NULL;
}

/* moe_forward — crates/peregrine-model/src/mlp.rs:46-120 from a routing table
 * (the router itself is orc_route_*), without the shared expert. Each routed
 * expert runs Mlp::swiglu over its rows (gathered in ascending token order);
 * out[s] accumulates w*y in batch-union order (mul, then add). The expert loop
 * runs on `nthreads` threads (par_map, mlp.rs:96-104); per-row results do not
 * depend on the thread count. tok_subset (optional) restricts the tokens
 * computed and written, for sampled checks at full size; the union order is
 * always taken over the whole batch. Returns the number of distinct experts. */
int orc_moe_forward(float *out, const float *x, int s_n, int D, const int32_t *idx, const float *w, int k,
                    const OrcExpert *experts, int e_n, int ga, const int32_t *tok_subset, int n_subset,
                    int nthreads, int use_simd) {
    const size_t R = (size_t)s_n * k;
    int32_t *uexp = malloc(sizeof(int32_t) * e_n), *off = malloc(sizeof(int32_t) * (e_n + 1));
    int32_t *row_tok = malloc(sizeof(int32_t) * R), *row_kk = malloc(sizeof(int32_t) * R);
    int32_t *tok_rows = malloc(sizeof(int32_t) * R);
    int n_u = orc_expert_table(idx, s_n, k, e_n, uexp, off, row_tok, row_kk, tok_rows);
    char *want_tok = calloc((size_t)s_n, 1);
    if (tok_subset) {
        for (int i = 0; i < n_subset; i++)
            if (tok_subset[i] >= 0 && tok_subset[i] < s_n) want_tok[tok_subset[i]] = 1;
    } else {
        memset(want_tok, 1, (size_t)s_n);
    }
    char *want = malloc(R ? R : 1);
    for (int r = 0; r < off[n_u]; r++) want[r] = want_tok[row_tok[r]];
    float *y = malloc(sizeof(float) * (R ? R : 1) * D);
    if (nthreads < 1) nthreads = 1;
    MoeJob *jobs = malloc(sizeof(MoeJob) * nthreads);
    pthread_t *th = malloc(sizeof(pthread_t) * nthreads);
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = (MoeJob){x, D, experts[0].gate.O, ga, use_simd, n_u, nthreads, t, experts, uexp, off, row_tok, want, y};
        if (nthreads > 1) pthread_create(&th[t], NULL, moe_worker, &jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    else
        moe_worker(&jobs[0]);
    for (int s = 0; s < s_n; s++) {
        if (!want_tok[s]) continue;
        float *dst = out + (size_t)s * D;
        for (int d = 0; d < D; d++) dst[d] = 0.0f;
        for (int j = 0; j < k; j++) {
            int r = tok_rows[(size_t)s * k + j];
            if (r < 0) break;
            float wgt = w[(size_t)s * k + row_kk[r]];
            const float *src = y + (size_t)r * D;
            for (int d = 0; d < D; d++) dst[d] += wgt * src[d];
        }
    }
    free(jobs); free(th); free(y); free(want); free(want_tok);
    free(uexp); free(off); free(row_tok); free(row_kk); free(tok_rows);
    return n_u;
}
