/*
 * oracle.h — CPU restatement of peregrine's integer-dot (IDOT) MoE expert path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker the GPU path is
 * compared against; only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it. The product library (libperegrine_hip.so)
 * never links, loads or calls it.
 *
 * Every function cites the reference file:line it restates (paths relative to
 * the peregrine repository root). Two behaviours have no reference and are
 * defined here, then restated bit-for-bit by the GPU kernels:
 *   - per-32-block activation quantisation ("act group" ga = 32), and its
 *     fp32 epilogue acc = fmaf(sw*sx_b, (float)d_b, acc) over blocks b;
 *   - the device-side expert-offset table (orc_expert_table).
 *
 * Weight formats (peregrine-core/src/qt.rs:14-45, extended):
 *   fmt 1  int8, one scale per row          (QtFmt::Int8)
 *   fmt 2  int4, one scale per row          (QtFmt::Int4)
 *   fmt 4  int4, one scale per gs weights   (QtFmt::Int4Grouped)
 *   fmt 8  int8, one scale per gs weights   (new: BASELINE int8 block weights)
 * int4 bytes are QT: element i is the low nibble of byte i/2 when i is even,
 * the high nibble when odd, stored biased as v+8 (idot.rs:8-10).
 */
#ifndef PEREGRINE_ORACLE_H
#define PEREGRINE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- activation quantisation ---- */
float orc_qrow_i8(const float *x, int n, int8_t *q);
void orc_quant_rows(const float *x, int rows, int n, int ga, int8_t *q, float *sx);

/* ---- integer dots ---- */
int32_t orc_dot_i8i8(const int8_t *w, const int8_t *x, int n);
int32_t orc_dot_i4i8(const uint8_t *w4, const int8_t *x, int n);
float orc_dot_i4i8_grouped(const uint8_t *w4, const int8_t *x, const float *scales, int n, int gs);
int32_t orc_dot_i4i8_avx2(const uint8_t *w4, const int8_t *x, int n);
int orc_have_avx2(void);

/* ---- matmuls ---- */
typedef struct {
    const void *q;        /* QT bytes, row-major [O][row_bytes(fmt, I)] */
    const float *scale;   /* [O] per-row or [O][ceil(I/gs)] grouped */
    int fmt, I, O, gs;    /* gs ignored for per-row formats */
} OrcTensor;

void orc_linear(float *y, const int8_t *xq, const float *sx, int ga, const OrcTensor *w, int S);
void orc_block_dots(int32_t *d, const int8_t *xq, const OrcTensor *w, int S);
void orc_matmul_f32(float *y, const float *x, const float *w, int s_n, int d_n, int o_n);

/* ---- SwiGLU expert ---- */
float orc_silu(float x);
void orc_silu_mul(float *g, const float *u, int n);
void orc_expert_swiglu(float *y, const float *x, int S, const OrcTensor *gate, const OrcTensor *up,
                       const OrcTensor *down, int ga, float *h_out);

/* ---- routing ---- */
int orc_negligible_tail(const float *w, int kept, float min_share);
int orc_route_sigmoid(const float *logits, const float *bias, int s_n, int e_n, int k, int norm_topk,
                      float routed_scale, float min_share, int32_t *idx, float *w, int32_t *keff);
void orc_route_softmax_topk(const float *logits, int s_n, int e_n, int k, int32_t *idx, float *w);
int orc_batch_union(const int32_t *idx, const int32_t *keff, int s_n, int k, int e_n, int32_t *uniq);

/* ---- expert-offset table and combine ---- */
int orc_expert_table(const int32_t *idx, int s_n, int k, int e_n, int32_t *uexp, int32_t *off,
                     int32_t *row_tok, int32_t *row_kk, int32_t *tok_rows);
int orc_reduce_layout_build(const int32_t *dst, int n, int s_n, int32_t *row_ptr, int32_t *row_idx);
void orc_grouped_reduce(float *out, const float *y, const int32_t *row_ptr, const int32_t *row_idx,
                        const float *rw, int s_n, int D);

/* ---- the whole routed MoE layer (mlp.rs moe_forward minus router/shared) ---- */
typedef struct {
    OrcTensor gate, up, down;
} OrcExpert;

int orc_moe_forward(float *out, const float *x, int s_n, int D, const int32_t *idx, const float *w, int k,
                    const OrcExpert *experts, int e_n, int ga, const int32_t *tok_subset, int n_subset,
                    int nthreads, int use_simd);

#ifdef __cplusplus
}
#endif
#endif
