/*
 * peregrine_hip.h — C ABI of libperegrine_hip.so, the MI355X (gfx950) GPU lane
 * for peregrine's quantised MoE expert matmuls.
 *
 * Drop-in for the CUDA backend's expert-group surface: every entry point
 * below named after a `coli_cuda_*` function takes the same arguments, keeps
 * the same ownership and returns 1 on success / 0 on failure with a
 * diagnostic on stderr (cuda/backend_cuda.h:30-192, bound from Rust at
 * crates/peregrine-cuda/src/lib.rs:40-109). Entry points marked NEW have no
 * counterpart in the reference.
 *
 * Arithmetic: int8 activations dotted against int4/int8 QT weights with exact
 * int32 per-block dots; fp32 epilogues in the order of peregrine-kernels
 * (crates/peregrine-kernels/src/matmul.rs:61-106). This follows the CPU IDOT
 * lane, not the CUDA backend's fp32-activation arm.
 *
 * Threading: like the reference, per-device scratch is shared and calls are
 * not re-entrant per device; one GPU-lane thread issues them.
 */
#ifndef PEREGRINE_HIP_H
#define PEREGRINE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define COLI_HIP_MAX_DEVICES 16

/* Weight formats (peregrine-core/src/qt.rs:14-45). */
#define COLI_HIP_FMT_I8 1   /* int8, one f32 scale per row */
#define COLI_HIP_FMT_I4 2   /* QT int4 (v+8 nibbles, low first), one scale per row */
#define COLI_HIP_FMT_I4G 4  /* QT int4, one scale per gs weights (gs = 32, 64, 128, 256) */
#define COLI_HIP_FMT_I8G 8  /* NEW: int8, one scale per gs weights */

/* Kernel arms reported through arm_out (codes keep backend_cuda.h:81-97). */
#define COLI_HIP_ARM_MFMA 0 /* grouped int8 MFMA GEMM (the reference's int4 TC slot) */
#define COLI_HIP_ARM_GEMV 2 /* per-row GEMV (the reference's packed-W4 slot) */

typedef struct ColiHipTensor ColiHipTensor;
typedef struct ColiHipGraph ColiHipGraph;
typedef struct ColiHipExpertSet ColiHipExpertSet;

/* ---- devices: replaces backend_cuda.h:30-40 ---- */
/* One context (non-blocking stream) per listed ordinal, 1 <= count <= 16.
 * Returns 0 when an ordinal names no visible device or repeats; the contexts
 * of an earlier init are then left as they were. Otherwise they are replaced. */
int coli_hip_init(const int *devices, int count);                  /* coli_cuda_init */
void coli_hip_shutdown(void);                                      /* coli_cuda_shutdown */
int coli_hip_device_count(void);                                   /* coli_cuda_device_count */
int coli_hip_probe_device_count(void);                             /* coli_cuda_probe_device_count */
int coli_hip_device_at(int index);                                 /* coli_cuda_device_at */
int coli_hip_mem_info(int device, size_t *free_bytes, size_t *total_bytes); /* coli_cuda_mem_info */
void coli_hip_stats(int device, size_t *tensor_count, size_t *tensor_bytes); /* coli_cuda_stats */
void coli_hip_group_stats(uint64_t *calls, uint64_t *experts, uint64_t *rows, double *h2d_ms,
                          double *kernel_ms, double *d2h_ms);     /* coli_cuda_group_stats */

/* ---- resident tensors: replaces backend_cuda.h:42-45, 139-145 ---- */
/* fmt 1 (int8) or 2 (int4) with O per-row scales; blocks until resident.
 * If *tensor is set, only checks that fmt/I/O/device match (as the reference). */
int coli_hip_tensor_upload(ColiHipTensor **tensor, const void *weights, const float *scales, int fmt, int I,
                           int O, int device);                     /* coli_cuda_tensor_upload */
/* NEW: any format, grouped formats take gs; scales are O*ceil(I/gs) laid out
 * sc[o*ng + g] (peregrine-core/src/qt.rs:154-160). */
int coli_hip_tensor_upload_grouped(ColiHipTensor **tensor, const void *weights, const float *scales, int fmt,
                                   int I, int O, int gs, int device);
/* NEW: same, with weights and scales already in device memory (no H2D). */
int coli_hip_tensor_upload_dev(ColiHipTensor **tensor, const void *weights_dev, const float *scales_dev, int fmt,
                               int I, int O, int gs, int device);
void coli_hip_tensor_free(ColiHipTensor *tensor);                  /* coli_cuda_tensor_free */
size_t coli_hip_tensor_bytes(const ColiHipTensor *tensor);          /* coli_cuda_tensor_bytes */
int coli_hip_tensor_device(const ColiHipTensor *tensor);            /* coli_cuda_tensor_device */
int coli_hip_tensor_update(ColiHipTensor *tensor, const void *weights, const float *scales); /* coli_cuda_tensor_update */

/* ---- the expert group: replaces backend_cuda.h:67-110 ----
 * y = down(silu(gate(x)) * up(x)) for `count` experts; x and y are host
 * [sum(rows)][D] f32, rows consecutive in call order, every rows[c] >= 1,
 * count <= 256. Blocks until y is written. */
int coli_hip_expert_group(ColiHipTensor *const *gates, ColiHipTensor *const *ups, ColiHipTensor *const *downs,
                          const int *rows, int count, float *y, const float *x); /* coli_cuda_expert_group */
/* tile_* are accepted and ignored (no WMMA fragment shapes on CDNA); arm_out
 * reports COLI_HIP_ARM_*. */
int coli_hip_expert_group_tiled(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                ColiHipTensor *const *downs, const int *rows, int count, float *y, const float *x,
                                int tile_m, int tile_n, int tile_k, int *arm_out); /* coli_cuda_expert_group_tiled */
/* out[s] = sum over row_idx[row_ptr[s]..row_ptr[s+1]] of rw[k]*y[k], ascending,
 * no atomics. */
int coli_hip_expert_group_reduce(ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                                 ColiHipTensor *const *downs, const int *rows, int count, const int *row_ptr,
                                 const int *row_idx, const float *rw, int s_n, float *out,
                                 const float *x);                 /* coli_cuda_expert_group_reduce */

/* ---- graphs: replaces backend_cuda.h:172-190 ----
 * With COLI_HIP_GRAPH=1 in the environment (COLI_CUDA_GRAPH=1, the
 * reference's name, is read as an alias), expert_group* calls are captured
 * once per launch shape (arm, expert count, widths, rows per expert, reduce
 * rows, formats) and replayed; descriptors and activations reach the graph
 * through mapped host staging that the replayed kernels read (and the output
 * is written back the same way), so a replay uses the current experts and
 * inputs. A new shape's next calls alternate replay and eager launch (three
 * timed probes each) and the faster is kept; a shape where eager wins runs
 * eagerly from then on (COLI_HIP_GRAPH_ADAPT=0 always replays). Not cached:
 * calls under profiling or with the debug-dot hook set. graph_cache_stats
 * counts every call that ran eagerly with the cache on as uncacheable. */
int coli_hip_graph_begin(int device);                             /* coli_cuda_graph_begin */
int coli_hip_graph_end(int device, ColiHipGraph **out);           /* coli_cuda_graph_end */
/* graph_launch refuses (returns 0) a graph captured before the device's
 * scratch buffers were reallocated by a larger call; scratch never grows
 * during a capture (run each call shape eagerly once before capturing it). */
int coli_hip_graph_launch(ColiHipGraph *g);                       /* coli_cuda_graph_launch */
void coli_hip_graph_free(ColiHipGraph *g);                        /* coli_cuda_graph_free */
void coli_hip_graph_cache_stats(uint64_t *captures, uint64_t *replays, uint64_t *invalidations,
                                uint64_t *uncacheable);          /* coli_cuda_graph_cache_stats */
int coli_hip_pipe_sync(int device);                                /* coli_cuda_pipe_sync */

/* ---- device memory: replaces backend_cuda.h:147-151 (pipe_* primitives) ---- */
void *coli_hip_pipe_alloc(int device, size_t bytes);                 /* coli_cuda_pipe_alloc */
void coli_hip_pipe_free(int device, void *p);                        /* coli_cuda_pipe_free */
int coli_hip_pipe_upload(int device, void *dst, const void *src, size_t bytes);   /* coli_cuda_pipe_upload */
int coli_hip_pipe_download(int device, const void *src, void *dst, size_t bytes); /* coli_cuda_pipe_download */

/* ---- NEW: stream timing and synthetic fills (benchmarks, tests) ---- */
/* Record event `slot` (0..15) on the device stream; elapsed ms between two. */
int coli_hip_event_record(int device, int slot);
float coli_hip_event_elapsed(int device, int slot_a, int slot_b);
/* Seeded device-side fill of n elements: kind 0 = uniform random bytes,
 * 1 = normal(a, b) f32, 2 = lognormal(mu = a, sigma = b) f32. Deterministic
 * for a given (seed, n); async on the device stream. */
int coli_hip_synth_fill(int device, void *dst, size_t n, int kind, float a, float b, uint64_t seed);

/* ---- NEW: knobs ---- */
/* Activation scale granularity for expert_group* calls: 0 = one scale per
 * row (the reference, default), 32 = one scale per 32-element block. */
int coli_hip_set_act_group(int ga);
int coli_hip_get_act_group(void);
/* Force an arm for later calls: -1 automatic, COLI_HIP_ARM_GEMV or _MFMA. */
int coli_hip_set_arm(int arm);
/* One-token layers with router logits (coli_hip_moe_forward_logits_dev, S = 1,
 * GEMV arm, at most 256 experts): route and quantise inside the gate/up GEMV
 * instead of a separate router launch. -1 automatic (when the gate/up grid has
 * at least 256 workgroups: config 1's 48-workgroup grid measured 15.6 us per
 * layer fused against 15.1 us apart), 0 never, 1 whenever eligible.
 * COLI_HIP_FUSED_ROUTE=0 or =1 in the environment sets 0 or 1 at first use. */
int coli_hip_set_fused_route(int mode);
/* One-token layers on the GEMV arm: the down projection also applies the
 * router weights in top-k order (one launch instead of down + combine; the
 * same bits). Eligible for k <= 8 and K <= 1536 (the down projection's input
 * width). -1 automatic (default: eligible and k <= 2), 0 never, 1 whenever
 * eligible. COLI_HIP_FUSED_COMBINE=0 or =1 in the environment sets 0 or 1 at
 * first use. */
int coli_hip_set_fused_combine(int mode);
/* Split-K GEMV arm (NEW, no counterpart in backend_cuda.h): the K blocks of
 * each (row, output tile) are spread over several workgroups so that decode
 * launches cover the chip; the workgroup that finishes a tile's count runs
 * its exact f32 chain, so results are the same bits as the unsplit kernel.
 * target_wgs is the workgroup count a GEMV launch aims for; 0 never splits
 * (the default: on MI355X the hand-off between workgroups costs more than the
 * extra CUs gain at the BASELINE decode shapes); -1 restores the default.
 * COLI_HIP_GEMV_SPLIT=<n> in the environment sets it at first use. A split gate/up GEMV takes the router launch apart (the fused
 * router prologue runs in the unsplit kernel only), and in automatic mode a
 * split down projection combines in its tail instead of the fused kernel. */
int coli_hip_set_gemv_split(int target_wgs);

/* ---- NEW: device-resident MoE layer (inputs already in HBM) ---- */
/* A fixed expert table: expert id e -> (gates[e], ups[e], downs[e]). */
int coli_hip_expert_set_create(ColiHipExpertSet **set, ColiHipTensor *const *gates, ColiHipTensor *const *ups,
                               ColiHipTensor *const *downs, int count);
void coli_hip_expert_set_free(ColiHipExpertSet *set);
/* Router for the BASELINE configs: top-k of logits[S][E] (ties to the lower
 * index), weights softmax-renormalised over the kept k. Async on the device
 * stream. */
int coli_hip_route_softmax_topk_dev(int device, const float *logits_dev, int S, int E, int k, int *ids_dev,
                                    float *w_dev);
/* The reference's router on the device (router.rs:52-170 after the router
 * matmul; the reference runs it on the host): sigmoid scores, greedy top-k
 * over score + bias[e] (bias_dev may be NULL: zero), weight = the sigmoid,
 * unfilled slots (0, 0), the negligible tail dropped when min_share > 0
 * (router.rs:191-209), optional renormalisation (+1e-20), times routed_scale.
 * keff_dev[S] (may be NULL) receives each token's kept count. Async. */
int coli_hip_route_sigmoid_topk_dev(int device, const float *logits_dev, const float *bias_dev, int S, int E, int k,
                                    int norm_topk, float routed_scale, float min_share, int *ids_dev, float *w_dev,
                                    int *keff_dev);
/* One routed MoE layer: out[S][D] = sum over each token's k experts, in
 * batch-union order, of w * SwiGLU_e(x). ids/w are [S][k] (device). act_group
 * 0 or 32; arm -1 automatic. The expert-offset table is built on the device.
 * Async on the device stream (coli_hip_pipe_sync waits). */
int coli_hip_moe_forward_dev(const ColiHipExpertSet *set, const float *x_dev, int S, const int *ids_dev,
                             const float *w_dev, int k, float *out_dev, int act_group, int arm);
/* The same layer as coli_hip_moe_forward_dev, allocating nothing: no
 * hipMalloc, hipFree or other allocating call, so callers that cannot
 * allocate (code under stream/graph capture, tight serving loops, harnesses
 * that forbid it) can use it from the first call. No counterpart in the
 * reference. Its scratch (activation quant, h, y, the expert-offset table) is
 * a fixed COLI_HIP_FIXED_SCRATCH_BYTES array per device, mapped at init; a
 * call needing more returns 0 with a message (about S * k <= 2300 rows at
 * D = 5120, I = 1536). Every call on a device shares that device's array and
 * leaves its contents behind: calls that overlap on one device (other host
 * threads, other streams) race. No profiling on this path. */
#define COLI_HIP_FIXED_SCRATCH_BYTES (64 << 20)
int coli_hip_moe_forward_dev_noalloc(const ColiHipExpertSet *set, const float *x_dev, int S, const int *ids_dev,
                                     const float *w_dev, int k, float *out_dev, int act_group, int arm);
/* Same layer with the router fused in: logits[S][E] (device) are routed
 * (as coli_hip_route_softmax_topk_dev) into ids_dev/w_dev [S][k], then the
 * layer runs. One token (S = 1) on the GEMV arm needs no expert table. */
int coli_hip_moe_forward_logits_dev(const ColiHipExpertSet *set, const float *x_dev, int S, const float *logits_dev,
                                    int k, int *ids_dev, float *w_dev, float *out_dev, int act_group, int arm);
/* The device stream (hipStream_t) of an initialised device, for interop. */
void *coli_hip_stream(int device);

/* ---- NEW: instrumentation ---- */
/* Per-kernel timings recorded with HIP events on the device stream while
 * COLI_HIP_PROFILE=1 (or coli_hip_set_profile(1)); which = COLI_HIP_K_*. */
#define COLI_HIP_K_TABLE 0
#define COLI_HIP_K_QUANT_X 1
#define COLI_HIP_K_GATEUP 2
#define COLI_HIP_K_QUANT_H 3
#define COLI_HIP_K_DOWN 4
#define COLI_HIP_K_COMBINE 5
#define COLI_HIP_K_COUNT 6
int coli_hip_set_profile(int on);
void coli_hip_kernel_stats(int which, uint64_t *launches, double *total_ms);
void coli_hip_reset_stats(void);
/* Parity hook: when set (device pointers, may be NULL), the next dispatches
 * also write every per-32-block int32 dot they compute: gate/up as
 * [R][2][I][ceil(D/32)], down as [R][D][ceil(I/32)]. */
int coli_hip_set_debug_dots(int32_t *gateup_dev, int32_t *down_dev);
/* Test hook: polls a GEMV's bounded wait (between its streaming waves and its
 * chain wave) makes before giving up; 0 restores the default (2^22). A wait
 * that gives up sets a host-visible flag: the next coli_hip_pipe_sync,
 * coli_hip_graph_launch or expert_group* call on the device returns 0 with a
 * diagnostic, and clears it. */
int coli_hip_set_spin_limit(int polls);
/* Last row plan of the device-resident path, copied to host (for tests):
 * hdr[4] = {rows, tiles, distinct experts, 0}. */
int coli_hip_last_table(int device, int *hdr, int *uexp, int *off, int *row_tok, int *tok_rows, int e_cap,
                        int r_cap);

#ifdef __cplusplus
}
#endif

#endif
