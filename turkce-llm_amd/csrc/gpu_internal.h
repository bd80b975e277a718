/* gpu_internal.h -- pieces of the GPU trainer (gpu_train.c) that the KV-cache
 * decoder (gpu_decode.c) and the queued driver loop (train_loop.c) reuse.
 * Not part of the C ABI: every symbol here has hidden visibility in
 * libtrlm_hip.so. */
#ifndef TRLM_GPU_INTERNAL_H
#define TRLM_GPU_INTERNAL_H

#include "trlm_ext.h"

#pragma GCC visibility push(hidden)

#ifdef __cplusplus
extern "C" {
#endif

/* lm_collect_params order (model/gpu_train.c:8-13): [0] embedding; layer l
 * at 1 + 10*l + k; last = final norm weight. */
enum { PK_ATTN_NORM = 0, PK_WQKV, PK_BQKV, PK_WO, PK_BO, PK_FFN_NORM, PK_WGU, PK_BGU, PK_WDOWN, PK_BDOWN };
static inline u32 trlm_pidx(u32 layer, u32 k) { return 1u + 10u * layer + k; }

typedef enum { GEMM_NN, GEMM_NT, GEMM_TN } GemmKind;

/* Called after a layer's QKV projection and RoPE, with that layer's qkv
 * ([g->N, 3D]: rotated Q, rotated K, V). */
typedef void (*TrlmLayerHook)(void* ctx, GpuTrainer* g, u32 layer, hipDeviceptr_t qkv);

void trlm_bind(GpuTrainer* g);
hipDeviceptr_t trlm_param_ptr(const GpuTrainer* g, u32 i);
/* Embedding, L blocks and final norm over g->N = g->B * g->T rows; the
 * result is left in g->nf. */
void trlm_forward_hidden(GpuTrainer* g, const u32* ids, TrlmLayerHook hook, void* hook_ctx);
void trlm_rmsnorm_rows(GpuTrainer* g, hipDeviceptr_t x, hipDeviceptr_t w, hipDeviceptr_t out, hipDeviceptr_t rinv,
                       u32 rows);
void trlm_gemm_rows(GpuTrainer* g, GemmKind kind, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C, i32 M, i32 N,
                    i32 K, i32 lda, i32 ldb, i32 ldc, hipDeviceptr_t bias, hipDeviceptr_t resid);
void trlm_swiglu_rows(GpuTrainer* g, hipDeviceptr_t gu, hipDeviceptr_t h, u32 rows);
void trlm_embed_rows(GpuTrainer* g, hipDeviceptr_t ids, hipDeviceptr_t x, u32 rows);
void trlm_argmax_rows(GpuTrainer* g, hipDeviceptr_t logits, i32 ld, u32 rows, hipDeviceptr_t out);

/* trlm_gemm (trlm_ext.h) with optional epilogue extras (NULL: none):
 *   stats: per-row softmax statistics of C ([M][stats_cap] float2: (max,
 *          sum exp(v - max)) of each wave's column half of each tile); single
 *          GEMM, beta 0, no bias / residual; no split-K;
 *   csum:  the column sums of op(B) over k ([N]: a bias gradient next to a
 *          weight gradient); single GEMM, B stored [K,N];
 *   rope:  columns [0, rope_cols) of C rotated as RoPE pairs of heads of
 *          rope_hd columns at position row % rope_T (tables [rope_T][rope_hd/2]),
 *          after bias; single GEMM; no split-K;
 *   tgt / tgt_val (with stats): tgt_val[m] = C[m, tgt[m]], the value the
 *          epilogue computes for that element (tgt[m] < N);
 *   no_store (with stats): C is not written -- the statistics (and tgt_val)
 *          are the whole output;
 *   glu_h / glu_F: the gate/up projection with its SwiGLU: C = [gate | up]
 *          (N = 2 glu_F) is written as usual and glu_h [M, glu_F] receives
 *          silu(gate) * up; single aligned NN GEMM, glu_F % 32 == 0,
 *          K % 32 == 0, bias allowed, nothing else.
 * Returns the stats entries written per row (0 without stats). */
typedef struct TrlmGemmExtra {
    hipDeviceptr_t stats;
    i32 stats_cap;
    hipDeviceptr_t csum;
    const f32* rope_cos;
    const f32* rope_sin;
    i32 rope_T, rope_hd, rope_cols;
    hipDeviceptr_t tgt;
    hipDeviceptr_t tgt_val;
    i32 no_store;
    hipDeviceptr_t glu_h;
    i32 glu_F;
} TrlmGemmExtra;
i32 trlm_gemm_ex(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
                 i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
                 f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr, const TrlmGemmExtra* x);

/* trlm_gemm_ex with the split-K partials in a caller-given workspace of
 * fixed_floats floats (fixed_ws != NULL): no allocation; a plan whose
 * partials do not fit runs with the most splits that do (down to one split,
 * which needs no workspace), as if forced to that count.  fixed_ws == NULL
 * is trlm_gemm_ex (the engine's grow-only workspace). */
i32 trlm_gemm_ws(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
                 i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
                 f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr, const TrlmGemmExtra* x,
                 hipDeviceptr_t fixed_ws, u64 fixed_floats);
/* The device of the context the engine was created in. */
i32 trlm_gemm_device(const TrlmGemm* e);
/* noalloc.hip: resolves the device address of the GEMM scratch array on
 * `device` (once per device; trlm_gemm_create calls it). */
void trlm_noalloc_setup(i32 device);

/* Queued driver steps (train_loop.c): see gpu_train.c. */
void trlm_check_ids(const GpuTrainer* g, const u32* ids, const char* what);
u32 trlm_embed_groups(GpuTrainer* g, const u32* ids, u32* order, u32* seg);
void trlm_train_step_queued(GpuTrainer* g, AdamOptimizer* opt, f32 weight_decay, f64 clip, hipDeviceptr_t loss_out,
                            hipDeviceptr_t norm_out, hipDeviceptr_t scale_buf);
void trlm_loss_mean_queued(GpuTrainer* g, hipDeviceptr_t out, i32 acc);
void trlm_eval_queued(GpuTrainer* g, hipDeviceptr_t sum, i32 acc);

#ifdef __cplusplus
}
#endif

#pragma GCC visibility pop

#endif
