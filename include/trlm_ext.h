/* trlm_ext.h -- additive entry points of the MI355X GPU path.
 *
 * None of these exist in the reference's API (model/gpu_train.h,
 * model/gpu_ops.h); they cover what BASELINE's configurations ask for and
 * the reference does not offer:
 *   - forward to logits, with or without the mean cross-entropy, and greedy
 *     argmax (the reference's CE overwrites logits with their gradient,
 *     train_kernels.cu:742-772, and it has no GPU argmax);
 *   - AdamW (decoupled weight decay; the reference's Adam has none,
 *     training/adam.c:43-52);
 *   - a raw fp32 GEMM on device buffers and stream-event timing, for the
 *     model-shape GEMM sweep and its tests;
 *   - TRLM v1 checkpoints straight from / to the device, a KV-cache decoder,
 *     and the training driver's loop (lr schedule, clipping, validation
 *     windows) queued on the device.
 */
#ifndef TRLM_EXT_H
#define TRLM_EXT_H

#include "gpu_train.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Forward pass only; copies logits [B*T, V] (row-major, unpadded) to
 * host_logits when it is not NULL.  Leaves the logits on the device for
 * gpu_trainer_greedy_argmax. */
void gpu_trainer_forward_logits(GpuTrainer* g, const u32* ids, f32* host_logits);

/* Forward pass plus mean cross-entropy (same definition and bits as
 * gpu_trainer_eval_loss) without overwriting the logits; copies them to
 * host_logits when not NULL. */
f32 gpu_trainer_forward_loss_logits(GpuTrainer* g, const u32* ids, const u32* targets, f32* host_logits);

/* Greedy next token of every row of the logits left on the device by the
 * last forward: first index of the row maximum (ties -> lowest index). */
void gpu_trainer_greedy_argmax(GpuTrainer* g, u32* host_ids_out);

/* AdamW: t++, then p -= lr*m_hat/(sqrt(v_hat)+eps) + lr*weight_decay*p on
 * all parameters (the reference has no exclusion list).  weight_decay = 0
 * gives exactly gpu_trainer_adam_step_scaled. */
void gpu_trainer_adamw_step_scaled(GpuTrainer* g, AdamOptimizer* opt, f32 weight_decay, f32 grad_scale);

/* ---- raw GEMM on device buffers (current context of the calling thread) ----
 * C = alpha*op(A)@op(B) (+ beta*C) (+ bias[n]) (+ resid[m,n]), batched with
 * element strides; trans_a/trans_b as k_gemm_nn/nt/tn of the reference
 * (train_kernels.cu:97-105).  bias/resid may be NULL. */
typedef struct TrlmGemm TrlmGemm;
TrlmGemm* trlm_gemm_create(HipCtx* ctx);
void trlm_gemm_destroy(TrlmGemm* e);
void trlm_gemm(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
               i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
               f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr);
/* trlm_gemm for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  It
 * has no counterpart in the reference.  Same arguments, plan, kernels and
 * results (bit for bit) as trlm_gemm on an engine from trlm_gemm_create,
 * but the split-K partials go to a fixed 32 MiB scratch array that each GPU
 * holds from the first trlm_gemm_create on it until the process ends, so
 * the call allocates nothing.  A plan whose partials need more than 32 MiB
 * (splits x M x N floats; of the model's GEMMs only the full-size LM-head dX)
 * runs with the most splits whose partials fit, down to one split, which
 * needs none; its result then equals trlm_gemm on an engine forced to that
 * split count (trlm_gemm_force(e, NULL, splits)), and trlm_gemm_last_variant
 * reports it.  Returns 0; or -1, with a message on stderr and nothing
 * launched, when the engine's device is not the calling thread's current
 * device.  All calls on one GPU share its scratch: calls that overlap in time
 * on one GPU (other streams, contexts or threads) race. */
i32 trlm_gemm_noalloc(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
                      i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
                      f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr);
/* Name of the kernel variant and split-K factor the last trlm_gemm call used. */
const char* trlm_gemm_last_variant(TrlmGemm* e, i32* splits);
/* The variant and split-K factor trlm_gemm picks for 16-byte-aligned operands
 * of this shape (host-only; no device call). */
const char* trlm_gemm_plan(i32 trans_a, i32 trans_b, i32 M, i32 N, i32 K, u32 batch, i32* splits);
/* Tuning hook: make later calls on this engine use the named aligned tile
 * variant ("256x128", "128x256", "128x128", "128x128_k32", "64x128",
 * "64x128_k32", "64x64", "64x64_k32") and, when splits > 0, that split-K
 * factor (single GEMMs only).  tile NULL restores automatic selection.
 * Returns 0, or -1 for an unknown name (selection is then automatic). */
i32 trlm_gemm_force(TrlmGemm* e, const char* tile, i32 splits);
/* The GEMM engine of a trainer's main stream (the forward, the LM head and
 * the backward's dX products), for trlm_gemm_force and
 * trlm_gemm_last_variant. */
TrlmGemm* gpu_trainer_gemm_engine(GpuTrainer* g);

/* Placement of the causal attention forward's jobs (host-only; no device
 * call).  For a grid of `heads` (batch x heads) by n query blocks that is
 * exactly three workgroups per compute unit (heads * n == 3 * cus, heads / 3
 * a multiple of xcds), fills jobs[heads * n] -- workgroup L = query-block
 * index * heads + head index takes query block jobs[L] >> 16 of head
 * jobs[L] & 0xffff -- so that the three workgroups L, L + cus, L + 2 cus
 * that share a compute unit hold floor or ceil of 3(n + 1)/2 key-block
 * stages between them and every head's jobs have the same L mod xcds (one
 * XCD), and returns 1; otherwise returns 0 and leaves jobs alone.  The
 * trainer builds it when the forward kernel holds three workgroups per
 * compute unit; any table that is a permutation gives the same bits. */
i32 trlm_attn_job_table(u32 heads, u32 n, u32 cus, u32 xcds, i32* jobs);

/* ---- checkpoints: TRLM v1 (training/checkpoint.h:6-12), the reference's
 * format and rules (checkpoint.c:22-137), straight from / to the device.
 * save: shapes from params (the caller's CPU mirror nodes), values and, when
 * opt != NULL, Adam m / v from the device, t from opt; written to
 * path ".tmp" and renamed over path only when complete.  load: validates
 * the whole file against params (count, ndim, shapes, exact size; optimizer
 * state required when opt != NULL) and changes nothing on failure; on
 * success fills the device buffers, the host mirror params[i]->value and, when
 * opt != NULL, opt->m / opt->v / opt->t.  Both return TRUE / FALSE. */
bool32 gpu_trainer_checkpoint_save(GpuTrainer* g, const char* path, Node** params, const AdamOptimizer* opt);
bool32 gpu_trainer_checkpoint_load(GpuTrainer* g, const char* path, Node** params, AdamOptimizer* opt);

/* ---- KV-cache decode (generate.c:57-73,186-212 without the per-step
 * full-window recompute).  The decoder uses the trainer's resident
 * parameters, kernels, stream and GEMM engine; it owns a K/V cache of
 * L x batch x H x max_ctx x hd floats each.  All sequences of a batch share
 * one length.  Errors (tokens outside the vocabulary, a full context, a step
 * before the prefill) print "[HIP ERROR] gpu_decode: ..." and _exit(1). */
typedef struct TrlmDecoder TrlmDecoder;
TrlmDecoder* gpu_decoder_create(GpuTrainer* g, u32 batch, u32 max_ctx);
void gpu_decoder_destroy(TrlmDecoder* d);
/* ids [batch][len] -> cache positions 0..len-1; logits of position len-1 */
void gpu_decoder_prefill(TrlmDecoder* d, const u32* ids, u32 len);
/* ids [batch]: one new token per sequence at position length(); its logits */
void gpu_decoder_step(TrlmDecoder* d, const u32* ids);
u32 gpu_decoder_length(const TrlmDecoder* d);
/* logits of the last prefill/step position, [batch][V] */
void gpu_decoder_logits(TrlmDecoder* d, f32* host_logits);
/* first index of each row's maximum */
void gpu_decoder_greedy(TrlmDecoder* d, u32* out_ids);
/* sample_next (generate.c:57-73) per row; rngs[batch] each advance by one
 * pcg_uniform draw, exactly as the reference's loop consumes them */
void gpu_decoder_sample(TrlmDecoder* d, PCGState* rngs, f32 temperature, u32* out_ids);
/* prefill + greedy generation of `steps` tokens per sequence; out
 * [batch][steps] (prompt_len + steps <= max_ctx) */
void gpu_decoder_generate_greedy(TrlmDecoder* d, const u32* prompt, u32 prompt_len, u32 steps, u32* out);
/* prefill + sampled generation (sample_next at `temperature`, generate.c:
 * 57-73,186-212, without its end-of-text stop): out [batch][steps], the same
 * picks as prefill + (gpu_decoder_sample, gpu_decoder_step) per token, with
 * rngs[b] advanced by one pcg_uniform per token of sequence b as the
 * reference's loop draws them (all drawn up front; no host round trip per
 * token) */
void gpu_decoder_generate_sampled(TrlmDecoder* d, const u32* prompt, u32 prompt_len, u32 steps, PCGState* rngs,
                                  f32 temperature, u32* out);

/* ---- training driver loop (training/train_lm_gpu.c:212-223, 241-258) ----
 * The reference's driver, per step: lr = lr_warmup_cosine(step, ...);
 * batch = gpu_trainer_sample_batch(..., seed_base + step); loss =
 * forward_backward; norm = grad_norm; scale = clip/norm when norm > clip,
 * else 1; adam_step_scaled(scale).  gpu_trainer_train_steps runs steps
 * first_step .. first_step+n_steps-1 of that loop with the same results bit
 * for bit, but queued: the batches are prepared on the host while the device
 * runs, and the loss mean, grad norm and clip scale stay on the device until
 * the call returns (one wait per call instead of several per step).
 * losses / grad_norms / lrs (each n_steps long, any may be NULL) receive each
 * step's loss, norm and learning rate; opt->lr holds the last step's rate. */
typedef struct TrlmSchedule {
    u64 warmup_steps, total_steps;   /* lr_warmup_cosine(step, warmup, total, peak, min) */
    f32 peak_lr, min_lr;
    f64 grad_clip;                   /* clip when the norm exceeds this; <= 0: never */
    f32 weight_decay;                /* 0: the reference's Adam; > 0: AdamW (decoupled) */
    u64 seed_base;                   /* step s samples with seed_base + s (reference: 2026) */
} TrlmSchedule;
void gpu_trainer_train_steps(GpuTrainer* g, AdamOptimizer* opt, const u32* tokens, u64 num_tokens,
                             const TrlmSchedule* s, u64 first_step, u32 n_steps, f32* losses, f64* grad_norms,
                             f32* lrs);
/* The driver's validation loss: val_batches x batch fixed windows spread
 * evenly over tokens[train_tokens .. train_tokens+val_tokens) (stride
 * (val_tokens - T - 1) / (val_batches * batch)), the f32 sum of the
 * batches' eval losses in order, divided by val_batches.  tokens holds at
 * least train_tokens + val_tokens ids. */
f32 gpu_trainer_eval_windows(GpuTrainer* g, const u32* tokens, u64 train_tokens, u64 val_tokens, u32 val_batches);
/* lr_warmup_cosine (training/lr_schedule.c:6-15): linear warmup to peak over
 * warmup steps, then half a cosine from peak to min by total_steps. */
f32 trlm_lr_warmup_cosine(u64 step, u64 warmup_steps, u64 total_steps, f32 peak_lr, f32 min_lr);

/* ---- node_matmul2d_gpu operand pinning (gpu_ops.h path) ----
 * gpu_ops_pin(data, count): the caller promises that data[0..count) stays
 * unchanged until gpu_ops_unpin_all().  A matmul operand (plain, transposed
 * or column-sliced view) lying wholly inside a pinned range is then read
 * from a device copy, made once per GPU on first use, instead of being
 * uploaded on every call -- for generate/chat, pin every parameter after
 * loading the model.  Results are unchanged.  gpu_ops_unpin_all frees the
 * copies; it must not run concurrently with matmuls; gpu_ops_shutdown calls
 * it. */
void gpu_ops_pin(const f32* data, u64 count);
void gpu_ops_unpin_all(void);

/* Stream-event timing on the current context's stream. */
typedef struct TrlmTimer { hipEvent_t start, stop; } TrlmTimer;
void trlm_timer_create(TrlmTimer* t);
void trlm_timer_destroy(TrlmTimer* t);
void trlm_timer_start(TrlmTimer* t);
f32 trlm_timer_stop_ms(TrlmTimer* t);   /* waits for the stop event */

/* Library version string (build identification) and the sizes of the
 * by-value structures, for bindings that must allocate them. */
const char* trlm_version(void);
u64 trlm_sizeof_gpu_trainer(void);
u64 trlm_sizeof_hip_ctx(void);

#ifdef __cplusplus
}
#endif

#endif /* TRLM_EXT_H */
