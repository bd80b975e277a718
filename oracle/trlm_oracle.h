/* trlm_oracle.h -- TEST INFRASTRUCTURE ONLY.
 *
 * CPU restatement of turkce-llm's fp32 CPU path (the path its GPU trainer is
 * checked against), used as the parity checker for the HIP path.  Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library.  Nothing in the product (turkce-llm_amd/, include/) links,
 * loads or calls it.
 *
 * Every function cites the reference file:line whose algorithm it restates.
 * Pinning (what checks each function beyond re-typing its formula):
 *   or_pcg_*                PCG32 known-answer vector (public pcg32 demo,
 *                           seed 42/54), plus bit-equality with oracle/_ref.
 *   or_m_*                  test_mathlib.c known-answer constants, libm
 *                           within 1 ulp, bit-equality with oracle/_ref.
 *   or_lm_init              bit-equality with oracle/_ref lm_init.
 *   or_matmul               fp64 brute force on off-grid shapes; exact on
 *                           small-integer inputs (test_cuda.c:55-94 case);
 *                           bit-equality with oracle/_ref tensor_matmul2d.
 *   or_forward_logits       bit-equality with oracle/_ref lm_forward; the
 *                           initial loss ~ ln V invariant.
 *   or_forward_backward     oracle/_ref autograd (data_parallel semantics),
 *                           central-difference gradient check on a tiny model.
 *   or_adam_step            oracle/_ref adam_step bit-equality; closed form
 *                           first step ~ lr*sign(g); AdamW(wd=0) == Adam.
 *   or_sample_batch         bit-equality with the reference's own
 *                           gpu_trainer_sample_batch (model/gpu_train.c,
 *                           compiled into oracle/_ref) and its frozen
 *                           windows in tests/golden/.
 *   or_argmax               numpy's first maximum on NaN-free rows and the
 *                           explicit NaN / -inf cases of its rule.
 */
#ifndef TRLM_ORACLE_H
#define TRLM_ORACLE_H

#include <stdint.h>

typedef struct OrPcg {
    uint64_t state;
    uint64_t inc;
    uint32_t has_cached;
    double cached;
} OrPcg;

typedef struct OrCfg {
    uint32_t V, D, H, L, F;
    float eps;
} OrCfg;

/* mathlib restatement (runtime/mathlib.c) */
double or_m_sqrt(double x);
double or_m_exp(double x);
double or_m_log(double x);
double or_m_pow(double b, double e);
double or_m_sin(double x);
double or_m_cos(double x);
/* lr_warmup_cosine (training/lr_schedule.c:6-15) */
float or_lr_warmup_cosine(uint64_t step, uint64_t warmup, uint64_t total, float peak, float min_lr);
float or_m_sqrtf(float x);
float or_m_expf(float x);
float or_m_logf(float x);
float or_m_powf(float b, float e);
float or_m_sinf(float x);
float or_m_cosf(float x);

/* PCG32 + helpers (runtime/prng.c) */
void or_pcg_seed(OrPcg* r, uint64_t initstate, uint64_t initseq);
uint32_t or_pcg_next_u32(OrPcg* r);
int64_t or_pcg_range_i64(OrPcg* r, int64_t lo, int64_t hi);
double or_pcg_gaussian(OrPcg* r, double mean, double stddev);

/* model layout (model/lm_model.c:134-148) */
uint32_t or_num_params(const OrCfg* c);
uint64_t or_param_layout(const OrCfg* c, uint64_t* offsets, uint64_t* numels);
void or_lm_init(const OrCfg* c, uint64_t seed_a, uint64_t seed_b, float* params);
void or_rope_tables(uint32_t T, uint32_t hd, float* cos_t, float* sin_t);
void or_sample_batch(const uint32_t* tokens, uint64_t num_tokens, uint32_t T, uint32_t B,
                     uint64_t seed_base, uint32_t* ids, uint32_t* tgt);

/* C[M,N] = A[M,K] @ B[K,N] with the reference's per-element summation order. */
void or_matmul(uint32_t M, uint32_t N, uint32_t K,
               const float* A, int64_t a_rs, int64_t a_cs,
               const float* B, int64_t b_rs, int64_t b_cs, float* C);

/* logits[B*T, V] of B independent sequences (one thread per sequence). */
void or_forward_logits(const OrCfg* c, const float* params, const uint32_t* ids,
                       uint32_t B, uint32_t T, float* logits, int nthreads);
/* loss and grads with data_parallel_step semantics; grads may be NULL. */
float or_forward_backward(const OrCfg* c, const float* params, const uint32_t* ids,
                          const uint32_t* tgt, uint32_t B, uint32_t T, float* grads,
                          float* loss_rows, int nthreads);

/* Adam (training/adam.c:70-95); wd > 0 adds the decoupled AdamW term. */
void or_adam_step(float* p, const float* g, float* m, float* v, uint64_t n, uint64_t t,
                  float lr, float b1, float b2, float eps, float wd, float grad_scale);

/* Greedy pick: the reference's max scan (generate.c:57-58) -- best starts at
 * index 0 and moves only to a strictly greater value, so ties keep the first
 * index, a NaN at index 0 keeps 0 and other NaNs are never picked. */
uint32_t or_argmax(const float* row, uint32_t n);
/* sample_next (training/generate.c:57-73) on one row of logits; scratch [n]. */
uint32_t or_sample_next(const float* logits, uint32_t n, float temperature, OrPcg* rng, float* scratch);

#endif
