/* ref_harness.c -- TEST INFRASTRUCTURE ONLY.
 *
 * Drives the reference's own CPU path, compiled from its sources under
 * /root/reference into oracle/_ref/libtrlm_ref.so (see oracle/Makefile),
 * through a flat C interface that ctypes can call.  Used to pin the oracle
 * restatement (trlm_oracle.c) and as bench.py's "reference" CPU baseline.
 *
 * The reference library is opened with RTLD_LAZY: its model files reference
 * the GPU matmul entry points (model/gpu_ops.h), which are not built here
 * and are never called on this path (use_gpu_layers = use_gpu_output = 0);
 * likewise model/gpu_train.c is in the library only for its host-side batch
 * sampler, and its cuda_* calls are never reached.
 *
 * The per-sequence threading and gradient averaging below restate
 * data_parallel_step (training/data_parallel.c:156-199), whose own worker
 * calls a GPU entry point unconditionally (data_parallel.c:87) and so
 * cannot run without a GPU build.
 */
#include <dlfcn.h>
#include <pthread.h>
#include <string.h>
#include <time.h>

#include "runtime/types.h"
#include "runtime/memory.h"
#include "runtime/prng.h"
#include "tensor/tensor.h"
#include "autograd/node.h"
#include "model/lm_model.h"
#include "model/transformer_block.h"
#include "model/embedding.h"
#include "model/model_ops.h"
#include "model/attention.h"
#include "model/rope.h"
#include "model/loss.h"
#include "training/adam.h"
#include "training/checkpoint.h"

static struct {
    Allocator (*allocator_create)(u64);
    void (*allocator_destroy)(Allocator*);
    PCGState (*pcg_seed)(u64, u64);
    u32 (*pcg_next_u32)(PCGState*);
    i64 (*pcg_range_i64)(PCGState*, i64, i64);
    f64 (*pcg_gaussian)(PCGState*, f64, f64);
    LMModel (*lm_init)(Allocator*, PCGState*, u32, u32, u32, u32, u32, f32);
    u32 (*lm_collect_params)(LMModel*, Node**);
    Node* (*lm_forward)(Allocator*, LMModel*, const u32*, u32, u64, Node*, Node*, Node*, i32, i32);
    Tensor (*tensor_create)(Allocator*, const u64*, u32);
    Tensor (*tensor_matmul2d)(Allocator*, const Tensor*, const Tensor*);
    Node* (*node_leaf)(Allocator*, Tensor, bool32);
    void (*rope_build_tables)(Tensor*, Tensor*, u64, u64, f32);
    void (*build_causal_mask)(Tensor*);
    Node* (*node_cross_entropy_loss)(Allocator*, Node*, const u32*);
    void (*backward)(Allocator*, Node*);
    AdamOptimizer (*adam_create)(Allocator*, Node**, u32, f32, f32, f32, f32);
    void (*adam_step)(AdamOptimizer*);
    void (*adam_step_parallel)(AdamOptimizer*, u32);
    f64 (*m_sqrt)(f64); f64 (*m_exp)(f64); f64 (*m_log)(f64); f64 (*m_pow)(f64, f64);
    f64 (*m_sin)(f64); f64 (*m_cos)(f64);
    f32 (*m_powf)(f32, f32); f32 (*m_expf)(f32); f32 (*m_logf)(f32); f32 (*m_sqrtf)(f32);
    f32 (*m_sinf)(f32); f32 (*m_cosf)(f32);
    bool32 (*checkpoint_save)(const char*, Node**, u32, const AdamOptimizer*);
    bool32 (*checkpoint_load)(Allocator*, const char*, Node**, u32, AdamOptimizer*);
    f32 (*lr_warmup_cosine)(u64, u64, u64, f32, f32);
    void (*gpu_trainer_sample_batch)(const u32*, u64, u32, u32, u64, u32*, u32*);
    Node* (*transformer_block)(Allocator*, Node*, const BlockWeights*, u32, u32, u64, Node*, Node*, Node*, f32, i32);
    Node* (*node_embedding_lookup)(Allocator*, Node*, const u32*, u64);
    Node* (*node_rmsnorm)(Allocator*, Node*, Node*, f32);
    Node* (*node_transpose)(Allocator*, Node*, u32, u32);
    Node* (*node_matmul2d)(Allocator*, Node*, Node*);
    Node* (*node_sum_all)(Allocator*, Node*);
    int ok;
} R;

#define LOAD(name) do { *(void**)(&R.name) = dlsym(h, #name); if (!R.name) return -2; } while (0)

int refh_open(const char* lib_path) {
    void* h = dlopen(lib_path, RTLD_LAZY | RTLD_LOCAL);
    if (!h) return -1;
    LOAD(allocator_create); LOAD(allocator_destroy);
    LOAD(pcg_seed); LOAD(pcg_next_u32); LOAD(pcg_range_i64); LOAD(pcg_gaussian);
    LOAD(lm_init); LOAD(lm_collect_params); LOAD(lm_forward);
    LOAD(tensor_create); LOAD(tensor_matmul2d); LOAD(node_leaf);
    LOAD(rope_build_tables); LOAD(build_causal_mask); LOAD(node_cross_entropy_loss);
    LOAD(backward); LOAD(adam_create); LOAD(adam_step); LOAD(adam_step_parallel);
    LOAD(m_sqrt); LOAD(m_exp); LOAD(m_log); LOAD(m_pow); LOAD(m_sin); LOAD(m_cos);
    LOAD(m_powf); LOAD(m_expf); LOAD(m_logf); LOAD(m_sqrtf); LOAD(m_sinf); LOAD(m_cosf);
    LOAD(checkpoint_save); LOAD(checkpoint_load);
    LOAD(lr_warmup_cosine);
    LOAD(gpu_trainer_sample_batch);
    LOAD(transformer_block); LOAD(node_embedding_lookup); LOAD(node_rmsnorm);
    LOAD(node_transpose); LOAD(node_matmul2d); LOAD(node_sum_all);
    R.ok = 1;
    return 0;
}

/* ---- scalar maths and PRNG ---- */
double refh_m(int which, double x, double y) {
    switch (which) {
        case 0: return R.m_sqrt(x);
        case 1: return R.m_exp(x);
        case 2: return R.m_log(x);
        case 3: return R.m_pow(x, y);
        case 4: return R.m_sin(x);
        case 5: return R.m_cos(x);
        case 10: return (double)R.m_sqrtf((f32)x);
        case 11: return (double)R.m_expf((f32)x);
        case 12: return (double)R.m_logf((f32)x);
        case 13: return (double)R.m_powf((f32)x, (f32)y);
        case 14: return (double)R.m_sinf((f32)x);
        case 15: return (double)R.m_cosf((f32)x);
        default: return 0.0;
    }
}

/* lr_warmup_cosine (training/lr_schedule.c) for steps first..first+n-1. */
void refh_lr_schedule(u64 first, u32 n, u64 warmup, u64 total, f32 peak, f32 min_lr, f32* out) {
    for (u32 i = 0; i < n; i++) out[i] = R.lr_warmup_cosine(first + i, warmup, total, peak, min_lr);
}

/* The reference's batch sampler (model/gpu_train.c:296-307), host code only. */
void refh_sample_batch(const u32* tokens, u64 num_tokens, u32 T, u32 B, u64 seed_base, u32* ids, u32* tgt) {
    R.gpu_trainer_sample_batch(tokens, num_tokens, T, B, seed_base, ids, tgt);
}

void refh_pcg_u32(u64 sa, u64 sb, u32 n, u32* out) {
    PCGState r = R.pcg_seed(sa, sb);
    for (u32 i = 0; i < n; i++) out[i] = R.pcg_next_u32(&r);
}

void refh_pcg_range(u64 sa, u64 sb, i64 lo, i64 hi, u32 n, i64* out) {
    PCGState r = R.pcg_seed(sa, sb);
    for (u32 i = 0; i < n; i++) out[i] = R.pcg_range_i64(&r, lo, hi);
}

void refh_pcg_gauss(u64 sa, u64 sb, u32 n, f64* out) {
    PCGState r = R.pcg_seed(sa, sb);
    for (u32 i = 0; i < n; i++) out[i] = R.pcg_gaussian(&r, 0.0, 1.0);
}

void refh_rope_tables(u32 T, u32 hd, f32* cos_out, f32* sin_out) {
    Allocator a = R.allocator_create(1ull << 26);
    u64 sh[2] = { T, hd / 2 };
    Tensor c = R.tensor_create(&a, sh, 2), s = R.tensor_create(&a, sh, 2);
    R.rope_build_tables(&c, &s, T, hd, 10000.0f);
    memcpy(cos_out, c.data, c.numel * sizeof(f32));
    memcpy(sin_out, s.data, s.numel * sizeof(f32));
    R.allocator_destroy(&a);
}

/* ---- model ---- */
typedef struct RefCfg { u32 V, D, H, L, F; f32 eps; } RefCfg;

static u64 arena_for(const RefCfg* c, u32 T) {
    u64 per = (u64)T * T * c->H * 48ull + (u64)T * c->V * 24ull + (u64)T * c->D * 400ull * c->L
            + (u64)c->V * c->D * 16ull + (u64)c->L * c->D * c->F * 64ull + (1ull << 30);
    return 2 * per;   /* a reservation: pages are committed only as the arena is used */
}

void refh_lm_init(const RefCfg* c, u64 sa, u64 sb, f32* params_out) {
    Allocator a = R.allocator_create(arena_for(c, 1));
    PCGState rng = R.pcg_seed(sa, sb);
    LMModel m = R.lm_init(&a, &rng, c->V, c->D, c->H, c->L, c->F, c->eps);
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np = R.lm_collect_params(&m, ps);
    u64 off = 0;
    for (u32 i = 0; i < np; i++) {
        memcpy(params_out + off, ps[i]->value.data, ps[i]->value.numel * sizeof(f32));
        off += ps[i]->value.numel;
    }
    R.allocator_destroy(&a);
}

/* A model whose parameter Nodes hold copies of the flat buffer, assembled in
 * lm_collect_params order (model/lm_model.c:134-148) without drawing weights. */
static Node* leaf_copy(Allocator* a, const f32* src, u64 rows, u64 cols, u32 ndim) {
    u64 sh[2] = { rows, cols };
    Tensor t = R.tensor_create(a, ndim == 2 ? sh : &sh[1], ndim);
    memcpy(t.data, src, t.numel * sizeof(f32));
    return R.node_leaf(a, t, TRUE);
}

static LMModel model_from_flat(Allocator* a, const RefCfg* c, const f32* params, Node** ps, u32* np) {
    LMModel m;
    memset(&m, 0, sizeof(m));
    m.num_layers = c->L; m.num_heads = c->H; m.d_model = c->D; m.vocab_size = c->V; m.eps = c->eps;
    u64 D = c->D, F = c->F, off = 0;
    m.embed_table = leaf_copy(a, params + off, c->V, D, 2); off += (u64)c->V * D;
    for (u32 l = 0; l < c->L; l++) {
        BlockWeights* b = &m.blocks[l];
        b->attn_norm_w = leaf_copy(a, params + off, 1, D, 1); off += D;
        b->attn.w_qkv = leaf_copy(a, params + off, D, 3 * D, 2); off += 3 * D * D;
        b->attn.b_qkv = leaf_copy(a, params + off, 1, 3 * D, 1); off += 3 * D;
        b->attn.wo = leaf_copy(a, params + off, D, D, 2); off += D * D;
        b->attn.bo = leaf_copy(a, params + off, 1, D, 1); off += D;
        b->ffn_norm_w = leaf_copy(a, params + off, 1, D, 1); off += D;
        b->ffn.w_gate_up = leaf_copy(a, params + off, D, 2 * F, 2); off += 2 * F * D;
        b->ffn.b_gate_up = leaf_copy(a, params + off, 1, 2 * F, 1); off += 2 * F;
        b->ffn.w_down = leaf_copy(a, params + off, F, D, 2); off += F * D;
        b->ffn.b_down = leaf_copy(a, params + off, 1, D, 1); off += D;
    }
    m.final_norm_w = leaf_copy(a, params + off, 1, D, 1);
    *np = R.lm_collect_params(&m, ps);
    return m;
}

typedef struct Work {
    const RefCfg* c; const f32* params; const u32* ids; const u32* tgt; u32 T;
    f32* grads; f32* logits; f32 loss; u64 total;
} Work;

static void* work_run(void* arg) {
    Work* w = (Work*)arg;
    const RefCfg* c = w->c;
    Allocator a = R.allocator_create(arena_for(c, w->T));
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np;
    LMModel m = model_from_flat(&a, c, w->params, ps, &np);
    u32 hd = c->D / c->H;
    u64 cs[2] = { w->T, hd / 2 }, ms[2] = { w->T, w->T };
    Tensor ct = R.tensor_create(&a, cs, 2), st = R.tensor_create(&a, cs, 2), mt = R.tensor_create(&a, ms, 2);
    R.rope_build_tables(&ct, &st, w->T, hd, 10000.0f);
    R.build_causal_mask(&mt);
    Node* cl = R.node_leaf(&a, ct, FALSE);
    Node* sl = R.node_leaf(&a, st, FALSE);
    Node* ml = R.node_leaf(&a, mt, FALSE);
    Node* logits = R.lm_forward(&a, &m, w->ids, 1, w->T, cl, sl, ml, 0, 0);
    if (w->logits) {
        memcpy(w->logits, logits->value.data, logits->value.numel * sizeof(f32));
    } else {
        Node* loss = R.node_cross_entropy_loss(&a, logits, w->tgt);
        if (w->grads) {
            R.backward(&a, loss);
            u64 off = 0;
            for (u32 i = 0; i < np; i++) {
                memcpy(w->grads + off, ps[i]->grad.data, ps[i]->grad.numel * sizeof(f32));
                off += ps[i]->grad.numel;
            }
        }
        w->loss = loss->value.data[0];
    }
    R.allocator_destroy(&a);
    return NULL;
}

static void run_all(Work* ws, u32 B, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    for (u32 s = 0; s < B; s += (u32)nthreads) {
        pthread_t th[64];
        u32 e = s + (u32)nthreads < B ? s + (u32)nthreads : B;
        for (u32 w = s; w < e; w++) pthread_create(&th[w - s], NULL, work_run, &ws[w]);
        for (u32 w = s; w < e; w++) pthread_join(th[w - s], NULL);
    }
}

void refh_forward_logits(const RefCfg* c, const f32* params, const u32* ids, u32 B, u32 T, f32* logits, int nthreads) {
    Work ws[64];
    for (u32 w = 0; w < B; w++) {
        memset(&ws[w], 0, sizeof(Work));
        ws[w].c = c; ws[w].params = params; ws[w].ids = ids + (u64)w * T; ws[w].T = T;
        ws[w].logits = logits + (u64)w * T * c->V;
    }
    run_all(ws, B, nthreads);
}

/* grads: [total] averaged over B; scratch: [B * total] per-sequence grads. */
f32 refh_forward_backward(const RefCfg* c, const f32* params, const u32* ids, const u32* tgt, u32 B, u32 T,
                          u64 total, f32* grads, f32* scratch, int nthreads) {
    Work ws[64];
    for (u32 w = 0; w < B; w++) {
        memset(&ws[w], 0, sizeof(Work));
        ws[w].c = c; ws[w].params = params; ws[w].ids = ids + (u64)w * T; ws[w].tgt = tgt + (u64)w * T;
        ws[w].T = T; ws[w].total = total;
        ws[w].grads = grads ? scratch + (u64)w * total : NULL;
    }
    run_all(ws, B, nthreads);
    if (grads) {
        f32 inv = 1.0f / (f32)B;
        for (u64 k = 0; k < total; k++) grads[k] = 0.0f;
        for (u32 w = 0; w < B; w++) for (u64 k = 0; k < total; k++) grads[k] += scratch[(u64)w * total + k];
        for (u64 k = 0; k < total; k++) grads[k] *= inv;
    }
    f32 ls = 0.0f;
    for (u32 w = 0; w < B; w++) ls += ws[w].loss;
    return ls / (f32)B;
}

/* One Adam step of the reference (training/adam.c) over a flat buffer. */
void refh_adam_step(const RefCfg* c, f32* params, const f32* grads, f32* m, f32* v, u64 t_before,
                    f32 lr, f32 b1, f32 b2, f32 eps) {
    Allocator a = R.allocator_create(arena_for(c, 1));
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np;
    model_from_flat(&a, c, params, ps, &np);
    AdamOptimizer opt = R.adam_create(&a, ps, np, lr, b1, b2, eps);
    opt.t = t_before;
    u64 off = 0;
    for (u32 i = 0; i < np; i++) {
        u64 n = ps[i]->value.numel;
        memcpy(ps[i]->grad.data, grads + off, n * sizeof(f32));
        memcpy(opt.m[i].data, m + off, n * sizeof(f32));
        memcpy(opt.v[i].data, v + off, n * sizeof(f32));
        off += n;
    }
    R.adam_step(&opt);
    off = 0;
    for (u32 i = 0; i < np; i++) {
        u64 n = ps[i]->value.numel;
        memcpy(params + off, ps[i]->value.data, n * sizeof(f32));
        memcpy(m + off, opt.m[i].data, n * sizeof(f32));
        memcpy(v + off, opt.v[i].data, n * sizeof(f32));
        off += n;
    }
    R.allocator_destroy(&a);
}

/* C = A @ B through tensor_matmul2d (tensor/tensor.c:351-373). */
void refh_matmul(u32 M, u32 N, u32 K, const f32* A, const f32* B, f32* C) {
    Allocator a = R.allocator_create(((u64)M * K + (u64)K * N + (u64)M * N) * 4ull + (1ull << 24));
    u64 sa[2] = { M, K }, sb[2] = { K, N };
    Tensor ta = R.tensor_create(&a, sa, 2), tb = R.tensor_create(&a, sb, 2);
    memcpy(ta.data, A, (u64)M * K * 4);
    memcpy(tb.data, B, (u64)K * N * 4);
    Tensor tc = R.tensor_matmul2d(&a, &ta, &tb);
    memcpy(C, tc.data, (u64)M * N * 4);
    R.allocator_destroy(&a);
}

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

/* Wall seconds of one reference training step (forward, backward, average,
 * adam_step_parallel) for B sequences of T tokens on nthreads threads. */
double refh_time_train_step(const RefCfg* c, f32* params, const u32* ids, const u32* tgt, u32 B, u32 T,
                            u64 total, f32* grads, f32* scratch, int nthreads) {
    double t0 = now_s();
    refh_forward_backward(c, params, ids, tgt, B, T, total, grads, scratch, nthreads);
    double t1 = now_s();
    Allocator a = R.allocator_create(arena_for(c, 1));
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np;
    model_from_flat(&a, c, params, ps, &np);
    AdamOptimizer opt = R.adam_create(&a, ps, np, 3e-4f, 0.9f, 0.95f, 1e-8f);
    u64 off = 0;
    for (u32 i = 0; i < np; i++) { memcpy(ps[i]->grad.data, grads + off, ps[i]->grad.numel * 4); off += ps[i]->grad.numel; }
    double t2 = now_s();   /* the harness-side model rebuild above is not timed */
    R.adam_step_parallel(&opt, (u32)nthreads);
    double t3 = now_s();
    R.allocator_destroy(&a);
    return (t1 - t0) + (t3 - t2);
}

double refh_time_forward(const RefCfg* c, const f32* params, const u32* ids, u32 B, u32 T, f32* logits, int nthreads) {
    double t0 = now_s();
    refh_forward_logits(c, params, ids, B, T, logits, nthreads);
    return now_s() - t0;
}

/* ---- the reference's CPU step in pieces, for a bounded baseline ----
 *
 * A full B=8, T=1024 step of the 12-layer model takes minutes on the host
 * cores, so the timed sample is its two kinds of piece, each run by
 * nthreads concurrent threads (one sequence each, as data_parallel_step
 * gives every sequence a thread), all released together by a barrier:
 *   block: one transformer_block (model/transformer_block.c) over T rows,
 *          forward, then node_sum_all + backward (gradients of the block's
 *          weights and of its input, as inside the full model);
 *   head:  node_embedding_lookup over R rows, the final node_rmsnorm, the
 *          tied node_matmul2d against node_transpose(embed_table), and
 *          node_cross_entropy_loss (model/lm_model.c:62-82), forward then
 *          backward.
 * Every row of the head piece costs the same whatever T is (no attention),
 * so a step is  L * block(T) + (T / R) * head(R)  plus the optimizer.
 * out[0] / out[1]: block forward / forward+backward wall seconds;
 * out[2] / out[3]: head forward / forward+backward wall seconds.  Wall =
 * latest finish minus earliest start over the threads. */
typedef struct PieceWork {
    const RefCfg* c; const f32* params; const u32* ids; const u32* tgt; u32 T, R;
    pthread_barrier_t* bar;
    double t0[2], t1[2], t2[2];
} PieceWork;

static void* piece_run(void* arg) {
    PieceWork* w = (PieceWork*)arg;
    const RefCfg* c = w->c;
    Allocator a = R.allocator_create(arena_for(c, w->T));
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np;
    LMModel m = model_from_flat(&a, c, w->params, ps, &np);
    u32 hd = c->D / c->H;
    u64 cs[2] = { w->T, hd / 2 }, ms[2] = { w->T, w->T }, xs[2] = { w->T, c->D };
    Tensor ct = R.tensor_create(&a, cs, 2), st = R.tensor_create(&a, cs, 2), mt = R.tensor_create(&a, ms, 2);
    R.rope_build_tables(&ct, &st, w->T, hd, 10000.0f);
    R.build_causal_mask(&mt);
    Node* cl = R.node_leaf(&a, ct, FALSE);
    Node* sl = R.node_leaf(&a, st, FALSE);
    Node* ml = R.node_leaf(&a, mt, FALSE);
    Tensor xt = R.tensor_create(&a, xs, 2);   /* the block's input: the sequence's embedding rows */
    for (u32 t = 0; t < w->T; t++)
        memcpy(xt.data + (u64)t * c->D, w->params + (u64)w->ids[t] * c->D, c->D * sizeof(f32));
    Node* x = R.node_leaf(&a, xt, TRUE);

    pthread_barrier_wait(w->bar);
    w->t0[0] = now_s();
    Node* y = R.transformer_block(&a, x, &m.blocks[0], c->H, 1, w->T, cl, sl, ml, m.eps, 0);
    Node* s = R.node_sum_all(&a, y);
    w->t1[0] = now_s();
    R.backward(&a, s);
    w->t2[0] = now_s();

    pthread_barrier_wait(w->bar);
    w->t0[1] = now_s();
    Node* e = R.node_embedding_lookup(&a, m.embed_table, w->ids, w->R);
    Node* h = R.node_rmsnorm(&a, e, m.final_norm_w, m.eps);
    Node* et = R.node_transpose(&a, m.embed_table, 0, 1);
    Node* lg = R.node_matmul2d(&a, h, et);
    Node* loss = R.node_cross_entropy_loss(&a, lg, w->tgt);
    w->t1[1] = now_s();
    R.backward(&a, loss);
    w->t2[1] = now_s();
    R.allocator_destroy(&a);
    return NULL;
}

int refh_time_pieces(const RefCfg* c, const f32* params, const u32* ids, const u32* tgt, u32 T, u32 R_rows,
                     int nthreads, double* out) {
    if (nthreads < 1 || nthreads > 64 || R_rows < 1 || R_rows > T || c->L < 1) return -1;
    PieceWork ws[64];
    pthread_t th[64];
    pthread_barrier_t bar;
    pthread_barrier_init(&bar, NULL, (unsigned)nthreads);
    for (int w = 0; w < nthreads; w++) {
        memset(&ws[w], 0, sizeof(PieceWork));
        ws[w].c = c; ws[w].params = params; ws[w].ids = ids + (u64)w * T; ws[w].tgt = tgt + (u64)w * T;
        ws[w].T = T; ws[w].R = R_rows; ws[w].bar = &bar;
    }
    for (int w = 0; w < nthreads; w++) pthread_create(&th[w], NULL, piece_run, &ws[w]);
    for (int w = 0; w < nthreads; w++) pthread_join(th[w], NULL);
    pthread_barrier_destroy(&bar);
    for (int k = 0; k < 2; k++) {
        double s0 = ws[0].t0[k], e1 = ws[0].t1[k], e2 = ws[0].t2[k];
        for (int w = 1; w < nthreads; w++) {
            if (ws[w].t0[k] < s0) s0 = ws[w].t0[k];
            if (ws[w].t1[k] > e1) e1 = ws[w].t1[k];
            if (ws[w].t2[k] > e2) e2 = ws[w].t2[k];
        }
        out[2 * k] = e1 - s0;
        out[2 * k + 1] = e2 - s0;
    }
    return 0;
}

/* Wall seconds of adam_step_parallel (training/adam.c:70-102) over the whole
 * model's parameters with the gradients given, on nthreads threads. */
double refh_time_adam(const RefCfg* c, f32* params, const f32* grads, int nthreads) {
    Allocator a = R.allocator_create(arena_for(c, 1));
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np;
    model_from_flat(&a, c, params, ps, &np);
    AdamOptimizer opt = R.adam_create(&a, ps, np, 3e-4f, 0.9f, 0.95f, 1e-8f);
    u64 off = 0;
    for (u32 i = 0; i < np; i++) { memcpy(ps[i]->grad.data, grads + off, ps[i]->grad.numel * 4); off += ps[i]->grad.numel; }
    double t0 = now_s();
    R.adam_step_parallel(&opt, (u32)nthreads);
    double t1 = now_s();
    R.allocator_destroy(&a);
    return t1 - t0;
}

/* Wall seconds of an M x N x K product through tensor_matmul2d
 * (tensor/tensor.c:351-373) split by rows over nthreads concurrent threads,
 * each running the reference's single-threaded loop on its own rows. */
typedef struct MmWork { u32 M, N, K; const f32* A; const f32* B; f32* C; } MmWork;

static void* mm_run(void* arg) {
    MmWork* w = (MmWork*)arg;
    if (w->M) refh_matmul(w->M, w->N, w->K, w->A, w->B, w->C);
    return NULL;
}

double refh_time_matmul_threads(u32 M, u32 N, u32 K, const f32* A, const f32* B, f32* C, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 64) nthreads = 64;
    MmWork ws[64];
    pthread_t th[64];
    u32 per = (M + (u32)nthreads - 1) / (u32)nthreads;
    double t0 = now_s();
    for (int w = 0; w < nthreads; w++) {
        u32 r0 = (u32)w * per < M ? (u32)w * per : M;
        u32 r1 = r0 + per < M ? r0 + per : M;
        ws[w].M = r1 - r0; ws[w].N = N; ws[w].K = K;
        ws[w].A = A + (u64)r0 * K; ws[w].B = B; ws[w].C = C + (u64)r0 * N;
        pthread_create(&th[w], NULL, mm_run, &ws[w]);
    }
    for (int w = 0; w < nthreads; w++) pthread_join(th[w], NULL);
    return now_s() - t0;
}

double refh_time_matmul(u32 M, u32 N, u32 K, const f32* A, const f32* B, f32* C) {
    double t0 = now_s();
    refh_matmul(M, N, K, A, B, C);
    return now_s() - t0;
}

/* ---- checkpoint TRLM v1 (training/checkpoint.c) over flat buffers ---- */

/* checkpoint_save of the model whose parameters are `params` (flat, in
 * lm_collect_params order) and, when has_opt, Adam state m, v, t. */
int refh_checkpoint_save(const RefCfg* c, const f32* params, const f32* m, const f32* v, u64 t, int has_opt,
                         const char* path) {
    Allocator a = R.allocator_create(arena_for(c, 1));
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np;
    model_from_flat(&a, c, params, ps, &np);
    AdamOptimizer opt = R.adam_create(&a, ps, np, 3e-4f, 0.9f, 0.95f, 1e-8f);
    opt.t = t;
    if (has_opt) {
        u64 off = 0;
        for (u32 i = 0; i < np; i++) {
            u64 n = ps[i]->value.numel;
            memcpy(opt.m[i].data, m + off, n * sizeof(f32));
            memcpy(opt.v[i].data, v + off, n * sizeof(f32));
            off += n;
        }
    }
    int ok = (int)R.checkpoint_save(path, ps, np, has_opt ? &opt : NULL);
    R.allocator_destroy(&a);
    return ok;
}

/* checkpoint_load into flat buffers (params always; m, v, *t when want_opt).
 * Returns the reference's result; on failure nothing is written. */
int refh_checkpoint_load(const RefCfg* c, const char* path, f32* params, f32* m, f32* v, u64* t, int want_opt) {
    Allocator a = R.allocator_create(arena_for(c, 1));
    Allocator scratch = R.allocator_create(4 * arena_for(c, 1));
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np;
    model_from_flat(&a, c, params, ps, &np);
    AdamOptimizer opt = R.adam_create(&a, ps, np, 3e-4f, 0.9f, 0.95f, 1e-8f);
    int ok = (int)R.checkpoint_load(&scratch, path, ps, np, want_opt ? &opt : NULL);
    if (ok) {
        u64 off = 0;
        for (u32 i = 0; i < np; i++) {
            u64 n = ps[i]->value.numel;
            memcpy(params + off, ps[i]->value.data, n * sizeof(f32));
            if (want_opt) {
                memcpy(m + off, opt.m[i].data, n * sizeof(f32));
                memcpy(v + off, opt.v[i].data, n * sizeof(f32));
            }
            off += n;
        }
        if (want_opt) *t = opt.t;
    }
    R.allocator_destroy(&scratch);
    R.allocator_destroy(&a);
    return ok;
}

/* checkpoint_save of a model built by the reference's own lm_init (so the
 * file's shapes are lm_init's), without optimizer state. */
int refh_checkpoint_save_init(const RefCfg* c, u64 sa, u64 sb, const char* path) {
    Allocator a = R.allocator_create(arena_for(c, 1));
    PCGState rng = R.pcg_seed(sa, sb);
    LMModel m = R.lm_init(&a, &rng, c->V, c->D, c->H, c->L, c->F, c->eps);
    Node* ps[LM_MAX_LAYERS * 12 + 2];
    u32 np = R.lm_collect_params(&m, ps);
    int ok = (int)R.checkpoint_save(path, ps, np, NULL);
    R.allocator_destroy(&a);
    return ok;
}
