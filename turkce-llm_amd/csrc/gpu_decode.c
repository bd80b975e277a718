/* gpu_decode.c -- KV-cache decode over a GpuTrainer's resident parameters.
 *
 * The reference generates text by running lm_forward over the whole window
 * for every new token and sampling the last row (training/generate.c:186-212,
 * sample_next at :57-73).  Within the model's context (no window slide) the
 * logits of the last position only depend on the keys and values of the
 * earlier positions, so this decoder keeps them:
 *   prefill: the trainer's own forward (trlm_forward_hidden) over
 *            batch x len rows, with a per-layer hook that copies the rotated
 *            K and V into the cache; the LM head runs on the last row of
 *            each sequence only;
 *   step:    one new token per sequence, four fused kernels per layer
 *            (kernels/decode_fused.hip): per (sequence, head) a workgroup
 *            forms the head's RMSNorm + QKV + RoPE, appends k and v to the
 *            cache and attends over it, its 8 waves splitting the context
 *            and merging in wave order; out-projection + residual;
 *            RMSNorm + gate/up + SwiGLU; down-projection + residual; then the
 *            final norm + LM head on `batch` rows.  Layer 0 reads its input
 *            rows straight from the embedding table.
 * Greedy selection is the first maximum of each row (k_argmax_rows);
 * sampling is sample_next's arithmetic on the device (k_sample_rows) with the
 * uniform drawn from the caller's PCG stream on the host, as pcg_uniform does
 * (runtime/prng.c:33-36).
 *
 * Cache layout: per layer [batch][H][max_ctx][hd] for K and for V; one cache
 * row per position, so the decode attention streams contiguous rows.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "trlm_ext.h"
#include "gpu_internal.h"

#define F4 ((u64)sizeof(f32))
#define DEC_QA_SEQ 2u      /* sequences per QKV + attention workgroup (as in decode_fused.hip) */
#define DEC_QA_WPS 4u      /* waves per sequence there */
#define DEC_HEAD_WAVES 8u  /* waves per LM-head workgroup (as in decode_fused.hip) */
#define DEC_HEAD_KMAX 512u /* d_model bound of the LM-head kernel's LDS rows */

#include "kernel_params.h"   /* DecGemmParams: the argument block the kernels read */

struct TrlmDecoder {
    GpuTrainer* g;
    u32 B, ctx, len;
    u32 L, H, hd, D, F, V, ldv;
    f32 scale;
    hipDeviceptr_t kc, vc;              /* [L][B][H][ctx][hd] each */
    hipDeviceptr_t cos_t, sin_t;        /* [ctx][hd/2] */
    /* step buffers, B rows */
    hipDeviceptr_t ids, x, x2, att, h, nf, logits, out_ids;
    /* sampling scratch */
    hipDeviceptr_t e, prefix, u;
    /* prefill buffers, grown to batch x len rows on demand */
    u64 pre_rows;
    hipDeviceptr_t p_x, p_x2, p_n, p_r1, p_r2, p_qkv, p_att, p_lse, p_gu, p_h, p_nf, p_rf, p_ids;
    hipFunction_t k_fill, k_gather, k_sample_exp, k_sample, k_sample_hist, k_argmax_hist;
    hipDeviceptr_t u_all;                /* sampled generation: the uniforms of every step */
    u64 u_cap;
    hipFunction_t k_qkv_attn, k_out, k_gu, k_down, k_head;
    /* step replay: the position lives on the device (pos_dev), so every step
     * is the same launch sequence -- captured once as a HIP graph on the
     * second step */
    hipDeviceptr_t pos_dev, hist;
    u32 hist_cap;
    u32 eager_steps;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

static void dec_fatal(const char* msg) {
    fprintf(stderr, "[HIP ERROR] gpu_decode: %s\n", msg);
    fflush(stderr);
    _exit(1);
}

static void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "[HIP ERROR] gpu_decode: %s -> %s: %s\n", what, hipGetErrorName(e), hipGetErrorString(e));
        fflush(stderr);
        _exit(1);
    }
}

static u32 cdiv32(u64 a, u64 b) { return (u32)((a + b - 1) / b); }
static hipDeviceptr_t fl(u64 floats) { return hip_alloc(floats * F4); }
static hipDeviceptr_t at(hipDeviceptr_t base, u64 floats) { return (hipDeviceptr_t)((char*)base + floats * F4); }

TrlmDecoder* gpu_decoder_create(GpuTrainer* g, u32 batch, u32 max_ctx) {
    if (batch == 0 || max_ctx == 0) dec_fatal("batch and max_ctx must be positive");
    /* the fused step kernels take 16-column output blocks that never straddle
     * a head or the q / k / v boundary, and 16-byte operand rows */
    if (g->D % 16 || g->hd % 16 || g->F % 4 || g->D > DEC_HEAD_KMAX)
        dec_fatal("decoding needs d_model and head_dim multiples of 16, d_model <= 512 and d_ff a multiple of 4");
    trlm_bind(g);
    TrlmDecoder* d = (TrlmDecoder*)calloc(1, sizeof(TrlmDecoder));
    d->g = g;
    d->B = batch; d->ctx = max_ctx; d->len = 0;
    d->L = g->L; d->H = g->H; d->hd = g->hd; d->D = g->D; d->F = g->F; d->V = g->V; d->ldv = g->ldv;
    d->scale = 1.0f / m_sqrtf((f32)g->hd);   /* attention.c:78 */

    u64 B = batch, D = g->D, F = g->F;
    u64 cache = (u64)g->L * B * g->H * max_ctx * g->hd;
    d->kc = fl(cache);
    d->vc = fl(cache);
    d->ids = hip_alloc(B * sizeof(u32));
    d->x = fl(B * D);
    d->x2 = fl(B * D);
    d->att = fl(B * D);
    d->h = fl(B * F);
    d->nf = fl(B * D);
    d->logits = fl(B * g->ldv);
    hip_memset_zero(d->logits, B * g->ldv * F4);
    d->out_ids = hip_alloc(B * sizeof(u32));
    d->e = fl(B * g->ldv);
    d->prefix = hip_alloc(B * g->V * sizeof(f64));
    d->u = hip_alloc(B * sizeof(f64));

    /* RoPE tables for every position of the context, built on the host as
     * the reference builds them (model/rope.c) */
    Tensor ct, st;
    memset(&ct, 0, sizeof(ct));
    ct.ndim = 2;
    ct.shape[0] = max_ctx;
    ct.shape[1] = g->hd / 2;
    ct.strides[0] = (i64)(g->hd / 2);
    ct.strides[1] = 1;
    ct.numel = (u64)max_ctx * (g->hd / 2);
    st = ct;
    ct.data = (f32*)malloc(ct.numel * F4);
    st.data = (f32*)malloc(st.numel * F4);
    if (!ct.data || !st.data) dec_fatal("out of host memory");
    rope_build_tables(&ct, &st, max_ctx, g->hd, 10000.0f);
    d->cos_t = fl(ct.numel);
    d->sin_t = fl(st.numel);
    hip_h2d(d->cos_t, ct.data, ct.numel * F4);
    hip_h2d(d->sin_t, st.data, st.numel * F4);
    hip_sync();
    free(ct.data);
    free(st.data);

    HipCtx* c = &g->hip;
    char name[64];
    d->k_fill = hip_get_kernel(c, "k_cache_fill");
    d->k_gather = hip_get_kernel(c, "k_gather_rows");
    d->k_sample_exp = hip_get_kernel(c, "k_sample_exp");
    d->k_sample = hip_get_kernel(c, "k_sample_rows");
    d->k_sample_hist = hip_get_kernel(c, "k_sample_hist");
    d->k_argmax_hist = hip_get_kernel(c, "k_argmax_hist");
    d->k_out = hip_get_kernel(c, "k_dec_out");
    d->k_gu = hip_get_kernel(c, "k_dec_gu");
    d->k_down = hip_get_kernel(c, "k_dec_down");
    /* the LM head holds a whole 16-column block of E in registers: the
     * instantiation with the fewest 16-deep steps covering d_model */
    d->k_head = hip_get_kernel(c, g->D <= 128 ? "k_dec_head_k8" : g->D <= 384 ? "k_dec_head_k24" : "k_dec_head_k32");
    snprintf(name, sizeof(name), "k_dec_qkv_attn_hd%u", g->hd);
    d->k_qkv_attn = hip_get_kernel(c, name);
    d->pos_dev = hip_alloc(sizeof(i32));
    hip_sync();
    return d;
}

static void free_prefill(TrlmDecoder* d) {
    hipDeviceptr_t* bufs[] = { &d->p_x, &d->p_x2, &d->p_n, &d->p_r1, &d->p_r2, &d->p_qkv, &d->p_att, &d->p_lse,
                               &d->p_gu, &d->p_h, &d->p_nf, &d->p_rf, &d->p_ids };
    for (u32 i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
        if (*bufs[i]) { hip_free(*bufs[i]); *bufs[i] = NULL; }
    d->pre_rows = 0;
}

static void drop_graph(TrlmDecoder* d) {
    if (d->exec) { hipGraphExecDestroy(d->exec); d->exec = NULL; }
    if (d->graph) { hipGraphDestroy(d->graph); d->graph = NULL; }
}

void gpu_decoder_destroy(TrlmDecoder* d) {
    if (!d) return;
    trlm_bind(d->g);
    hip_sync();
    drop_graph(d);
    free_prefill(d);
    if (d->hist) hip_free(d->hist);
    if (d->u_all) hip_free(d->u_all);
    hip_free(d->pos_dev);
    hipDeviceptr_t bufs[] = { d->kc, d->vc, d->ids, d->x, d->x2, d->att, d->h, d->nf,
                              d->logits, d->out_ids, d->e, d->prefix, d->u, d->cos_t, d->sin_t };
    for (u32 i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++) hip_free(bufs[i]);
    free(d);
}

u32 gpu_decoder_length(const TrlmDecoder* d) { return d->len; }

static void check_tokens(const TrlmDecoder* d, const u32* ids, u64 n) {
    for (u64 i = 0; i < n; i++)
        if (ids[i] >= d->V) {
            fprintf(stderr, "[HIP ERROR] gpu_decode: token %u at %llu is outside the vocabulary (%u)\n", ids[i],
                    (unsigned long long)i, d->V);
            fflush(stderr);
            _exit(1);
        }
}

static void cache_hook(void* ctx, GpuTrainer* pf, u32 layer, hipDeviceptr_t qkv) {
    TrlmDecoder* d = (TrlmDecoder*)ctx;
    u64 per_layer = (u64)d->B * d->H * d->ctx * d->hd;
    hipDeviceptr_t kc = at(d->kc, layer * per_layer), vc = at(d->vc, layer * per_layer);
    i32 ldq = 3 * (i32)d->D, B = (i32)d->B, len = (i32)pf->T, H = (i32)d->H, hd = (i32)d->hd, D = (i32)d->D;
    i32 ctxn = (i32)d->ctx;
    void* args[] = { &qkv, &ldq, &B, &len, &H, &hd, &D, &kc, &vc, &ctxn };
    hip_launch(d->k_fill, cdiv32((u64)d->B * pf->T * d->H * (d->hd / 4), 256), 1, 1, 256, 1, 1, 0, args);
}

/* logits [B, ldv] = nf [B, D] @ E^T */
static void head(TrlmDecoder* d) {
    GpuTrainer* g = d->g;
    i32 B = (i32)d->B, V = (i32)d->V, D = (i32)d->D;
    trlm_gemm_rows(g, GEMM_NT, d->nf, trlm_param_ptr(g, 0), d->logits, B, V, D, D, D, (i32)d->ldv, NULL, NULL);
}

void gpu_decoder_prefill(TrlmDecoder* d, const u32* ids, u32 len) {
    GpuTrainer* g = d->g;
    if (len == 0 || len > d->ctx) dec_fatal("prefill length must be in [1, max_ctx]");
    check_tokens(d, ids, (u64)d->B * len);
    trlm_bind(g);
    u64 R = (u64)d->B * len, D = d->D, F = d->F;
    if (R > d->pre_rows) {
        free_prefill(d);
        d->p_x = fl(R * D);
        d->p_x2 = fl(R * D);
        d->p_n = fl(R * D);
        d->p_r1 = fl(R);
        d->p_r2 = fl(R);
        d->p_qkv = fl(R * 3 * D);
        d->p_att = fl(R * D);
        d->p_lse = fl(R * d->H);
        d->p_gu = fl(R * 2 * F);
        d->p_h = fl(R * F);
        d->p_nf = fl(R * D);
        d->p_rf = fl(R);
        d->p_ids = hip_alloc(R * sizeof(u32));
        d->pre_rows = R;
    }
    /* The trainer's forward on batch x len rows: a copy of the trainer with
     * the same parameters, kernels and GEMM engine, whose activations are one
     * set of buffers shared by every layer (nothing is kept for a backward). */
    GpuTrainer pf = *g;
    pf.B = d->B; pf.T = len; pf.N = (u32)R;
    for (u32 l = 0; l < g->L; l++) {
        GpuLayerActs* a = &pf.layers[l];
        a->x_in = d->p_x; a->n1 = d->p_n; a->r1 = d->p_r1; a->qkv = d->p_qkv; a->att = d->p_att;
        a->lse = d->p_lse; a->x2 = d->p_x2; a->n2 = d->p_n; a->r2 = d->p_r2; a->gu = d->p_gu; a->h = d->p_h;
    }
    pf.x_final = d->p_x;
    pf.nf = d->p_nf;
    pf.rf = d->p_rf;
    pf.ids = d->p_ids;
    pf.cos_t = d->cos_t;
    pf.sin_t = d->sin_t;
    trlm_forward_hidden(&pf, ids, cache_hook, d);
    /* last row of every sequence -> head */
    {
        hipDeviceptr_t src = d->p_nf, dst = d->nf;
        i32 ld = (i32)D, stride = (i32)len, off = (i32)len - 1, cols = (i32)D, n = (i32)d->B;
        void* args[] = { &src, &ld, &stride, &off, &cols, &n, &dst };
        hip_launch(d->k_gather, cdiv32((u64)d->B * D, 256), 1, 1, 256, 1, 1, 0, args);
    }
    head(d);
    d->len = len;
    i32 lenv = (i32)len;
    hip_h2d(d->pos_dev, &lenv, sizeof(i32));
}

/* Workgroups of a fused decode GEMM: rt row tiles of 16*rb rows times the
 * column blocks, rounded up to a multiple of the 8 XCDs (the kernel maps
 * workgroup i to XCD i % 8 and skips the spare ones). */
static void dec_gemm_launch(hipFunction_t f, DecGemmParams* p, u32 rb, u32 waves) {
    u32 nrt = cdiv32((u64)p->M, 16u * rb), total = nrt * (u32)p->ncb;
    u32 per_xcd = cdiv32(total, 8);
    void* args[] = { p };
    hip_launch(f, 8 * per_xcd, 1, 1, 64 * waves, 1, 1, 0, args);
}

/* One decode step on the device: the token d->ids of every sequence at
 * position *pos_dev through the L layers and the head into d->logits, then
 * *pos_dev += 1.  Every argument is the same from step to step. */
static void step_body(TrlmDecoder* d) {
    GpuTrainer* g = d->g;
    const i32 Bc = (i32)d->B, D = (i32)d->D, F = (i32)d->F, H = (i32)d->H, hd = (i32)d->hd, ctxn = (i32)d->ctx;
    const float* E = (const float*)trlm_param_ptr(g, 0);
    const u64 per_layer = (u64)d->B * d->H * d->ctx * d->hd;
    hipDeviceptr_t x = d->x, x2 = d->x2, att = d->att, h = d->h, logits = d->logits, posd = d->pos_dev;
    DecGemmParams base;
    memset(&base, 0, sizeof(base));
    base.E = E;
    base.ids = (const u32*)d->ids;
    base.eps = g->eps;
    base.M = Bc;
    base.F = F;
    base.H = H; base.hd = hd; base.D = D; base.ctx = ctxn;
    base.cos_t = (const float*)d->cos_t; base.sin_t = (const float*)d->sin_t;
    base.pos = (const i32*)posd;
    for (u32 l = 0; l < d->L; l++) {
#define PP(k) ((const float*)trlm_param_ptr(g, trlm_pidx(l, k)))
        float* kc = (float*)at(d->kc, l * per_layer);
        float* vc = (float*)at(d->vc, l * per_layer);
        /* per (sequence, head): q | k -> cache | v -> cache = RoPE(RMSNorm(x) @ Wqkv + b),
         * then att = the attention of q over the cache and the new key */
        DecGemmParams p = base;
        p.A = (const float*)x; p.a_ids = l == 0; p.lda = D;
        p.W = PP(PK_WQKV); p.ldw = 3 * D; p.bias = PP(PK_BQKV); p.norm_w = PP(PK_ATTN_NORM);
        p.C = (float*)att; p.ldc = D;
        p.N = 3 * D; p.K = D;
        p.kc = kc; p.vc = vc;
        p.scale = d->scale;
        {
            void* args[] = { &p };
            hip_launch(d->k_qkv_attn, cdiv32(d->B, DEC_QA_SEQ) * d->H, 1, 1, 64 * DEC_QA_SEQ * DEC_QA_WPS, 1, 1, 0,
                       args);
        }
        /* x2 = x + (att @ Wo + bo) */
        p = base;
        p.A = (const float*)att; p.lda = D;
        p.W = PP(PK_WO); p.ldw = D; p.bias = PP(PK_BO);
        p.resid = (const float*)x; p.resid_ids = l == 0; p.ldr = D;
        p.C = (float*)x2; p.ldc = D;
        p.N = D; p.K = D; p.ncb = (i32)cdiv32((u64)D, 16);
        dec_gemm_launch(d->k_out, &p, 1, 4);
        /* h = SwiGLU(RMSNorm(x2) @ Wgu + bgu) */
        p = base;
        p.A = (const float*)x2; p.lda = D;
        p.W = PP(PK_WGU); p.ldw = 2 * F; p.bias = PP(PK_BGU); p.norm_w = PP(PK_FFN_NORM);
        p.C = (float*)h; p.ldc = F;
        p.N = 2 * F; p.K = D; p.ncb = (i32)cdiv32((u64)F, 16);
        dec_gemm_launch(d->k_gu, &p, 1, 4);
        /* x = x2 + (h @ Wd + bd) */
        p = base;
        p.A = (const float*)h; p.lda = F;
        p.W = PP(PK_WDOWN); p.ldw = D; p.bias = PP(PK_BDOWN);
        p.resid = (const float*)x2; p.ldr = D;
        p.C = (float*)x; p.ldc = D;
        p.N = D; p.K = F; p.ncb = (i32)cdiv32((u64)D, 16);
        dec_gemm_launch(d->k_down, &p, 1, 8);
#undef PP
    }
    /* logits = RMSNorm(x) @ E^T; the position moves on */
    DecGemmParams p = base;
    p.A = (const float*)x; p.a_ids = d->L == 0; p.lda = D;
    p.W = E; p.ldw = D; p.norm_w = (const float*)trlm_param_ptr(g, trlm_pidx(d->L, 0));
    p.C = (float*)logits; p.ldc = (i32)d->ldv;
    p.N = (i32)d->V; p.K = D; p.ncb = (i32)cdiv32((u64)d->V, 16);
    p.pos_inc = (i32*)posd;
    {
        /* persistent: at most one workgroup per CU (its rows fill most of the
         * CU's LDS), each of its 8 waves walking column blocks */
        u32 groups = cdiv32((u64)p.ncb, DEC_HEAD_WAVES);
        if (groups > 256) groups = 256;
        void* args[] = { &p };
        hip_launch(d->k_head, groups, cdiv32((u64)Bc, 64), 1, 64 * DEC_HEAD_WAVES, 1, 1, 0, args);
    }
}

/* Steps run eagerly the first time, then as replays of the step captured on
 * the second call.  With TRLM_DECODE_EAGER=1 in the environment every step runs eagerly --
 * the same kernels in the same order, for kernel tracers (rocprofv3
 * --kernel-trace faults on this ROCm while it intercepts a graph replay). */
static int eager_only(void) {
    static int v = -1;
    if (v < 0) {
        const char* e = getenv("TRLM_DECODE_EAGER");
        v = (e && e[0] == '1') ? 1 : 0;
    }
    return v;
}

static void run_step(TrlmDecoder* d) {
    hipStream_t st = hip_current_stream();
    if (eager_only() || d->eager_steps == 0) {
        step_body(d);
    } else if (d->exec) {
        check_hip(hipGraphLaunch(d->exec, st), "hipGraphLaunch");
    } else {
        check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        step_body(d);
        check_hip(hipStreamEndCapture(st, &d->graph), "hipStreamEndCapture");
        check_hip(hipGraphInstantiate(&d->exec, d->graph, NULL, NULL, 0), "hipGraphInstantiate");
        check_hip(hipGraphLaunch(d->exec, st), "hipGraphLaunch");
    }
    d->eager_steps++;
}

void gpu_decoder_step(TrlmDecoder* d, const u32* ids) {
    if (d->len == 0) dec_fatal("step before prefill");
    if (d->len >= d->ctx) dec_fatal("context is full (max_ctx reached)");
    check_tokens(d, ids, d->B);
    trlm_bind(d->g);
    hip_h2d(d->ids, ids, (u64)d->B * sizeof(u32));
    run_step(d);
    d->len++;
}

void gpu_decoder_logits(TrlmDecoder* d, f32* host_logits) {
    trlm_bind(d->g);
    for (u32 b = 0; b < d->B; b++)
        hip_d2h(host_logits + (u64)b * d->V, at(d->logits, (u64)b * d->ldv), (u64)d->V * F4);
}

void gpu_decoder_greedy(TrlmDecoder* d, u32* out_ids) {
    trlm_bind(d->g);
    trlm_argmax_rows(d->g, d->logits, (i32)d->ldv, d->B, d->out_ids);
    hip_d2h(out_ids, d->out_ids, (u64)d->B * sizeof(u32));
}

#define DEC_SAMPLE_THREADS 1024u   /* threads per workgroup of the sampling kernels */
#define DEC_SAMPLE_CHUNKS 8u       /* k_sample_exp workgroups per row (as in decode.hip) */

/* e = sample_next's exponentials of every row of the current logits */
static void sample_exp(TrlmDecoder* d, f32 temperature) {
    hipDeviceptr_t lg = d->logits, e = d->e;
    i32 ld = (i32)d->ldv, V = (i32)d->V;
    void* args[] = { &lg, &ld, &V, &temperature, &e };
    hip_launch(d->k_sample_exp, d->B, DEC_SAMPLE_CHUNKS, 1, DEC_SAMPLE_THREADS, 1, 1, 0, args);
}

/* TRLM_SAMPLE_SEQUENTIAL=1: every row takes the kernel's sequential path
 * (the reference's f64 sums on one thread) instead of the parallel exact
 * decision -- for checking that the two agree. */
static i32 sample_sequential(void) {
    const char* e = getenv("TRLM_SAMPLE_SEQUENTIAL");
    return (e && e[0] == '1') ? 1 : 0;
}

void gpu_decoder_sample(TrlmDecoder* d, PCGState* rngs, f32 temperature, u32* out_ids) {
    trlm_bind(d->g);
    f64* u = (f64*)malloc((u64)d->B * sizeof(f64));
    if (!u) dec_fatal("out of host memory");
    for (u32 b = 0; b < d->B; b++) u[b] = (f64)pcg_next_u32(&rngs[b]) * (1.0 / 4294967296.0);   /* pcg_uniform */
    hip_h2d(d->u, u, (u64)d->B * sizeof(f64));
    hipDeviceptr_t e = d->e, pr = d->prefix, up = d->u, out = d->out_ids;
    i32 V = (i32)d->V, ld = (i32)d->ldv, seq = sample_sequential();
    void* args[] = { &V, &ld, &up, &e, &pr, &out, &seq };
    sample_exp(d, temperature);
    hip_launch(d->k_sample, d->B, 1, 1, DEC_SAMPLE_THREADS, 1, 1, 0, args);
    hip_d2h(out_ids, d->out_ids, (u64)d->B * sizeof(u32));
    free(u);
}

/* History buffer of `steps` picks per sequence (grow-only). */
static void ensure_hist(TrlmDecoder* d, u32 steps) {
    if (d->hist_cap < d->B * steps) {
        if (d->hist) hip_free(d->hist);
        d->hist = hip_alloc((u64)d->B * steps * sizeof(u32));
        d->hist_cap = d->B * steps;
    }
}

void gpu_decoder_generate_sampled(TrlmDecoder* d, const u32* prompt, u32 prompt_len, u32 steps, PCGState* rngs,
                                  f32 temperature, u32* out) {
    if (steps == 0) return;
    if ((u64)prompt_len + steps > d->ctx) dec_fatal("prompt_len + steps exceeds max_ctx");
    gpu_decoder_prefill(d, prompt, prompt_len);
    ensure_hist(d, steps);
    /* every uniform up front, in the order the reference's loop draws them:
     * one pcg_uniform per sequence and token, from that sequence's stream */
    u64 n = (u64)steps * d->B;
    f64* u = (f64*)malloc(n * sizeof(f64));
    if (!u) dec_fatal("out of host memory");
    for (u32 s = 0; s < steps; s++)
        for (u32 b = 0; b < d->B; b++) u[(u64)s * d->B + b] = (f64)pcg_next_u32(&rngs[b]) * (1.0 / 4294967296.0);
    if (d->u_cap < n) {
        if (d->u_all) hip_free(d->u_all);
        d->u_all = hip_alloc(n * sizeof(f64));
        d->u_cap = n;
    }
    hip_h2d(d->u_all, u, n * sizeof(f64));
    free(u);
    /* pick s is taken when *pos_dev = prompt_len + s; it becomes the ids of
     * the next step directly on the device */
    hipDeviceptr_t ua = d->u_all, e = d->e, pr = d->prefix, ids = d->ids, hist = d->hist, posd = d->pos_dev;
    i32 V = (i32)d->V, ld = (i32)d->ldv, hl = (i32)steps, base = (i32)prompt_len, seq = sample_sequential();
    void* args[] = { &V, &ld, &ua, &e, &pr, &ids, &hist, &hl, &posd, &base, &seq };
    sample_exp(d, temperature);
    hip_launch(d->k_sample_hist, d->B, 1, 1, DEC_SAMPLE_THREADS, 1, 1, 0, args);
    for (u32 s = 1; s < steps; s++) {
        run_step(d);
        d->len++;
        sample_exp(d, temperature);
        hip_launch(d->k_sample_hist, d->B, 1, 1, DEC_SAMPLE_THREADS, 1, 1, 0, args);
    }
    hip_d2h(out, d->hist, (u64)d->B * steps * sizeof(u32));
}

void gpu_decoder_generate_greedy(TrlmDecoder* d, const u32* prompt, u32 prompt_len, u32 steps, u32* out) {
    if (steps == 0) return;
    if ((u64)prompt_len + steps > d->ctx) dec_fatal("prompt_len + steps exceeds max_ctx");
    gpu_decoder_prefill(d, prompt, prompt_len);
    ensure_hist(d, steps);
    /* pick s (s = 0 .. steps-1) is taken when *pos_dev = prompt_len + s; it
     * becomes the ids of the next step directly on the device */
    hipDeviceptr_t lg = d->logits, ids = d->ids, hist = d->hist, posd = d->pos_dev;
    i32 ld = (i32)d->ldv, V = (i32)d->V, hl = (i32)steps, base = (i32)prompt_len;
    void* args[] = { &lg, &ld, &V, &ids, &hist, &hl, &posd, &base };
    hip_launch(d->k_argmax_hist, d->B, 1, 1, 1024, 1, 1, 0, args);
    for (u32 s = 1; s < steps; s++) {
        run_step(d);
        d->len++;
        hip_launch(d->k_argmax_hist, d->B, 1, 1, 1024, 1, 1, 0, args);
    }
    hip_d2h(out, d->hist, (u64)d->B * steps * sizeof(u32));
}
