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
 *   step:    one new token per sequence -- the layer GEMMs on `batch` rows,
 *            RoPE at the token's position, append to the cache, attention of
 *            the new query over the cache (k_decode_attn_hd*, split over the
 *            context, merged in chunk order), head on `batch` rows.
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
#define DEC_CHUNK 256u   /* keys per decode-attention block (<= 1024) */

struct TrlmDecoder {
    GpuTrainer* g;
    u32 B, ctx, len;
    u32 L, H, hd, D, F, V, ldv;
    u32 nsplit_max;
    f32 scale;
    hipDeviceptr_t kc, vc;              /* [L][B][H][ctx][hd] each */
    hipDeviceptr_t cos_t, sin_t;        /* [ctx][hd/2] */
    /* step buffers, B rows */
    hipDeviceptr_t ids, x, x2, n, r, qkv, att, gu, h, nf, logits, part, out_ids;
    /* sampling scratch */
    hipDeviceptr_t e, prefix, u;
    /* prefill buffers, grown to batch x len rows on demand */
    u64 pre_rows;
    hipDeviceptr_t p_x, p_x2, p_n, p_r1, p_r2, p_qkv, p_att, p_lse, p_gu, p_h, p_nf, p_rf, p_ids;
    hipFunction_t k_fill, k_append, k_attn, k_merge, k_gather, k_sample, k_advance, k_argmax_hist;
    /* step replay: the position lives on the device (pos_dev), the attention
     * grid is fixed at nsplit_max, and the step's GEMMs use the decoder's own
     * engine, so every step is the same launch sequence -- captured once as
     * a HIP graph after one eager step has sized the GEMM workspace */
    hipDeviceptr_t pos_dev, hist;
    u32 hist_cap;
    TrlmGemm* gemm;
    u32 eager_steps;
    hipGraph_t graph;
    hipGraphExec_t exec;
};

static void dec_fatal(const char* msg) {
    fprintf(stderr, "[HIP ERROR] gpu_decode: %s\n", msg);
    fflush(stderr);
    _exit(1);
}

static u32 cdiv32(u64 a, u64 b) { return (u32)((a + b - 1) / b); }
static hipDeviceptr_t fl(u64 floats) { return hip_alloc(floats * F4); }
static hipDeviceptr_t at(hipDeviceptr_t base, u64 floats) { return (hipDeviceptr_t)((char*)base + floats * F4); }

TrlmDecoder* gpu_decoder_create(GpuTrainer* g, u32 batch, u32 max_ctx) {
    if (batch == 0 || max_ctx == 0) dec_fatal("batch and max_ctx must be positive");
    trlm_bind(g);
    TrlmDecoder* d = (TrlmDecoder*)calloc(1, sizeof(TrlmDecoder));
    d->g = g;
    d->B = batch; d->ctx = max_ctx; d->len = 0;
    d->L = g->L; d->H = g->H; d->hd = g->hd; d->D = g->D; d->F = g->F; d->V = g->V; d->ldv = g->ldv;
    d->scale = 1.0f / m_sqrtf((f32)g->hd);   /* attention.c:78 */
    d->nsplit_max = cdiv32(max_ctx, DEC_CHUNK);

    u64 B = batch, D = g->D, F = g->F;
    u64 cache = (u64)g->L * B * g->H * max_ctx * g->hd;
    d->kc = fl(cache);
    d->vc = fl(cache);
    d->ids = hip_alloc(B * sizeof(u32));
    d->x = fl(B * D);
    d->x2 = fl(B * D);
    d->n = fl(B * D);
    d->r = fl(B);
    d->qkv = fl(B * 3 * D);
    d->att = fl(B * D);
    d->gu = fl(B * 2 * F);
    d->h = fl(B * F);
    d->nf = fl(B * D);
    d->logits = fl(B * g->ldv);
    hip_memset_zero(d->logits, B * g->ldv * F4);
    d->part = fl(B * g->H * d->nsplit_max * (g->hd + 4));
    d->out_ids = hip_alloc(B * sizeof(u32));
    d->e = fl(B * g->V);
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
    d->k_append = hip_get_kernel(c, "k_decode_qkv_append");
    snprintf(name, sizeof(name), "k_decode_attn_hd%u", g->hd);
    d->k_attn = hip_get_kernel(c, name);
    snprintf(name, sizeof(name), "k_decode_merge_hd%u", g->hd);
    d->k_merge = hip_get_kernel(c, name);
    d->k_gather = hip_get_kernel(c, "k_gather_rows");
    d->k_sample = hip_get_kernel(c, "k_sample_rows");
    d->k_advance = hip_get_kernel(c, "k_decode_advance");
    d->k_argmax_hist = hip_get_kernel(c, "k_argmax_hist");
    d->pos_dev = hip_alloc(sizeof(i32));
    d->gemm = trlm_gemm_create(c);
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
    hip_free(d->pos_dev);
    trlm_gemm_destroy(d->gemm);
    hipDeviceptr_t bufs[] = { d->kc, d->vc, d->ids, d->x, d->x2, d->n, d->r, d->qkv, d->att, d->gu, d->h, d->nf,
                              d->logits, d->part, d->out_ids, d->e, d->prefix, d->u, d->cos_t, d->sin_t };
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

/* One decode step on the device: embed d->ids at position *pos_dev, the L
 * blocks with the cache append and decode attention, final norm, head into
 * d->logits, *pos_dev += 1.  Every argument is the same from step to step. */
static void step_body(TrlmDecoder* d) {
    GpuTrainer ps = *d->g;   /* the trainer's kernels and parameters, the decoder's GEMM engine */
    ps.gemm = d->gemm;
    GpuTrainer* g = &ps;
    const u32 B = d->B;
    const i32 Bi = (i32)B, D = (i32)d->D, F = (i32)d->F, H = (i32)d->H, hd = (i32)d->hd, ldq = 3 * D;
    const i32 ctxn = (i32)d->ctx, chunk = (i32)DEC_CHUNK, nsg = (i32)d->nsplit_max;
    hipDeviceptr_t posd = d->pos_dev;
    trlm_embed_rows(g, d->ids, d->x, B);
    u64 per_layer = (u64)B * d->H * d->ctx * d->hd;
    for (u32 l = 0; l < d->L; l++) {
        hipDeviceptr_t kc = at(d->kc, l * per_layer), vc = at(d->vc, l * per_layer);
#define PP(k) trlm_param_ptr(g, trlm_pidx(l, k))
        trlm_rmsnorm_rows(g, d->x, PP(PK_ATTN_NORM), d->n, d->r, B);
        trlm_gemm_rows(g, GEMM_NN, d->n, PP(PK_WQKV), d->qkv, Bi, 3 * D, D, D, 3 * D, 3 * D, PP(PK_BQKV), NULL);
        {
            hipDeviceptr_t qkv = d->qkv, ct = d->cos_t, st = d->sin_t;
            void* args[] = { &qkv, (void*)&ldq, &ct, &st, &posd, (void*)&Bi, (void*)&H, (void*)&hd, (void*)&D,
                             &kc, &vc, (void*)&ctxn };
            hip_launch(d->k_append, cdiv32((u64)B * d->H * (d->hd / 2), 256), 1, 1, 256, 1, 1, 0, args);
        }
        {
            hipDeviceptr_t qkv = d->qkv, part = d->part, att = d->att;
            f32 scale = d->scale;
            void* args[] = { &qkv, (void*)&ldq, &kc, &vc, &posd, (void*)&ctxn, (void*)&H, (void*)&chunk, &scale,
                             &part };
            hip_launch(d->k_attn, B * d->H, d->nsplit_max, 1, 256, 1, 1, 0, args);
            void* args2[] = { &part, &posd, (void*)&chunk, (void*)&nsg, (void*)&H, (void*)&D, &att };
            hip_launch(d->k_merge, B * d->H, 1, 1, 64, 1, 1, 0, args2);
        }
        /* x2 = x + (att @ Wo + bo); x = x2 + (swiglu(norm(x2) @ Wgu + bgu) @ Wd + bd) */
        trlm_gemm_rows(g, GEMM_NN, d->att, PP(PK_WO), d->x2, Bi, D, D, D, D, D, PP(PK_BO), d->x);
        trlm_rmsnorm_rows(g, d->x2, PP(PK_FFN_NORM), d->n, d->r, B);
        trlm_gemm_rows(g, GEMM_NN, d->n, PP(PK_WGU), d->gu, Bi, 2 * F, D, D, 2 * F, 2 * F, PP(PK_BGU), NULL);
        trlm_swiglu_rows(g, d->gu, d->h, B);
        trlm_gemm_rows(g, GEMM_NN, d->h, PP(PK_WDOWN), d->x, Bi, D, F, F, D, D, PP(PK_BDOWN), d->x2);
#undef PP
    }
    trlm_rmsnorm_rows(g, d->x, trlm_param_ptr(g, trlm_pidx(d->L, 0)), d->nf, d->r, B);
    trlm_gemm_rows(g, GEMM_NT, d->nf, trlm_param_ptr(g, 0), d->logits, Bi, (i32)d->V, D, D, D, (i32)d->ldv, NULL,
                   NULL);
    void* args[] = { &posd };
    hip_launch(d->k_advance, 1, 1, 1, 64, 1, 1, 0, args);
}

static void check_hip(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        fprintf(stderr, "[HIP ERROR] gpu_decode: %s -> %s: %s\n", what, hipGetErrorName(e), hipGetErrorString(e));
        fflush(stderr);
        _exit(1);
    }
}

/* Runs one step: eagerly the first time (the GEMM engine sizes its
 * workspace), then as a replay of the step captured on the second call. */
static void run_step(TrlmDecoder* d) {
    if (d->exec) {
        check_hip(hipGraphLaunch(d->exec, hip_current_stream()), "hipGraphLaunch");
    } else if (d->eager_steps == 0) {
        step_body(d);
        d->eager_steps++;
    } else {
        hipStream_t st = hip_current_stream();
        check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        step_body(d);
        check_hip(hipStreamEndCapture(st, &d->graph), "hipStreamEndCapture");
        check_hip(hipGraphInstantiate(&d->exec, d->graph, NULL, NULL, 0), "hipGraphInstantiate");
        check_hip(hipGraphLaunch(d->exec, st), "hipGraphLaunch");
    }
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

void gpu_decoder_sample(TrlmDecoder* d, PCGState* rngs, f32 temperature, u32* out_ids) {
    trlm_bind(d->g);
    f64* u = (f64*)malloc((u64)d->B * sizeof(f64));
    if (!u) dec_fatal("out of host memory");
    for (u32 b = 0; b < d->B; b++) u[b] = (f64)pcg_next_u32(&rngs[b]) * (1.0 / 4294967296.0);   /* pcg_uniform */
    hip_h2d(d->u, u, (u64)d->B * sizeof(f64));
    hipDeviceptr_t lg = d->logits, e = d->e, pr = d->prefix, up = d->u, out = d->out_ids;
    i32 ld = (i32)d->ldv, V = (i32)d->V;
    void* args[] = { &lg, &ld, &V, &temperature, &up, &e, &pr, &out };
    hip_launch(d->k_sample, d->B, 1, 1, 256, 1, 1, 0, args);
    hip_d2h(out_ids, d->out_ids, (u64)d->B * sizeof(u32));
    free(u);
}

void gpu_decoder_generate_greedy(TrlmDecoder* d, const u32* prompt, u32 prompt_len, u32 steps, u32* out) {
    if (steps == 0) return;
    if ((u64)prompt_len + steps > d->ctx) dec_fatal("prompt_len + steps exceeds max_ctx");
    gpu_decoder_prefill(d, prompt, prompt_len);
    if (d->hist_cap < d->B * steps) {
        if (d->hist) hip_free(d->hist);
        d->hist = hip_alloc((u64)d->B * steps * sizeof(u32));
        d->hist_cap = d->B * steps;
    }
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
