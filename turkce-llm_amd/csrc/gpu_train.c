/* gpu_train.c -- GPU-resident forward, backward and Adam on MI355X.
 *
 * Same API and semantics as the reference's model/gpu_train.c (cited per
 * function), re-planned for gfx950:
 *   - every projection and the tied LM head run on the fp32 MFMA GEMM
 *     (trlm_gemm.c) with bias and residual fused into the epilogue;
 *   - attention is flash style (attention.hip): no [B,H,T,T] tensor, Q/K/V
 *     read in place from the qkv projection, O written in place into the
 *     [N,D] attention output, so the head split/merge passes disappear;
 *   - bias / norm-weight gradients are two-stage fixed-order column sums and
 *     the embedding backward is a per-token segmented sum in ascending row
 *     order, so no reduction uses atomics;
 *   - one HIP stream per trainer; the blocking points are the reference's
 *     (loss readback, grad-norm readback, end of the Adam step).
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "trlm_ext.h"
#include "gpu_internal.h"

static u32 pidx(u32 layer, u32 k) { return trlm_pidx(layer, k); }

#define F4 ((u64)sizeof(f32))

static hipDeviceptr_t dptr(hipDeviceptr_t base, u64 floats) { return (hipDeviceptr_t)((char*)base + floats * F4); }
static hipDeviceptr_t P_(const GpuTrainer* g, u32 i) { return dptr(g->params, g->offsets[i]); }
static hipDeviceptr_t G_(const GpuTrainer* g, u32 i) { return dptr(g->grads, g->offsets[i]); }

static void fatal(const char* msg) {
    fprintf(stderr, "[HIP ERROR] gpu_train: %s\n", msg);
    fflush(stderr);
    _exit(1);
}

/* ---------------- launch helpers ---------------- */

static u32 cdiv_u64(u64 a, u64 b) { return (u32)((a + b - 1) / b); }

/* C[M,N] = op(A) op(B) (+ beta C) (+ bias) (+ resid), single matrices with
 * the reference's leading-dimension conventions (gpu_train.c:53-63). */

static void gemm1(GpuTrainer* g, GemmKind kind, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C, i32 M, i32 N,
                  i32 K, i32 lda, i32 ldb, i32 ldc, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid) {
    trlm_gemm(g->gemm, kind == GEMM_TN, kind == GEMM_NT, A, B, C, M, N, K, lda, ldb, ldc, 1, 0, 0, 0, 1.0f, beta,
              bias, resid, ldc);
}

/* Weight and bias gradient of a linear layer in one GEMM:
 * dW [M, N] = X^T @ dY (TN, X [K=rows, M], dY [rows, N]) and db [N] =
 * column sums of dY, which the GEMM adds up from the dY tiles it loads
 * (model/gpu_train.c:415-432 runs k_colsum_acc separately).  Issued inside
 * a side-stream section, on the side GEMM context. */
static void gemm_wb(GpuTrainer* g, hipDeviceptr_t X, hipDeviceptr_t dY, hipDeviceptr_t dW, hipDeviceptr_t db, i32 M,
                    i32 N, i32 K) {
    TrlmGemmExtra x;
    memset(&x, 0, sizeof(x));
    x.csum = db;
    trlm_gemm_ex(g->gemm_side, 1, 0, X, dY, dW, M, N, K, M, N, N, 1, 0, 0, 0, 1.0f, 0.0f, NULL, NULL, N, &x);
}

/* threads of k_swiglu_fwd / k_swiglu_bwd: one float4 each when F % 4 == 0 */
static u32 swiglu_blocks(const GpuTrainer* g, u64 rows) {
    u64 work = rows * g->F;
    if (g->F % 4 == 0) work /= 4;
    return cdiv_u64(work, 256);
}

/* float4 chunks per lane of the 16-lanes-per-row RMSNorm kernels for
 * rows of D floats (k_rmsnorm_{fwd,bwd}_q<n>), 0 when D needs the generic
 * one-wave-per-row kernels (D % 4 != 0 or D > 1024). */
static u32 rms_nq(u32 D) {
    static const u32 NQ[] = { 1, 2, 4, 6, 8, 16 };
    if (D % 4 || D > 1024) return 0;
    for (u32 i = 0; i < sizeof(NQ) / sizeof(NQ[0]); i++)
        if (64 * NQ[i] >= D) return NQ[i];
    return 0;
}

static void rmsnorm_rows(GpuTrainer* g, hipDeviceptr_t x, hipDeviceptr_t w, hipDeviceptr_t out, hipDeviceptr_t rinv,
                         u32 nrows) {
    i32 rows = (i32)nrows, cols = (i32)g->D;
    f32 eps = g->eps;
    void* args[] = { &x, &w, &out, &rinv, &rows, &cols, &eps };
    hip_launch(g->k.rmsnorm_fwd, cdiv_u64(nrows, rms_nq(g->D) ? 16 : 4), 1, 1, 256, 1, 1, 0, args);
}

static void rmsnorm_fwd(GpuTrainer* g, hipDeviceptr_t x, hipDeviceptr_t w, hipDeviceptr_t out, hipDeviceptr_t rinv) {
    rmsnorm_rows(g, x, w, out, rinv, g->N);
}

#define RMS_ROWS 16u

/* RMSNorm backward (gpu_train.c:132-140) on the current stream: dx = dxin
 * (zero when dxin is 0) + the norm's input gradient, and the weight
 * gradient dw = sum over rows of dy*x*r as per-block partials into part
 * (rows in order; colsum_partials adds them up, on the side stream in the
 * backward). */
static void rmsnorm_bwd(GpuTrainer* g, hipDeviceptr_t x, hipDeviceptr_t w, hipDeviceptr_t rinv, hipDeviceptr_t dy,
                        hipDeviceptr_t dxin, hipDeviceptr_t dx, hipDeviceptr_t part) {
    i32 rows = (i32)g->N, cols = (i32)g->D;
    u32 nb = cdiv_u64(g->N, RMS_ROWS);
    void* args[] = { &x, &w, &rinv, &dy, &dxin, &dx, &part, &rows, &cols };
    hip_launch(g->k.rmsnorm_bwd, nb, 1, 1, 256, 1, 1, 4u * (u32)cols * (u32)F4, args);
}

#define COLSUM_GROUP 16u

/* Rows of a partial buffer: the RMSNorm backward's per-block partials, then
 * room for colsum_partials' group sums. */
static u64 part_buffer_rows(u64 N) {
    u64 nb = cdiv_u64(N, RMS_ROWS);
    return nb + cdiv_u64(nb, COLSUM_GROUP);
}

/* dw = sum of an RMSNorm backward's partial rows: sums of 16-row groups in
 * block order (one block per 64 columns x group, so the reduction spreads
 * over the GPU), then the group sums in group order.  The group sums go to
 * the partial buffer's own spare rows, so calls on different buffers may
 * run concurrently. */
static void colsum_partials(GpuTrainer* g, hipDeviceptr_t part, hipDeviceptr_t dw) {
    u32 nb = cdiv_u64(g->N, RMS_ROWS), ng = cdiv_u64(nb, COLSUM_GROUP);
    i32 inb = (i32)nb, cols = (i32)g->D, acc = 0, grp = (i32)COLSUM_GROUP;
    hipDeviceptr_t stage = (hipDeviceptr_t)((char*)part + (u64)nb * g->D * F4);
    void* a1[] = { &part, &inb, &cols, &stage, &acc, &grp };
    hip_launch(g->k.colsum_final, cdiv_u64((u64)cols, 64), ng, 1, 256, 1, 1, 0, a1);
    i32 ing = (i32)ng;
    void* a2[] = { &stage, &ing, &cols, &dw, &acc, &ing };
    hip_launch(g->k.colsum_final, cdiv_u64((u64)cols, 64), 1, 1, 256, 1, 1, 0, a2);
}

#include "kernel_params.h"   /* AttnParams: the argument block the kernels read */

static AttnParams attn_params(GpuTrainer* g) {
    AttnParams a;
    memset(&a, 0, sizeof(a));
    a.B = (int)g->B; a.T = (int)g->T; a.H = (int)g->H; a.D = (int)g->D;
    a.ldq = 3 * (int)g->D; a.ldo = (int)g->D;
    a.scale = 1.0f / m_sqrtf((f32)g->hd);   /* attention.c:78 */
    return a;
}

/* The causal attention forward's job of each workgroup.  Query block q of a
 * head is a job of q + 1 key-block stages, so a head's jobs have the sizes
 * 1 .. n (n query blocks).  When the grid is exactly three resident
 * workgroups per compute unit, workgroups L, L + cus and L + 2 cus share one
 * unit (the dispatcher fills every unit once per round of `cus`
 * workgroups), and the unit's time follows the sum of its three sizes.
 * Three heads' jobs (three copies of 1 .. n) split into n triples whose sums
 * are all floor or ceil of 3(n + 1)/2: row a is i = 1 .. n, row b is a
 * shifted cyclically by n/2, and row c gives rank 1 .. n to the columns in
 * descending order of a + b (ties: lower i first) -- each row a
 * permutation of 1 .. n, so every (head, query block) is taken once.  Three
 * heads per n units; B8 T1024 (48 heads, 16 blocks, 256 units): every unit
 * gets 25 or 26 stages, against 23 to 28 in the kernel's snake order.  Each
 * triple of heads stays on one XCD, as the snake order keeps each head. */
#define GFX950_XCDS 8u   /* MI355X: 8 XCDs of 32 compute units, each with its own L2 */

i32 trlm_attn_job_table(u32 heads, u32 n, u32 cus, u32 xcds, i32* jobs) {
    if (n == 0 || cus == 0 || xcds == 0 || heads % 3 != 0 || (u64)heads * n != 3ull * cus || n > 32767 ||
        heads > 65535 || (heads / 3) % xcds != 0)
        return 0;
    u32* row = (u32*)malloc(3ull * n * sizeof(u32));
    if (!row) fatal("out of host memory");
    u32 *ra = row, *rb = row + n, *rc = row + 2 * n;
    for (u32 i = 0; i < n; i++) {
        ra[i] = i + 1;
        rb[i] = (i + n / 2) % n + 1;
    }
    for (u32 i = 0; i < n; i++) {
        u32 rank = 0;
        for (u32 j = 0; j < n; j++) {
            const u32 pi = ra[i] + rb[i], pj = ra[j] + rb[j];
            rank += (pj > pi || (pj == pi && j < i)) ? 1u : 0u;
        }
        rc[i] = rank + 1;
    }
    /* replica r (heads 3r .. 3r + 2) takes units x, x + xcds, x + 2 xcds, ...
     * of one XCD x = r mod xcds: workgroups go to the XCDs in turn (L mod
     * xcds), so each head's K and V are read into one XCD's L2 only */
    for (u32 r = 0; r < heads / 3; r++)
        for (u32 t = 0; t < n; t++)
            for (u32 k = 0; k < 3; k++) {
                const u32 size = row[k * n + t], head = 3 * r + k;
                const u32 unit = r % xcds + xcds * ((r / xcds) * n + t);
                jobs[k * cus + unit] = (i32)(((size - 1) << 16) | head);
            }
    free(row);
    return 1;
}

/* ---------------- create / destroy ---------------- */

/* Every device buffer of a trainer lives in one allocation, carved into
 * 256-byte aligned slices: the buffer plan below lists (slot, floats) pairs,
 * carve() sizes and places them all, then assigns the slots. */
#define CARVE_ALIGN 256u
#define GPU_TRAIN_PLAN_MAX (4u + 11u * LM_MAX_LAYERS + 64u)   /* flat buffers, layer activations, the rest */
typedef struct CarvePlan {
    hipDeviceptr_t* slot[GPU_TRAIN_PLAN_MAX];
    u64 bytes[GPU_TRAIN_PLAN_MAX];
    u32 n;
} CarvePlan;

static void want(CarvePlan* cp, hipDeviceptr_t* slot, u64 bytes) {
    if (cp->n == GPU_TRAIN_PLAN_MAX) fatal("too many trainer buffers");
    cp->slot[cp->n] = slot;
    cp->bytes[cp->n] = bytes;
    cp->n++;
}

static void want_f(CarvePlan* cp, hipDeviceptr_t* slot, u64 floats) { want(cp, slot, floats * F4); }

static void carve(CarvePlan* cp) {
    u64 total = 0;
    for (u32 i = 0; i < cp->n; i++) total += (cp->bytes[i] + CARVE_ALIGN - 1) / CARVE_ALIGN * CARVE_ALIGN;
    char* base = (char*)hip_alloc(total);
    for (u32 i = 0; i < cp->n; i++) {
        *cp->slot[i] = (hipDeviceptr_t)base;
        base += (cp->bytes[i] + CARVE_ALIGN - 1) / CARVE_ALIGN * CARVE_ALIGN;
    }
}

/* The buffers of a B x T trainer (sizes in floats unless noted). */
static void plan_buffers(GpuTrainer* g, CarvePlan* cp) {
    const u64 N = g->N, D = g->D, F = g->F, BHT = (u64)g->B * g->H * g->T;
    const u64 nqb = ((u64)g->T + 63) / 64, part_rows = part_buffer_rows(N);
    /* the flat parameter-sized buffers, lm_collect_params order */
    hipDeviceptr_t* flat[4] = { &g->params, &g->grads, &g->adam_m, &g->adam_v };
    for (u32 i = 0; i < 4; i++) want_f(cp, flat[i], g->total_scalars);
    /* what each layer keeps from its forward for the backward */
    for (u32 l = 0; l < g->L; l++) {
        GpuLayerActs* a = &g->layers[l];
        const struct { hipDeviceptr_t* p; u64 n; } acts[] = {
            { &a->x_in, N * D }, { &a->n1, N * D }, { &a->r1, N },     { &a->qkv, N * 3 * D },
            { &a->att, N * D },  { &a->lse, BHT },  { &a->x2, N * D }, { &a->n2, N * D },
            { &a->r2, N },       { &a->gu, N * 2 * F }, { &a->h, N * F },
        };
        for (u32 i = 0; i < sizeof(acts) / sizeof(acts[0]); i++) want_f(cp, acts[i].p, acts[i].n);
    }
    /* head and loss */
    want_f(cp, &g->x_final, N * D);
    want_f(cp, &g->nf, N * D);
    want_f(cp, &g->rf, N);
    want_f(cp, &g->logits, N * (u64)g->ldv);
    want_f(cp, &g->ce_stats, N * (u64)g->ce_stats_cap * 2);
    want_f(cp, &g->ce_zt, N);
    want_f(cp, &g->loss_rows, N);
    want_f(cp, &g->norm_partial, GPU_TRAIN_NORM_BLOCKS);
    /* backward scratch: the residual-gradient ring, the by-parity pairs the
     * side stream reads, the causal dS blocks of one layer, norm partials */
    for (u32 i = 0; i < GPU_TRAIN_DRES_RING; i++) want_f(cp, &g->dres[i], N * D);
    for (u32 i = 0; i < 2; i++) {
        want_f(cp, &g->dqkv[i], N * 3 * D);
        want_f(cp, &g->dgu[i], N * 2 * F);
        want_f(cp, &g->part[i][0], part_rows * D);
        want_f(cp, &g->part[i][1], part_rows * D);
    }
    want_f(cp, &g->part_final, part_rows * D);
    want_f(cp, &g->dn, N * D);
    want_f(cp, &g->datt, N * D);
    want_f(cp, &g->dh, N * F);
    want_f(cp, &g->dvec, BHT);
    want_f(cp, &g->att_ds, (u64)g->B * g->H * (nqb * (nqb + 1) / 2) * 4096);
    want(cp, &g->attn_jobs, (u64)g->B * g->H * nqb * sizeof(i32));
    /* token ids and the embedding backward's row groups (u32) */
    want(cp, &g->ids, N * sizeof(u32));
    want(cp, &g->targets, N * sizeof(u32));
    want(cp, &g->emb_order, N * sizeof(u32));
    want(cp, &g->emb_seg, (2 * N + 1) * sizeof(u32));
    /* RoPE tables [T][hd/2] */
    want_f(cp, &g->cos_t, (u64)g->T * (g->hd / 2));
    want_f(cp, &g->sin_t, (u64)g->T * (g->hd / 2));
}

GpuTrainer gpu_trainer_create(Allocator* alloc, const char* ptx_path, const LMModel* model,
                              Node** params, u32 num_params, u32 batch_size, u32 seq_len) {
    GpuTrainer g;
    memset(&g, 0, sizeof(g));
    /* model and batch geometry; F is the feed-forward width, read off the
     * first block's down projection [F, D] */
    const u32 d_model = model->d_model, heads = model->num_heads;
    g.V = model->vocab_size;
    g.L = model->num_layers;
    g.D = d_model;
    g.H = heads;
    g.hd = heads ? d_model / heads : 0;
    g.F = (u32)model->blocks[0].ffn.w_down->value.shape[0];
    g.eps = model->eps;
    g.B = batch_size;
    g.T = seq_len;
    g.N = batch_size * seq_len;
    g.ldv = (g.V + 3u) & ~3u;
    g.ce_stats_cap = 2 * (i32)((g.V + 63) / 64);     /* two entries per 64-wide (smallest) tile column */
    if (g.L > LM_MAX_LAYERS || num_params != 10u * g.L + 2u) fatal("parameter list does not match the model");
    if (g.D % g.H != 0 || g.D % 4 != 0) fatal("d_model must be a multiple of 4 and of num_heads");
    if (g.hd != 16 && g.hd != 32 && g.hd != 64) fatal("head_dim must be 16, 32 or 64");

    g.hip = hip_init(alloc, ptx_path);
    hip_set_current(&g.hip);
    g.gemm = NULL;   /* created below, after g.hip has its final address in the caller */

    /* flat layout: tensor i at offsets[i] of every parameter-sized buffer */
    g.num_params = num_params;
    g.total_scalars = 0;
    for (u32 i = 0; i < num_params; i++) {
        g.numels[i] = params[i]->value.numel;
        g.offsets[i] = g.total_scalars;
        g.total_scalars += g.numels[i];
    }
    CarvePlan* cp = (CarvePlan*)calloc(1, sizeof(CarvePlan));
    if (!cp) fatal("out of host memory");
    plan_buffers(&g, cp);
    carve(cp);
    free(cp);
    hip_memset_zero(g.grads, g.total_scalars * F4);
    hip_memset_zero(g.adam_m, g.total_scalars * F4);
    hip_memset_zero(g.adam_v, g.total_scalars * F4);
    hip_memset_zero(g.logits, (u64)g.N * g.ldv * F4);

    const u64 N = g.N;
    g.host_loss_rows = (f32*)allocator_alloc(alloc, N * F4);
    g.host_emb = (u32*)allocator_alloc(alloc, (3 * N + 1 + (u64)g.V + 1) * sizeof(u32));
    g.host_norm_partial = (f32*)allocator_alloc(alloc, GPU_TRAIN_NORM_BLOCKS * F4);

    /* RoPE tables, built on the host exactly as the CPU path builds them
     * (gpu_train.c:239-247, model/rope.c) */
    u64 cshape[2] = { g.T, g.hd / 2 };   /* the slots planned above */
    Tensor cos_t = tensor_create(alloc, cshape, 2);
    Tensor sin_t = tensor_create(alloc, cshape, 2);
    rope_build_tables(&cos_t, &sin_t, g.T, g.hd, 10000.0f);
    hip_h2d(g.cos_t, cos_t.data, cos_t.numel * F4);
    hip_h2d(g.sin_t, sin_t.data, sin_t.numel * F4);

    HipCtx* c = &g.hip;
    g.k.embed_fwd = hip_get_kernel(c, "k_embed_fwd");
    g.k.embed_bwd = hip_get_kernel(c, "k_embed_bwd");
    {
        const u32 nq = rms_nq(g.D);
        char fname[40], bname[40];
        if (nq) {
            snprintf(fname, sizeof(fname), "k_rmsnorm_fwd_q%u", nq);
            snprintf(bname, sizeof(bname), "k_rmsnorm_bwd_q%u", nq);
        } else {
            snprintf(fname, sizeof(fname), "k_rmsnorm_fwd");
            snprintf(bname, sizeof(bname), "k_rmsnorm_bwd");
        }
        g.k.rmsnorm_fwd = hip_get_kernel(c, fname);
        g.k.rmsnorm_bwd = hip_get_kernel(c, bname);
    }
    g.k.colsum_final = hip_get_kernel(c, "k_colsum_final");
    g.k.swiglu_fwd = hip_get_kernel(c, "k_swiglu_fwd");
    g.k.swiglu_bwd = hip_get_kernel(c, "k_swiglu_bwd");
    g.k.cross_entropy = hip_get_kernel(c, "k_cross_entropy");
    g.k.argmax_rows = hip_get_kernel(c, "k_argmax_rows");
    g.k.sumsq_partial = hip_get_kernel(c, "k_sumsq_partial");
    g.k.adam = hip_get_kernel(c, "k_adam");
    g.k.loss_mean = hip_get_kernel(c, "k_loss_mean");
    g.k.norm_clip = hip_get_kernel(c, "k_norm_clip");
    g.k.adam_ds = hip_get_kernel(c, "k_adam_ds");
    char name[64];
    snprintf(name, sizeof(name), "k_attn_fwd_hd%u", g.hd);
    g.k.attn_fwd = hip_get_kernel(c, name);
    snprintf(name, sizeof(name), "k_attn_bwd_dkv_hd%u", g.hd);
    g.k.attn_bwd_dkv = hip_get_kernel(c, name);
    snprintf(name, sizeof(name), "k_attn_bwd_dq_hd%u", g.hd);
    g.k.attn_bwd_dq = hip_get_kernel(c, name);
    snprintf(name, sizeof(name), "k_attn_dvec_hd%u", g.hd);
    g.k.attn_dvec = hip_get_kernel(c, name);
    /* the attention forward's placement table, where the grid is exactly
     * three resident workgroups per compute unit (TRLM_ATTN_SNAKE=1 keeps
     * the kernel's own order; the results are the same bits either way) */
    g.attn_fwd_jobs = 0;
    {
        const char* snake = getenv("TRLM_ATTN_SNAKE");
        const u32 heads = g.B * g.H, nqb = (g.T + 63) / 64;
        if (!(snake && snake[0] == '1') && hip_blocks_per_cu(g.k.attn_fwd, 256) == 3) {
            i32* t = (i32*)malloc((u64)heads * nqb * sizeof(i32));
            if (!t) fatal("out of host memory");
            if (trlm_attn_job_table(heads, nqb, hip_cu_count(), GFX950_XCDS, t)) {
                hip_h2d(g.attn_jobs, t, (u64)heads * nqb * sizeof(i32));
                g.attn_fwd_jobs = g.attn_jobs;
            }
            free(t);
        }
    }

    gpu_trainer_upload(&g, params, NULL_PTR);
    hip_sync();
    return g;
}

/* The GEMM engine keeps a pointer to the trainer's HipCtx, and the trainer
 * is returned by value, so the engine is bound lazily on first use. */
static void bind(GpuTrainer* g) {
    hip_set_current(&g->hip);
    if (!g->gemm) g->gemm = trlm_gemm_create(&g->hip);
    if (!g->gemm_side) g->gemm_side = trlm_gemm_create(&g->hip);
}

void gpu_trainer_destroy(GpuTrainer* g) {
    hip_set_current(&g->hip);
    hip_sync();
    if (g->gemm) { trlm_gemm_destroy(g->gemm); g->gemm = NULL; }
    if (g->gemm_side) { trlm_gemm_destroy(g->gemm_side); g->gemm_side = NULL; }
    hip_shutdown(&g->hip);   /* frees every buffer allocated for this trainer */
}

/* ---------------- CPU mirror <-> GPU (gpu_train.c:258-294) ---------------- */

/* Copies between one flat device buffer and the caller's per-tensor host
 * arrays (host[i]: tensor i, numels[i] floats at offsets[i] of the buffer),
 * synchronously.  Tensors that lie back to back in host memory -- the
 * runtime's arena places a model's parameters that way -- travel as one
 * transfer. */
static void mirror(GpuTrainer* g, hipDeviceptr_t flat, f32* const* host, int to_device) {
    u32 i = 0;
    while (i < g->num_params) {
        u64 run = g->numels[i];
        u32 j = i + 1;
        while (j < g->num_params && host[j] == host[i] + run) run += g->numels[j++];
        hipDeviceptr_t dev = dptr(flat, g->offsets[i]);
        if (to_device) hip_h2d(dev, host[i], run * F4);
        else hip_d2h(host[i], dev, run * F4);
        i = j;
    }
}

enum { HOST_VALUE, HOST_GRAD, HOST_ADAM_M, HOST_ADAM_V };

/* The host arrays of one kind for every tensor. */
static void host_arrays(const GpuTrainer* g, Node** params, const AdamOptimizer* opt, int kind, f32** out) {
    for (u32 i = 0; i < g->num_params; i++) {
        switch (kind) {
            case HOST_VALUE: out[i] = params[i]->value.data; break;
            case HOST_GRAD: out[i] = params[i]->grad.data; break;
            case HOST_ADAM_M: out[i] = opt->m[i].data; break;
            default: out[i] = opt->v[i].data; break;
        }
    }
}

static void mirror_kind(GpuTrainer* g, Node** params, const AdamOptimizer* opt, int kind, int to_device) {
    f32* host[GPU_TRAIN_MAX_PARAMS];
    const hipDeviceptr_t flat[4] = { g->params, g->grads, g->adam_m, g->adam_v };
    hip_set_current(&g->hip);
    host_arrays(g, params, opt, kind, host);
    mirror(g, flat[kind], host, to_device);
}

void gpu_trainer_upload(GpuTrainer* g, Node** params, const AdamOptimizer* opt) {
    mirror_kind(g, params, opt, HOST_VALUE, 1);
    if (opt != NULL_PTR) {
        mirror_kind(g, params, opt, HOST_ADAM_M, 1);
        mirror_kind(g, params, opt, HOST_ADAM_V, 1);
    }
}

void gpu_trainer_download(GpuTrainer* g, Node** params, AdamOptimizer* opt) {
    mirror_kind(g, params, opt, HOST_VALUE, 0);
    if (opt != NULL_PTR) {
        mirror_kind(g, params, opt, HOST_ADAM_M, 0);
        mirror_kind(g, params, opt, HOST_ADAM_V, 0);
    }
}

void gpu_trainer_download_grads(GpuTrainer* g, Node** params) { mirror_kind(g, params, NULL_PTR, HOST_GRAD, 0); }

void gpu_trainer_upload_grads(GpuTrainer* g, Node** params) { mirror_kind(g, params, NULL_PTR, HOST_GRAD, 1); }

void gpu_trainer_sample_batch(const u32* tokens, u64 num_tokens, u32 seq_len, u32 batch_size,
                              u64 seed_base, u32* ids_out, u32* targets_out) {
    i64 max_start = (i64)(num_tokens - seq_len - 1);
    for (u32 w = 0; w < batch_size; w++) {
        PCGState rng = pcg_seed(seed_base * 1000003ull + w, 99ull + w);
        i64 start = pcg_range_i64(&rng, 0, max_start);
        for (u32 t = 0; t < seq_len; t++) {
            ids_out[(u64)w * seq_len + t] = tokens[start + t];
            targets_out[(u64)w * seq_len + t] = tokens[start + t + 1];
        }
    }
}

/* ---------------- forward / backward ---------------- */

/* Stable counting sort of the rows by token id: rows of one token form a
 * segment, listed in ascending row order (the order in which the reference
 * adds them, embedding.c:10-14). */
/* Rows of the batch grouped by token for the embedding backward: order[N]
 * (row indices, stable within a token) and seg = seg_start[nseg+1] then
 * seg_tok[nseg]; returns nseg. */
u32 trlm_embed_groups(GpuTrainer* g, const u32* ids, u32* order, u32* seg) {
    u32 N = g->N, V = g->V;
    u32* count = g->host_emb + 3 * N + 1;    /* [V+1] */
    memset(count, 0, ((u64)V + 1) * sizeof(u32));
    for (u32 n = 0; n < N; n++) {
        if (ids[n] >= V) fatal("token id outside the vocabulary");
        count[ids[n] + 1]++;
    }
    u32 nseg = 0;
    for (u32 v = 0; v < V; v++) if (count[v + 1]) nseg++;
    u32* seg_start = seg;
    u32* seg_tok = seg + nseg + 1;
    u32 s = 0;
    for (u32 v = 0; v < V; v++) {
        u32 c = count[v + 1];
        count[v + 1] = count[v] + c;   /* count[v] = first slot of token v */
        if (c) { seg_start[s] = count[v]; seg_tok[s] = v; s++; }
    }
    seg_start[nseg] = N;
    for (u32 n = 0; n < N; n++) order[count[ids[n]]++] = n;
    return nseg;
}

static void embed_segments(GpuTrainer* g, const u32* ids) {
    u32* order = g->host_emb;
    u32* seg = order + g->N;
    u32 nseg = trlm_embed_groups(g, ids, order, seg);
    g->emb_nseg = nseg;
    hip_h2d(g->emb_order, order, (u64)g->N * sizeof(u32));
    hip_h2d(g->emb_seg, seg, (2ull * nseg + 1) * sizeof(u32));
}

/* Embedding, L blocks, final norm, tied head (model/gpu_train.c:312-378). */
void trlm_check_ids(const GpuTrainer* g, const u32* ids, const char* what) {
    for (u32 n = 0; n < g->N; n++)
        if (ids[n] >= g->V) {
            fprintf(stderr, "[HIP ERROR] gpu_train: %s[%u] = %u is outside the vocabulary (%u)\n", what, n, ids[n],
                    g->V);
            fflush(stderr);
            _exit(1);
        }
}

/* Embedding, the L blocks and the final norm (-> g->nf).  hook (if any) runs
 * after each layer's QKV projection and RoPE, with that layer's qkv.  ids
 * NULL: the batch's ids are already in g->ids. */
void trlm_forward_hidden(GpuTrainer* g, const u32* ids, TrlmLayerHook hook, void* hook_ctx) {
    i32 N = (i32)g->N, D = (i32)g->D, F = (i32)g->F;
    if (ids) {
        trlm_check_ids(g, ids, "ids");
        hip_h2d(g->ids, ids, (u64)N * sizeof(u32));
    }
    {
        hipDeviceptr_t E = P_(g, 0), idp = g->ids, x0 = g->layers[0].x_in;
        void* args[] = { &E, &idp, &x0, &N, &D };
        u64 work = (D % 4 == 0) ? (u64)N * D / 4 : (u64)N * D;
        hip_launch(g->k.embed_fwd, cdiv_u64(work, 256), 1, 1, 256, 1, 1, 0, args);
    }
    AttnParams ap = attn_params(g);
    for (u32 l = 0; l < g->L; l++) {
        GpuLayerActs* a = &g->layers[l];
        hipDeviceptr_t x_out = (l + 1 < g->L) ? g->layers[l + 1].x_in : g->x_final;
        rmsnorm_fwd(g, a->x_in, P_(g, pidx(l, PK_ATTN_NORM)), a->n1, a->r1);
        /* qkv = n1 @ Wqkv + b, with RoPE applied to the Q and K columns in
         * the GEMM's epilogue */
        {
            TrlmGemmExtra x;
            memset(&x, 0, sizeof(x));
            x.rope_cos = (const f32*)g->cos_t;
            x.rope_sin = (const f32*)g->sin_t;
            x.rope_T = (i32)g->T;
            x.rope_hd = (i32)g->hd;
            x.rope_cols = 2 * D;
            trlm_gemm_ex(g->gemm, 0, 0, a->n1, P_(g, pidx(l, PK_WQKV)), a->qkv, N, 3 * D, D, D, 3 * D, 3 * D, 1, 0,
                         0, 0, 1.0f, 0.0f, P_(g, pidx(l, PK_BQKV)), NULL, 3 * D, &x);
        }
        if (hook) hook(hook_ctx, g, l, a->qkv);
        ap.qkv = (const float*)a->qkv; ap.out = (float*)a->att; ap.lse = (float*)a->lse;
        ap.jobs = (const int*)g->attn_fwd_jobs;
        {
            void* args[] = { &ap };
            hip_launch(g->k.attn_fwd, g->B * g->H, cdiv_u64(g->T, 64), 1, 256, 1, 1, 0, args);
        }
        /* x2 = x_in + (att @ Wo + bo) */
        gemm1(g, GEMM_NN, a->att, P_(g, pidx(l, PK_WO)), a->x2, N, D, D, D, D, D, 0.0f, P_(g, pidx(l, PK_BO)),
              a->x_in);
        rmsnorm_fwd(g, a->x2, P_(g, pidx(l, PK_FFN_NORM)), a->n2, a->r2);
        /* gu = n2 @ Wgu + bgu, and h = SwiGLU(gu): in the GEMM's epilogue
         * where the widths allow it, else as a separate pass */
        if (F % 32 == 0 && D % 32 == 0) {
            TrlmGemmExtra x;
            memset(&x, 0, sizeof(x));
            x.glu_h = a->h;
            x.glu_F = F;
            trlm_gemm_ex(g->gemm, 0, 0, a->n2, P_(g, pidx(l, PK_WGU)), a->gu, N, 2 * F, D, D, 2 * F, 2 * F, 1, 0, 0,
                         0, 1.0f, 0.0f, P_(g, pidx(l, PK_BGU)), NULL, 2 * F, &x);
        } else {
            gemm1(g, GEMM_NN, a->n2, P_(g, pidx(l, PK_WGU)), a->gu, N, 2 * F, D, D, 2 * F, 2 * F, 0.0f,
                  P_(g, pidx(l, PK_BGU)), NULL);
            hipDeviceptr_t gu = a->gu, h = a->h;
            void* args[] = { &gu, &h, &N, &F };
            hip_launch(g->k.swiglu_fwd, swiglu_blocks(g, (u64)N), 1, 1, 256, 1, 1, 0, args);
        }
        /* x_out = x2 + (h @ Wd + bd) */
        gemm1(g, GEMM_NN, a->h, P_(g, pidx(l, PK_WDOWN)), x_out, N, D, F, F, D, D, 0.0f, P_(g, pidx(l, PK_BDOWN)),
              a->x2);
    }
    rmsnorm_fwd(g, g->x_final, P_(g, pidx(g->L, 0)), g->nf, g->rf);
}

static void forward_to_logits(GpuTrainer* g, const u32* ids) {
    i32 N = (i32)g->N, D = (i32)g->D, V = (i32)g->V, ldv = (i32)g->ldv;
    trlm_forward_hidden(g, ids, NULL, NULL);
    /* logits = nf @ E^T  (tied head, NT with B = E [V, D]); the epilogue also
     * leaves each row's softmax statistics per column block for the CE */
    TrlmGemmExtra x;
    memset(&x, 0, sizeof(x));
    x.stats = g->ce_stats;
    x.stats_cap = g->ce_stats_cap;
    g->ce_nst = trlm_gemm_ex(g->gemm, 0, 1, g->nf, P_(g, 0), g->logits, N, V, D, D, D, ldv, 1, 0, 0, 0, 1.0f, 0.0f,
                             NULL, NULL, ldv, &x);
}

/* The evaluation forward (forward + mean CE, no gradient): the LM-head
 * GEMM's epilogue leaves only what the cross-entropy reads -- each row's
 * softmax statistics and its target's logit -- and never writes the
 * [N, V] logits, so the loss needs no logits round trip through HBM
 * (model/gpu_train.c:378-384 writes them and reads them back).  The
 * targets must already be on the device. */
static void forward_to_loss_stats(GpuTrainer* g, const u32* ids) {
    i32 N = (i32)g->N, D = (i32)g->D, V = (i32)g->V, ldv = (i32)g->ldv;
    trlm_forward_hidden(g, ids, NULL, NULL);
    TrlmGemmExtra x;
    memset(&x, 0, sizeof(x));
    x.stats = g->ce_stats;
    x.stats_cap = g->ce_stats_cap;
    x.tgt = g->targets;
    x.tgt_val = g->ce_zt;
    x.no_store = 1;
    g->ce_nst = trlm_gemm_ex(g->gemm, 0, 1, g->nf, P_(g, 0), g->logits, N, V, D, D, D, ldv, 1, 0, 0, 0, 1.0f, 0.0f,
                             NULL, NULL, ldv, &x);
}

static void upload_targets(GpuTrainer* g, const u32* targets) {
    trlm_check_ids(g, targets, "targets");
    hip_h2d(g->targets, targets, (u64)g->N * sizeof(u32));
}

/* targets NULL: already in g->targets.  from_stats: the logits were not
 * stored (forward_to_loss_stats); the loss comes from the statistics and
 * the target logits alone, and no gradient is formed. */
static void cross_entropy_ex(GpuTrainer* g, const u32* targets, i32 write_grad, i32 from_stats) {
    if (targets) upload_targets(g, targets);
    hipDeviceptr_t lg = g->logits, tg = g->targets, lr = g->loss_rows, st = g->ce_stats;
    hipDeviceptr_t zt = from_stats ? g->ce_zt : NULL;
    i32 ld = (i32)g->ldv, V = (i32)g->V, nst = g->ce_nst;
    f32 grad_scale = 1.0f / (f32)g->N;
    if (from_stats) write_grad = 0;
    void* args[] = { &lg, &ld, &tg, &lr, &V, &grad_scale, &write_grad, &st, &nst, &zt };
    hip_launch(g->k.cross_entropy, g->N, 1, 1, 256, 1, 1, 0, args);
}

static void cross_entropy(GpuTrainer* g, const u32* targets, i32 write_grad) {
    cross_entropy_ex(g, targets, write_grad, 0);
}

/* Gradients of every parameter from dlogits left in g->logits
 * (model/gpu_train.c:390-474).  Weight-gradient GEMMs write (beta = 0):
 * each weight receives exactly one contribution per step. */
static void backward_pass(GpuTrainer* g) {
    i32 N = (i32)g->N, D = (i32)g->D, F = (i32)g->F, V = (i32)g->V, ldv = (i32)g->ldv;
    u32 p_final = pidx(g->L, 0);
    const u32 R = GPU_TRAIN_DRES_RING;

    /* tied head, dnf = dlogits @ E (dE = dlogits^T @ nf comes last, below) */
    gemm1(g, GEMM_NN, g->logits, P_(g, 0), g->dn, N, D, V, ldv, D, D, 0.0f, NULL, NULL);
    rmsnorm_bwd(g, g->x_final, P_(g, p_final), g->rf, g->dn, 0, g->dres[0], g->part_final);

    AttnParams ap = attn_params(g);
    ap.rope_cos = (const float*)g->cos_t;   /* dQ, dK rotated back as they are stored */
    ap.rope_sin = (const float*)g->sin_t;
    /* The weight gradients (GEMMs with their bias sums, norm-weight sums)
     * run on the side stream, each section issued as soon as the main
     * stream's dX chain has produced what it reads, so it overlaps the
     * chain's next kernels.  What the sections of layer step j read -- its
     * two residual-gradient versions, dgu, dqkv and the norm partials of its
     * parity -- is next written in step j + 2, which first waits for side
     * mark 0: the end of step j + 1's first section, issued after all of
     * step j's. */
    u32 v = 0;   /* dres[v % R]: gradient at the current layer's output */
    hipDeviceptr_t part_prev = g->part_final, w_prev = G_(g, p_final);   /* norm partials still to sum */
    for (i32 l = (i32)g->L - 1; l >= 0; l--) {
        GpuLayerActs* a = &g->layers[l];
        const u32 ul = (u32)l, step = g->L - 1u - ul, par = step & 1u;
        hipDeviceptr_t d_out = g->dres[v % R], d_mid = g->dres[(v + 1) % R], d_in = g->dres[(v + 2) % R];
        hipDeviceptr_t dgu = g->dgu[par], dqkv = g->dqkv[par];
        if (step >= 2) hip_main_wait(0);
        /* FFN: x3 = x2 + (h @ Wd + bd); d_out = dx3 */
        hip_side_begin();
        colsum_partials(g, part_prev, w_prev);
        gemm_wb(g, a->h, d_out, G_(g, pidx(ul, PK_WDOWN)), G_(g, pidx(ul, PK_BDOWN)), F, D, N);
        hip_side_end(0);
        gemm1(g, GEMM_NT, d_out, P_(g, pidx(ul, PK_WDOWN)), g->dh, N, F, D, D, D, F, 0.0f, NULL, NULL);
        {
            hipDeviceptr_t gu = a->gu, dh = g->dh;
            void* args[] = { &gu, &dh, &dgu, &N, &F };
            hip_launch(g->k.swiglu_bwd, swiglu_blocks(g, (u64)N), 1, 1, 256, 1, 1, 0, args);
        }
        hip_side_begin();
        gemm_wb(g, a->n2, dgu, G_(g, pidx(ul, PK_WGU)), G_(g, pidx(ul, PK_BGU)), D, 2 * F, N);
        hip_side_end(1);
        gemm1(g, GEMM_NT, dgu, P_(g, pidx(ul, PK_WGU)), g->dn, N, D, 2 * F, 2 * F, 2 * F, D, 0.0f, NULL, NULL);
        rmsnorm_bwd(g, a->x2, P_(g, pidx(ul, PK_FFN_NORM)), a->r2, g->dn, d_out, d_mid, g->part[par][1]);
        /* attention: x2 = x + (att @ Wo + bo); d_mid = dx2 */
        hip_side_begin();
        colsum_partials(g, g->part[par][1], G_(g, pidx(ul, PK_FFN_NORM)));
        gemm_wb(g, a->att, d_mid, G_(g, pidx(ul, PK_WO)), G_(g, pidx(ul, PK_BO)), D, D, N);
        hip_side_end(2);
        gemm1(g, GEMM_NT, d_mid, P_(g, pidx(ul, PK_WO)), g->datt, N, D, D, D, D, D, 0.0f, NULL, NULL);
        ap.qkv = (const float*)a->qkv; ap.O = (const float*)a->att; ap.dO = (const float*)g->datt;
        ap.lse = (float*)a->lse; ap.dvec = (float*)g->dvec; ap.out = (float*)dqkv;
        ap.ds = (float*)g->att_ds;
        {
            /* D, then dK/dV (leaving dS), then dQ from dS */
            void* args[] = { &ap };
            hip_launch(g->k.attn_dvec, cdiv_u64((u64)g->N * g->D / 4, 256), 1, 1, 256, 1, 1, 0, args);
            hip_launch(g->k.attn_bwd_dkv, g->B * g->H, cdiv_u64(g->T, 64), 1, 256, 1, 1, 0, args);
            hip_launch(g->k.attn_bwd_dq, g->B * g->H, cdiv_u64(g->T, 64), 1, 256, 1, 1, 0, args);
        }
        hip_side_begin();
        gemm_wb(g, a->n1, dqkv, G_(g, pidx(ul, PK_WQKV)), G_(g, pidx(ul, PK_BQKV)), D, 3 * D, N);
        hip_side_end(3);
        gemm1(g, GEMM_NT, dqkv, P_(g, pidx(ul, PK_WQKV)), g->dn, N, D, 3 * D, 3 * D, 3 * D, D, 0.0f, NULL, NULL);
        rmsnorm_bwd(g, a->x_in, P_(g, pidx(ul, PK_ATTN_NORM)), a->r1, g->dn, d_mid, d_in, g->part[par][0]);
        part_prev = g->part[par][0];
        w_prev = G_(g, pidx(ul, PK_ATTN_NORM));
        v += 2;
    }
    colsum_partials(g, part_prev, w_prev);
    /* tied head: dE = dlogits^T @ nf, overlapping the last side sections */
    gemm1(g, GEMM_TN, g->logits, g->nf, G_(g, 0), V, D, N, ldv, D, D, 0.0f, NULL, NULL);
    /* join: every weight gradient is complete before anything reads it */
    hip_side_join();
    /* embedding: dE[tok] += rows of the input gradient, per token in
     * ascending row order */
    {
        hipDeviceptr_t dx = g->dres[v % R], order = g->emb_order, seg = g->emb_seg, dE = G_(g, 0);
        hipDeviceptr_t seg_tok = dptr(seg, g->emb_nseg + 1);
        i32 nseg = (i32)g->emb_nseg;
        void* args[] = { &dx, &order, &seg, &seg_tok, &nseg, &dE, &D };
        hip_launch(g->k.embed_bwd, g->emb_nseg, cdiv_u64((u64)D, 256), 1, 256, 1, 1, 0, args);
    }
}

/* Per-sequence mean then mean over sequences (gpu_train.c:476-487). */
static f32 mean_loss(GpuTrainer* g) {
    hip_d2h(g->host_loss_rows, g->loss_rows, (u64)g->N * F4);
    f32 loss_sum = 0.0f;
    for (u32 b = 0; b < g->B; b++) {
        f32 s = 0.0f;
        for (u32 t = 0; t < g->T; t++) s += g->host_loss_rows[(u64)b * g->T + t];
        loss_sum += s / (f32)g->T;
    }
    return loss_sum / (f32)g->B;
}

f32 gpu_trainer_forward_backward(GpuTrainer* g, const u32* ids, const u32* targets) {
    bind(g);
    embed_segments(g, ids);
    forward_to_logits(g, ids);
    cross_entropy(g, targets, 1);
    backward_pass(g);
    return mean_loss(g);
}

/* The loss rows come from the LM head's row statistics and target logits
 * alone, so eval writes no logits and forms no gradient (the reference's
 * kernel overwrites the logits with their gradient here, which no caller can
 * observe): the same loss as forward_backward, bit for bit. */
f32 gpu_trainer_eval_loss(GpuTrainer* g, const u32* ids, const u32* targets) {
    bind(g);
    upload_targets(g, targets);
    forward_to_loss_stats(g, ids);
    cross_entropy_ex(g, NULL, 0, 1);
    return mean_loss(g);
}

/* Deterministic L2 norm: fixed grid of partial sums, f64 host sum in order
 * (gpu_train.c:502-512). */
f64 gpu_trainer_grad_norm(GpuTrainer* g) {
    bind(g);
    hipDeviceptr_t x = g->grads, part = g->norm_partial;
    long long n = (long long)g->total_scalars;
    void* args[] = { &x, &n, &part };
    hip_launch(g->k.sumsq_partial, GPU_TRAIN_NORM_BLOCKS, 1, 1, 256, 1, 1, 0, args);
    hip_d2h(g->host_norm_partial, g->norm_partial, GPU_TRAIN_NORM_BLOCKS * F4);
    f64 ss = 0.0;
    for (u32 i = 0; i < GPU_TRAIN_NORM_BLOCKS; i++) ss += (f64)g->host_norm_partial[i];
    return m_sqrt(ss);
}

static void adam_launch(GpuTrainer* g, AdamOptimizer* opt, f32 grad_scale, f32 weight_decay) {
    bind(g);
    opt->t++;
    f32 bc1 = 1.0f - m_powf(opt->beta1, (f32)opt->t);
    f32 bc2 = 1.0f - m_powf(opt->beta2, (f32)opt->t);
    hipDeviceptr_t p = g->params, gr = g->grads, m = g->adam_m, v = g->adam_v;
    long long n = (long long)g->total_scalars;
    f32 lr = opt->lr, b1 = opt->beta1, b2 = opt->beta2, eps = opt->eps;
    f32 lrwd = lr * weight_decay;
    void* args[] = { &p, &gr, &m, &v, &n, &lr, &b1, &b2, &eps, &bc1, &bc2, &grad_scale, &lrwd };
    u32 blocks = cdiv_u64((u64)(n / 4) > 0 ? (u64)(n / 4) : 1, 256);
    hip_launch(g->k.adam, blocks, 1, 1, 256, 1, 1, 0, args);
    hip_sync();
}

void gpu_trainer_adam_step(GpuTrainer* g, AdamOptimizer* opt) { gpu_trainer_adam_step_scaled(g, opt, 1.0f); }

void gpu_trainer_adam_step_scaled(GpuTrainer* g, AdamOptimizer* opt, f32 grad_scale) {
    adam_launch(g, opt, grad_scale, 0.0f);
}

/* ---------------- queued driver steps (train_loop.c) ---------------- */

/* One training step of the driver loop with the batch already on the device
 * (g->ids, g->targets, g->emb_order/emb_seg, g->emb_nseg): forward, CE,
 * backward, the loss mean into loss_out (f32), the grad norm into norm_out
 * (f64) and the clip scale into scale_buf (f32), then Adam/AdamW with that
 * scale.  Nothing waits for the device. */
void trlm_train_step_queued(GpuTrainer* g, AdamOptimizer* opt, f32 weight_decay, f64 clip, hipDeviceptr_t loss_out,
                            hipDeviceptr_t norm_out, hipDeviceptr_t scale_buf) {
    forward_to_logits(g, NULL);
    cross_entropy(g, NULL, 1);
    backward_pass(g);
    trlm_loss_mean_queued(g, loss_out, 0);
    {
        hipDeviceptr_t x = g->grads, part = g->norm_partial;
        long long n = (long long)g->total_scalars;
        void* args[] = { &x, &n, &part };
        hip_launch(g->k.sumsq_partial, GPU_TRAIN_NORM_BLOCKS, 1, 1, 256, 1, 1, 0, args);
        i32 np = (i32)GPU_TRAIN_NORM_BLOCKS;
        void* args2[] = { &part, &np, &clip, &norm_out, &scale_buf };
        hip_launch(g->k.norm_clip, 1, 1, 1, 256, 1, 1, 0, args2);
    }
    opt->t++;
    f32 bc1 = 1.0f - m_powf(opt->beta1, (f32)opt->t);
    f32 bc2 = 1.0f - m_powf(opt->beta2, (f32)opt->t);
    hipDeviceptr_t p = g->params, gr = g->grads, m = g->adam_m, v = g->adam_v;
    long long n = (long long)g->total_scalars;
    f32 lr = opt->lr, b1 = opt->beta1, b2 = opt->beta2, eps = opt->eps;
    f32 lrwd = lr * weight_decay;
    void* args[] = { &p, &gr, &m, &v, &n, &lr, &b1, &b2, &eps, &bc1, &bc2, &scale_buf, &lrwd };
    u32 blocks = cdiv_u64((u64)(n / 4) > 0 ? (u64)(n / 4) : 1, 256);
    hip_launch(g->k.adam_ds, blocks, 1, 1, 256, 1, 1, 0, args);
}

/* mean_loss of g->loss_rows on the device into *out (acc: added onto it). */
void trlm_loss_mean_queued(GpuTrainer* g, hipDeviceptr_t out, i32 acc) {
    hipDeviceptr_t rows = g->loss_rows;
    i32 B = (i32)g->B, T = (i32)g->T;
    void* args[] = { &rows, &B, &T, &out, &acc };
    hip_launch(g->k.loss_mean, 1, 1, 1, 256, 1, 1, 0, args);
}

/* eval_loss with the batch already on the device; the loss is added onto
 * *sum (acc = 0 starts the sum). */
void trlm_eval_queued(GpuTrainer* g, hipDeviceptr_t sum, i32 acc) {
    forward_to_loss_stats(g, NULL);
    cross_entropy_ex(g, NULL, 0, 1);
    trlm_loss_mean_queued(g, sum, acc);
}

/* ---------------- additive entry points (trlm_ext.h) ---------------- */

static void logits_to_host(GpuTrainer* g, f32* host) {
    hipError_t r = hipMemcpy2DAsync(host, (size_t)g->V * F4, g->logits, (size_t)g->ldv * F4, (size_t)g->V * F4,
                                    g->N, hipMemcpyDeviceToHost, g->hip.stream);
    if (r != hipSuccess) fatal("logits copy failed");
    hip_sync();
}

void gpu_trainer_forward_logits(GpuTrainer* g, const u32* ids, f32* host_logits) {
    bind(g);
    forward_to_logits(g, ids);
    if (host_logits) logits_to_host(g, host_logits);
    else hip_sync();
}

f32 gpu_trainer_forward_loss_logits(GpuTrainer* g, const u32* ids, const u32* targets, f32* host_logits) {
    bind(g);
    forward_to_logits(g, ids);
    cross_entropy(g, targets, 0);
    f32 loss = mean_loss(g);
    if (host_logits) logits_to_host(g, host_logits);
    return loss;
}

void gpu_trainer_greedy_argmax(GpuTrainer* g, u32* host_ids_out) {
    bind(g);
    hipDeviceptr_t lg = g->logits, out = g->emb_order;   /* [N] u32 scratch */
    i32 ld = (i32)g->ldv, V = (i32)g->V;
    void* args[] = { &lg, &ld, &V, &out };
    hip_launch(g->k.argmax_rows, g->N, 1, 1, 256, 1, 1, 0, args);
    hip_d2h(host_ids_out, out, (u64)g->N * sizeof(u32));
}

void gpu_trainer_adamw_step_scaled(GpuTrainer* g, AdamOptimizer* opt, f32 weight_decay, f32 grad_scale) {
    adam_launch(g, opt, grad_scale, weight_decay);
}

TrlmGemm* gpu_trainer_gemm_engine(GpuTrainer* g) {
    bind(g);
    return g->gemm;
}

/* ---------------- helpers shared with the decoder (gpu_decode.c) ---------------- */

void trlm_bind(GpuTrainer* g) { bind(g); }

hipDeviceptr_t trlm_param_ptr(const GpuTrainer* g, u32 i) { return P_(g, i); }

void trlm_rmsnorm_rows(GpuTrainer* g, hipDeviceptr_t x, hipDeviceptr_t w, hipDeviceptr_t out, hipDeviceptr_t rinv,
                       u32 rows) {
    rmsnorm_rows(g, x, w, out, rinv, rows);
}

void trlm_gemm_rows(GpuTrainer* g, GemmKind kind, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C, i32 M, i32 N,
                    i32 K, i32 lda, i32 ldb, i32 ldc, hipDeviceptr_t bias, hipDeviceptr_t resid) {
    gemm1(g, kind, A, B, C, M, N, K, lda, ldb, ldc, 0.0f, bias, resid);
}

void trlm_swiglu_rows(GpuTrainer* g, hipDeviceptr_t gu, hipDeviceptr_t h, u32 rows) {
    i32 n = (i32)rows, F = (i32)g->F;
    void* args[] = { &gu, &h, &n, &F };
    hip_launch(g->k.swiglu_fwd, swiglu_blocks(g, rows), 1, 1, 256, 1, 1, 0, args);
}

void trlm_embed_rows(GpuTrainer* g, hipDeviceptr_t ids, hipDeviceptr_t x, u32 rows) {
    hipDeviceptr_t E = P_(g, 0);
    i32 n = (i32)rows, D = (i32)g->D;
    void* args[] = { &E, &ids, &x, &n, &D };
    u64 work = (g->D % 4 == 0) ? (u64)rows * g->D / 4 : (u64)rows * g->D;
    hip_launch(g->k.embed_fwd, cdiv_u64(work, 256), 1, 1, 256, 1, 1, 0, args);
}

void trlm_argmax_rows(GpuTrainer* g, hipDeviceptr_t logits, i32 ld, u32 rows, hipDeviceptr_t out) {
    i32 V = (i32)g->V;
    void* args[] = { &logits, &ld, &V, &out };
    hip_launch(g->k.argmax_rows, rows, 1, 1, 256, 1, 1, 0, args);
}
