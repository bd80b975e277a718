/* trlm_gemm.c -- host dispatch of the fp32 MFMA GEMM kernels (gemm.hip).
 *
 * Plays the role of the reference's gemm()/gemm1()/bf16_gemm*() launch
 * helpers (model/gpu_train.c:42-118): same operand conventions (NN, NT, TN;
 * batched with element strides; alpha/beta; bias and residual epilogue),
 * with the tile shape and split-K chosen per problem for 256 CUs:
 *   - (tile, split-K) minimise a load-balance cost model (select_plan): the
 *     busiest CU's share of workgroups, the variant's residency and
 *     efficiency, and the split partials' HBM round trip.  The plan depends
 *     on (M, N, K, batch) only, so reruns are bit-identical;
 *   - split-K (single GEMMs: weight gradients with K = B*T, dX with
 *     K = vocab, short-M shapes): splits write raw partials to a workspace
 *     that k_gemm_splitk_reduce sums in split order, so the result stays
 *     deterministic (no atomics);
 *   - operands whose rows are not 16-byte aligned go to the _u variants,
 *     which use scalar loads.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "gpu_internal.h"

#include "kernel_params.h"   /* GemmParams: the argument block the kernels read */

enum { L_NN = 0, L_NT = 1, L_TN = 2 };
static const char* LAYOUT_NAME[4] = { "nn", "nt", "tn", "tt" };

/* Aligned tile variants (gemm.hip): name suffix, tile rows/cols, k step. */
typedef struct TileDef { const char* name; int bm, bn, bk; } TileDef;
enum { T_256x128, T_128x256, T_128x128, T_128x128_K32, T_64x128, T_64x128_K32, T_64x64, T_64x64_K32, T_COUNT };
static const TileDef TILES[T_COUNT] = {
    { "256x128", 256, 128, 16 }, { "128x256", 128, 256, 16 }, { "128x128", 128, 128, 16 },
    { "128x128_k32", 128, 128, 32 }, { "64x128", 64, 128, 16 }, { "64x128_k32", 64, 128, 32 },
    { "64x64", 64, 64, 16 }, { "64x64_k32", 64, 64, 32 },
};

#define CUS 256
#define KCHUNK_ALIGN 32  /* split-K chunks are multiples of every variant's k step */

struct TrlmGemm {
    HipCtx* ctx;
    hipFunction_t k[3][T_COUNT];
    hipFunction_t ku[4];
    hipFunction_t reduce;
    hipFunction_t reduce4;   /* four columns per thread, for 16-byte aligned operands */
    hipFunction_t glu;   /* k_gemm_nn_64x64_k32_glu */
    hipDeviceptr_t ws;
    u64 ws_floats;
    char last[48];
    i32 last_splits;
    i32 force_tile;    /* -1: automatic selection */
    i32 force_splits;  /* 0: automatic split-K */
};

TrlmGemm* trlm_gemm_create(HipCtx* ctx) {
    TrlmGemm* e = (TrlmGemm*)calloc(1, sizeof(TrlmGemm));
    e->ctx = ctx;
    e->force_tile = -1;
    char name[64];
    for (int l = 0; l < 3; l++)
        for (int t = 0; t < T_COUNT; t++) {
            snprintf(name, sizeof(name), "k_gemm_%s_%s", LAYOUT_NAME[l], TILES[t].name);
            e->k[l][t] = hip_get_kernel(ctx, name);
        }
    for (int l = 0; l < 4; l++) {
        snprintf(name, sizeof(name), "k_gemm_%s_64x64_u", LAYOUT_NAME[l]);
        e->ku[l] = hip_get_kernel(ctx, name);
    }
    e->reduce = hip_get_kernel(ctx, "k_gemm_splitk_reduce");
    e->reduce4 = hip_get_kernel(ctx, "k_gemm_splitk_reduce4");
    e->glu = hip_get_kernel(ctx, "k_gemm_nn_64x64_k32_glu");
    trlm_noalloc_setup(ctx->device);
    return e;
}

void trlm_gemm_destroy(TrlmGemm* e) {
    if (!e) return;
    if (e->ws) hip_free(e->ws);
    free(e);
}

i32 trlm_gemm_device(const TrlmGemm* e) { return e->ctx->device; }

const char* trlm_gemm_last_variant(TrlmGemm* e, i32* splits) {
    if (splits) *splits = e->last_splits;
    return e->last;
}

i32 trlm_gemm_force(TrlmGemm* e, const char* tile, i32 splits) {
    e->force_tile = -1;
    e->force_splits = splits > 0 ? splits : 0;
    if (!tile || !tile[0]) return 0;
    for (int t = 0; t < T_COUNT; t++)
        if (strcmp(tile, TILES[t].name) == 0) {
            e->force_tile = t;
            return 0;
        }
    return -1;
}

static int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

static int aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

/* Row statistics: 2 entries per tile column (one per wave column half);
 * the caller's buffer holds stats_cap entries per row. */
static void set_stats(GemmParams* p, hipDeviceptr_t stats, i32 stats_cap, int bn) {
    int n = 2 * cdiv(p->N, bn);
    if (n > stats_cap) {
        fprintf(stderr, "[HIP ERROR] trlm_gemm: row statistics need %d entries per row, buffer has %d\n", n, stats_cap);
        _exit(1);
    }
    p->stats = (float*)stats;
    p->stats_ld = n;
}

static void launch(hipFunction_t f, GemmParams* p, u32 gz) {
    void* args[] = { p };
    hip_launch(f, (u32)(p->tiles_m * p->tiles_n), 1, gz, 256, 1, 1, 0, args);
}

static long long tiles_of(int t, int M, int N, u32 batch) {
    return (long long)cdiv(M, TILES[t].bm) * cdiv(N, TILES[t].bn) * batch;
}

/* Split-K factor for a single GEMM with few output tiles and a long K:
 * enough splits for ~2 workgroups per CU, each split >= 256 deep.  Used
 * when a tile is forced without a split factor. */
static int auto_splits(long long tiles, int K) {
    if (K < 512 || tiles >= CUS) return 1;
    int s = cdiv(2 * CUS, tiles);
    if (s > K / 256) s = K / 256;
    if (s > 32) s = 32;
    return s < 1 ? 1 : s;
}

/* Plan model: the tiles' workgroups are spread evenly over the 256 CUs, so
 * the busiest CU runs n = ceil(workgroups / 256) of them, `occ` at a time
 * (the variant's resident workgroups per CU).  A CU with c resident
 * workgroups runs at cu_rate(c) of its steady-state rate (one resident
 * 4-wave workgroup cannot hide its own load latency), and each variant has
 * its own steady-state efficiency.  The last resident batch adds an
 * imbalance term proportional to a workgroup's duration.  Split-K adds the
 * partials' round trip through HBM plus the reduction launch.  Constants
 * fitted to MI355X timings of every variant/split on the model's GEMMs at
 * 512-8192 rows (within 0.6 % of the per-shape best over those 45 shapes). */
typedef struct PlanTile { int tile; int occ; double eff; } PlanTile;
static const PlanTile PLAN_TILES[] = {
    { T_128x128, 3, 1.047 }, { T_128x256, 2, 0.977 }, { T_256x128, 2, 1.008 },
    { T_64x128_K32, 2, 0.955 }, { T_64x64_K32, 4, 0.992 },
};
static const int PLAN_SPLITS[] = { 1, 2, 3, 4, 6, 7, 8, 12, 16, 24, 32 };
#define PLAN_CU_FLOPS 0.6e12     /* per-CU steady-state fp32 MFMA rate, FLOP/s */
#define PLAN_SPLIT_BW 1.63e12    /* effective bytes/s of the partials' round trip */
#define PLAN_SPLIT_FIXED 1.25e-6 /* reduction launch, s */
#define PLAN_TAIL 0.075          /* last-round imbalance, in resident-batch durations */

static double cu_rate(int c) { return c <= 1 ? 0.916 : 1.0; }

static double plan_cost(const PlanTile* pt, int M, int N, int K, u32 batch, int splits) {
    const TileDef* td = &TILES[pt->tile];
    double wg = (double)cdiv(M, td->bm) * cdiv(N, td->bn) * batch * splits;
    int kch = splits > 1 ? cdiv(cdiv(K, splits), KCHUNK_ALIGN) * KCHUNK_ALIGN : K;
    long long n = (long long)((wg + CUS - 1) / CUS);
    double w = 2.0 * td->bm * td->bn * (double)kch / (pt->eff * PLAN_CU_FLOPS);
    long long full = n / pt->occ, rest = n % pt->occ;
    double t = (double)full * pt->occ * w / cu_rate(pt->occ);
    if (rest) t += (double)rest * w / cu_rate((int)rest);
    /* workgroups of one resident batch finish unevenly: long workgroups
     * leave CUs idle at the end, which more, shorter ones even out */
    t += PLAN_TAIL * pt->occ * w / cu_rate((int)(n < pt->occ ? n : pt->occ));
    if (splits > 1) t += (splits + 1) * (double)M * N * 4.0 / PLAN_SPLIT_BW + PLAN_SPLIT_FIXED;
    return t;
}

static void select_plan(int M, int N, int K, u32 batch, int* tile, int* splits) {
    double best = 0.0;
    *tile = T_128x128;
    *splits = 1;
    /* Decode-sized products (M <= 128 rows, few tiles): each workgroup's
     * k loop is latency-bound (~1 us per 32-deep step), so split K down to
     * 64-deep chunks over up to 8 partitions, one workgroup per CU at most.
     * Measured on MI355X at M = 64: QKV 12.8 -> 9.0 us, attention-out 11.8
     * -> 8.6, gate_up 12.4 -> 8.2, down (K = 1024) 12.6 -> 10.4, reduction
     * included. */
    if (M <= 128 && batch == 1) {
        long long tiles = (long long)cdiv(M, 64) * cdiv(N, 64);
        if (tiles < 128) {
            long long smax = K / 64;
            if (smax > 8) smax = 8;
            if (smax > CUS / tiles) smax = CUS / tiles;
            *tile = T_64x64_K32;
            for (size_t j = 0; j < sizeof(PLAN_SPLITS) / sizeof(PLAN_SPLITS[0]); j++)
                if (PLAN_SPLITS[j] <= smax) *splits = PLAN_SPLITS[j];
            return;
        }
    }
    for (size_t i = 0; i < sizeof(PLAN_TILES) / sizeof(PLAN_TILES[0]); i++)
        for (size_t j = 0; j < sizeof(PLAN_SPLITS) / sizeof(PLAN_SPLITS[0]); j++) {
            int sp = PLAN_SPLITS[j];
            if (sp > 1 && (batch != 1 || K / sp < 256)) continue;
            double c = plan_cost(&PLAN_TILES[i], M, N, K, batch, sp);
            if ((i == 0 && j == 0) || c < best) {
                best = c;
                *tile = PLAN_TILES[i].tile;
                *splits = sp;
            }
        }
}

const char* trlm_gemm_plan(i32 trans_a, i32 trans_b, i32 M, i32 N, i32 K, u32 batch, i32* splits) {
    static __thread char name[48];
    int layout = trans_a ? (trans_b ? 3 : L_TN) : (trans_b ? L_NT : L_NN);
    int tile, sp;
    if (layout == 3) {
        snprintf(name, sizeof(name), "k_gemm_tt_64x64_u");
        sp = 1;
    } else {
        select_plan(M, N, K, batch ? batch : 1, &tile, &sp);
        if (sp > 1) sp = cdiv(K, cdiv(cdiv(K, sp), KCHUNK_ALIGN) * KCHUNK_ALIGN);
        snprintf(name, sizeof(name), "k_gemm_%s_%s", LAYOUT_NAME[layout], TILES[tile].name);
    }
    if (splits) *splits = sp;
    return name;
}

void trlm_gemm(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
               i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
               f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr) {
    trlm_gemm_ex(e, trans_a, trans_b, A, B, C, M, N, K, lda, ldb, ldc, batch, sA, sB, sC, alpha, beta, bias, resid,
                 ldr, NULL);
}

i32 trlm_gemm_ex(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
                 i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
                 f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr, const TrlmGemmExtra* x) {
    return trlm_gemm_ws(e, trans_a, trans_b, A, B, C, M, N, K, lda, ldb, ldc, batch, sA, sB, sC, alpha, beta, bias,
                        resid, ldr, x, NULL, 0);
}

i32 trlm_gemm_ws(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
                 i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
                 f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr, const TrlmGemmExtra* x,
                 hipDeviceptr_t fixed_ws, u64 fixed_floats) {
    hipDeviceptr_t stats = x ? x->stats : NULL, csum = x ? x->csum : NULL;
    i32 stats_cap = x ? x->stats_cap : 0;
    int rope = x && x->rope_cos;
    if (M <= 0 || N <= 0 || batch == 0) return 0;
    if (rope && (batch != 1 || x->rope_T <= 0 || x->rope_hd <= 0 || x->rope_hd % 4 || x->rope_cols % 4)) {
        fprintf(stderr, "[HIP ERROR] trlm_gemm: RoPE epilogue needs a single GEMM and head width a multiple of 4\n");
        _exit(1);
    }
    if (stats && (batch != 1 || beta != 0.0f || bias || resid || trans_a || !trans_b)) {
        fprintf(stderr, "[HIP ERROR] trlm_gemm: row statistics need a single NT GEMM (the LM head's) with no beta, "
                        "bias or residual\n");
        _exit(1);
    }
    if (x && (x->tgt || x->tgt_val || x->no_store) && (!stats || (x->tgt == NULL) != (x->tgt_val == NULL))) {
        fprintf(stderr, "[HIP ERROR] trlm_gemm: target values and no_store need row statistics (and both target buffers)\n");
        _exit(1);
    }
    if (x && x->glu_h) {
        /* the SwiGLU epilogue: one fixed kernel, so only the shapes it tiles exactly */
        if (trans_a || trans_b || batch != 1 || beta != 0.0f || resid || stats || csum || rope || fixed_ws ||
            x->glu_F <= 0 || x->glu_F % 32 || N != 2 * x->glu_F || K <= 0 || K % 32 || !aligned16(A) ||
            !aligned16(B) || !aligned16(C) || !aligned16(x->glu_h) || lda % 4 || ldb % 4 || ldc % 4 ||
            (bias && !aligned16(bias))) {
            fprintf(stderr, "[HIP ERROR] trlm_gemm: the SwiGLU epilogue needs a single aligned NN GEMM, N = 2F with "
                            "F %% 32 == 0, K %% 32 == 0, no beta, residual or other epilogue\n");
            _exit(1);
        }
        GemmParams p;
        memset(&p, 0, sizeof(p));
        p.A = (const float*)A; p.B = (const float*)B; p.C = (float*)C; p.bias = (const float*)bias;
        p.M = M; p.N = N; p.K = K; p.lda = lda; p.ldb = ldb; p.ldc = ldc; p.ldr = ldr;
        p.splits = 1; p.kchunk = K; p.alpha = alpha; p.beta = 0.0f;
        p.tiles_m = cdiv(M, 64); p.tiles_n = cdiv(N, 64);
        p.glu_h = (float*)x->glu_h; p.glu_F = x->glu_F;
        snprintf(e->last, sizeof(e->last), "k_gemm_nn_64x64_k32_glu");
        e->last_splits = 1;
        launch(e->glu, &p, 1);
        return 0;
    }
    if (csum && (batch != 1 || trans_b)) {
        fprintf(stderr, "[HIP ERROR] trlm_gemm: column sums need a single GEMM with B stored [K,N]\n");
        _exit(1);
    }
    if (M > (1 << 30) || N > (1 << 30) || K < 0) {
        fprintf(stderr, "[HIP ERROR] trlm_gemm: bad shape M=%d N=%d K=%d\n", M, N, K);
        _exit(1);
    }
    GemmParams p;
    memset(&p, 0, sizeof(p));
    p.A = (const float*)A; p.B = (const float*)B; p.C = (float*)C;
    p.bias = (const float*)bias; p.resid = (const float*)resid;
    p.sA = sA; p.sB = sB; p.sC = sC; p.sW = 0;
    p.M = M; p.N = N; p.K = K;
    p.lda = lda; p.ldb = ldb; p.ldc = ldc; p.ldr = ldr;
    p.splits = 1; p.kchunk = K > 0 ? K : 1;
    p.alpha = alpha; p.beta = beta;
    p.csum = (float*)csum;
    if (stats) {
        p.tgt = (const u32*)x->tgt;
        p.tgt_val = (float*)x->tgt_val;
        p.no_store = x->no_store != 0;
    }
    if (rope) {
        p.rope_cos = x->rope_cos; p.rope_sin = x->rope_sin;
        p.rope_T = x->rope_T; p.rope_hd = x->rope_hd; p.rope_cols = x->rope_cols;
    }

    int layout = trans_a ? (trans_b ? 3 : L_TN) : (trans_b ? L_NT : L_NN);
    int aligned = layout != 3 && aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                  (batch == 1 || ((sA % 4 == 0) && (sB % 4 == 0)));
    if (!aligned) {
        p.tiles_m = cdiv(M, 64); p.tiles_n = cdiv(N, 64);
        snprintf(e->last, sizeof(e->last), "k_gemm_%s_64x64_u", LAYOUT_NAME[layout]);
        e->last_splits = 1;
        if (stats) set_stats(&p, stats, stats_cap, 64);
        launch(e->ku[layout], &p, batch);
        return p.stats ? 2 * p.tiles_n : 0;
    }

    int tile, splits;
    select_plan(M, N, K, batch, &tile, &splits);
    if (e->force_tile >= 0) {
        tile = e->force_tile;
        splits = batch == 1 ? auto_splits(tiles_of(tile, M, N, 1), K) : 1;
    }
    if (e->force_splits > 0 && batch == 1) splits = e->force_splits;
    if (stats || rope) splits = 1;         /* these epilogues need whole sums */
    p.tiles_m = cdiv(M, TILES[tile].bm);
    p.tiles_n = cdiv(N, TILES[tile].bn);
    if (stats) set_stats(&p, stats, stats_cap, TILES[tile].bn);
    int kchunk = K;
    if (splits > 1 && K < 2 * KCHUNK_ALIGN) splits = 1;
    if (splits > 1) {
        kchunk = cdiv(cdiv(K, splits), KCHUNK_ALIGN) * KCHUNK_ALIGN;
        splits = cdiv(K, kchunk);
    }
    /* split-K: raw partials into the workspace, then an ordered reduction;
     * with column sums each split's slab has one more row, M, for them */
    u64 slab = ((u64)M + (csum ? 1u : 0u)) * (u64)N;
    if (fixed_ws && splits > 1 && (u64)splits * slab > fixed_floats) {
        /* A fixed workspace that cannot hold the plan's partials: run the
         * most splits whose partials fit (one split needs none).  The k
         * chunks are formed as for a forced split count, so the result
         * equals this engine's trlm_gemm forced to that many splits. */
        u64 fit = fixed_floats / slab;
        splits = fit < 2 ? 1 : (int)fit;
        kchunk = K;
        if (splits > 1) {
            kchunk = cdiv(cdiv(K, splits), KCHUNK_ALIGN) * KCHUNK_ALIGN;
            splits = cdiv(K, kchunk);
        }
    }
    snprintf(e->last, sizeof(e->last), "k_gemm_%s_%s", LAYOUT_NAME[layout], TILES[tile].name);
    e->last_splits = splits;
    if (splits <= 1) {
        launch(e->k[layout][tile], &p, batch);
        return p.stats ? 2 * p.tiles_n : 0;
    }
    u64 need = (u64)splits * slab;
    hipDeviceptr_t W = fixed_ws;
    if (!fixed_ws) {
        if (need > e->ws_floats) {
            if (e->ws) hip_free(e->ws);
            e->ws = hip_alloc(need * sizeof(f32));
            e->ws_floats = need;
        }
        W = e->ws;
    }
    GemmParams q = p;
    q.C = (float*)W;
    q.ldc = N;
    q.sW = (long long)slab;
    q.kchunk = kchunk;
    q.splits = splits;
    q.alpha = 1.0f; q.beta = 0.0f; q.bias = NULL; q.resid = NULL;
    launch(e->k[layout][tile], &q, (u32)splits);
    long long total = (long long)slab;
    i32 sp = splits;
    i64 sW = (i64)slab;
    void* args[] = { &W, &sp, &sW, &C, &M, &N, &ldc, &alpha, &beta, &bias, &resid, &ldr, &csum };
    /* four columns per thread when every row segment of four is 16-byte
     * aligned in each operand: same per-element order, same bits */
    const int vec4 = (N % 4) == 0 && (ldc % 4) == 0 && (!resid || (ldr % 4) == 0) &&
                     (((uintptr_t)W | (uintptr_t)C | (uintptr_t)bias | (uintptr_t)resid | (uintptr_t)csum) & 15u) == 0;
    if (vec4)
        hip_launch(e->reduce4, (u32)((total / 4 + 255) / 256), 1, 1, 256, 1, 1, 0, args);
    else
        hip_launch(e->reduce, (u32)((total + 255) / 256), 1, 1, 256, 1, 1, 0, args);
    return 0;
}

void trlm_timer_create(TrlmTimer* t) {
    hipEventCreate(&t->start);
    hipEventCreate(&t->stop);
}

void trlm_timer_destroy(TrlmTimer* t) {
    hipEventDestroy(t->start);
    hipEventDestroy(t->stop);
}

void trlm_timer_start(TrlmTimer* t) { hipEventRecord(t->start, hip_current_stream()); }

f32 trlm_timer_stop_ms(TrlmTimer* t) {
    float ms = 0.f;
    hipEventRecord(t->stop, hip_current_stream());
    hipEventSynchronize(t->stop);
    hipEventElapsedTime(&ms, t->start, t->stop);
    return ms;
}

const char* trlm_version(void) { return "trlm-mi355x 0.1 (gfx950, fp32 MFMA)"; }

u64 trlm_sizeof_gpu_trainer(void) { return (u64)sizeof(GpuTrainer); }
u64 trlm_sizeof_hip_ctx(void) { return (u64)sizeof(HipCtx); }
