/* trlm_gemm.c -- host dispatch of the fp32 MFMA GEMM kernels (gemm.hip).
 *
 * Plays the role of the reference's gemm()/gemm1()/bf16_gemm*() launch
 * helpers (model/gpu_train.c:42-118): same operand conventions (NN, NT, TN;
 * batched with element strides; alpha/beta; bias and residual epilogue),
 * with the tile shape and split-K chosen per problem for 256 CUs:
 *   - 128x128 tiles when that gives >= 2 workgroups per CU,
 *     else 64x128, else 64x64;
 *   - split-K for single GEMMs with a large K and too few tiles (the
 *     weight-gradient TN forms, K = B*T; dX with K = vocab): splits write
 *     raw partials to a workspace that k_gemm_splitk_reduce sums in split
 *     order, so the result stays deterministic (no atomics);
 *   - operands whose rows are not 16-byte aligned go to the _u variants,
 *     which use scalar loads.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "trlm_ext.h"

/* Kernel argument block; layout identical to struct GemmParams in gemm.hip. */
typedef struct GemmParams {
    const float* A;
    const float* B;
    float* C;
    const float* bias;
    const float* resid;
    long long sA, sB, sC, sW;
    int M, N, K;
    int lda, ldb, ldc, ldr;
    int splits, kchunk;
    float alpha, beta;
    int tiles_m, tiles_n;
} GemmParams;

enum { L_NN = 0, L_NT = 1, L_TN = 2 };
enum { T_128x128 = 0, T_64x128 = 1, T_64x64 = 2 };
static const int TILE_BM[3] = { 128, 64, 64 };
static const int TILE_BN[3] = { 128, 128, 64 };
static const char* LAYOUT_NAME[4] = { "nn", "nt", "tn", "tt" };
static const char* TILE_NAME[3] = { "128x128", "64x128", "64x64" };

#define CUS 256
#define GBK 16

struct TrlmGemm {
    HipCtx* ctx;
    hipFunction_t k[3][3];
    hipFunction_t ku[4];
    hipFunction_t reduce;
    hipDeviceptr_t ws;
    u64 ws_floats;
    char last[48];
    i32 last_splits;
};

TrlmGemm* trlm_gemm_create(HipCtx* ctx) {
    TrlmGemm* e = (TrlmGemm*)calloc(1, sizeof(TrlmGemm));
    e->ctx = ctx;
    char name[64];
    for (int l = 0; l < 3; l++)
        for (int t = 0; t < 3; t++) {
            snprintf(name, sizeof(name), "k_gemm_%s_%s", LAYOUT_NAME[l], TILE_NAME[t]);
            e->k[l][t] = hip_get_kernel(ctx, name);
        }
    for (int l = 0; l < 4; l++) {
        snprintf(name, sizeof(name), "k_gemm_%s_64x64_u", LAYOUT_NAME[l]);
        e->ku[l] = hip_get_kernel(ctx, name);
    }
    e->reduce = hip_get_kernel(ctx, "k_gemm_splitk_reduce");
    return e;
}

void trlm_gemm_destroy(TrlmGemm* e) {
    if (!e) return;
    if (e->ws) hip_free(e->ws);
    free(e);
}

const char* trlm_gemm_last_variant(TrlmGemm* e, i32* splits) {
    if (splits) *splits = e->last_splits;
    return e->last;
}

static int cdiv(long long a, long long b) { return (int)((a + b - 1) / b); }

static int aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static void launch(hipFunction_t f, GemmParams* p, u32 gz) {
    void* args[] = { p };
    hip_launch(f, (u32)(p->tiles_m * p->tiles_n), 1, gz, 256, 1, 1, 0, args);
}

void trlm_gemm(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B, hipDeviceptr_t C,
               i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA, i64 sB, i64 sC,
               f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid, i32 ldr) {
    if (M <= 0 || N <= 0 || batch == 0) return;
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

    int layout = trans_a ? (trans_b ? 3 : L_TN) : (trans_b ? L_NT : L_NN);
    int aligned = layout != 3 && aligned16(A) && aligned16(B) && (lda % 4 == 0) && (ldb % 4 == 0) &&
                  (batch == 1 || ((sA % 4 == 0) && (sB % 4 == 0)));
    if (!aligned) {
        p.tiles_m = cdiv(M, 64); p.tiles_n = cdiv(N, 64);
        snprintf(e->last, sizeof(e->last), "k_gemm_%s_64x64_u", LAYOUT_NAME[layout]);
        e->last_splits = 1;
        launch(e->ku[layout], &p, batch);
        return;
    }

    long long t128 = (long long)cdiv(M, 128) * cdiv(N, 128) * batch;
    long long t64x128 = (long long)cdiv(M, 64) * cdiv(N, 128) * batch;
    int tile;
    int splits = 1;
    if (batch == 1 && K >= 512 && t128 < CUS) {
        /* few output tiles, long K: split K across workgroups */
        tile = T_128x128;
        splits = cdiv(2 * CUS, t128);
        if (splits > K / 256) splits = K / 256;
        if (splits > 32) splits = 32;
        if (splits < 1) splits = 1;
    } else if (t128 >= 2 * CUS) {
        tile = T_128x128;
    } else if (t64x128 >= 2 * CUS) {
        tile = T_64x128;
    } else {
        tile = T_64x64;
    }
    p.tiles_m = cdiv(M, TILE_BM[tile]);
    p.tiles_n = cdiv(N, TILE_BN[tile]);
    if (splits > 1) {
        int kchunk = cdiv(cdiv(K, splits), GBK) * GBK;
        splits = cdiv(K, kchunk);
    }
    snprintf(e->last, sizeof(e->last), "k_gemm_%s_%s", LAYOUT_NAME[layout], TILE_NAME[tile]);
    e->last_splits = splits;
    if (splits <= 1) {
        launch(e->k[layout][tile], &p, batch);
        return;
    }
    /* split-K: raw partials into the workspace, then an ordered reduction */
    u64 need = (u64)splits * (u64)M * (u64)N;
    if (need > e->ws_floats) {
        if (e->ws) hip_free(e->ws);
        e->ws = hip_alloc(need * sizeof(f32));
        e->ws_floats = need;
    }
    GemmParams q = p;
    q.C = (float*)e->ws;
    q.ldc = N;
    q.sW = (long long)M * N;
    q.kchunk = cdiv(cdiv(K, splits), GBK) * GBK;
    q.splits = splits;
    q.alpha = 1.0f; q.beta = 0.0f; q.bias = NULL; q.resid = NULL;
    launch(e->k[layout][tile], &q, (u32)splits);
    long long total = (long long)M * N;
    hipDeviceptr_t W = e->ws;
    i32 sp = splits;
    i64 sW = (i64)M * N;
    void* args[] = { &W, &sp, &sW, &C, &M, &N, &ldc, &alpha, &beta, &bias, &resid, &ldr };
    hip_launch(e->reduce, (u32)((total + 255) / 256), 1, 1, 256, 1, 1, 0, args);
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
