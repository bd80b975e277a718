/* kernel_params.h -- argument blocks of the kernels that take a struct by
 * value, shared by the kernels (the .hip files under kernels) and the host code that fills
 * them (trlm_gemm.c, gpu_train.c, gpu_decode.c): one definition, so the
 * bytes the host passes and the layout the kernel reads cannot disagree.
 * Plain C types only; the same text compiles as C and as HIP C++. */
#ifndef TRLM_KERNEL_PARAMS_H
#define TRLM_KERNEL_PARAMS_H

/* GEMM engine (kernels/gemm.hip, host trlm_gemm.c) */
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
    float* stats;      // optional: per-row (max, sum exp(v - max)) of each wave's columns
    int stats_ld;      // float2 entries per row of stats
    float* csum;       // optional (TB = 0): column sums of B over k (a bias gradient);
                       // with split-K each split writes its partial as row M of its slab
    const float* rope_cos;   // optional: RoPE on columns [0, rope_cols) (see rope4)
    const float* rope_sin;
    int rope_T, rope_hd, rope_cols;
    const unsigned* tgt;     // optional, with stats: row m's target column; its value goes
    float* tgt_val;          // to tgt_val[m] (the cross-entropy's z[t])
    int no_store;            // with stats: C is not written (the statistics are the output)
    float* glu_h;            // optional (SwiGLU epilogue, k_gemm_nn_64x64_k32_glu): h [M, glu_F] =
    int glu_F;               // silu(gate) * up of C = [gate | up] (N = 2 * glu_F), C still written
} GemmParams;

/* Flash attention (kernels/attention.hip, host gpu_train.c) */
typedef struct AttnParams {
    const float* qkv;  // [B*T, ldq]
    float* out;        // forward: O [B*T, ldo]; backward: dqkv [B*T, ldq]
    const float* O;    // backward: O [B*T, ldo]
    const float* dO;   // backward: dO [B*T, ldo]
    float* lse;        // [B*H*T] base-2 log-sum-exp of scaled scores
    float* dvec;       // [B*H*T] D_i = <dO_i, O_i>
    int B, T, H, D;
    int ldq, ldo;
    float scale;       // 1/sqrt(HD)
    // backward: when set, dQ and dK leave through the transpose of the RoPE
    // rotation (tables [T][HD/2]), so dqkv is the gradient of the un-rotated
    // projection
    const float* rope_cos;
    const float* rope_sin;
    // backward: the dK/dV pass leaves every causal 64x64 block of
    // dS = P o (dP - D) * scale here for the dQ pass: [B*H][nqb(nqb+1)/2]
    // blocks (query block i, key block j <= i at i(i+1)/2 + j), each in the
    // dK/dV pass's register order [key group g][query half c][r][lane]: key
    // 32g + l%32, query 32c + 8(r/4) + 4(l/32) + r%4 (one 256-byte row per r)
    float* ds;
    // forward, optional: the job of workgroup L = blockIdx.y * gridDim.x +
    // blockIdx.x as query block << 16 | (batch * H + head); without it the
    // kernel takes its jobs in its own longest-first snake order
    const int* jobs;
} AttnParams;

/* Fused decode GEMMs and head (kernels/decode_fused.hip, host gpu_decode.c) */
typedef struct DecGemmParams {
    const float* A;          // [M, lda] (unused when a_ids)
    const unsigned* ids;     // token ids [M] for a_ids / resid_ids
    const float* E;          // embedding table [V, D] for ids
    int a_ids;               // row m of A is E[ids[m]] (layer 0's input), row stride lda
    int lda;
    const float* W;          // NN: [K, ldw]; NT: [N, ldw] (the head's E)
    int ldw;
    const float* bias;       // [N] or null
    const float* norm_w;     // RMSNorm weight [K] (kernels with the norm prologue)
    float eps;
    const float* resid;      // [M, ldr] or null
    int resid_ids;           // row m of resid is E[ids[m]] (layer 0), row stride ldr
    int ldr;
    float* C;                // [M, ldc]
    int ldc;
    int M, N, K;
    int ncb;                 // column blocks of 16
    int F;                   // SwiGLU: the up half starts at column F; h has F columns
    const float* cos_t;      // QKV: RoPE tables [ctx][hd/2]
    const float* sin_t;
    const int* pos;          // the token's position (device-resident)
    int H, hd, D;
    float* kc;               // this layer's caches [M][H][ctx][hd]
    float* vc;
    int ctx;
    int* pos_inc;            // head: block 0 adds 1 to *pos_inc after its stores
    float scale;             // QKV + attention: the score scale 1/sqrt(hd)
} DecGemmParams;

#endif /* TRLM_KERNEL_PARAMS_H */
