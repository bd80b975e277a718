// attention.hip -- causal attention on FP32 matrix cores, flash style.
//
// Replaces the reference's materialised-P attention (QK^T GEMM, in-place
// masked softmax, PV GEMM and their backward: train_kernels.cu:631-664,
// gpu_train.c:346-353,445-455) with kernels that never store P:
//   forward : S = QK^T*scale, online softmax, O = PV; saves the per-row
//             log-sum-exp (base 2) for the backward;
//   backward: D_i = <dO_i, O_i>; dK,dV over key blocks; dQ over query blocks.
// Masked entries (j > i) are exactly zero in the reference (exp of -1e9 is 0,
// mathlib.c:142), so key blocks above the diagonal are skipped outright.
// No atomics: dQ is produced by its own pass instead of being accumulated
// across key blocks, so results are bit-identical run to run.
//
// Layout: Q, K, V are read straight from qkv [B*T, ld] (head h at columns
// h*HD, D+h*HD, 2D+h*HD, RoPE already applied) and O is written straight
// into att [B*T, D] at columns h*HD -- no head split/merge passes.
//
// MFMA mapping (v_mfma_f32_32x32x2f32, lane l, register r):
//   A operand: A[l%32][k], B operand: B[k][l%32], k = step pair (l/32);
//   result   : D[8*(r/4) + 4*(l/32) + r%4][l%32].
// Computing S^T = K Q^T puts one query per lane (column) and its keys in the
// lane's registers, so row max / sum need no cross-lane work except one
// exchange with lane l^32; the exponentiated S^T registers are then directly
// the B operand of O^T += V^T P^T, step r using register r.
#include "common.h"

#define ATT_LOG2E 1.4426950408889634f

struct AttnParams {
    const float* qkv;  // [B*T, ldq]
    float* out;        // forward: O [B*T, ldo]; backward: dqkv [B*T, ldq]
    const float* O;    // backward: O [B*T, ldo]
    const float* dO;   // backward: dO [B*T, ldo]
    float* lse;        // [B*H*T] base-2 log-sum-exp of scaled scores
    float* dvec;       // [B*H*T] D_i = <dO_i, O_i>
    int B, T, H, D;
    int ldq, ldo;
    float scale;       // 1/sqrt(HD)
};

// Load a [64 rows x HD] tile (rows r0.., columns col0..) of a row-major
// matrix with row stride ld into registers (rows >= rlim read as 0).
template <int HD>
__device__ __forceinline__ void att_load(const float* base, int ld, int r0, int rlim, int col0, f32x4* regs) {
    constexpr int NQ = 64 * HD / 4 / 256;   // float4 per thread
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        int idx = threadIdx.x + i * 256;
        int r = idx / (HD / 4), c = (idx % (HD / 4)) * 4;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (r0 + r < rlim) v = *(const f32x4*)(base + (long long)(r0 + r) * ld + col0 + c);
        regs[i] = v;
    }
}

template <int HD>
__device__ __forceinline__ void att_store_lds(float* lds, const f32x4* regs) {
    constexpr int NQ = 64 * HD / 4 / 256;
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        int idx = threadIdx.x + i * 256;
        int r = idx / (HD / 4), c = (idx % (HD / 4)) * 4;
        *(f32x4*)(lds + r * (HD + 4) + c) = regs[i];
    }
}

// Row-fragment of 32 rows for the d-steps of chunk j: lane l gets
// X[rb + l%32][8j + 4*(l/32) + s], s = 0..3.
template <int HD>
__device__ __forceinline__ f32x4 att_frag(const float* lds, int rb, int j, int lane) {
    return *(const f32x4*)(lds + (rb + (lane & 31)) * (HD + 4) + 8 * j + 4 * (lane >> 5));
}

// Same fragment straight from global memory (for per-wave register operands).
template <int HD>
__device__ __forceinline__ void att_frag_global(const float* base, int ld, int row, bool valid, int col0, int lane,
                                                f32x4* out) {
#pragma unroll
    for (int j = 0; j < HD / 8; j++) {
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (valid) v = *(const f32x4*)(base + (long long)row * ld + col0 + 8 * j + 4 * (lane >> 5));
        out[j] = v;
    }
}

// =========================================================== forward
template <int HD>
__device__ void flash_fwd(const AttnParams& p) {
    constexpr int DB = (HD + 31) / 32;         // 32-row d blocks of O^T
    constexpr int NQ = 64 * HD / 4 / 256;
    constexpr int LD = HD + 4;
    __shared__ __attribute__((aligned(16))) float Ks[64 * LD];
    __shared__ __attribute__((aligned(16))) float Vs[64 * LD];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5;
    const int nqb = (p.T + 127) / 128;
    const int qb = nqb - 1 - (int)blockIdx.x;   // heavy (late) query blocks first
    const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
    const long long rowbase = (long long)b * p.T;
    const float* qkv = p.qkv + rowbase * p.ldq;
    const int qcol = h * HD, kcol = p.D + h * HD, vcol = 2 * p.D + h * HD;

    const int qw0 = qb * 128 + wave * 32;       // first query of this wave
    const int qpos = qw0 + (lane & 31);         // this lane's query
    const float c2 = p.scale * ATT_LOG2E;

    f32x4 qf[HD / 8];
    att_frag_global<HD>(qkv, p.ldq, qpos, qpos < p.T, qcol, lane, qf);

    f32x16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[d][r] = 0.f;
    float m = -INFINITY, l = 0.f;

    int kv_end = (qb + 1) * 128;
    if (kv_end > p.T) kv_end = p.T;
    const int nkv = (kv_end + 63) / 64;

    f32x4 rk[NQ], rv[NQ];
    att_load<HD>(qkv, p.ldq, 0, p.T, kcol, rk);
    att_load<HD>(qkv, p.ldq, 0, p.T, vcol, rv);
    for (int kb = 0; kb < nkv; kb++) {
        const int kv0 = kb * 64;
        __syncthreads();
        att_store_lds<HD>(Ks, rk);
        att_store_lds<HD>(Vs, rv);
        __syncthreads();
        if (kb + 1 < nkv) {
            att_load<HD>(qkv, p.ldq, kv0 + 64, p.T, kcol, rk);
            att_load<HD>(qkv, p.ldq, kv0 + 64, p.T, vcol, rv);
        }
        if (kv0 > qw0 + 31) continue;           // fully above the diagonal for this wave

        // S^T = K Q^T for two 32-key sub-blocks
        f32x16 s[2];
#pragma unroll
        for (int c = 0; c < 2; c++) {
#pragma unroll
            for (int r = 0; r < 16; r++) s[c][r] = 0.f;
#pragma unroll
            for (int j = 0; j < HD / 8; j++) {
                f32x4 kf = att_frag<HD>(Ks, c * 32, j, lane);
#pragma unroll
                for (int t = 0; t < 4; t++) s[c] = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[t], qf[j][t], s[c], 0, 0, 0);
            }
        }
        // scale to base-2 units, mask, running max
        const bool diag = (kv0 + 63 > qw0);
        float mx = m;
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int kpos = kv0 + c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                float v = s[c][r] * c2;
                if (diag && kpos > qpos) v = -INFINITY;
                s[c][r] = v;
                mx = fmaxf(mx, v);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
        const float alpha = exp2f(m - mx);      // m = -inf on the first block -> 0
        m = mx;
        float ls = 0.f;
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float e = exp2f(s[c][r] - mx);
                s[c][r] = e;
                ls += e;
            }
        l = l * alpha + ls;
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[d][r] *= alpha;
        // O^T += V^T P^T
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int kr = c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
#pragma unroll
                for (int d = 0; d < DB; d++) {
                    const int dc = d * 32 + (lane & 31);
                    float vv = (dc < HD) ? Vs[kr * LD + dc] : 0.f;
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vv, s[c][r], o[d], 0, 0, 0);
                }
            }
    }
    l = l + __shfl_xor(l, 32, WAVE);
    if (qpos < p.T) {
        const float inv = 1.0f / l;
        float* orow = p.out + (rowbase + qpos) * p.ldo + qcol;
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d0 = d * 32 + 8 * g + 4 * half;
                if (d0 < HD) {
                    f32x4 v = {o[d][4 * g] * inv, o[d][4 * g + 1] * inv, o[d][4 * g + 2] * inv, o[d][4 * g + 3] * inv};
                    *(f32x4*)(orow + d0) = v;
                }
            }
        if (half == 0) p.lse[(long long)bh * p.T + qpos] = m + __log2f(l);
    }
}

// =========================================================== backward prep
// D_i = sum_d dO[i,d] * O[i,d] for every (row, head).
extern "C" __global__ void __launch_bounds__(256) k_attn_bwd_prep(AttnParams p) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)p.B * p.T * p.H;
    if (i >= total) return;
    int h = (int)(i % p.H);
    long long n = i / p.H;
    int hd = p.D / p.H;
    const float* a = p.O + n * p.ldo + h * hd;
    const float* g = p.dO + n * p.ldo + h * hd;
    float s = 0.f;
    for (int d = 0; d < hd; d++) s += a[d] * g[d];
    long long b = n / p.T, t = n - b * p.T;
    p.dvec[(b * p.H + h) * p.T + t] = s;
}

// =========================================================== backward dK, dV
// Workgroup: 128 keys (4 waves x 32); loops over 64-query blocks at or below
// the diagonal.  S and dP are formed as [q x kv] (one key per lane), so the
// exponentiated P and dS registers feed dV^T += dO^T P and dK^T += Q^T dS.
template <int HD>
__device__ void flash_bwd_dkv(const AttnParams& p) {
    constexpr int DB = (HD + 31) / 32;
    constexpr int NQ = 64 * HD / 4 / 256;
    constexpr int LD = HD + 4;
    __shared__ __attribute__((aligned(16))) float Qs[64 * LD];
    __shared__ __attribute__((aligned(16))) float Gs[64 * LD];   // dO tile
    __shared__ float Ls[64], Ds[64];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5;
    const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
    const long long rowbase = (long long)b * p.T;
    const float* qkv = p.qkv + rowbase * p.ldq;
    const float* dO = p.dO + rowbase * p.ldo;
    const int qcol = h * HD, kcol = p.D + h * HD, vcol = 2 * p.D + h * HD;
    const float* lse = p.lse + (long long)bh * p.T;
    const float* dv = p.dvec + (long long)bh * p.T;
    const float c2 = p.scale * ATT_LOG2E;

    const int kw0 = blockIdx.x * 128 + wave * 32;
    const int kpos = kw0 + (lane & 31);
    f32x4 kf[HD / 8], vf[HD / 8];
    att_frag_global<HD>(qkv, p.ldq, kpos, kpos < p.T, kcol, lane, kf);
    att_frag_global<HD>(qkv, p.ldq, kpos, kpos < p.T, vcol, lane, vf);

    f32x16 dk[DB], dvv[DB];
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) { dk[d][r] = 0.f; dvv[d][r] = 0.f; }

    const int q_begin = (blockIdx.x * 128) / 64;
    const int nqb = (p.T + 63) / 64;
    f32x4 rq[NQ], rg[NQ];
    float rl = 0.f, rd = 0.f;
    auto gload = [&](int qb) {
        att_load<HD>(qkv, p.ldq, qb * 64, p.T, qcol, rq);
        att_load<HD>(dO, p.ldo, qb * 64, p.T, qcol, rg);
        if (threadIdx.x < 64) {
            int q = qb * 64 + threadIdx.x;
            rl = (q < p.T) ? lse[q] : 0.f;
            rd = (q < p.T) ? dv[q] : 0.f;
        }
    };
    if (q_begin < nqb) gload(q_begin);
    for (int qb = q_begin; qb < nqb; qb++) {
        const int q0 = qb * 64;
        __syncthreads();
        att_store_lds<HD>(Qs, rq);
        att_store_lds<HD>(Gs, rg);
        if (threadIdx.x < 64) { Ls[threadIdx.x] = rl; Ds[threadIdx.x] = rd; }
        __syncthreads();
        if (qb + 1 < nqb) gload(qb + 1);
        if (q0 + 63 < kw0) continue;            // every query precedes every key of this wave

#pragma unroll
        for (int c = 0; c < 2; c++) {           // 32-query sub-blocks
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; r++) { s[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
            for (int j = 0; j < HD / 8; j++) {
                f32x4 qa = att_frag<HD>(Qs, c * 32, j, lane);
                f32x4 ga = att_frag<HD>(Gs, c * 32, j, lane);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[t], kf[j][t], s, 0, 0, 0);
                    dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga[t], vf[j][t], dp, 0, 0, 0);
                }
            }
            // P and dS for rows q = q0 + c*32 + 8*(r/4) + 4*half + r%4, column = this lane's key
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int ql = c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                const int qpos = q0 + ql;
                float pr = exp2f(s[r] * c2 - Ls[ql]);
                if (kpos > qpos || qpos >= p.T) pr = 0.f;
                s[r] = pr;
                dp[r] = pr * (dp[r] - Ds[ql]) * p.scale;
            }
            // dV^T += dO^T P ; dK^T += Q^T dS   (step r uses register r)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int ql = c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
#pragma unroll
                for (int d = 0; d < DB; d++) {
                    const int dc = d * 32 + (lane & 31);
                    float ga = (dc < HD) ? Gs[ql * LD + dc] : 0.f;
                    float qa = (dc < HD) ? Qs[ql * LD + dc] : 0.f;
                    dvv[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(ga, s[r], dvv[d], 0, 0, 0);
                    dk[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(qa, dp[r], dk[d], 0, 0, 0);
                }
            }
        }
    }
    if (kpos < p.T) {
        float* row = p.out + (rowbase + kpos) * p.ldq;
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d0 = d * 32 + 8 * g + 4 * half;
                if (d0 < HD) {
                    f32x4 a = {dk[d][4 * g], dk[d][4 * g + 1], dk[d][4 * g + 2], dk[d][4 * g + 3]};
                    f32x4 v = {dvv[d][4 * g], dvv[d][4 * g + 1], dvv[d][4 * g + 2], dvv[d][4 * g + 3]};
                    *(f32x4*)(row + kcol + d0) = a;
                    *(f32x4*)(row + vcol + d0) = v;
                }
            }
    }
}

// =========================================================== backward dQ
// Workgroup: 128 queries (4 waves x 32); loops over 64-key blocks up to the
// diagonal.  S^T and dP^T put one query per lane; dQ^T += K^T dS^T.
template <int HD>
__device__ void flash_bwd_dq(const AttnParams& p) {
    constexpr int DB = (HD + 31) / 32;
    constexpr int NQ = 64 * HD / 4 / 256;
    constexpr int LD = HD + 4;
    __shared__ __attribute__((aligned(16))) float Ks[64 * LD];
    __shared__ __attribute__((aligned(16))) float Vs[64 * LD];

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5;
    const int nqb = (p.T + 127) / 128;
    const int qb = nqb - 1 - (int)blockIdx.x;
    const int bh = blockIdx.y, b = bh / p.H, h = bh - b * p.H;
    const long long rowbase = (long long)b * p.T;
    const float* qkv = p.qkv + rowbase * p.ldq;
    const float* dO = p.dO + rowbase * p.ldo;
    const int qcol = h * HD, kcol = p.D + h * HD, vcol = 2 * p.D + h * HD;
    const float c2 = p.scale * ATT_LOG2E;

    const int qw0 = qb * 128 + wave * 32;
    const int qpos = qw0 + (lane & 31);
    const bool qvalid = qpos < p.T;
    f32x4 qf[HD / 8], gf[HD / 8];
    att_frag_global<HD>(qkv, p.ldq, qpos, qvalid, qcol, lane, qf);
    att_frag_global<HD>(dO, p.ldo, qpos, qvalid, qcol, lane, gf);
    const float lq = qvalid ? p.lse[(long long)bh * p.T + qpos] : 0.f;
    const float dq_i = qvalid ? p.dvec[(long long)bh * p.T + qpos] : 0.f;

    f32x16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[d][r] = 0.f;

    int kv_end = (qb + 1) * 128;
    if (kv_end > p.T) kv_end = p.T;
    const int nkv = (kv_end + 63) / 64;
    f32x4 rk[NQ], rv[NQ];
    att_load<HD>(qkv, p.ldq, 0, p.T, kcol, rk);
    att_load<HD>(qkv, p.ldq, 0, p.T, vcol, rv);
    for (int kb = 0; kb < nkv; kb++) {
        const int kv0 = kb * 64;
        __syncthreads();
        att_store_lds<HD>(Ks, rk);
        att_store_lds<HD>(Vs, rv);
        __syncthreads();
        if (kb + 1 < nkv) {
            att_load<HD>(qkv, p.ldq, kv0 + 64, p.T, kcol, rk);
            att_load<HD>(qkv, p.ldq, kv0 + 64, p.T, vcol, rv);
        }
        if (kv0 > qw0 + 31) continue;
#pragma unroll
        for (int c = 0; c < 2; c++) {
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; r++) { s[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
            for (int j = 0; j < HD / 8; j++) {
                f32x4 ka = att_frag<HD>(Ks, c * 32, j, lane);
                f32x4 va = att_frag<HD>(Vs, c * 32, j, lane);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(ka[t], qf[j][t], s, 0, 0, 0);
                    dp = __builtin_amdgcn_mfma_f32_32x32x2f32(va[t], gf[j][t], dp, 0, 0, 0);
                }
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int kpos = kv0 + c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                float pr = exp2f(s[r] * c2 - lq);
                if (kpos > qpos) pr = 0.f;
                dp[r] = pr * (dp[r] - dq_i) * p.scale;
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int kr = c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
#pragma unroll
                for (int d = 0; d < DB; d++) {
                    const int dc = d * 32 + (lane & 31);
                    float ka = (dc < HD) ? Ks[kr * LD + dc] : 0.f;
                    acc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(ka, dp[r], acc[d], 0, 0, 0);
                }
            }
        }
    }
    if (qvalid) {
        float* row = p.out + (rowbase + qpos) * p.ldq + qcol;
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const int d0 = d * 32 + 8 * g + 4 * half;
                if (d0 < HD) {
                    f32x4 v = {acc[d][4 * g], acc[d][4 * g + 1], acc[d][4 * g + 2], acc[d][4 * g + 3]};
                    *(f32x4*)(row + d0) = v;
                }
            }
    }
}

#define ATT_KERNELS(HD)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) k_attn_fwd_hd##HD(AttnParams p) { flash_fwd<HD>(p); } \
    extern "C" __global__ void __launch_bounds__(256) k_attn_bwd_dkv_hd##HD(AttnParams p) {              \
        flash_bwd_dkv<HD>(p);                                                                             \
    }                                                                                                     \
    extern "C" __global__ void __launch_bounds__(256) k_attn_bwd_dq_hd##HD(AttnParams p) { flash_bwd_dq<HD>(p); }

ATT_KERNELS(16)
ATT_KERNELS(32)
ATT_KERNELS(64)
ATT_KERNELS(128)
