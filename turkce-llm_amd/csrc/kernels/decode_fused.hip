// decode_fused.hip -- the KV-cache decode step as four kernels per layer.
//
// A decode step runs the model on one new token per sequence: every product
// has only `batch` rows (64 in the benchmark), so the step is bound by
// latency and HBM, not by the matrix cores.  The reference computes it as
// the full-window lm_forward (training/generate.c:186-212); within the
// context the last row needs only the cached keys and values, so a step is:
//   k_dec_qkv_attn  per head and pair of sequences: RMSNorm(x) @ Wqkv + b
//               for the head's columns, RoPE on q and k at the position, k
//               and v appended to the cache, then q over the cached keys and
//               the new one, 4 waves per sequence splitting the context,
//               merged in wave order                   (layer 0: x = E[ids])
//   k_dec_out   x2 = x + (att @ Wo + bo)
//   k_dec_gu    h = SwiGLU(RMSNorm(x2) @ Wgu + bgu)
//   k_dec_down  x = x2 + (h @ Wd + bd)
//   k_dec_head_k*  logits = RMSNorm(x) @ E^T, then the position moves on
//
// GEMM tiling.  The output is cut into 16 x 16 blocks, one per workgroup
// (two for the gate/up pair), so even a 64-row product spreads over
// hundreds of CUs; the workgroup's KW waves split K, each accumulating its
// share with v_mfma_f32_16x16x4f32, and the partial blocks are added in wave
// order through LDS.  Workgroups are mapped so that each XCD takes a
// contiguous range of column blocks (the weight slices it streams share its
// L2 with its neighbours').  Operands are read straight from global memory,
// 16 bytes per lane: lane (i, kq) of a wave holds A[row i][k0 + 4kq .. +3]
// and feeds component u to MFMA step u, i.e. the MFMA's k index kq at step u
// stands for k0 + 4kq + u; the B operand is read with the same mapping, so
// the dot products are unchanged.
//
// RMSNorm is applied as out[m, n] = r[m] * sum_k (x[m, k] w[k]) W[k, n] with
// r = 1/sqrt(mean(x^2) + eps) taken in f64 (as the reference's
// k_rmsnorm_fwd), the waves' sums of squares added in wave order.
#include "common.h"

typedef float f32x4_t __attribute__((ext_vector_type(4)));

#define DEC_LOG2E_F 1.4426950408889634f

enum { DM_PLAIN = 0, DM_SWIGLU = 2 };

// Argument block of the fused GEMMs; layout mirrored by DecGemmParams in
// gpu_decode.c.
#include "../kernel_params.h"   // GemmParams, AttnParams, DecGemmParams

__device__ __forceinline__ f32x4_t ld4(const float* p) { return *(const f32x4_t*)p; }
// a streamed load (the KV cache is read once per step): the non-temporal hint
// keeps it from displacing the weights the step's GEMMs re-read from cache
__device__ __forceinline__ f32x4_t ld4_stream(const float* p) { return __builtin_nontemporal_load((const f32x4_t*)p); }

template <int KW, int RB, bool NT, int MODE, bool NORM>
__device__ __forceinline__ void dec_gemm(const DecGemmParams& p) {
    constexpr int NACC = (MODE == DM_SWIGLU) ? 2 : 1;   // gate and up blocks
    __shared__ float red[KW][RB * NACC][4][64];
    __shared__ float ssq[KW][RB * 16];
    __shared__ float rn[RB * 16];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int li = lane & 15, kq = lane >> 4;

    // workgroup -> (row tile, column block): XCD x = blockIdx.x % 8 takes a
    // contiguous range of column blocks, its row tiles next to each other
    const int nrt = (p.M + 16 * RB - 1) / (16 * RB);
    const int total = nrt * p.ncb;
    const int per_xcd = (total + 7) >> 3;
    const int t = (blockIdx.x & 7) * per_xcd + (blockIdx.x >> 3);
    if (t >= total) return;
    const int rt = t % nrt, cb = t / nrt;
    const int m0 = rt * 16 * RB;

    // this wave's k range: a multiple of 16 per wave
    const int kper = (((p.K + KW - 1) / KW) + 15) & ~15;
    const int k0 = w * kper;
    int k1 = k0 + kper;
    if (k1 > p.K) k1 = p.K;

    // A rows this lane reads (clamped to valid rows; their results are not stored)
    const float* arow[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        int m = m0 + 16 * rb + li;
        if (m > p.M - 1) m = p.M - 1;
        arow[rb] = p.a_ids ? p.E + (long long)p.ids[m] * p.lda : p.A + (long long)m * p.lda;
    }
    // B columns this lane reads (clamped; masked below)
    const int ncols = (MODE == DM_SWIGLU) ? p.F : p.N;
    const int c = 16 * cb + li;
    const bool cvalid = c < ncols;
    int bcol[NACC];
    bcol[0] = cvalid ? c : 0;
    if (NACC == 2) bcol[NACC - 1] = cvalid ? p.F + c : 0;

    // wave 0's epilogue inputs, loaded now so they arrive with the operands:
    // bias and residual rows (this lane's 4 rows per row block)
    // No load sits under a per-element branch: a branch that joins after a
    // load makes the join wait for it, which chained these loads one after
    // another in front of the operand stream.
    float ebias[NACC], eres[RB][4];
    if (w == 0) {
        // any valid address when there is no bias (the value is then not
        // used: the epilogue selects 0, so nothing waits for it here)
        const float* bsrc = p.bias ? p.bias : p.W;
#pragma unroll
        for (int a = 0; a < NACC; a++) ebias[a] = bsrc[bcol[a]];
#pragma unroll
        for (int rb = 0; rb < RB; rb++)
#pragma unroll
            for (int r = 0; r < 4; r++) eres[rb][r] = 0.f;
        if (MODE == DM_PLAIN && p.resid_ids) {
            unsigned id[RB][4];
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + 16 * rb + 4 * kq + r;
                    id[rb][r] = p.ids[m < p.M ? m : p.M - 1];
                }
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int r = 0; r < 4; r++) eres[rb][r] = p.E[(long long)id[rb][r] * p.ldr + bcol[0]];
        } else if (MODE == DM_PLAIN && p.resid) {
#pragma unroll
            for (int rb = 0; rb < RB; rb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + 16 * rb + 4 * kq + r;
                    eres[rb][r] = p.resid[(long long)(m < p.M ? m : p.M - 1) * p.ldr + bcol[0]];
                }
        }
    }

    f32x4_t acc[RB][NACC];
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int a = 0; a < NACC; a++) acc[rb][a] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    float ss[RB];
#pragma unroll
    for (int rb = 0; rb < RB; rb++) ss[rb] = 0.f;

    // batches of up to 8 k-blocks of 16: every load of a batch is issued
    // (unconditionally, from clamped valid addresses) before any of its
    // arithmetic -- a load under a branch would be waited for inside it --
    // then lanes past K or N are zeroed, the norm weight applied, and the
    // MFMAs issued
    for (int kb = k0; kb < k1; kb += 128) {
        f32x4_t av[8][RB];
        f32x4_t bv[8][NACC];
        f32x4_t nw[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = kb + 16 * j + 4 * kq;
            const int ks = k < k1 ? k : 0;
#pragma unroll
            for (int rb = 0; rb < RB; rb++) av[j][rb] = ld4(arow[rb] + ks);
#pragma unroll
            for (int a = 0; a < NACC; a++) {
                if (NT) {
                    bv[j][a] = ld4(p.W + (long long)bcol[a] * p.ldw + ks);
                } else {
                    const float* wp = p.W + (long long)ks * p.ldw + bcol[a];
#pragma unroll
                    for (int u = 0; u < 4; u++) bv[j][a][u] = wp[(long long)u * p.ldw];
                }
            }
            if (NORM) nw[j] = ld4(p.norm_w + ks);
        }
        const f32x4_t zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const bool kv = kb + 16 * j + 4 * kq < k1;
#pragma unroll
            for (int rb = 0; rb < RB; rb++) {
                const f32x4_t x = kv ? av[j][rb] : zero;
                if (NORM) {
                    ss[rb] += x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3];
                    av[j][rb] = x * nw[j];
                } else {
                    av[j][rb] = x;
                }
            }
#pragma unroll
            for (int a = 0; a < NACC; a++) bv[j][a] = (kv && cvalid) ? bv[j][a] : zero;
        }
#pragma unroll
        for (int j = 0; j < 8; j++)
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int rb = 0; rb < RB; rb++)
#pragma unroll
                    for (int a = 0; a < NACC; a++)
                        acc[rb][a] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[j][rb][u], bv[j][a][u], acc[rb][a], 0, 0, 0);
    }

    // partial blocks -> LDS; wave 0 adds them in wave order
#pragma unroll
    for (int rb = 0; rb < RB; rb++)
#pragma unroll
        for (int a = 0; a < NACC; a++)
#pragma unroll
            for (int r = 0; r < 4; r++) red[w][rb * NACC + a][r][lane] = acc[rb][a][r];
    if (NORM) {
        // sum of squares of row li over this wave's k range: the four kq lane groups
#pragma unroll
        for (int rb = 0; rb < RB; rb++) {
            float s = ss[rb];
            s += __shfl_xor(s, 16, WAVE);
            s += __shfl_xor(s, 32, WAVE);
            if (kq == 0) ssq[w][rb * 16 + li] = s;
        }
    }
    __syncthreads();
    if (NORM && threadIdx.x < RB * 16) {
        float s = ssq[0][threadIdx.x];
#pragma unroll
        for (int q = 1; q < KW; q++) s += ssq[q][threadIdx.x];
        rn[threadIdx.x] = 1.0f / (float)sqrt((double)(s / (float)p.K + p.eps));
    }
    __syncthreads();
    if (w != 0) return;

#pragma unroll
    for (int rb = 0; rb < RB; rb++) {
        float v[NACC][4];
#pragma unroll
        for (int a = 0; a < NACC; a++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float s = red[0][rb * NACC + a][r][lane];
#pragma unroll
                for (int q = 1; q < KW; q++) s += red[q][rb * NACC + a][r][lane];
                v[a][r] = s;
            }
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int mrow = 16 * rb + 4 * kq + r;   // row within the tile (result layout of the MFMA)
            const int m = m0 + mrow;
            const float scale = NORM ? rn[mrow] : 1.0f;
            float o[NACC];
#pragma unroll
            for (int a = 0; a < NACC; a++) o[a] = v[a][r] * scale + (p.bias ? ebias[a] : 0.f);
            if (MODE == DM_SWIGLU) {
                const float g = o[0], u = o[NACC - 1];
                const float sg = 1.0f / (1.0f + expf(-g));
                if (m < p.M && cvalid) p.C[(long long)m * p.ldc + c] = (g * sg) * u;
            } else {
                if (m < p.M && cvalid) p.C[(long long)m * p.ldc + c] = (p.resid || p.resid_ids) ? eres[rb][r] + o[0] : o[0];
            }
        }
    }
    if (p.pos_inc && blockIdx.x == 0 && threadIdx.x == 0) *p.pos_inc = *p.pos_inc + 1;
}

extern "C" __global__ void __launch_bounds__(256) k_dec_out(DecGemmParams p) { dec_gemm<4, 1, false, DM_PLAIN, false>(p); }
extern "C" __global__ void __launch_bounds__(256) k_dec_gu(DecGemmParams p) { dec_gemm<4, 1, false, DM_SWIGLU, true>(p); }
extern "C" __global__ void __launch_bounds__(512) k_dec_down(DecGemmParams p) { dec_gemm<8, 1, false, DM_PLAIN, false>(p); }

// ---------------------------------------------------------------- LM head
// logits[m, n] = sum_k (x[m, k] r[m] w[k]) E[n, k] for the (up to) 64 rows of
// row tile blockIdx.y, with r the row's RMSNorm reciprocal.  A persistent
// grid of 8-wave workgroups, wave w of workgroup g taking the 16-column
// blocks of E g*8 + w, g*8 + w + 8*grid, ...  Every wave first issues all its
// loads: its 8 rows of x, then the whole first column block of E (NKB
// 16-deep steps, one f32x4 per lane each), so the E stream has the block in
// flight while the rows are normalised into LDS (x was issued first, so the
// in-order memory counter lets the staging start before E arrives).  Then
// four 16-row MFMA blocks share every E fragment.  LDS rows are padded by 4
// floats so the 16 rows of a fragment read fall in different banks.
// K <= 16*NKB <= DEC_HEAD_KMAX, K % 16 == 0.
#define DEC_HEAD_KMAX 512
#define DEC_HEAD_WAVES 8
template <int NKB>
__device__ __forceinline__ void dec_head(const DecGemmParams& p) {
    constexpr int LDK = DEC_HEAD_KMAX + 4;
    constexpr int RPW = 64 / DEC_HEAD_WAVES;   // rows staged per wave
    __shared__ float xs[64 * LDK];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int li = lane & 15, kq = lane >> 4;
    const int m0 = blockIdx.y * 64;
    const int K = p.K, K4 = K >> 2;   // K4 <= 128: two float4 per lane and row
    const int nwaves = gridDim.x * DEC_HEAD_WAVES;

    // this wave's rows w, w + 8, ... and the norm weight (clamped loads)
    // (the row addresses are formed first, under one branch on a_ids: a
    // per-row branch around the id load made every row wait for the rows
    // before it)
    f32x4_t xv[RPW][2], nw[2];
    const float* xr[RPW];
    if (p.a_ids) {
        unsigned id[RPW];
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int m = m0 + w + DEC_HEAD_WAVES * r;
            id[r] = p.ids[m < p.M ? m : p.M - 1];
        }
#pragma unroll
        for (int r = 0; r < RPW; r++) xr[r] = p.E + (long long)id[r] * p.lda;
    } else {
#pragma unroll
        for (int r = 0; r < RPW; r++) {
            const int m = m0 + w + DEC_HEAD_WAVES * r;
            xr[r] = p.A + (long long)(m < p.M ? m : p.M - 1) * p.lda;
        }
    }
#pragma unroll
    for (int r = 0; r < RPW; r++)
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int q = lane + 64 * t;
            xv[r][t] = ld4(xr[r] + 4 * (q < K4 ? q : 0));
        }
#pragma unroll
    for (int t = 0; t < 2; t++) {
        const int q = lane + 64 * t;
        nw[t] = ld4(p.norm_w + 4 * (q < K4 ? q : 0));
    }
    // the first column block of E, whole (steps past K load step 0 and are skipped)
    int cb = blockIdx.x * DEC_HEAD_WAVES + w;
    f32x4_t ev[NKB];
    auto eload = [&](int blk) {
        int c = 16 * blk + li;
        if (c > p.N - 1) c = p.N - 1;
        const float* er = p.W + (long long)c * p.ldw + 4 * kq;
#pragma unroll
        for (int j = 0; j < NKB; j++) ev[j] = ld4(er + (16 * j < K ? 16 * j : 0));
    };
    eload(cb < p.ncb ? cb : 0);

    // rows -> r = 1/sqrt(mean(x^2) + eps) in f64 -> x * r * w into LDS
#pragma unroll
    for (int r = 0; r < RPW; r++) {
        float ss = 0.f;
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const f32x4_t v = xv[r][t];
            if (lane + 64 * t < K4) ss += v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
        }
        ss = wave_sum(ss);
        const float rr = 1.0f / (float)sqrt((double)(ss / (float)K + p.eps));
        const int row = w + DEC_HEAD_WAVES * r;
#pragma unroll
        for (int t = 0; t < 2; t++) {
            const int q = lane + 64 * t;
            if (q < K4) {
                f32x4_t v = xv[r][t];
#pragma unroll
                for (int e = 0; e < 4; e++) v[e] = v[e] * rr * nw[t][e];
                *(f32x4_t*)(xs + row * LDK + 4 * q) = v;
            }
        }
    }
    __syncthreads();

    for (; cb < p.ncb; cb += nwaves) {
        f32x4_t acc[4];
#pragma unroll
        for (int rb = 0; rb < 4; rb++) acc[rb] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < NKB; j++) {
            if (16 * j >= K) break;
            f32x4_t av[4];
#pragma unroll
            for (int rb = 0; rb < 4; rb++) av[rb] = *(const f32x4_t*)(xs + (16 * rb + li) * LDK + 16 * j + 4 * kq);
#pragma unroll
            for (int u = 0; u < 4; u++)
#pragma unroll
                for (int rb = 0; rb < 4; rb++)
                    acc[rb] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[rb][u], ev[j][u], acc[rb], 0, 0, 0);
        }
        const int c = 16 * cb + li;
        if (c < p.N) {
#pragma unroll
            for (int rb = 0; rb < 4; rb++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int m = m0 + 16 * rb + 4 * kq + r;
                    if (m < p.M) p.C[(long long)m * p.ldc + c] = acc[rb][r];
                }
        }
        if (cb + nwaves < p.ncb) eload(cb + nwaves);
    }
    if (p.pos_inc && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) *p.pos_inc = *p.pos_inc + 1;
}

// instantiations by the number of 16-deep steps the register block holds
#define DEC_HEAD_KERNEL(NKB)                                                                              \
    extern "C" __global__ void __launch_bounds__(64 * DEC_HEAD_WAVES) k_dec_head_k##NKB(DecGemmParams p) { \
        dec_head<NKB>(p);                                                                                 \
    }
DEC_HEAD_KERNEL(8)
DEC_HEAD_KERNEL(24)
DEC_HEAD_KERNEL(32)

// ---------------------------------------------------------------- attention
// One wave's share of a decode attention: q (this lane's 4 components, LPR =
// HD/4 lanes per key row) over the cached key rows [j0, j1) of one (sequence,
// head), with an online softmax in base 2.  The wave walks its rows in passes
// of NIT*RPI; kn / vn hold the first pass's rows, loaded by the caller
// (unconditionally, from rows clamped to row 0, which always holds a key), and
// every pass loads the next one's before its arithmetic.  Returns the wave's
// running max (-inf without keys), its sum of exponentials and its O (the
// wave's row groups added), the same in every lane of a column quad.
template <int HD, int NIT>
__device__ __forceinline__ void dec_attn_range(const f32x4_t qv, const float* __restrict__ kb,
                                               const float* __restrict__ vb, int j0, int j1, int sub, float c2,
                                               f32x4_t (&kn)[NIT], f32x4_t (&vn)[NIT], float& mx_out,
                                               float& l_out, f32x4_t& o_out) {
    constexpr int LPR = HD / 4, RPI = 64 / LPR, PASS = NIT * RPI;
    const int c4 = (threadIdx.x & 63) % LPR;
    float mx = -INFINITY, ls = 0.f;
    f32x4_t o = {0.f, 0.f, 0.f, 0.f};
    for (int p0 = j0; p0 < j1; p0 += PASS) {
        f32x4_t kr[NIT], vr[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            kr[it] = kn[it];
            vr[it] = vn[it];
            const int j = p0 + PASS + it * RPI + sub;
            const long long off = (long long)(j < j1 ? j : 0) * HD;
            kn[it] = ld4_stream(kb + off);
            vn[it] = ld4_stream(vb + off);
        }
        float sc[NIT];
        float pm = -INFINITY;
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int j = p0 + it * RPI + sub;
            float d = kr[it][0] * qv[0] + kr[it][1] * qv[1] + kr[it][2] * qv[2] + kr[it][3] * qv[3];
#pragma unroll
            for (int sh = 1; sh < LPR; sh <<= 1) d += __shfl_xor(d, sh, WAVE);
            sc[it] = j < j1 ? d * c2 : -INFINITY;
            pm = fmaxf(pm, sc[it]);
        }
        pm = wave_max(pm);
        const float nm = fmaxf(mx, pm);        // finite: the pass holds at least one key
        const float corr = exp2f(mx - nm);     // 0 on the first pass (mx = -inf)
        ls *= corr;
        o *= corr;
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const float e = exp2f(sc[it] - nm);   // 0 for rows past the wave's keys
            ls += e;
            o += e * vr[it];
        }
        mx = nm;
    }
    // the wave's sum counts each key row once (lane c4 == 0 of its group),
    // its O adds the RPI row groups
    float lrow = c4 == 0 ? ls : 0.f;
    lrow = wave_sum(lrow);
#pragma unroll
    for (int sh = LPR; sh < 64; sh <<= 1) {
        o[0] += __shfl_xor(o[0], sh, WAVE);
        o[1] += __shfl_xor(o[1], sh, WAVE);
        o[2] += __shfl_xor(o[2], sh, WAVE);
        o[3] += __shfl_xor(o[3], sh, WAVE);
    }
    mx_out = mx;
    l_out = lrow;
    o_out = o;
}

// ------------------------------------------------- QKV projection + attention
// One workgroup per head h and pair of sequences (b0, b0 + 1), 4 waves per
// sequence: it forms the head's q, k and v of each sequence's new token
// itself -- RMSNorm(x[b]) @ Wqkv[:, head columns] + b, RoPE on q and k at the
// position -- appends k and v to the cache, and runs the attention of q over
// the cached keys 0 .. pos-1 (each wave of the sequence a contiguous range,
// dec_attn_range) and the new key, merged in wave order with the new key
// last.  This removes the step's separate QKV kernel and its boundary: the
// inputs of a head's attention are the row x[b] and a 3*HD-column slice of
// Wqkv, which the workgroup reads once for its two sequences (measured
// against one sequence of 8 waves, four of 2 or 4 waves and two of 8 waves
// per workgroup: two of 4 is the fastest step).
//
// Projection: the workgroup's 8 waves split the rows of the slice; lane
// (sub, c4) reads W[k][seg*D + h*HD + 4c4 .. +3] of the three segments for
// rows k = k0 + RPI*g + sub, so one wave instruction covers RPI whole rows of
// a segment, and multiplies them into both sequences' sums.  The
// normalisation is applied after the sum, out = r * sum_k (x[k] w[k])
// W[k][c] + bias, r = 1/sqrt(mean(x^2) + eps) in f64 as in k_rmsnorm_fwd.
// The per-row values x[k] w[k] reach the lanes by lane shuffles, and the
// partial sums go through LDS to the first wave of each sequence, which adds
// them in wave order.  The projection's loads (x, the norm weight, the row's
// quads for the sum of squares, the first batch of the slice) are issued
// first and the cache stream's first pass right after them (it does not
// depend on q), so the pass is in flight during the projection while the
// projection's waits -- the memory counter is in order -- cover only its own
// loads (same-box: decode 111.2 k -> 111.9 k tokens/s, logits unchanged bit
// for bit; before, the sum of squares waited for the whole pass).
template <int HD, int SEQ, int WPS, int NIT = 4>
__device__ __forceinline__ void dec_qkv_attn(const DecGemmParams& p) {
    constexpr int LPR = HD / 4, RPI = 64 / LPR;
    constexpr int TW = SEQ * WPS;               // waves of the workgroup
    constexpr int GB = 12;                      // row groups per load batch of the projection
    __shared__ f32x4_t red[TW][SEQ][3][LPR];    // the waves' partial q | k | v sums
    __shared__ f32x4_t hv[SEQ][3][LPR];         // each sequence's q, new k, new v
    __shared__ float wm[TW], wl[TW];
    __shared__ f32x4_t wo[TW][LPR];
    __shared__ float s_new[SEQ];
    const int pos = *p.pos;                     // the new token's position = cached keys
    // consecutive workgroups take different heads, so the workgroups on one
    // XCD (every 8th) read only a few of the heads' Wqkv slices
    const int pr = blockIdx.x / p.H, h = blockIdx.x - pr * p.H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sq = wave / WPS, wr = wave - sq * WPS;   // this wave's sequence and its rank there
    const int sub = lane / LPR, c4 = lane % LPR;
    const int D = p.D;
    const float c2 = p.scale * DEC_LOG2E_F;
    // the workgroup's sequences (a missing last one recomputes the first's
    // values and stores nothing)
    int bs[SEQ];
#pragma unroll
    for (int s = 0; s < SEQ; s++) {
        const int bb = pr * SEQ + s;
        bs[s] = bb < p.M ? bb : pr * SEQ;
    }
    const int b = bs[sq];
    const bool b_ok = pr * SEQ + sq < p.M;

    // this wave's range of cached keys
    const int n = pos;
    const int per = ((n + WPS - 1) / WPS + RPI - 1) / RPI * RPI;
    const int j0 = wr * per;
    int j1 = j0 + per;
    if (j1 > n) j1 = n;
    const long long head_rows = ((long long)b * p.H + h) * p.ctx;
    const float* kb = p.kc + head_rows * HD + 4 * c4;
    const float* vb = p.vc + head_rows * HD + 4 * c4;

    // ---- projection inputs first, then the cache stream's first pass: the
    // memory counter is in order, so the projection's waits then cover only
    // its own loads (x, the norm weight, the Wqkv slice), not the HBM pass
    const float* xr[SEQ];
#pragma unroll
    for (int s = 0; s < SEQ; s++)
        xr[s] = p.a_ids ? p.E + (long long)p.ids[bs[s]] * p.lda : p.A + (long long)bs[s] * p.lda;
    const int rw = ((D + TW - 1) / TW + RPI - 1) / RPI * RPI;   // rows per wave (<= 64 for D <= 512)
    const int k0 = wave * rw;
    int k1 = k0 + rw;
    if (k1 > D) k1 = D;
    const int kx = k0 + lane;
    const int kxs = kx < k1 ? kx : 0;
    const float wn = p.norm_w[kxs];
    float xv[SEQ];
#pragma unroll
    for (int s = 0; s < SEQ; s++) xv[s] = xr[s][kxs];
    // the row's float4 quads lane and lane + 64 (D <= 512), for the sum of squares
    const int qa = lane < D / 4 ? lane : 0, qb = lane + 64 < D / 4 ? lane + 64 : 0;
    // (the row chosen by selects: indexing xr by the runtime sq would turn
    // these into flat loads, which make the compiler wait for every load)
    const float* xq = xr[0];
#pragma unroll
    for (int s = 1; s < SEQ; s++) xq = sq == s ? xr[s] : xq;
    const f32x4_t sa = ld4(xq + 4 * qa), sb = ld4(xq + 4 * qb);
    __builtin_amdgcn_sched_barrier(0);
    const float* wcol = p.W + h * HD + 4 * c4;   // q column quad; k at + D, v at + 2D
    f32x4_t wv[GB][3];
    auto wload = [&](int g0) {
#pragma unroll
        for (int j = 0; j < GB; j++) {
            const int k = k0 + g0 + j * RPI + sub;
            const long long ks = k < k1 ? k : 0;
#pragma unroll
            for (int g = 0; g < 3; g++) wv[j][g] = ld4(wcol + ks * p.ldw + g * D);
        }
    };
    // every load of a batch is issued before the first use (left to itself
    // the scheduler keeps a few in flight and waits on each in turn)
    wload(0);
    __builtin_amdgcn_sched_barrier(0);
    // this wave's first pass of cached keys (clamped to row 0, which the
    // prefill always wrote; rows past the wave's keys weigh 0)
    f32x4_t kn[NIT], vn[NIT];
#pragma unroll
    for (int it = 0; it < NIT; it++) {
        const int j = j0 + it * RPI + sub;
        const long long off = (long long)(j < j1 ? j : 0) * HD;
        kn[it] = ld4_stream(kb + off);
        vn[it] = ld4_stream(vb + off);
    }
    __builtin_amdgcn_sched_barrier(0);

    // lane i < rw holds x[b][k0 + i] * w[k0 + i] of each sequence
    float xw[SEQ];
#pragma unroll
    for (int s = 0; s < SEQ; s++) xw[s] = (kx < k1 && lane < rw) ? xv[s] * wn : 0.f;
    // the first wave of each sequence also forms its row's sum of squares for r
    float ss = 0.f;
    if (wr == 0) {
        if (lane < D / 4) ss += sa[0] * sa[0] + sa[1] * sa[1] + sa[2] * sa[2] + sa[3] * sa[3];
        if (lane + 64 < D / 4) ss += sb[0] * sb[0] + sb[1] * sb[1] + sb[2] * sb[2] + sb[3] * sb[3];
        ss = wave_sum(ss);
    }
    f32x4_t acc[SEQ][3];
#pragma unroll
    for (int s = 0; s < SEQ; s++)
#pragma unroll
        for (int g = 0; g < 3; g++) acc[s][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    auto wfma = [&](int g0) {
#pragma unroll
        for (int j = 0; j < GB; j++) {
            const int i = g0 + j * RPI + sub;           // row offset inside the wave's range
            const bool kv = i < rw && k0 + i < k1;
#pragma unroll
            for (int s = 0; s < SEQ; s++) {
                const float xk = __shfl(xw[s], i < 64 ? i : 63, WAVE);
#pragma unroll
                for (int g = 0; g < 3; g++) acc[s][g] += (kv ? xk : 0.f) * wv[j][g];
            }
        }
    };
    wfma(0);
    // further batches (d_model > 384: rows per wave above GB * RPI)
    for (int g0 = GB * RPI; g0 < rw; g0 += GB * RPI) {
        wload(g0);
        __builtin_amdgcn_sched_barrier(0);
        wfma(g0);
    }
    // rows of the wave -> one partial per column quad
#pragma unroll
    for (int sh = LPR; sh < 64; sh <<= 1)
#pragma unroll
        for (int s = 0; s < SEQ; s++)
#pragma unroll
            for (int g = 0; g < 3; g++)
#pragma unroll
                for (int e = 0; e < 4; e++) acc[s][g][e] += __shfl_xor(acc[s][g][e], sh, WAVE);
    if (sub == 0) {
#pragma unroll
        for (int s = 0; s < SEQ; s++)
#pragma unroll
            for (int g = 0; g < 3; g++) red[wave][s][g][c4] = acc[s][g];
    }
    __syncthreads();
    if (wr == 0 && lane < 3 * LPR) {
        const int g = lane / LPR, cq = lane % LPR;
        f32x4_t y = red[0][sq][g][cq];
#pragma unroll
        for (int w = 1; w < TW; w++) y += red[w][sq][g][cq];
        const float r = 1.0f / (float)sqrt((double)(ss / (float)D + p.eps));
        const f32x4_t bv = ld4(p.bias + g * D + h * HD + 4 * cq);
#pragma unroll
        for (int e = 0; e < 4; e++) y[e] = y[e] * r + bv[e];
        if (g < 2) {
            // RoPE on the pairs (4cq, 4cq+1) and (4cq+2, 4cq+3)
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const int t = pos * (HD / 2) + 2 * cq + i;
                const float cs = p.cos_t[t], sn = p.sin_t[t];
                const float ye = y[2 * i], yo = y[2 * i + 1];
                y[2 * i] = ye * cs - yo * sn;
                y[2 * i + 1] = ye * sn + yo * cs;
            }
        }
        hv[sq][g][cq] = y;
        if (g > 0 && b_ok) *(f32x4_t*)((g == 1 ? p.kc : p.vc) + (head_rows + pos) * HD + 4 * cq) = y;
    }
    __syncthreads();
    const f32x4_t qv = hv[sq][0][c4];
    if (wr == 0) {
        // the new key's score, formed as the cached keys' scores are
        const f32x4_t kv = hv[sq][1][c4];
        float d = kv[0] * qv[0] + kv[1] * qv[1] + kv[2] * qv[2] + kv[3] * qv[3];
#pragma unroll
        for (int sh = 1; sh < LPR; sh <<= 1) d += __shfl_xor(d, sh, WAVE);
        if (lane == 0) s_new[sq] = d * c2;
    }

    // ---- attention over the cached keys, merged with the new key
    float mx, lrow;
    f32x4_t o;
    dec_attn_range<HD, NIT>(qv, kb, vb, j0, j1, sub, c2, kn, vn, mx, lrow, o);
    if (sub == 0) wo[wave][c4] = o;
    if (lane == 0) { wm[wave] = mx; wl[wave] = lrow; }
    __syncthreads();
    if (wr == 0 && lane < LPR && b_ok) {
        const int w0 = sq * WPS;
        const float sn = s_new[sq];
        float M = sn;
#pragma unroll
        for (int w = 0; w < WPS; w++) M = fmaxf(M, wm[w0 + w]);
        float L = 0.f;
        f32x4_t a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < WPS; w++) {
            const float wt = wm[w0 + w] == -INFINITY ? 0.f : exp2f(wm[w0 + w] - M);   // waves without keys weigh 0
            L += wt * wl[w0 + w];
            a += wt * wo[w0 + w][lane];
        }
        const float wt = exp2f(sn - M);
        L += wt;
        a += wt * hv[sq][2][lane];
        *(f32x4_t*)(p.C + (long long)b * p.ldc + h * HD + 4 * lane) = a / L;
    }
}

// DEC_QA_SEQ sequences per workgroup, DEC_QA_WPS waves each
#define DEC_QA_SEQ 2
#define DEC_QA_WPS 4
#define DEC_QKV_ATTN_KERNEL(HD)                                                                         \
    extern "C" __global__ void __launch_bounds__(64 * DEC_QA_SEQ * DEC_QA_WPS)                           \
        __attribute__((amdgpu_waves_per_eu(2))) k_dec_qkv_attn_hd##HD(DecGemmParams p) {               \
        dec_qkv_attn<HD, DEC_QA_SEQ, DEC_QA_WPS>(p);                                                    \
    }
DEC_QKV_ATTN_KERNEL(16)
DEC_QKV_ATTN_KERNEL(32)
DEC_QKV_ATTN_KERNEL(64)

// Lane layout of v_mfma_f32_16x16x4f32 (checked exactly by a test):
// out[lane*4 + r] = result register r of lane `lane`.
extern "C" __global__ void k_mfma16_layout_probe(const float* a, const float* b, float* out) {
    const int l = threadIdx.x;
    f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[l], b[l], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 4; r++) out[l * 4 + r] = acc[r];
}
