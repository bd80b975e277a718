// attention.hip -- causal attention on FP32 matrix cores, flash style.
//
// Replaces the reference's materialised-P attention (QK^T GEMM, in-place
// masked softmax, PV GEMM and their backward: train_kernels.cu:631-664,
// gpu_train.c:346-353,445-455) with kernels that never store P:
//   forward : S = QK^T*scale, online softmax, O = PV; saves the per-row
//             log-sum-exp (base 2) for the backward;
//   backward: D_i = <dO_i, O_i>; dK, dV over key blocks, which also store
//             every causal 64x64 block of dS = P o (dP - D) * scale; then
//             dQ = dS K over query blocks from those blocks (S and dP are
//             formed once, not once per pass).
// Masked entries (j > i) are exactly zero in the reference (exp of -1e9 is 0,
// mathlib.c:142), so key blocks above the diagonal are skipped outright.
// No atomics: dQ is produced by its own pass instead of being accumulated
// across key blocks, so results are bit-identical run to run.
//
// Work split (causal blocks differ a lot in length: the last query block sees
// every key): a workgroup owns 64 rows (queries, or keys for dK/dV) as two
// 32-row groups, and each group's loop over the other axis is shared by two
// wavefronts: in the forward and dQ passes each takes one 32-key half of
// every 64-key block, in dK/dV alternate 64-query blocks.  The two partial
// results are merged through LDS in a fixed order at the end, which halves
// the longest per-wavefront loop without losing reproducibility.
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

#include "../kernel_params.h"   // GemmParams, AttnParams, DecGemmParams

// First float of dS block (query block qb, key block kb <= qb) of head bh.
__device__ __forceinline__ float* att_ds_block(const AttnParams& p, int bh, int qb, int kb) {
    const long long nqb = (p.T + 63) / 64;
    return p.ds + (((long long)bh * (nqb * (nqb + 1) / 2)) + (long long)qb * (qb + 1) / 2 + kb) * 4096;
}

// One [64 x HD] tile (rows r0.., columns col0.., row stride ld) held in
// registers across the 256 threads of a workgroup: thread t holds the
// f32x4 at row (t + 256 i) / (HD/4), column 4 ((t + 256 i) % (HD/4)).
// Loading and storing are separate steps so that all of a stage's loads are
// in flight together (and can be issued one stage ahead of the LDS store).
template <int HD>
struct AttTile {
    static constexpr int NQ = 64 * HD / 4 / 256;
    f32x4 v[NQ];
    // Row addresses are clamped to row rlim-1, so every load stays inside the
    // tensor; rows >= rlim are zeroed by store(), not here, so that a
    // prefetch does not have to wait for its data.
    __device__ __forceinline__ void load(const float* base, int ld, int r0, int rlim, int col0) {
        if (r0 + 64 <= rlim) {
            // whole tile in range: one wave-uniform row base, per-thread
            // 32-bit offsets
            const float* b = base + (long long)r0 * ld + col0;
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                int idx = threadIdx.x + i * 256;
                int r = idx / (HD / 4), c = (idx % (HD / 4)) * 4;
                v[i] = *(const f32x4*)(b + (r * ld + c));
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            int idx = threadIdx.x + i * 256;
            int r = idx / (HD / 4), c = (idx % (HD / 4)) * 4;
            int row = r0 + r;
            v[i] = *(const f32x4*)(base + (long long)(row < rlim ? row : rlim - 1) * ld + col0 + c);
        }
    }
    // LDS layout [64][HD + 4]; rows r0 + r >= rlim are written as 0
    __device__ __forceinline__ void store(float* lds, int r0, int rlim) const {
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            int idx = threadIdx.x + i * 256;
            int r = idx / (HD / 4), c = (idx % (HD / 4)) * 4;
            f32x4 x = v[i];
            if (r0 + r >= rlim) x = f32x4{0.f, 0.f, 0.f, 0.f};
            *(f32x4*)(lds + r * (HD + 4) + c) = x;
        }
    }
};

// A [64 x HD] tile stored transposed in LDS, [HD][ATT_LDT] (row index
// contiguous), so that 4 consecutive rows of one column are one 128-bit LDS
// read.  Each load instruction of a wave covers 16 rows x 4 column groups
// (rows 64 bytes apart in LDS per column), which keeps the transposing
// 32-bit stores at the minimum two LDS cycles per instruction.
#define ATT_LDT 68
template <int HD>
struct AttTileT {
    static constexpr int NQ = 64 * HD / 4 / 256;
    f32x4 v[NQ];
    __device__ __forceinline__ void coords(int i, int& r, int& c) const {
        const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
        const int blk = w * NQ + i;
        r = 16 * (blk & 3) + (l & 15);
        c = 4 * (4 * (blk >> 2) + (l >> 4));
    }
    __device__ __forceinline__ void load(const float* base, int ld, int r0, int rlim, int col0) {
        if (r0 + 64 <= rlim) {
            const float* b = base + (long long)r0 * ld + col0;
#pragma unroll
            for (int i = 0; i < NQ; i++) {
                int r, c;
                coords(i, r, c);
                v[i] = *(const f32x4*)(b + (r * ld + c));
            }
            return;
        }
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            int r, c;
            coords(i, r, c);
            int row = r0 + r;
            v[i] = *(const f32x4*)(base + (long long)(row < rlim ? row : rlim - 1) * ld + col0 + c);
        }
    }
    __device__ __forceinline__ void store(float* lds, int r0, int rlim) const {
#pragma unroll
        for (int i = 0; i < NQ; i++) {
            int r, c;
            coords(i, r, c);
            f32x4 x = v[i];
            if (r0 + r >= rlim) x = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int e = 0; e < 4; e++) lds[(c + e) * ATT_LDT + r] = x[e];
        }
    }
};

// Row-fragment of 32 rows for the d-steps of chunk j: lane l gets
// X[rb + l%32][8j + 4*(l/32) + s], s = 0..3.
template <int HD>
__device__ __forceinline__ f32x4 att_frag(const float* lds, int rb, int j, int lane) {
    return *(const f32x4*)(lds + (rb + (lane & 31)) * (HD + 4) + 8 * j + 4 * (lane >> 5));
}

// Same fragment straight from global memory (per-wave register operands).
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

// Make the compiler wait for loaded operand registers here, once: later
// loads issued inside a loop would otherwise be waited for together with
// them (the memory counter is in order) at their first use in the loop.
template <int N>
__device__ __forceinline__ void att_settle(const f32x4* x) {
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" ::"v"(x[i]));
}

// Store a [HD x 32] accumulator set (rows d, one column per lane) to the
// row of `row` (columns col0 + d): float4 over 4 consecutive d.  With rope
// tables, the pairs (d0, d0+1), (d0+2, d0+3) are rotated back by position t
// (the transpose of the forward rotation, model_ops.c:130-155).
template <int HD>
__device__ __forceinline__ void att_store_rows(float* rowp, const f32x16* acc, int half, float scale,
                                               const float* rc = nullptr, const float* rs = nullptr, int t = 0) {
    constexpr int DB = (HD + 31) / 32;
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int d0 = d * 32 + 8 * g + 4 * half;
            if (d0 < HD) {
                f32x4 v = {acc[d][4 * g] * scale, acc[d][4 * g + 1] * scale, acc[d][4 * g + 2] * scale,
                           acc[d][4 * g + 3] * scale};
                if (rc) {
                    const int k = t * (HD / 2) + (d0 >> 1);
                    const float c0 = rc[k], c1 = rc[k + 1], s0 = rs[k], s1 = rs[k + 1];
                    const f32x4 a = v;
                    v[0] = a[0] * c0 + a[1] * s0;
                    v[1] = -a[0] * s0 + a[1] * c0;
                    v[2] = a[2] * c1 + a[3] * s1;
                    v[3] = -a[2] * s1 + a[3] * c1;
                }
                *(f32x4*)(rowp + d0) = v;
            }
        }
}

// Causal work per query block grows with its index, so the workgroup ->
// (head, query block) map ranks the jobs longest first (rank r: query block
// nqb-1 - r/BH, head r%BH, BH = gridDim.x heads) and lets dispatch round k
// (256 workgroups, one per CU, consecutive workgroups going to different
// CUs) take its ranks in reverse order when k is odd: a CU then holds a long,
// a short and a middle block (per-CU key blocks 23..28 instead of 18..33 for
// 768 workgroups of 16 blocks).
__device__ __forceinline__ void att_snake_job(int nqb, int& qb, int& bh) {
    const int BH = gridDim.x, total = BH * gridDim.y;
    const int L = blockIdx.y * BH + blockIdx.x, r = L / 256, lo = r * 256;
    const int m = (total - lo) < 256 ? (total - lo) : 256;
    const int rank = (r & 1) ? lo + (m - 1) - (L - lo) : L;
    qb = nqb - 1 - rank / BH;
    bh = rank - (rank / BH) * BH;
}

// =========================================================== forward
// grid (B*H, ceil(T/64)), 256 threads, three workgroups per CU.  Wave w:
// query group g = w&1 (32 queries), key half part = w>>1: every stage loads
// one 64-key block (K and V^T in LDS, the next block fetched into registers
// meanwhile) and part p takes its keys 32p .. 32p+31; each wave keeps its own
// online softmax, and the two parts are merged at the end.  One K and one V^T
// tile per stage (35 KB of LDS) and 167 registers let three workgroups share
// a CU, so all 768 workgroups of B8 T1024 are resident at once and the
// snake order (att_snake_job) evens out the causal work per CU: 23 to 28 key
// blocks.  When the grid is exactly three workgroups per CU, the host's job
// table (p.jobs, trlm_attn_job_table) gives every CU 25 or 26 and keeps each
// head on one XCD as the snake does (B8 T1024, same bits: 70.8 -> 66.7 us
// launched back to back; within noise in the model's forward).
template <int HD>
__device__ void flash_fwd(const AttnParams& p) {
    constexpr int DB = (HD + 31) / 32;
    constexpr int LD = HD + 4;
    constexpr int KS = 64 * LD, VS = HD * ATT_LDT;                     // K [64][LD], V^T [HD][ATT_LDT]
    __shared__ __attribute__((aligned(16))) float lds[KS + VS];        // K | V^T of the stage's key block

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, half = lane >> 5;
    const int grp = wave & 1, part = wave >> 1;
    const int nqb = (p.T + 63) / 64;
    int qb, bh;
    if (p.jobs) {
        // the host's placement: workgroups L, L + CUs, L + 2 CUs share a
        // compute unit, and their jobs' key-block counts sum to the same
        // total (+-1) on every unit
        const int j = p.jobs[blockIdx.y * gridDim.x + blockIdx.x];
        qb = j >> 16;
        bh = j & 0xffff;
    } else {
        att_snake_job(nqb, qb, bh);
    }
    const int b = bh / p.H, h = bh - b * p.H;
    const long long rowbase = (long long)b * p.T;
    const float* qkv = p.qkv + rowbase * p.ldq;
    const int qcol = h * HD, kcol = p.D + h * HD, vcol = 2 * p.D + h * HD;
    const int qw0 = qb * 64 + grp * 32;
    const int qpos = qw0 + (lane & 31);
    const float c2 = p.scale * ATT_LOG2E;

    f32x4 qf[HD / 8];
    att_frag_global<HD>(qkv, p.ldq, qpos, qpos < p.T, qcol, lane, qf);
    f32x16 o[DB];
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[d][r] = 0.f;
    float m = -INFINITY, l = 0.f;

    int kv_end = (qb + 1) * 64;
    if (kv_end > p.T) kv_end = p.T;
    const int nkv = (kv_end + 63) / 64;
    const float* Ks = lds;
    const float* Vt = lds + KS;
    // one key block per stage: part p of the wave pair takes its keys
    // 32p .. 32p+31; K and V^T of the next block are fetched one stage ahead
    AttTile<HD> tk;
    AttTileT<HD> tv;
    auto fetch = [&](int kb) {
        tk.load(qkv, p.ldq, kb * 64, p.T, kcol);
        tv.load(qkv, p.ldq, kb * 64, p.T, vcol);
    };
    fetch(0);
    att_settle<HD / 8>(qf);
    for (int kb = 0; kb < nkv; kb++) {
        __syncthreads();
        tk.store(lds, kb * 64, kv_end);
        tv.store(lds + KS, kb * 64, kv_end);
        __syncthreads();
        fetch(kb + 1);
        const int kv0 = kb * 64 + part * 32;
        if (kv0 > qw0 + 31) continue;

        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; r++) s[r] = 0.f;
#pragma unroll
        for (int j = 0; j < HD / 8; j++) {
            f32x4 kf = att_frag<HD>(Ks, part * 32, j, lane);
#pragma unroll
            for (int t = 0; t < 4; t++) s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[t], qf[j][t], s, 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < HD / 8; q++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }
        if (kv0 + 31 > qw0) {
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int kpos = kv0 + 8 * (r >> 2) + 4 * half + (r & 3);
                if (kpos > qpos) s[r] = -INFINITY;
            }
        }
        float mr = s[0];
#pragma unroll
        for (int r = 0; r < 16; r++) mr = fmaxf(mr, s[r]);
        mr = fmaxf(mr, __shfl_xor(mr, 32, WAVE));
        const float mx = fmaxf(m, mr * c2);
        const float alpha = __builtin_amdgcn_exp2f(m - mx);
        m = mx;
        float ls = 0.f;
#pragma unroll
        for (int r = 0; r < 16; r++) {
            float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c2, -mx));
            s[r] = e;
            ls += e;
        }
        l = l * alpha + ls;
        if (__ballot(alpha != 1.0f)) {
#pragma unroll
            for (int d = 0; d < DB; d++)
#pragma unroll
                for (int r = 0; r < 16; r++) o[d][r] *= alpha;
        }
#pragma unroll
        for (int g = 0; g < 4; g++) {
            f32x4 vt[DB];
#pragma unroll
            for (int d = 0; d < DB; d++) {
                const int dc = d * 32 + (lane & 31);
                vt[d] = (dc < HD) ? *(const f32x4*)(Vt + dc * ATT_LDT + part * 32 + 8 * g + 4 * half)
                                  : f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int t = 0; t < 4; t++)
#pragma unroll
                for (int d = 0; d < DB; d++)
                    o[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt[d][t], s[4 * g + t], o[d], 0, 0, 0);
        }
#pragma unroll
        for (int q = 0; q < 4 * DB; q++) {
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
        }
    }
    // merge the two key partitions of each query group: (m, l, O) of part 1
    // go through LDS to the part-0 wave, which rescales, adds and stores.
    __syncthreads();
    float* xch = lds + grp * (DB * 16 * 64 + 128);
    if (part == 1) {
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) xch[(d * 16 + r) * 64 + lane] = o[d][r];
        xch[DB * 16 * 64 + lane] = m;
        xch[DB * 16 * 64 + 64 + lane] = l;
    }
    __syncthreads();
    if (part == 0) {
        const float m1 = xch[DB * 16 * 64 + lane], l1 = xch[DB * 16 * 64 + 64 + lane];
        const float mm = fmaxf(m, m1);
        const float a0 = exp2f(m - mm), a1 = (m1 == -INFINITY) ? 0.f : exp2f(m1 - mm);
        float lt = l * a0 + l1 * a1;
        lt = lt + __shfl_xor(lt, 32, WAVE);
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[d][r] = o[d][r] * a0 + xch[(d * 16 + r) * 64 + lane] * a1;
        if (qpos < p.T) {
            att_store_rows<HD>(p.out + (rowbase + qpos) * p.ldo + qcol, o, half, 1.0f / lt);
            if (half == 0) p.lse[(long long)bh * p.T + qpos] = mm + __log2f(lt);
        }
    }
}


// =========================================================== backward dK, dV
// grid (B*H, ceil(T/64)).  Wave w: key group g = w&1 (32 keys), query
// partition part = w>>1 (64-query blocks at or after the keys' block,
// alternating).  S and dP are formed as [q x kv] (one key per lane), so the
// P and dS registers feed dV^T += dO^T P and dK^T += Q^T dS directly.  A
// stage's four Q / dO tiles go straight from global memory into LDS, all in
// flight together: one memory round trip per stage where register staging
// (room for one tile beside the K, V operands and four accumulators) took
// four (B8 T1024 hd64: 138.3 -> 135.0 us, same bits).
// LDS address space for global_load_lds destinations
typedef __attribute__((address_space(3))) void att_lds_void;
template <int HD>
__device__ void flash_bwd_dkv(const AttnParams& p) {
    constexpr int DB = (HD + 31) / 32;
    constexpr int LD = HD + 4;
    constexpr int TILE = 2 * 64 * LD + 128;                 // Q, dO, L, D of one query block
    constexpr int NCH = 64 * LD / 256;                       // 1 KB global_load_lds chunks per tile
    static_assert((64 * LD) % 256 == 0, "tile chunks");
    __shared__ __attribute__((aligned(16))) float lds[2 * TILE];

    const int lane = threadIdx.x & 63, half = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform, kept in SGPRs
    const int grp = wave & 1, part = wave >> 1;
    const int kb = blockIdx.y;                               // early keys (most queries) first
    const int bh = blockIdx.x, b = bh / p.H, h = bh - b * p.H;
    const long long rowbase = (long long)b * p.T;
    const float* qkv = p.qkv + rowbase * p.ldq;
    const float* dO = p.dO + rowbase * p.ldo;
    const int qcol = h * HD, kcol = p.D + h * HD, vcol = 2 * p.D + h * HD;
    const float* lse = p.lse + (long long)bh * p.T;
    const float* dv = p.dvec + (long long)bh * p.T;
    const float c2 = p.scale * ATT_LOG2E;

    const int kw0 = kb * 64 + grp * 32;
    const int kpos = kw0 + (lane & 31);
    f32x4 kf[HD / 8], vf[HD / 8];
    att_frag_global<HD>(qkv, p.ldq, kpos, kpos < p.T, kcol, lane, kf);
    att_frag_global<HD>(qkv, p.ldq, kpos, kpos < p.T, vcol, lane, vf);

    f32x16 dk[DB], dvv[DB];
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) { dk[d][r] = 0.f; dvv[d][r] = 0.f; }

    const int nqb = (p.T + 63) / 64;
    const int nblk = nqb - kb;                               // query blocks kb .. nqb-1
    const int niter = (nblk + 1) / 2;
    const float* Qs = lds + part * TILE;
    const float* Gs = Qs + 64 * LD;
    const float* Ls = Gs + 64 * LD;
    const float* Ds = Ls + 64;
    for (int it = 0; it < niter; it++) {
        // Q and dO of the stage's two query blocks go straight into LDS
        // (global_load_lds: 1 KB per wave instruction, rows [64][LD], pad
        // columns a copy of column 0 that is never read), all four tiles in
        // flight together; rows past the end are clamped to the last row:
        // their probabilities are masked to 0, so their products are 0.
        // L and D go through registers.  Unconditional: blocks past the end
        // load clamped rows and are skipped below.
        __syncthreads();                                     // every wave is done with the last stage
#pragma unroll
        for (int tt = 0; tt < 4; tt++) {
            const int pp = tt >> 1, q0 = (kb + 2 * it + pp) * 64;
            const bool isq = (tt & 1) == 0;
            const float* src = isq ? qkv + qcol : dO + qcol;
            const int ld = isq ? p.ldq : p.ldo;
            float* dst = lds + pp * TILE + (isq ? 0 : 64 * LD);
            for (int ci = wave; ci < NCH; ci += 4) {
                const int pos = 256 * ci + 4 * lane;
                const int r = pos / LD, col = pos - r * LD;
                const int row = q0 + r < p.T ? q0 + r : p.T - 1;
                __builtin_amdgcn_global_load_lds((const void*)(src + (long long)row * ld + (col < HD ? col : 0)),
                                                 (att_lds_void*)(dst + 256 * ci), 16, 0, 0);
            }
        }
        if (threadIdx.x < 128) {
            const int pp = threadIdx.x >> 6, q = (kb + 2 * it + pp) * 64 + (threadIdx.x & 63);
            const int qc = q < p.T ? q : p.T - 1;
            const float lv = lse[qc], dd = dv[qc];
            float* base = lds + pp * TILE + 2 * 64 * LD;
            base[threadIdx.x & 63] = q < p.T ? lv : 0.f;
            base[64 + (threadIdx.x & 63)] = q < p.T ? dd : 0.f;
        }
        __builtin_amdgcn_s_waitcnt(0);                       // this wave's tile chunks have landed
        __syncthreads();
        const int j = 2 * it + part;
        if (j >= nblk) continue;
        const int q0 = (kb + j) * 64;
        if (q0 + 63 < kw0) continue;                         // every query precedes this wave's keys
#pragma unroll
        for (int c = 0; c < 2; c++) {
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; r++) { s[r] = 0.f; dp[r] = 0.f; }
#pragma unroll
            for (int jj = 0; jj < HD / 8; jj++) {
                f32x4 qa = att_frag<HD>(Qs, c * 32, jj, lane);
                f32x4 ga = att_frag<HD>(Gs, c * 32, jj, lane);
#pragma unroll
                for (int t = 0; t < 4; t++) {
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[t], kf[jj][t], s, 0, 0, 0);
                    dp = __builtin_amdgcn_mfma_f32_32x32x2f32(ga[t], vf[jj][t], dp, 0, 0, 0);
                }
            }
            // mask (keys after the query, queries past the end) only where the
            // block can hold such pairs (wave-uniform test)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int ql = c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                s[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c2, -Ls[ql]));
            }
            if (q0 < kw0 + 32 || q0 + 64 > p.T) {
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int qpos = q0 + c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                    if (kpos > qpos || qpos >= p.T) s[r] = 0.f;
                }
            }
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int ql = c * 32 + 8 * (r >> 2) + 4 * half + (r & 3);
                dp[r] = s[r] * (dp[r] - Ds[ql]) * p.scale;
            }
            {
                // the registers as they are: 64 lanes = one 256-byte row per r
                // (wave-uniform block base: scalar address, lane as the offset)
                float* blk = att_ds_block(p, bh, kb + j, kb) + (grp * 2 + c) * 1024;
#pragma unroll
                for (int r = 0; r < 16; r++) blk[r * 64 + lane] = dp[r];
            }
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
    __syncthreads();
    float* xch = lds + grp * (2 * DB * 16 * 64);
    if (part == 1) {
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                xch[(d * 16 + r) * 64 + lane] = dk[d][r];
                xch[(DB * 16 + d * 16 + r) * 64 + lane] = dvv[d][r];
            }
    }
    __syncthreads();
    if (part == 0 && kpos < p.T) {
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                dk[d][r] = dk[d][r] + xch[(d * 16 + r) * 64 + lane];
                dvv[d][r] = dvv[d][r] + xch[(DB * 16 + d * 16 + r) * 64 + lane];
            }
        float* row = p.out + (rowbase + kpos) * p.ldq;
        att_store_rows<HD>(row + kcol, dk, half, 1.0f, p.rope_cos, p.rope_sin, kpos);
        att_store_rows<HD>(row + vcol, dvv, half, 1.0f);
    }
}

// =========================================================== backward dQ
// dQ_i = sum_{j <= i} dS_ij K_j from the dS blocks of the dK/dV pass.
// grid (B*H, ceil(T/64)), 256 threads, snake order (att_snake_job).  Wave w:
// query group g = w&1 (32 queries), key half part = w>>1: every stage takes
// one 64-key block, part p its keys 32p .. 32p+31 (the stored dS key group
// p), so the two parts always have equal work; their partial dQ^T merge
// through LDS at the end.  dQ^T accumulates as K^T dS^T: lane l feeds
// K[k][d0 + l%32] and dS[q + l%32][k] for k = 8c + 4(l/32) + s, so the dS
// operand of four k-steps is one 128-bit load (four consecutive keys are
// four consecutive lanes of the stored register rows).
// The K tile goes straight from global memory into LDS (global_load_lds: no
// staging registers, no transposing stores) in row-major [64][HD + 8] rows,
// two buffers, one barrier per stage; the rows a wave's two halves read
// together (4 apart) then sit 32 banks apart, and one ds_read2 gives both
// 32-column d blocks of a k-step.  114 registers and 36 KB of LDS: four
// workgroups fit a CU.  B8 T1024 hd64: 40.4 us against 49.5 for two key
// blocks per stage with a transposed register-staged K tile (and 54.7 for
// that form in plain longest-first order).
template <int HD>
__device__ void flash_bwd_dq_ds(const AttnParams& p) {
    constexpr int DB = (HD + 31) / 32;
    constexpr int LDK = HD + 8;                 // rows 4 apart are 32 banks apart
    constexpr int TS = 64 * LDK;                // floats per K tile
    constexpr int NCH = TS / 256;               // 1 KB global_load_lds chunks per tile
    static_assert(TS % 256 == 0 && 2 * TS >= 2 * DB * 16 * 64, "K tile layout");
    __shared__ __attribute__((aligned(16))) float lds[2 * TS];

    const int lane = threadIdx.x & 63, half = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform
    const int grp = wave & 1, part = wave >> 1;
    const int nqb = (p.T + 63) / 64;
    int qb, bh;
    att_snake_job(nqb, qb, bh);
    const int b = bh / p.H, h = bh - b * p.H;
    const long long rowbase = (long long)b * p.T;
    const float* kg = p.qkv + rowbase * p.ldq + p.D + h * HD;
    const int qcol = h * HD;
    const int qpos = qb * 64 + grp * 32 + (lane & 31);
    // this lane's query qq = l%32 of group grp sits in rows r(qq) of the
    // (key group part, grp) sub-block, in lane half (qq/4)&1
    const int qq = lane & 31;
    const int ds_off = part * 2048 + grp * 1024 + ((qq >> 3) * 4 + (qq & 3)) * 64 + ((qq >> 2) & 1) * 32 + 4 * half;
    const int nkv = qb + 1;
    // lanes past HD (HD = 16) read column 0 of their row and feed 0
    const int dl = (lane & 31) < HD ? (lane & 31) : 0;

    f32x16 acc[DB];
#pragma unroll
    for (int d = 0; d < DB; d++)
#pragma unroll
        for (int r = 0; r < 16; r++) acc[d][r] = 0.f;

    // K block kb into buf: chunk ci (256 floats) is one wave instruction,
    // lane l the 16 bytes at float 256 ci + 4 l of the padded layout (pad
    // columns take a copy of column 0, never read); rows past the end are
    // clamped to the last row: their dS entries are exactly 0 (causal mask).
    auto kload = [&](int kb, float* buf) {
        for (int ci = wave; ci < NCH; ci += 4) {
            const int pos = 256 * ci + 4 * lane;
            const int r = pos / LDK, col = pos - r * LDK;
            int key = kb * 64 + r;
            key = key < p.T ? key : p.T - 1;
            const float* src = kg + (long long)key * p.ldq + (col < HD ? col : 0);
            __builtin_amdgcn_global_load_lds((const void*)src, (att_lds_void*)(buf + 256 * ci), 16, 0, 0);
        }
    };
    auto sload = [&](int kb, f32x4* sv) {
        const float* row = att_ds_block(p, bh, qb, kb) + ds_off;
#pragma unroll
        for (int c = 0; c < 4; c++) sv[c] = *(const f32x4*)(row + 8 * c);
    };
    auto mma = [&](const float* buf, const f32x4* sv) {
        const float* kr = buf + (32 * part + 4 * half) * LDK + dl;
#pragma unroll
        for (int c = 0; c < 4; c++)
#pragma unroll
            for (int t = 0; t < 4; t++) {
                const float* kp = kr + (8 * c + t) * LDK;
#pragma unroll
                for (int d = 0; d < DB; d++) {
                    const float kv = (d * 32 + (lane & 31)) < HD ? kp[32 * d] : 0.f;
                    acc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(kv, sv[c][t], acc[d], 0, 0, 0);
                }
            }
    };
    // Stage kb: wait for this wave's loads of block kb, barrier (every wave's
    // loads have landed, and every wave is done with the other buffer), issue
    // block kb+1 into the other buffer, then the MFMAs of block kb.
    f32x4 s0[4], s1[4];
    kload(0, lds);
    sload(0, s0);
    for (int kb = 0; kb < nkv; kb += 2) {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (kb + 1 < nkv) { kload(kb + 1, lds + TS); sload(kb + 1, s1); }
        mma(lds, s0);
        if (kb + 1 >= nkv) break;
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
        if (kb + 2 < nkv) { kload(kb + 2, lds); sload(kb + 2, s0); }
        mma(lds + TS, s1);
    }
    __syncthreads();
    float* xch = lds + grp * (DB * 16 * 64);
    if (part == 1) {
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) xch[(d * 16 + r) * 64 + lane] = acc[d][r];
    }
    __syncthreads();
    if (part == 0 && qpos < p.T) {
#pragma unroll
        for (int d = 0; d < DB; d++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[d][r] = acc[d][r] + xch[(d * 16 + r) * 64 + lane];
        att_store_rows<HD>(p.out + (rowbase + qpos) * p.ldq + qcol, acc, half, 1.0f, p.rope_cos, p.rope_sin, qpos);
    }
}

// D_i = <dO_i, O_i> per (row, head) for the dK/dV pass: HD/4 threads per
// (row, head), one float4 product each, summed across them by shuffles.
template <int HD>
__device__ void attn_dvec(const AttnParams& p) {
    constexpr int G = HD / 4;
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long total = (long long)p.B * p.T * p.D / 4;
    float v = 0.f;
    long long rh = 0;
    if (i < total) {
        rh = i / G;                                       // row * H + h
        const long long row = rh / p.H;
        const int h = (int)(rh - row * p.H), c = (int)(i % G) * 4;
        const f32x4 g = *(const f32x4*)(p.dO + row * p.ldo + h * HD + c);
        const f32x4 o = *(const f32x4*)(p.O + row * p.ldo + h * HD + c);
        v = g[0] * o[0] + g[1] * o[1] + g[2] * o[2] + g[3] * o[3];
    }
#pragma unroll
    for (int m = G / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, WAVE);
    if (i < total && i % G == 0) {
        const long long row = rh / p.H;
        const int h = (int)(rh - row * p.H);
        const long long bb = row / p.T, t = row - bb * p.T;
        p.dvec[(bb * p.H + h) * p.T + t] = v;
    }
}

#define ATT_KERNELS(HD)                                                                                   \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) k_attn_fwd_hd##HD(AttnParams p) { \
        flash_fwd<HD>(p);                                                                                 \
    }                                                                                                     \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) k_attn_bwd_dkv_hd##HD(AttnParams p) { \
        flash_bwd_dkv<HD>(p);                                                                             \
    }                                                                                                     \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) k_attn_bwd_dq_hd##HD(AttnParams p) { \
        flash_bwd_dq_ds<HD>(p);                                                                           \
    }                                                                                                     \
    extern "C" __global__ void __launch_bounds__(256) k_attn_dvec_hd##HD(AttnParams p) { attn_dvec<HD>(p); }

ATT_KERNELS(16)
ATT_KERNELS(32)
ATT_KERNELS(64)
