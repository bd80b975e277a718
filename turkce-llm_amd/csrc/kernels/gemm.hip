// gemm.hip -- fp32 GEMMs on CDNA4 FP32 matrix cores (v_mfma_f32_32x32x2f32).
//
// C[M,N] = alpha * op(A) @ op(B) (+ beta*C) (+ bias[n]) (+ resid[m,n])
//   TA=0: A stored [M,K] (lda)     TA=1: A stored [K,M] -> op(A) = A^T
//   TB=0: B stored [K,N] (ldb)     TB=1: B stored [N,K] -> op(B) = B^T
// Batched through blockIdx.z (element strides sA/sB/sC), with an optional
// deterministic split-K: split s of a batch entry covers K-range
// [s*kchunk, (s+1)*kchunk) and writes its raw partial to C + s*sW; the
// partials are then summed in split order by k_gemm_splitk_reduce.
// Same contract as the reference's k_gemm_nn/nt/tn and k_bf16_gemm_nn_bias
// (train_kernels.cu:97-193,226-329), computed in fp32 only.
//
// Design (MI355X):
//  - 256-thread workgroups = 4 wave64 in a 2x2 grid; each wave owns a
//    (BM/2)x(BN/2) block of 32x32 MFMA accumulators.
//  - Operands are staged through double-buffered LDS, one barrier per
//    BK=16 (or 32) step; the next global tile is prefetched into registers while the
//    current one feeds the matrix cores.
//  - Interior tiles run a software-pipelined loop: the operand fragments of
//    the next 8-k chunk are read from LDS while the current chunk's MFMAs
//    run, the next tile is written to LDS before the last chunk, and that
//    chunk's MFMAs are issued after the barrier, where they cover the reads
//    of the next tile's first chunk.  A wave raises its priority while it
//    issues MFMAs, so the waves sharing a SIMD fall out of step and one
//    wave's LDS/barrier phase overlaps another's matrix work.
//  - A K-contiguous operand is kept K-contiguous in LDS and read with one
//    128-bit LDS read per 4 MFMA steps: lane l feeds k = kk+4*(l/32)+s at
//    step s, a permutation of k that both operands share.  An MN-contiguous
//    operand is kept MN-contiguous and read 32 consecutive floats per
//    half-wave (conflict-free), as 64-bit reads of two interleaved blocks
//    where the wave block is two MFMA blocks wide (GemmIlv).
//  - Tiles are visited XCD-aware: consecutive workgroups land on different
//    XCDs, so the tile index is remapped so that each XCD works on a
//    contiguous, M-grouped range of tiles and reuses operands in its own L2.
//  - Results leave through LDS where the operand tiles' LDS can hold them:
//    a wave's accumulators are written there 32 rows at a time and read back
//    as whole row segments, so each wave-wide store covers 4-8 rows of
//    128-256 bytes instead of 32 rows x 32 bytes.  The CU's vector-memory
//    path is the contended resource of these kernels (a store straight from
//    the accumulators waited ~0.5 us to issue), so fewer, fuller cache-line
//    transactions per store are what the epilogue is tuned for.
#include "common.h"

#include <type_traits>

#include "../kernel_params.h"   // GemmParams, AttnParams, DecGemmParams

// RoPE of four consecutive output columns n..n+3 of row `row` (model/rope.c:
// 20-40): pairs (2k, 2k+1) of a head of rope_hd columns rotated by
// (cos, sin)[t = row % rope_T, k]; the tables are [rope_T][rope_hd/2].
// n is a multiple of 4, so k is even and each table pair is one 8-byte load.
typedef float f32x2 __attribute__((ext_vector_type(2)));
// (cos, sin) of the two pairs of columns n..n+3 of row `row`
__device__ __forceinline__ void rope_tab(const GemmParams& p, int row, int n, f32x2& cc, f32x2& ss) {
    const int t = row % p.rope_T, k = (n % p.rope_hd) >> 1, hh = p.rope_hd >> 1;
    cc = *(const f32x2*)(p.rope_cos + t * hh + k);
    ss = *(const f32x2*)(p.rope_sin + t * hh + k);
}
__device__ __forceinline__ void rope_rot(f32x4& v, f32x2 cc, f32x2 ss) {
    const float c0 = cc[0], c1 = cc[1], s0 = ss[0], s1 = ss[1];
    const f32x4 a = v;
    v[0] = a[0] * c0 - a[1] * s0;
    v[1] = a[0] * s0 + a[1] * c0;
    v[2] = a[2] * c1 - a[3] * s1;
    v[3] = a[2] * s1 + a[3] * c1;
}
__device__ __forceinline__ void rope4(const GemmParams& p, int row, int n, f32x4& v) {
    f32x2 cc, ss;
    rope_tab(p, row, n, cc, ss);
    rope_rot(v, cc, ss);
}

__device__ __forceinline__ void gemm_tile_coords(const GemmParams& p, int& tm, int& tn, int& split) {
    const int num = p.tiles_m * p.tiles_n;
    // XCD-aware remap: hardware hands workgroup i to XCD (i % 8).  A split-K
    // launch (a single GEMM, blockIdx.z = split) is remapped over all its
    // workgroups in split-major order, so each XCD takes whole splits: the
    // tiles of one split share its k-range of both operands, which then stays
    // in that XCD's L2 instead of being fetched by every XCD.
    const int splits = p.splits > 1 ? p.splits : 1;
    const int all = num * splits;
    int bid = blockIdx.x + (splits > 1 ? (int)blockIdx.z * num : 0);
    const int per = all >> 3;
    int tile = bid;
    if (bid < (per << 3)) tile = (bid & 7) * per + (bid >> 3);
    split = 0;
    if (splits > 1) {
        split = tile / num;
        tile -= split * num;
    }
    // Group 8 M-tiles so tiles that run together share A and B panels.
    const int GROUP = 8;
    int group_size = GROUP * p.tiles_n;
    int g = tile / group_size;
    int first_m = g * GROUP;
    int gm = p.tiles_m - first_m;
    if (gm > GROUP) gm = GROUP;
    int in = tile - g * group_size;
    tm = first_m + in % gm;
    tn = in / gm;
}

// K-major tiles keep k contiguous, one row per m/n index.  With BK = 16 a
// row is 16 floats and its four 16-byte chunks are stored XOR-swizzled by
// (row/2) % 4: the 8 lanes an LDS cycle serves then touch 32 distinct banks
// both when a store covers two whole rows and when a fragment read takes one
// chunk of 8 consecutive rows (a 4-float row pad, the BK = 32 layout, leaves
// every store 2-way conflicted at BK = 16).
template <int BK>
__device__ __forceinline__ int kmajor_slot(int row, int chunk) {
    if (BK == 16) return row * 16 + 4 * (chunk ^ ((row >> 1) & 3));
    return row * (BK + 4) + 4 * chunk;
}

template <int R, int BK, bool KMAJOR>
struct TileLds {
    // KMAJOR: [R][BK] swizzled (BK = 16) or [R][BK+4]; else [BK][R] (m/n contiguous)
    static constexpr int SIZE = KMAJOR ? R * (BK == 16 ? BK : BK + 4) : BK * R;
};

// Interleaved fragments.  An MN-contiguous operand whose wave block is two
// 32-wide MFMA blocks (64 rows of A or columns of B) is read with block b
// taking rows rb0 + 2*(l%32) + b: one 64-bit LDS read per k-step then feeds
// both blocks (4 reads per 8-k chunk instead of 8 32-bit ones; LM-head dX /
// dW +2.7 / +3.5 %).  Each output element still sums its k in the same
// order, so the results are the same bits.  Only where the results leave
// through LDS (gemm_store_lds), which places every value at its real row
// and column; the epilogue's other paths map rows and columns the same way.
template <int TA, int TB, int BM, int BN, int BK>
struct GemmIlv {
    static constexpr int ASZ = TileLds<BM, BK, TA == 0>::SIZE, BSZ = TileLds<BN, BK, TB == 1>::SIZE;
    static constexpr bool LDS_STORE = 4 * 32 * (BN / 2) <= 2 * (ASZ + BSZ);
    static constexpr bool A = TA == 1 && BM == 128 && LDS_STORE;
    static constexpr bool B = TB == 0 && BN == 128 && LDS_STORE;
};

// Load one operand tile (R rows of m/n, BK of k) from global memory into
// registers.  KMAJOR: element (r, k) at base[r*ld + k]; else base[k*ld + r].
template <int R, int BK, bool KMAJOR, bool ALIGNED>
__device__ __forceinline__ void load_tile(const float* __restrict__ base, int ld, int r0, int rlim, int k0,
                                          int klim, f32x4* regs) {
    constexpr int NL = R * BK / 4 / 256;
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        int idx = t + i * 256;
        int r, k;
        if (KMAJOR) { r = idx / (BK / 4); k = (idx % (BK / 4)) * 4; }
        else { k = idx / (R / 4); r = (idx % (R / 4)) * 4; }
        int gr = r0 + r, gk = k0 + k;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (KMAJOR) {
            if (gr < rlim) {
                const float* src = base + (long long)gr * ld + gk;
                if (ALIGNED && gk + 3 < klim) {
                    v = *(const f32x4*)src;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = (gk + e < klim) ? src[e] : 0.f;
                }
            }
        } else {
            if (gk < klim) {
                const float* src = base + (long long)gk * ld + gr;
                if (ALIGNED && gr + 3 < rlim) {
                    v = *(const f32x4*)src;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) v[e] = (gr + e < rlim) ? src[e] : 0.f;
                }
            }
        }
        regs[i] = v;
    }
}

template <int R, int BK, bool KMAJOR>
__device__ __forceinline__ void store_tile(float* lds, const f32x4* regs) {
    constexpr int NL = R * BK / 4 / 256;
    const int t = threadIdx.x;
#pragma unroll
    for (int i = 0; i < NL; i++) {
        int idx = t + i * 256;
        if (KMAJOR) {
            int r = idx / (BK / 4), c = idx % (BK / 4);
            *(f32x4*)(lds + kmajor_slot<BK>(r, c)) = regs[i];
        } else {
            int k = idx / (R / 4), r = (idx % (R / 4)) * 4;
            *(f32x4*)(lds + k * R + r) = regs[i];
        }
    }
}

// Operand values of one 32-row MFMA block for the 4 steps of an 8-k chunk.
template <int R, int BK, bool KMAJOR>
__device__ __forceinline__ f32x4 fetch_frag(const float* lds, int rb, int kk, int lane) {
    const int row = rb + (lane & 31);
    const int kq = kk + 4 * (lane >> 5);
    if (KMAJOR) {
        return *(const f32x4*)(lds + kmajor_slot<BK>(row, kq >> 2));
    } else {
        f32x4 v;
#pragma unroll
        for (int s = 0; s < 4; s++) v[s] = lds[(kq + s) * R + row];
        return v;
    }
}

template <int R, int BK, bool KMAJOR, int NF, bool ILV = false>
__device__ __forceinline__ void fetch_frags(const float* lds, int rb0, int kk, int lane, f32x4 (&f)[NF]) {
    if constexpr (ILV) {
        static_assert(!KMAJOR && NF == 2, "interleaved fragments: MN-contiguous operand, two blocks");
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        const int kq = kk + 4 * (lane >> 5);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const f32x2 v = *(const f32x2*)(lds + (kq + s) * R + rb0 + 2 * (lane & 31));
            f[0][s] = v[0];
            f[1][s] = v[1];
        }
    } else {
#pragma unroll
        for (int i = 0; i < NF; i++) f[i] = fetch_frag<R, BK, KMAJOR>(lds, rb0 + i * 32, kk, lane);
    }
}

// Unchecked loads over whole BK steps: each thread streams f32x4s through
// fixed row pointers.  The k-range must lie inside the matrix; rows (KMAJOR)
// or columns (m/n-contiguous) past rlim are redirected to row rlim - 1 /
// column 0, so an edge tile reads only valid memory and its extra rows /
// columns hold copies that only reach the C rows / columns the epilogue
// does not store.  (A float4 that straddles rlim stays inside the row: the
// aligned kernels require ld % 4 == 0, so ld >= rlim rounded up to 4.)
template <int R, int BK, bool KMAJOR>
struct TileStream {
    static constexpr int NL = R * BK / 4 / 256;
    const float* ptr[NL];
    long long step;
    // glu_F (m/n-major, R = 64): the tile's columns 0..31 are gate columns
    // r0/2 .. of [gate | up] and 32..63 the matching up columns glu_F + r0/2 ..
    __device__ __forceinline__ void init(const float* __restrict__ base, int ld, int r0, int rlim, int k0,
                                         int glu_F = 0) {
        const int t = threadIdx.x;
#pragma unroll
        for (int i = 0; i < NL; i++) {
            int idx = t + i * 256;
            int r, k;
            if (KMAJOR) { r = idx / (BK / 4); k = (idx % (BK / 4)) * 4; }
            else { k = idx / (R / 4); r = (idx % (R / 4)) * 4; }
            int gr = r0 + r;
            if (!KMAJOR && glu_F) gr = (r < 32 ? 0 : glu_F - 32) + (r0 >> 1) + r;
            if (gr >= rlim) gr = KMAJOR ? rlim - 1 : 0;
            ptr[i] = KMAJOR ? base + (long long)gr * ld + (k0 + k) : base + (long long)(k0 + k) * ld + gr;
        }
        step = KMAJOR ? BK : (long long)BK * ld;
    }
    __device__ __forceinline__ void load(f32x4* regs) {
#pragma unroll
        for (int i = 0; i < NL; i++) {
            regs[i] = *(const f32x4*)ptr[i];
            ptr[i] += step;
        }
    }
};

// Column sums of B over k (TB = 0): every thread's B loads fall on the same
// four columns, so it keeps one f32x4 of running sums, added at the tile
// stores; the end of gemm_body adds up the threads of each column.
template <int BN, int BK, int NLB>
__device__ __forceinline__ void colsum_add(f32x4& cs, const f32x4 (&rb)[NLB]) {
#pragma unroll
    for (int i = 0; i < NLB; i++) cs += rb[i];
}

// Edge tiles and the scalar-load variants: every load checked.
template <int TA, int TB, int BM, int BN, int BK, bool ALIGNED>
__device__ __forceinline__ void gemm_mainloop(const GemmParams& p, const float* A, const float* B, int m0, int n0,
                                              int kb, int ke, float* lds, f32x16 (&acc)[BM / 64][BN / 64],
                                              bool cs_on, f32x4& cs) {
    constexpr bool AK = (TA == 0);   // A K-contiguous
    constexpr bool BK_ = (TB == 1);  // B K-contiguous
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int ASZ = TileLds<BM, BK, AK>::SIZE, BSZ = TileLds<BN, BK, BK_>::SIZE;
    constexpr int NLA = BM * BK / 4 / 256, NLB = BN * BK / 4 / 256;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

    f32x4 ra[NLA > 0 ? NLA : 1], rb[NLB > 0 ? NLB : 1];
    auto gload = [&](int k0) {
        load_tile<BM, BK, AK, ALIGNED>(A, p.lda, m0, p.M, k0, ke, ra);
        load_tile<BN, BK, BK_, ALIGNED>(B, p.ldb, n0, p.N, k0, ke, rb);
    };
    auto lstore = [&](int buf) {
        store_tile<BM, BK, AK>(lds + buf * (ASZ + BSZ), ra);
        store_tile<BN, BK, BK_>(lds + buf * (ASZ + BSZ) + ASZ, rb);
        if (!BK_ && cs_on) colsum_add<BN, BK, (NLB > 0 ? NLB : 1)>(cs, rb);
    };

    const int nk = (ke - kb + BK - 1) / BK;
    if (nk > 0) {
        gload(kb);
        lstore(0);
    }
    __syncthreads();
    for (int kt = 0; kt < nk; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < nk) gload(kb + (kt + 1) * BK);
        const float* la = lds + cur * (ASZ + BSZ);
        const float* lb = la + ASZ;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 8) {
            f32x4 fa[FM], fb[FN];
            fetch_frags<BM, BK, AK, FM, GemmIlv<TA, TB, BM, BN, BK>::A>(la, wm0, kk, lane, fa);
            fetch_frags<BN, BK, BK_, FN, GemmIlv<TA, TB, BM, BN, BK>::B>(lb, wn0, kk, lane, fb);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[j][s], fa[i][s], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) lstore(cur ^ 1);
        __syncthreads();
    }
}


// Interior tiles (every load in bounds, k-range a whole number of BK steps):
// fragments double-buffered per 8-k chunk, next tile stored before the last
// chunk, last chunk's MFMAs after the barrier.
template <int TA, int TB, int BM, int BN, int BK>
__device__ __forceinline__ void gemm_mainloop_full(const GemmParams& p, const float* A, const float* B, int m0,
                                                   int n0, int kb, int ke, float* lds,
                                                   f32x16 (&acc)[BM / 64][BN / 64], bool cs_on, f32x4& cs) {
    constexpr bool AK = (TA == 0);   // A K-contiguous
    constexpr bool BK_ = (TB == 1);  // B K-contiguous
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int ASZ = TileLds<BM, BK, AK>::SIZE, BSZ = TileLds<BN, BK, BK_>::SIZE;
    constexpr int NLA = BM * BK / 4 / 256, NLB = BN * BK / 4 / 256;
    constexpr int NC = BK / 8;
    static_assert(NC % 2 == 0, "fragment buffers alternate per 8-k chunk");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

    f32x4 ra[NLA], rb[NLB];
    TileStream<BM, BK, AK> sa;
    TileStream<BN, BK, BK_> sb;
    sa.init(A, p.lda, m0, p.M, kb);
    sb.init(B, p.ldb, n0, p.N, kb);
    const int nk = (ke - kb) / BK;
    sa.load(ra);
    sb.load(rb);
    store_tile<BM, BK, AK>(lds, ra);
    store_tile<BN, BK, BK_>(lds + ASZ, rb);
    if (!BK_ && cs_on) colsum_add<BN, BK, NLB>(cs, rb);
    if (nk > 1) {
        sa.load(ra);
        sb.load(rb);
    }
    __syncthreads();
    f32x4 fa[2][FM], fb[2][FN];
    fetch_frags<BM, BK, AK, FM, GemmIlv<TA, TB, BM, BN, BK>::A>(lds, wm0, 0, lane, fa[0]);
    fetch_frags<BN, BK, BK_, FN, GemmIlv<TA, TB, BM, BN, BK>::B>(lds + ASZ, wn0, 0, lane, fb[0]);
    for (int kt = 0; kt < nk; kt++) {
        const float* la = lds + (kt & 1) * (ASZ + BSZ);
        float* ln = lds + ((kt & 1) ^ 1) * (ASZ + BSZ);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int u = c & 1, v = u ^ 1;
            if (c + 1 < NC) {
                fetch_frags<BM, BK, AK, FM, GemmIlv<TA, TB, BM, BN, BK>::A>(la, wm0, (c + 1) * 8, lane, fa[v]);
                fetch_frags<BN, BK, BK_, FN, GemmIlv<TA, TB, BM, BN, BK>::B>(la + ASZ, wn0, (c + 1) * 8, lane, fb[v]);
            } else {
                // Last chunk of this tile: its fragments are in registers, so
                // the other buffer can take the next tile before the barrier.
                if (kt + 1 < nk) {
                    store_tile<BM, BK, AK>(ln, ra);
                    store_tile<BN, BK, BK_>(ln + ASZ, rb);
                    if (!BK_ && cs_on) colsum_add<BN, BK, NLB>(cs, rb);
                }
                __syncthreads();
                if (kt + 1 < nk) {
                    fetch_frags<BM, BK, AK, FM, GemmIlv<TA, TB, BM, BN, BK>::A>(ln, wm0, 0, lane, fa[v]);
                    fetch_frags<BN, BK, BK_, FN, GemmIlv<TA, TB, BM, BN, BK>::B>(ln + ASZ, wn0, 0, lane, fb[v]);
                    if (kt + 2 < nk) {
                        sa.load(ra);
                        sb.load(rb);
                    }
                }
            }
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[u][j][s], fa[u][i][s], acc[i][j], 0, 0, 0);
            __builtin_amdgcn_s_setprio(0);
        }
    }
}

// Epilogue: v = alpha*acc (+ beta*C) (+ bias[n]); C = resid + v, for one
// wave's (BM/2)x(BN/2) block at rows r0.., columns c0...
// The MFMAs take the B fragment as their first operand, so each 32x32
// accumulator block holds C^T: lane l owns row m = l%32 of the block and, in
// registers 4g..4g+3, its four consecutive columns 8g + 4*(l/32) + q -- one
// 16-byte run of a row of C.  Where the operands are 16-byte aligned and the
// tile's columns are all in range, each run is read and stored as one f32x4,
// and the loads of two column blocks are issued together ahead of their
// stores (the compiler cannot move a load above a store that may alias it,
// so interleaving them would expose every load's latency).  Everything else
// takes the per-element path.
//
// Where the wave blocks fit in the workgroup's operand LDS (free once the
// main loop's last barrier has passed) and the operands are 16-byte aligned,
// the values go out through LDS instead (gemm_store_lds): a store straight
// from the accumulators covers 32 rows x 32 bytes, one piece of 32 different
// cache lines, while the transposed store covers whole row segments of the
// wave's block.  The arithmetic per element is the same in both paths.
template <int BM, int BN, bool PLAIN, bool ILA, bool ILB>
__device__ __forceinline__ void gemm_store_lds(const GemmParams& p, float* C, const f32x16 (&acc)[BM / 64][BN / 64],
                                               int r0, int c0, int lane, float* lw) {
    constexpr int FM = BM / 64, FN = BN / 64;
    constexpr int W = FN * 32;         // floats per row of the wave's block
    constexpr int CPR = W / 4;         // 16-byte chunks per row (8 or 16)
    constexpr int RPI = 64 / CPR;      // rows per wave-wide store (8 or 4)
    const int half = lane >> 5, ml = lane & 31;
    const int ch = lane % CPR, n = c0 + 4 * ch;
    const bool full = n + 3 < p.N;
    const float* addp = p.beta != 0.f ? C : p.resid;   // the one operand read per element
    const int ldadd = p.beta != 0.f ? p.ldc : p.ldr;
    f32x4 bv = {0.f, 0.f, 0.f, 0.f};
    if (p.bias) {
#pragma unroll
        for (int q = 0; q < 4; q++) bv[q] = n + q < p.N ? p.bias[n + q] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < FM; i++) {
        // 32 rows of the block: lane (ml, half) holds row ml, 16-byte chunks
        // 8j + 2g + half; chunk k of row r sits at chunk k ^ (r % 8), so the
        // 8 lanes an LDS cycle serves hit distinct banks on both sides.
        // Interleaved rows (ILA): this pass's row ml is row 2*ml + i of the
        // wave block.  Interleaved columns (ILB): register q of blocks 0 / 1
        // holds column 2*(8g + 4*half + q) + 0 / 1, so each 16-byte chunk
        // takes two registers of each block.
        if constexpr (ILB) {
#pragma unroll
            for (int g = 0; g < 4; g++)
#pragma unroll
                for (int qp = 0; qp < 4; qp += 2) {
                    const f32x4 v = {p.alpha * acc[i][0][4 * g + qp], p.alpha * acc[i][1][4 * g + qp],
                                     p.alpha * acc[i][0][4 * g + qp + 1], p.alpha * acc[i][1][4 * g + qp + 1]};
                    *(f32x4*)(lw + ml * W + 4 * ((4 * g + 2 * half + qp / 2) ^ (ml & 7))) = v;
                }
        } else {
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    f32x4 v;
#pragma unroll
                    for (int q = 0; q < 4; q++) v[q] = p.alpha * acc[i][j][4 * g + q];
                    *(f32x4*)(lw + ml * W + 4 * ((8 * j + 2 * g + half) ^ (ml & 7))) = v;
                }
        }
        __builtin_amdgcn_wave_barrier();   // one wave's LDS accesses complete in order
        if constexpr (PLAIN) {
            if (r0 + 32 * FM <= p.M && c0 + W <= p.N) {
                // the wave block lies wholly inside C: every row of the pass
                // is read back before the first store, so the stores wait on
                // the LDS once per pass rather than once per row
                f32x4 v[32 / RPI];
#pragma unroll
                for (int it = 0; it < 32 / RPI; it++) {
                    const int rr = it * RPI + lane / CPR;
                    v[it] = *(const f32x4*)(lw + rr * W + 4 * (ch ^ (rr & 7)));
                }
                const int rl = lane / CPR;
                float* dst = C + (long long)(ILA ? r0 + 2 * rl + i : r0 + i * 32 + rl) * p.ldc + n;
                constexpr int STEP = ILA ? 2 * RPI : RPI;   // rows between the pass's stores
#pragma unroll
                for (int it = 0; it < 32 / RPI; it++) *(f32x4*)(dst + (long long)(it * STEP) * p.ldc) = v[it];
                __builtin_amdgcn_wave_barrier();
                continue;
            }
#pragma unroll
            for (int it = 0; it < 32 / RPI; it++) {
                const int rr = it * RPI + lane / CPR;
                const int row = ILA ? r0 + 2 * rr + i : r0 + i * 32 + rr;
                const f32x4 v = *(const f32x4*)(lw + rr * W + 4 * (ch ^ (rr & 7)));
                float* dst = C + (long long)row * p.ldc + n;
                if (row < p.M) {
                    if (full) *(f32x4*)dst = v;
                    else {
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            if (n + q < p.N) dst[q] = v[q];
                    }
                }
            }
            __builtin_amdgcn_wave_barrier();
            continue;
        }
        if (r0 + 32 * FM <= p.M && c0 + W <= p.N) {
            // interior wave block: per group of four rows, every global load
            // (addend rows, RoPE tables) and LDS read is issued before the
            // first store, so no store waits behind the next row's loads
            const bool rope = p.rope_cos && n < p.rope_cols;
#pragma unroll
            for (int it0 = 0; it0 < 32 / RPI; it0 += 4) {
                f32x4 av[4], a[4];
                f32x2 cc[4], ss[4];
                int row[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int rl = (it0 + u) * RPI + lane / CPR;
                    row[u] = ILA ? r0 + 2 * rl + i : r0 + i * 32 + rl;
                    av[u] = f32x4{0.f, 0.f, 0.f, 0.f};
                    if (addp) av[u] = *(const f32x4*)(addp + (long long)row[u] * ldadd + n);
                }
                if (rope) {
#pragma unroll
                    for (int u = 0; u < 4; u++) rope_tab(p, row[u], n, cc[u], ss[u]);
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int rr = (it0 + u) * RPI + lane / CPR;
                    a[u] = *(const f32x4*)(lw + rr * W + 4 * (ch ^ (rr & 7)));
                }
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    f32x4 v;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float x = a[u][q];
                        if (p.beta != 0.f) x = x + p.beta * av[u][q];
                        if (p.bias) x = x + bv[q];
                        if (p.resid) x = av[u][q] + x;
                        v[q] = x;
                    }
                    if (rope) rope_rot(v, cc[u], ss[u]);
                    *(f32x4*)(C + (long long)row[u] * p.ldc + n) = v;
                }
            }
            __builtin_amdgcn_wave_barrier();
            continue;
        }
#pragma unroll
        for (int it0 = 0; it0 < 32 / RPI; it0 += 4) {
            f32x4 av[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int rl = (it0 + u) * RPI + lane / CPR;
                const int row = ILA ? r0 + 2 * rl + i : r0 + i * 32 + rl;
                av[u] = f32x4{0.f, 0.f, 0.f, 0.f};
                if (addp && row < p.M) {
                    const float* ap = addp + (long long)row * ldadd + n;
                    if (full) av[u] = *(const f32x4*)ap;
                    else {
#pragma unroll
                        for (int q = 0; q < 4; q++) av[u][q] = n + q < p.N ? ap[q] : 0.f;
                    }
                }
            }
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const int rr = (it0 + u) * RPI + lane / CPR;
                const int row = ILA ? r0 + 2 * rr + i : r0 + i * 32 + rr;
                const f32x4 a = *(const f32x4*)(lw + rr * W + 4 * (ch ^ (rr & 7)));
                if (row >= p.M) continue;
                f32x4 v;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float x = a[q];
                    if (p.beta != 0.f) x = x + p.beta * av[u][q];
                    if (p.bias) x = x + bv[q];
                    if (p.resid) x = av[u][q] + x;
                    v[q] = x;
                }
                if (p.rope_cos && n < p.rope_cols) rope4(p, row, n, v);
                float* dst = C + (long long)row * p.ldc + n;
                if (full) *(f32x4*)dst = v;
                else {
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        if (n + q < p.N) dst[q] = v[q];
                }
            }
        }
        __builtin_amdgcn_wave_barrier();   // this pass's reads before the next pass's writes
    }
}

template <int BM, int BN, bool LDS_STORE = false, bool ILA = false, bool ILB = false>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, float* C, const f32x16 (&acc)[BM / 64][BN / 64],
                                              int r0, int c0, int lane, float* lw = nullptr) {
    constexpr int FM = BM / 64, FN = BN / 64;
    constexpr int JG = FN < 2 ? FN : 2;
    const int half = lane >> 5, ml = lane & 31;
    // the row of accumulator block i in this lane (interleaved fragments:
    // see GemmIlv; their columns are mapped in the paths below)
    auto row_of = [&](int i) { return ILA ? r0 + 2 * ml + i : r0 + i * 32 + ml; };
    // Row statistics: the NT layout only (the host refuses others), so never
    // with interleaved fragments
    if constexpr (!ILA && !ILB) {
    if (p.stats) {
        // Row statistics for a softmax over the row (the LM head's
        // cross-entropy): per row, the max of this wave's BN/2 columns of
        // v = alpha*acc and the sum of exp(v - max); columns >= N are left
        // out ((-inf, 0) when none is in range).  Entry (row, c0 / (BN/2)) =
        // (row, 2*tile column + wave column half).  Only for beta = 0 and no
        // bias / residual (the host asks for it on the LM head only).
        constexpr float L2E = 1.4426950408889634f;
        const int sc = c0 / (BN / 2);
#pragma unroll
        for (int i = 0; i < FM; i++) {
            float mx = -INFINITY;
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++)
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        if (c0 + j * 32 + 8 * g + 4 * half + q < p.N) mx = fmaxf(mx, p.alpha * acc[i][j][4 * g + q]);
            mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
            float sm = 0.f;
            if (mx != -INFINITY) {
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int g = 0; g < 4; g++)
#pragma unroll
                        for (int q = 0; q < 4; q++)
                            if (c0 + j * 32 + 8 * g + 4 * half + q < p.N)
                                sm += __builtin_amdgcn_exp2f((p.alpha * acc[i][j][4 * g + q] - mx) * L2E);
            }
            sm += __shfl_xor(sm, 32, WAVE);
            const int row = r0 + i * 32 + ml;
            if (half == 0 && row < p.M) {
                float* st = p.stats + 2 * ((long long)row * p.stats_ld + sc);
                st[0] = mx;
                st[1] = sm;
            }
            if (p.tgt && row < p.M) {
                // the lane holding column t of this row (if the wave's columns
                // include it) leaves that logit, the value C would hold
                const int t = (int)p.tgt[row] - c0;
                if (t >= 0 && t < BN / 2 && ((t >> 2) & 1) == half) {
                    float v = 0.f;
#pragma unroll
                    for (int j = 0; j < FN; j++)
#pragma unroll
                        for (int g = 0; g < 4; g++)
#pragma unroll
                            for (int q = 0; q < 4; q++)
                                if (t == j * 32 + 8 * g + 4 * half + q) v = p.alpha * acc[i][j][4 * g + q];
                    p.tgt_val[row] = v;
                }
            }
        }
        if (p.no_store) return;
    }
    }
    const float* addp = p.beta != 0.f ? C : p.resid;   // the one operand read per element
    const int ldadd = p.beta != 0.f ? p.ldc : p.ldr;
    const bool aligned = !(p.beta != 0.f && p.resid) &&
                         ((reinterpret_cast<uintptr_t>(C) | reinterpret_cast<uintptr_t>(p.resid) |
                           reinterpret_cast<uintptr_t>(p.bias)) & 15) == 0 &&
                         ((p.ldc | (p.resid ? p.ldr : 0)) & 3) == 0;
    if constexpr (LDS_STORE) {
        if (aligned) {   // the same for every wave of the workgroup
            __syncthreads();   // the main loop's LDS tiles (and column sums) are read
            // alpha only (the LM head, the split-K partials): a store loop with
            // no per-element selects
            if (p.beta == 0.f && !p.bias && !p.resid && !p.rope_cos)
                gemm_store_lds<BM, BN, true, ILA, ILB>(p, C, acc, r0, c0, lane, lw);
            else
                gemm_store_lds<BM, BN, false, ILA, ILB>(p, C, acc, r0, c0, lane, lw);
            return;
        }
    }
    if constexpr (!ILA && !ILB) {
        const bool vec = aligned && c0 + BN / 2 <= p.N;
        if (vec) {
#pragma unroll
            for (int i = 0; i < FM; i++) {
                const int row = r0 + i * 32 + ml;
                if (row >= p.M) continue;
                float* crow = C + (long long)row * p.ldc;
                const float* arow = addp + (long long)row * ldadd;
#pragma unroll
                for (int j0 = 0; j0 < FN; j0 += JG) {
                    f32x4 av[JG][4], bv[JG][4];
#pragma unroll
                    for (int jj = 0; jj < JG; jj++)
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            const int n = c0 + (j0 + jj) * 32 + 8 * g + 4 * half;
                            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
                            av[jj][g] = addp ? *(const f32x4*)(arow + n) : z;
                            bv[jj][g] = p.bias ? *(const f32x4*)(p.bias + n) : z;
                        }
#pragma unroll
                    for (int jj = 0; jj < JG; jj++)
#pragma unroll
                        for (int g = 0; g < 4; g++) {
                            f32x4 v;
#pragma unroll
                            for (int q = 0; q < 4; q++) {
                                float x = p.alpha * acc[i][j0 + jj][4 * g + q];
                                if (p.beta != 0.f) x = x + p.beta * av[jj][g][q];
                                if (p.bias) x = x + bv[jj][g][q];
                                if (p.resid) x = av[jj][g][q] + x;
                                v[q] = x;
                            }
                            const int n = c0 + (j0 + jj) * 32 + 8 * g + 4 * half;
                            if (p.rope_cos && n < p.rope_cols) rope4(p, row, n, v);
                            *(f32x4*)(crow + n) = v;
                        }
                }
            }
            return;
        }
    }
    if constexpr (!ILA && !ILB) {
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const int row = r0 + i * 32 + ml;
            if (row >= p.M) continue;
            float* crow = C + (long long)row * p.ldc;
            const float* rrow = p.resid + (long long)row * p.ldr;
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int g = 0; g < 4; g++) {
                    float cv[4], rv[4], bv[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int n = c0 + j * 32 + 8 * g + 4 * half + q;
                        const bool ok = n < p.N;
                        cv[q] = (ok && p.beta != 0.f) ? crow[n] : 0.f;
                        rv[q] = (ok && p.resid) ? rrow[n] : 0.f;
                        bv[q] = (ok && p.bias) ? p.bias[n] : 0.f;
                    }
                    f32x4 v;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        float x = p.alpha * acc[i][j][4 * g + q];
                        if (p.beta != 0.f) x = x + p.beta * cv[q];
                        if (p.bias) x = x + bv[q];
                        if (p.resid) x = rv[q] + x;
                        v[q] = x;
                    }
                    const int n0g = c0 + j * 32 + 8 * g + 4 * half;
                    if (p.rope_cos && n0g < p.rope_cols) rope4(p, row, n0g, v);
#pragma unroll
                    for (int q = 0; q < 4; q++)
                        if (n0g + q < p.N) crow[n0g + q] = v[q];
                }
        }
        return;
    }
    // per element, in groups of four consecutive columns: block j's
    // registers 4g .. 4g+3, or (interleaved columns) registers 4g + qp and
    // 4g + qp + 1 of both blocks
#pragma unroll
    for (int i = 0; i < FM; i++) {
        const int row = row_of(i);
        if (row >= p.M) continue;
        float* crow = C + (long long)row * p.ldc;
        const float* rrow = p.resid + (long long)row * p.ldr;
#pragma unroll
        for (int gi = 0; gi < 4 * FN; gi++) {
            f32x4 a;
            int n0g;
            if constexpr (ILB) {
                const int g = gi >> 1, qp = 2 * (gi & 1);
                a = f32x4{acc[i][0][4 * g + qp], acc[i][1][4 * g + qp], acc[i][0][4 * g + qp + 1],
                          acc[i][1][4 * g + qp + 1]};
                n0g = c0 + 2 * (8 * g + 4 * half + qp);
            } else {
                const int j = gi >> 2, g = gi & 3;
                a = f32x4{acc[i][j][4 * g], acc[i][j][4 * g + 1], acc[i][j][4 * g + 2], acc[i][j][4 * g + 3]};
                n0g = c0 + j * 32 + 8 * g + 4 * half;
            }
            float cv[4], rv[4], bv[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int n = n0g + q;
                const bool ok = n < p.N;
                cv[q] = (ok && p.beta != 0.f) ? crow[n] : 0.f;
                rv[q] = (ok && p.resid) ? rrow[n] : 0.f;
                bv[q] = (ok && p.bias) ? p.bias[n] : 0.f;
            }
            f32x4 v;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float x = p.alpha * a[q];
                if (p.beta != 0.f) x = x + p.beta * cv[q];
                if (p.bias) x = x + bv[q];
                if (p.resid) x = rv[q] + x;
                v[q] = x;
            }
            if (p.rope_cos && n0g < p.rope_cols) rope4(p, row, n0g, v);
#pragma unroll
            for (int q = 0; q < 4; q++)
                if (n0g + q < p.N) crow[n0g + q] = v[q];
        }
    }
}

// SwiGLU epilogue of the gate/up projection (64x64 tiles, the B columns of
// tile tn paired as gate r0/2 + 0..31 and up glu_F + r0/2 + 0..31, see
// TileStream): every wave stores its 32x32 block of C = [gate | up] (+ bias)
// at the real columns, the up waves hand their values to the gate waves
// through LDS, and those store h = (g * sigmoid(g)) * u (feedforward.c:
// 146-150, the order of k_swiglu_fwd) -- the separate SwiGLU pass and its
// re-read of C disappear.
__device__ __forceinline__ void gemm_epilogue_glu(const GemmParams& p, const f32x16& acc, int r0, int tn, int wm,
                                                  int wn, int lane, float* lds) {
    const int half = lane >> 5, ml = lane & 31;
    const int row = r0 + ml;
    const int cb = (wn == 0 ? 0 : p.glu_F) + 32 * tn;
    f32x4 v[4], b[4];
    // the bias loads go out before the first store: a load issued after a
    // store waits behind it (the memory counter is in order)
#pragma unroll
    for (int g = 0; g < 4; g++)
        b[g] = p.bias ? *(const f32x4*)(p.bias + cb + 8 * g + 4 * half) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const int n = cb + 8 * g + 4 * half;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            float x = p.alpha * acc[4 * g + q];
            if (p.bias) x = x + b[g][q];
            v[g][q] = x;
        }
        if (row < p.M) *(f32x4*)(p.C + (long long)row * p.ldc + n) = v[g];
    }
    constexpr int LDX = 36;
    float* xs = lds + wm * 32 * LDX;
    __syncthreads();   // the main loop's last LDS reads are done
    if (wn == 1) {
#pragma unroll
        for (int g = 0; g < 4; g++) *(f32x4*)(xs + ml * LDX + 8 * g + 4 * half) = v[g];
    }
    __syncthreads();
    if (wn == 0 && row < p.M) {
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const f32x4 u = *(const f32x4*)(xs + ml * LDX + 8 * g + 4 * half);
            f32x4 o;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float sg = 1.0f / (1.0f + expf(-v[g][q]));
                o[q] = (v[g][q] * sg) * u[q];
            }
            *(f32x4*)(p.glu_h + (long long)row * p.glu_F + 32 * tn + 8 * g + 4 * half) = o;
        }
    }
}

// As gemm_mainloop_full, with the global loads two tiles ahead: tile j >= 1
// is staged in register set (j - 1) & 1, so the load of tile kt + 3 is
// issued at the end of tile kt and has two tiles of MFMAs to land before
// its LDS store at the end of tile kt + 2.  The k loop is unrolled by two so
// that the register set and the LDS buffer are compile-time indices.
template <int TA, int TB, int BM, int BN, int BK, bool GLU = false>
__device__ __forceinline__ void gemm_mainloop_pf2(const GemmParams& p, const float* A, const float* B, int m0,
                                                  int n0, int kb, int ke, float* lds,
                                                  f32x16 (&acc)[BM / 64][BN / 64], bool cs_on, f32x4& cs) {
    constexpr bool AK = (TA == 0);
    constexpr bool BK_ = (TB == 1);
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int ASZ = TileLds<BM, BK, AK>::SIZE, BSZ = TileLds<BN, BK, BK_>::SIZE;
    constexpr int NLA = BM * BK / 4 / 256, NLB = BN * BK / 4 / 256;
    constexpr int NC = BK / 8;
    static_assert(NC % 2 == 0, "fragment buffers alternate per 8-k chunk");
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

    f32x4 ra[2][NLA], rb[2][NLB];
    TileStream<BM, BK, AK> sa;
    TileStream<BN, BK, BK_> sb;
    sa.init(A, p.lda, m0, p.M, kb);
    sb.init(B, p.ldb, n0, p.N, kb, GLU ? p.glu_F : 0);
    const int nk = (ke - kb) / BK;
    sa.load(ra[0]);
    sb.load(rb[0]);
    store_tile<BM, BK, AK>(lds, ra[0]);
    store_tile<BN, BK, BK_>(lds + ASZ, rb[0]);
    if (!BK_ && cs_on) colsum_add<BN, BK, NLB>(cs, rb[0]);
    if (nk > 1) {
        sa.load(ra[0]);
        sb.load(rb[0]);
    }
    if (nk > 2) {
        sa.load(ra[1]);
        sb.load(rb[1]);
    }
    __syncthreads();
    f32x4 fa[2][FM], fb[2][FN];
    fetch_frags<BM, BK, AK, FM, GemmIlv<TA, TB, BM, BN, BK>::A>(lds, wm0, 0, lane, fa[0]);
    fetch_frags<BN, BK, BK_, FN, GemmIlv<TA, TB, BM, BN, BK>::B>(lds + ASZ, wn0, 0, lane, fb[0]);
    // one tile: kt is computed from LDS buffer S = kt & 1; tile kt + 1 sits in
    // register set S and goes to buffer S ^ 1; set S then takes tile kt + 3
    auto tile = [&](auto S_, int kt) {
        constexpr int S = decltype(S_)::value;
        const float* la = lds + S * (ASZ + BSZ);
        float* ln = lds + (S ^ 1) * (ASZ + BSZ);
#pragma unroll
        for (int c = 0; c < NC; c++) {
            const int u = c & 1, v = u ^ 1;
            if (c + 1 < NC) {
                fetch_frags<BM, BK, AK, FM, GemmIlv<TA, TB, BM, BN, BK>::A>(la, wm0, (c + 1) * 8, lane, fa[v]);
                fetch_frags<BN, BK, BK_, FN, GemmIlv<TA, TB, BM, BN, BK>::B>(la + ASZ, wn0, (c + 1) * 8, lane, fb[v]);
            } else {
                if (kt + 1 < nk) {
                    store_tile<BM, BK, AK>(ln, ra[S]);
                    store_tile<BN, BK, BK_>(ln + ASZ, rb[S]);
                    if (!BK_ && cs_on) colsum_add<BN, BK, NLB>(cs, rb[S]);
                }
                __syncthreads();
                if (kt + 1 < nk) {
                    fetch_frags<BM, BK, AK, FM, GemmIlv<TA, TB, BM, BN, BK>::A>(ln, wm0, 0, lane, fa[v]);
                    fetch_frags<BN, BK, BK_, FN, GemmIlv<TA, TB, BM, BN, BK>::B>(ln + ASZ, wn0, 0, lane, fb[v]);
                    if (kt + 3 < nk) {
                        sa.load(ra[S]);
                        sb.load(rb[S]);
                    }
                }
            }
#pragma unroll
            for (int s = 0; s < 4; s++)
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(fb[u][j][s], fa[u][i][s], acc[i][j], 0, 0, 0);
            // Spread this chunk's memory instructions between its MFMAs:
            // groups of SG MFMAs (2 for the 16-MFMA chunks of 128x128, else
            // 1), 1 LDS read, 1 global load, 1 LDS write (+2-4 % on the
            // LM-head GEMMs against issuing them in one run beside a raised
            // wave priority; the group size measured best per tile).
            constexpr int SG = FM * FN >= 4 ? 2 : 1;
#pragma unroll
            for (int q = 0; q < 4 * FM * FN / SG; q++) {
                __builtin_amdgcn_sched_group_barrier(0x008, SG, 0);  // MFMA
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
                __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);   // global load
                __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);   // LDS write
            }
        }
    };
    for (int kt = 0; kt < nk; kt += 2) {
        tile(std::integral_constant<int, 0>{}, kt);
        if (kt + 1 < nk) tile(std::integral_constant<int, 1>{}, kt + 1);
    }
}

template <int TA, int TB, int BM, int BN, int BK, bool ALIGNED, int PF = 1, bool GLU = false>
__device__ __forceinline__ void gemm_body(const GemmParams& p) {
    constexpr bool AK = (TA == 0);   // A K-contiguous
    constexpr bool BK_ = (TB == 1);  // B K-contiguous
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int ASZ = TileLds<BM, BK, AK>::SIZE, BSZ = TileLds<BN, BK, BK_>::SIZE;
    __shared__ __attribute__((aligned(16))) float lds[2 * (ASZ + BSZ)];

    int tm, tn, split;
    gemm_tile_coords(p, tm, tn, split);
    const int batch = p.splits > 1 ? 0 : (int)blockIdx.z;   // split-K launches are single GEMMs
    const float* A = p.A + batch * p.sA;
    const float* B = p.B + batch * p.sB;
    float* C = p.C + batch * p.sC + split * p.sW;
    const int m0 = tm * BM, n0 = tn * BN;
    const int kb = split * p.kchunk;
    int ke = kb + p.kchunk;
    if (ke > p.K) ke = p.K;

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm0 = (wave >> 1) * WM, wn0 = (wave & 1) * WN;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // The whole BK steps of the k-range take the pipelined, check-free loop
    // (edge tiles included: their out-of-range rows / columns are redirected,
    // see TileStream); a partial last step, and the scalar-load variants,
    // take the guarded loop.
    const int kfull = ke > kb ? kb + (ke - kb) / BK * BK : kb;
    // the first row of tiles also sums B's columns over its k-range
    const bool cs_on = TB == 0 && p.csum != nullptr && tm == 0;
    f32x4 cs = {0.f, 0.f, 0.f, 0.f};
    if constexpr (ALIGNED) {
        if (kfull > kb) {
            if constexpr (PF == 2) gemm_mainloop_pf2<TA, TB, BM, BN, BK, GLU>(p, A, B, m0, n0, kb, kfull, lds, acc, cs_on, cs);
            else gemm_mainloop_full<TA, TB, BM, BN, BK>(p, A, B, m0, n0, kb, kfull, lds, acc, cs_on, cs);
        }
        if (kfull < ke) {
            if (kfull > kb) __syncthreads();   // every wave is done reading the loop's LDS tiles
            gemm_mainloop<TA, TB, BM, BN, BK, true>(p, A, B, m0, n0, kfull, ke, lds, acc, cs_on, cs);
        }
    } else {
        gemm_mainloop<TA, TB, BM, BN, BK, false>(p, A, B, m0, n0, kb, ke, lds, acc, cs_on, cs);
    }
    if (TB == 0 && cs_on) {
        // threads t, t + BN/4, ... hold the same four columns: add them in
        // thread order through LDS (free after the main loop's last barrier)
        constexpr int G = BN / 4, R = 256 / G;
        f32x4* xs = reinterpret_cast<f32x4*>(lds);
        xs[threadIdx.x] = cs;
        __syncthreads();
        if (threadIdx.x < G) {
            f32x4 t = xs[threadIdx.x];
#pragma unroll
            for (int j = 1; j < R; j++) t += xs[threadIdx.x + j * G];
            float* dst = p.splits > 1 ? C + (long long)p.M * p.ldc : p.csum;
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (n0 + 4 * threadIdx.x + e < p.N) dst[n0 + 4 * threadIdx.x + e] = t[e];
        }
    }

    if constexpr (GLU) {
        static_assert(BM == 64 && BN == 64 && PF == 2 && ALIGNED, "SwiGLU epilogue: 64x64 pipelined tiles");
        gemm_epilogue_glu(p, acc[0][0], m0 + wm0, tn, wave >> 1, wave & 1, lane, lds);
    } else {
        // the transposed store needs 32 rows of every wave's block in the operand LDS
        constexpr bool LDS_STORE = 4 * 32 * (BN / 2) <= 2 * (ASZ + BSZ);
        using Ilv = GemmIlv<TA, TB, BM, BN, BK>;
        static_assert(Ilv::LDS_STORE == LDS_STORE, "one rule for the transposed store");
        gemm_epilogue<BM, BN, LDS_STORE, Ilv::A, Ilv::B>(p, C, acc, m0 + wm0, n0 + wn0, lane,
                                                         lds + wave * 32 * (BN / 2));
    }
}

#define GEMM_KERNEL(NAME, TA, TB, BM, BN, BK, AL, WPE, PF)                             \
    extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(WPE))) \
    NAME(GemmParams p) {                                                                 \
        gemm_body<TA, TB, BM, BN, BK, AL, PF>(p);                                        \
    }

#define GEMM_LAYOUTS(TILE, BM, BN, BK, WPE, PF)                                         \
    GEMM_KERNEL(k_gemm_nn_##TILE, 0, 0, BM, BN, BK, true, WPE, PF)                      \
    GEMM_KERNEL(k_gemm_nt_##TILE, 0, 1, BM, BN, BK, true, WPE, PF)                      \
    GEMM_KERNEL(k_gemm_tn_##TILE, 1, 0, BM, BN, BK, true, WPE, PF)

// name: k_gemm_<layout>_<BM>x<BN>[_k32][_u]
//   _k32: 32-deep k step (one barrier per 32 k instead of 16)
//   _u:   unaligned operands (scalar loads), 16-deep k step
// Waves own (BM/2)x(BN/2).  WPE is the register budget as resident waves per
// SIMD: the largest count the variant's LDS allows (2 for the
// 8-accumulator-block 256x128 / 128x256 tiles), short of spilling.  PF is the
// interior loop's global-load distance in tiles (2 where the second staging
// register set fits the budget: 2-5 % faster on the model's shapes).
GEMM_LAYOUTS(256x128, 256, 128, 16, 2, 1)
GEMM_LAYOUTS(128x256, 128, 256, 16, 2, 1)
GEMM_LAYOUTS(128x128, 128, 128, 16, 3, 2)
GEMM_LAYOUTS(128x128_k32, 128, 128, 32, 2, 1)
GEMM_LAYOUTS(64x128, 64, 128, 16, 4, 1)
GEMM_LAYOUTS(64x128_k32, 64, 128, 32, 2, 2)
GEMM_LAYOUTS(64x64, 64, 64, 16, 5, 1)
GEMM_LAYOUTS(64x64_k32, 64, 64, 32, 4, 2)
// the gate/up projection with the SwiGLU epilogue (host: K % 32 == 0, N = 2F, F % 32 == 0)
extern "C" __global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
k_gemm_nn_64x64_k32_glu(GemmParams p) {
    gemm_body<0, 0, 64, 64, 32, true, 2, true>(p);
}
GEMM_KERNEL(k_gemm_nn_64x64_u, 0, 0, 64, 64, 16, false, 1, 1)
GEMM_KERNEL(k_gemm_nt_64x64_u, 0, 1, 64, 64, 16, false, 1, 1)
GEMM_KERNEL(k_gemm_tn_64x64_u, 1, 0, 64, 64, 16, false, 1, 1)
GEMM_KERNEL(k_gemm_tt_64x64_u, 1, 1, 64, 64, 16, false, 1, 1)

// out[m,n] = alpha * sum_s W[s][m,n] (+ beta*out) (+ bias[n]); out = resid + v.
// Partials are summed in split order, so the result is reproducible.
extern "C" __global__ void __launch_bounds__(256)
k_gemm_splitk_reduce(const float* __restrict__ W, int splits, long long sW, float* __restrict__ C, int M, int N,
                     int ldc, float alpha, float beta, const float* __restrict__ bias,
                     const float* __restrict__ resid, int ldr, float* __restrict__ csum) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const long long rows = M + (csum ? 1 : 0);   // row M: the splits' column-sum partials
    if (i >= rows * N) return;
    int m = (int)(i / N), n = (int)(i - (long long)m * N);
    float s = W[i];
    for (int k = 1; k < splits; k++) s += W[k * sW + i];
    if (m == M) {
        csum[n] = s;
        return;
    }
    float v = alpha * s;
    float* dst = C + (long long)m * ldc + n;
    if (beta != 0.f) v = v + beta * *dst;
    if (bias) v = v + bias[n];
    if (resid) v = resid[(long long)m * ldr + n] + v;
    *dst = v;
}

// The same reduction four consecutive columns per thread (host: N, ldc, ldr
// multiples of 4 and every pointer 16-byte aligned): 16-byte loads of every
// split, the splits' loads issued four at a time ahead of their additions,
// each column's sum still taken in split order and its epilogue in the
// scalar kernel's order, so the results are the same bits.
extern "C" __global__ void __launch_bounds__(256)
k_gemm_splitk_reduce4(const float* __restrict__ W, int splits, long long sW, float* __restrict__ C, int M, int N,
                      int ldc, float alpha, float beta, const float* __restrict__ bias,
                      const float* __restrict__ resid, int ldr, float* __restrict__ csum) {
    const long long i = 4 * ((long long)blockIdx.x * blockDim.x + threadIdx.x);
    const long long rows = M + (csum ? 1 : 0);
    if (i >= rows * N) return;
    const int m = (int)(i / N), n = (int)(i - (long long)m * N);
    f32x4 s = *(const f32x4*)(W + i);
    int k = 1;
    for (; k + 4 <= splits; k += 4) {
        f32x4 w[4];
#pragma unroll
        for (int u = 0; u < 4; u++) w[u] = *(const f32x4*)(W + (long long)(k + u) * sW + i);
#pragma unroll
        for (int u = 0; u < 4; u++) s += w[u];
    }
    for (; k < splits; k++) s += *(const f32x4*)(W + (long long)k * sW + i);
    if (m == M) {
        *(f32x4*)(csum + n) = s;
        return;
    }
    float* dst = C + (long long)m * ldc + n;
    const f32x4 c = beta != 0.f ? *(const f32x4*)dst : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 b = bias ? *(const f32x4*)(bias + n) : f32x4{0.f, 0.f, 0.f, 0.f};
    const f32x4 r = resid ? *(const f32x4*)(resid + (long long)m * ldr + n) : f32x4{0.f, 0.f, 0.f, 0.f};
    f32x4 o;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        float v = alpha * s[q];
        if (beta != 0.f) v = v + beta * c[q];
        if (bias) v = v + b[q];
        if (resid) v = r[q] + v;
        o[q] = v;
    }
    *(f32x4*)dst = o;
}

// Writes the raw accumulator of one MFMA whose A and B operands are the
// lane's own values, so a host test can confirm the operand/result lane
// layout the GEMMs assume.  out: [64 lanes][16 registers].
extern "C" __global__ void k_mfma_layout_probe(const float* a, const float* b, float* out) {
    int l = threadIdx.x;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; r++) acc[r] = 0.f;
    acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[l], b[l], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; r++) out[l * 16 + r] = acc[r];
}
