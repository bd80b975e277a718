// decode.hip -- KV-cache decode on MI355X.
//
// The reference generates by recomputing the whole window each step
// (training/generate.c:186-212: lm_forward over the context, then
// sample_next on the last row).  Here every layer keeps its rotated keys and
// its values in a cache, [B][H][ctx][hd] per layer, so a step costs one
// token's projections plus one pass over the cached keys/values -- an HBM
// bound pass (decode attention reads ctx*hd*8 bytes per head and sequence).
//
// Kernels:
//   k_cache_fill        prefill: copy K, V of a [B*len, 3D] qkv into the cache
//   k_decode_qkv_append step: RoPE the new q, k at position pos (same
//                       arithmetic as the QKV GEMM's RoPE epilogue), append k, v to the cache
//   k_decode_attn_hd*   step: one (sequence, head, context chunk) per block;
//                       writes the chunk's (max, sum, unnormalised O)
//   k_decode_merge_hd*  step: combines the chunks in chunk order
//   k_decode_advance    step: moves the device-resident position on
//   k_argmax_hist       greedy generation: pick -> next ids and history
//   k_gather_rows       last prompt row of every sequence
//   k_sample_rows       sample_next (generate.c:57-73) on the device
#include "common.h"

#define DEC_LOG2E 1.4426950408889634f

// kc/vc[((b*H + h)*ctx + t)*hd + d] = K/V of token t of sequence b, from
// qkv[(b*len + t)*ldq + {D, 2D} + h*hd + d]; float4 per thread.
extern "C" __global__ void __launch_bounds__(256)
k_cache_fill(const float* __restrict__ qkv, int ldq, int B, int len, int H, int hd, int D, float* __restrict__ kc,
             float* __restrict__ vc, int ctx) {
    const int q4 = hd >> 2;
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long total = (long long)B * len * H * q4;
    if (i >= total) return;
    int c = (int)(i % q4);
    long long rest = i / q4;
    int h = (int)(rest % H);
    rest /= H;
    int t = (int)(rest % len);
    int b = (int)(rest / len);
    const float* row = qkv + ((long long)b * len + t) * ldq + h * hd + 4 * c;
    long long dst = (((long long)b * H + h) * ctx + t) * hd + 4 * c;
    *(f32x4*)(kc + dst) = *(const f32x4*)(row + D);
    *(f32x4*)(vc + dst) = *(const f32x4*)(row + 2 * D);
}

// One thread per (sequence b, head h, pair k): rotate q and k of the new
// token (row b of qkv) by position pos = *pos_dev as the QKV GEMM epilogue does,
// write q back, append the rotated k and the v pair at cache position pos.
// The position lives in device memory so that a captured step replays
// unchanged (k_decode_advance moves it on).
extern "C" __global__ void __launch_bounds__(256)
k_decode_qkv_append(float* __restrict__ qkv, int ldq, const float* __restrict__ cos_t,
                    const float* __restrict__ sin_t, const int* __restrict__ pos_dev, int B, int H, int hd, int D,
                    float* __restrict__ kc, float* __restrict__ vc, int ctx) {
    const int half = hd >> 1;
    const int pos = *pos_dev;
    int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= B * H * half) return;
    int k = i % half, h = (i / half) % H, b = i / (half * H);
    float c = cos_t[pos * half + k], s = sin_t[pos * half + k];
    float* row = qkv + (long long)b * ldq;
    float* q = row + h * hd + 2 * k;
    float* kk = row + D + h * hd + 2 * k;
    const float* v = row + 2 * D + h * hd + 2 * k;
    float a0 = q[0], a1 = q[1];
    q[0] = a0 * c - a1 * s;
    q[1] = a0 * s + a1 * c;
    a0 = kk[0]; a1 = kk[1];
    long long dst = (((long long)b * H + h) * ctx + pos) * hd + 2 * k;
    kc[dst] = a0 * c - a1 * s;
    kc[dst + 1] = a0 * s + a1 * c;
    vc[dst] = v[0];
    vc[dst + 1] = v[1];
}

// grid (B*H, nsplit), 256 threads.  Block (bh, s) covers keys
// [s*chunk, min((s+1)*chunk, n)) of sequence b, head h, for the query in
// row b of qkv, with n = *pos_dev + 1 (blocks past n write an empty chunk).  Lanes work in groups of LPR = HD/4 lanes per key row
// (float4 each, so a wave instruction reads whole rows, coalesced);
// a wave takes every 4th group of RPI = 64/LPR rows.  Output per block:
// part[(bh*nsplit + s)*(HD + 4) + {0..HD-1, HD, HD+1}] = O (unnormalised),
// m (base-2 max of the scaled scores), l (sum of 2^(score - m)).
// chunk <= 1024.  Every reduction has a fixed order.
template <int HD>
__device__ void decode_attn(const float* __restrict__ qkv, int ldq, const float* __restrict__ kc,
                            const float* __restrict__ vc, const int* __restrict__ pos_dev, int ctx, int H, int chunk,
                            float scale, float* __restrict__ part) {
    const int n = *pos_dev + 1;
    constexpr int LPR = HD / 4, RPI = 64 / LPR;
    __shared__ float sc[1024];
    __shared__ float red[8];
    __shared__ f32x4 oacc[4][LPR];
    const int bh = blockIdx.x, s = blockIdx.y, nsplit = gridDim.y;
    const int b = bh / H, h = bh - b * H;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane / LPR, c4 = lane % LPR;
    const int k0 = s * chunk;
    int k1 = k0 + chunk;
    if (k1 > n) k1 = n;
    const int cnt = k1 > k0 ? k1 - k0 : 0;
    const float c2 = scale * DEC_LOG2E;
    const long long cbase = ((long long)bh * ctx) * HD;
    const f32x4 q = *(const f32x4*)(qkv + (long long)b * ldq + h * HD + 4 * c4);

    // scores: a wave's rows of NIT iterations are loaded together (their
    // latency overlaps), then reduced across the LPR lanes of each row
    constexpr int NIT = 256 / (4 * RPI);
    for (int g0 = 0; g0 < cnt; g0 += NIT * 4 * RPI) {
        f32x4 kv[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int j = g0 + it * 4 * RPI + wave * RPI + sub;
            kv[it] = j < cnt ? *(const f32x4*)(kc + cbase + (long long)(k0 + j) * HD + 4 * c4)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int j = g0 + it * 4 * RPI + wave * RPI + sub;
            float d = kv[it][0] * q[0] + kv[it][1] * q[1] + kv[it][2] * q[2] + kv[it][3] * q[3];
#pragma unroll
            for (int o = 1; o < LPR; o <<= 1) d += __shfl_xor(d, o, WAVE);
            if (c4 == 0 && j < cnt) sc[j] = d * c2;
        }
    }
    __syncthreads();
    // max and sum of 2^(score - max) over the chunk (fixed order)
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < cnt; j += 256) mx = fmaxf(mx, sc[j]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float ls = 0.f;
    for (int j = threadIdx.x; j < cnt; j += 256) {
        float e = exp2f(sc[j] - mx);
        sc[j] = e;
        ls += e;
    }
    ls = wave_sum(ls);
    if (lane == 0) red[4 + wave] = ls;
    __syncthreads();
    // O = sum_j p_j V_j
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    for (int g0 = 0; g0 < cnt; g0 += NIT * 4 * RPI) {
        f32x4 vv[NIT];
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int j = g0 + it * 4 * RPI + wave * RPI + sub;
            vv[it] = j < cnt ? *(const f32x4*)(vc + cbase + (long long)(k0 + j) * HD + 4 * c4)
                             : f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int it = 0; it < NIT; it++) {
            const int j = g0 + it * 4 * RPI + wave * RPI + sub;
            if (j < cnt) o += sc[j] * vv[it];
        }
    }
#pragma unroll
    for (int w = LPR; w < 64; w <<= 1) {
        o[0] += __shfl_xor(o[0], w, WAVE);
        o[1] += __shfl_xor(o[1], w, WAVE);
        o[2] += __shfl_xor(o[2], w, WAVE);
        o[3] += __shfl_xor(o[3], w, WAVE);
    }
    if (sub == 0) oacc[wave][c4] = o;
    __syncthreads();
    float* dst = part + ((long long)bh * nsplit + s) * (HD + 4);
    if (threadIdx.x < LPR) {
        f32x4 t = oacc[0][threadIdx.x];
        t += oacc[1][threadIdx.x];
        t += oacc[2][threadIdx.x];
        t += oacc[3][threadIdx.x];
        *(f32x4*)(dst + 4 * threadIdx.x) = t;
    }
    if (threadIdx.x == 0) {
        dst[HD] = mx;
        dst[HD + 1] = ((red[4] + red[5]) + red[6]) + red[7];
    }
}

// One wave per (sequence, head): att[b, h*HD + d] = sum_s w_s O_s[d] /
// sum_s w_s l_s with w_s = 2^(m_s - max_s m_s), over the chunks that hold
// keys (n = *pos_dev + 1), in order; records are nsplit_grid per head.
template <int HD>
__device__ void decode_merge(const float* __restrict__ part, const int* __restrict__ pos_dev, int chunk,
                             int nsplit_grid, int H, int D, float* __restrict__ att) {
    const int bh = blockIdx.x, b = bh / H, h = bh - b * H;
    const int d = threadIdx.x;
    const int nsplit = (*pos_dev + chunk) / chunk;
    const float* p = part + (long long)bh * nsplit_grid * (HD + 4);
    float M = -INFINITY;
    for (int s = 0; s < nsplit; s++) M = fmaxf(M, p[s * (HD + 4) + HD]);
    float L = 0.f, o = 0.f;
    for (int s = 0; s < nsplit; s++) {
        const float m = p[s * (HD + 4) + HD];
        const float w = (m == -INFINITY) ? 0.f : exp2f(m - M);
        L += w * p[s * (HD + 4) + HD + 1];
        if (d < HD) o += w * p[s * (HD + 4) + d];
    }
    if (d < HD) att[(long long)b * D + h * HD + d] = o / L;
}

#define DECODE_KERNELS(HD)                                                                                  \
    extern "C" __global__ void __launch_bounds__(256)                                                       \
    k_decode_attn_hd##HD(const float* qkv, int ldq, const float* kc, const float* vc, const int* pos_dev,   \
                         int ctx, int H, int chunk, float scale, float* part) {                             \
        decode_attn<HD>(qkv, ldq, kc, vc, pos_dev, ctx, H, chunk, scale, part);                             \
    }                                                                                                       \
    extern "C" __global__ void __launch_bounds__(64)                                                        \
    k_decode_merge_hd##HD(const float* part, const int* pos_dev, int chunk, int nsplit_grid, int H, int D,  \
                          float* att) {                                                                     \
        decode_merge<HD>(part, pos_dev, chunk, nsplit_grid, H, D, att);                                     \
    }

DECODE_KERNELS(16)
DECODE_KERNELS(32)
DECODE_KERNELS(64)

// *pos_dev += 1: the step's token is in the cache.
extern "C" __global__ void k_decode_advance(int* __restrict__ pos_dev) {
    if (threadIdx.x == 0 && blockIdx.x == 0) *pos_dev = *pos_dev + 1;
}

// Greedy pick per row (argmax_finish's rule, as k_argmax_rows), written
// both as the next step's input ids[row] and into hist[row*hist_ld + step]
// with step = *pos_dev - pos_base, so generation needs no host round trip.
#define ARGMAX_THREADS 1024
extern "C" __global__ void __launch_bounds__(ARGMAX_THREADS)
k_argmax_hist(const float* __restrict__ logits, int ld, int V, unsigned* __restrict__ ids,
              unsigned* __restrict__ hist, int hist_ld, const int* __restrict__ pos_dev, int pos_base) {
    constexpr int NW = ARGMAX_THREADS / 64;
    __shared__ float bv[NW];
    __shared__ int bi[NW];
    const float* z = logits + (long long)blockIdx.x * ld;
    float best = -INFINITY;
    int idx = ARGMAX_NONE;
    // each thread scans its float4s in increasing index order, strict > keeps
    // the first occurrence; the reductions prefer the lower index on ties
    if ((ld & 3) == 0) {
        const int nq = V >> 2;
        for (int q = threadIdx.x; q < nq; q += ARGMAX_THREADS) {
            const f32x4 v = *(const f32x4*)(z + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (v[e] > best) { best = v[e]; idx = 4 * q + e; }
        }
        for (int j = 4 * nq + (int)threadIdx.x; j < V; j += ARGMAX_THREADS)
            if (z[j] > best) { best = z[j]; idx = j; }
    } else {
        for (int j = threadIdx.x; j < V; j += ARGMAX_THREADS)
            if (z[j] > best) { best = z[j]; idx = j; }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        float v2 = __shfl_xor(best, o, WAVE);
        int i2 = __shfl_xor(idx, o, WAVE);
        if (v2 > best || (v2 == best && i2 < idx)) { best = v2; idx = i2; }
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) { bv[wave] = best; bi[wave] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float b = bv[0];
        int k = bi[0];
        for (int w = 1; w < NW; w++)
            if (bv[w] > b || (bv[w] == b && bi[w] < k)) { b = bv[w]; k = bi[w]; }
        k = argmax_finish(z, k);
        ids[blockIdx.x] = (unsigned)k;
        hist[(long long)blockIdx.x * hist_ld + (*pos_dev - pos_base)] = (unsigned)k;
    }
}

// dst[i, :] = src[(i*stride + offset), :]  (cols floats per row)
extern "C" __global__ void __launch_bounds__(256)
k_gather_rows(const float* __restrict__ src, int ld, int stride, int offset, int cols, int n, float* __restrict__ dst) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (long long)n * cols) return;
    int r = (int)(i / cols), c = (int)(i - (long long)r * cols);
    dst[i] = src[((long long)r * stride + offset) * ld + c];
}

// ---------------------------------------------------------------- sampling
// The reference's m_expf: (float) of an f64 Taylor series around the
// nearest multiple of ln 2 (runtime/mathlib.c:87-106), restated with the
// same operation order; contraction off so every step rounds as on the CPU.
__device__ double dec_m_exp(double x) {
#pragma clang fp contract(off)
    if (x != x) return x;
    if (x > 709.782712893384) return __longlong_as_double(0x7FF0000000000000ll);
    if (x < -745.1332191019412) return 0.0;
    const double ln2 = 0.69314718055994530942;
    double kf = x / ln2;
    long long k = (long long)(kf + (kf >= 0.0 ? 0.5 : -0.5));
    double r = x - (double)k * ln2;
    double term = 1.0, acc = 1.0;
    for (int i = 1; i < 40; i++) {
        term *= r / (double)i;
        acc += term;
        if (term < 1e-18 && term > -1e-18) break;
    }
    // acc * 2^k by exponent arithmetic, flushing to 0 / inf
    if (acc == 0.0) return 0.0;
    unsigned long long bits = (unsigned long long)__double_as_longlong(acc);
    unsigned long long sgn = bits & 0x8000000000000000ull;
    long long ne = (long long)((bits >> 52) & 0x7FF) + k;
    if (ne >= 0x7FF) return __longlong_as_double((long long)(sgn | 0x7FF0000000000000ull));
    if (ne <= 0) return sgn ? -0.0 : 0.0;
    return __longlong_as_double((long long)(sgn | ((unsigned long long)ne << 52) | (bits & 0x000FFFFFFFFFFFFFull)));
}

// One 256-thread block per row, the reference's sample_next
// (training/generate.c:57-73) with r = u[row] * sum drawn on the host:
//   e_j = m_expf((z_j - max) / temperature)    (parallel, exact per element)
//   prefix_j = sum_{i<=j} (f64)e_i             (one thread, in order -- the
//                                               f64 sums of the reference)
//   out = first j with prefix_j >= r, else V-1
// e and prefix are per-row scratch ([rows][V] floats / doubles).
extern "C" __global__ void __launch_bounds__(256)
k_sample_rows(const float* __restrict__ logits, int ld, int V, float temperature, const double* __restrict__ u,
              float* __restrict__ e, double* __restrict__ prefix, unsigned* __restrict__ out) {
    __shared__ float red[4];
    __shared__ double total;
    __shared__ int found[4];
    const int row = blockIdx.x;
    const float* z = logits + (long long)row * ld;
    float* er = e + (long long)row * V;
    double* pr = prefix + (long long)row * V;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < V; j += 256) mx = fmaxf(mx, z[j]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (int j = threadIdx.x; j < V; j += 256) er[j] = (float)dec_m_exp((double)((z[j] - mx) / temperature));
    __syncthreads();
    if (threadIdx.x == 0) {
        double c = 0.0;
        for (int j = 0; j < V; j++) {
            c += (double)er[j];
            pr[j] = c;
        }
        total = c;
    }
    __syncthreads();
    const double r = u[row] * total;
    // first index whose prefix reaches r (prefixes never decrease)
    int best = 0x7fffffff;
    for (int j = threadIdx.x; j < V; j += 256)
        if (pr[j] >= r) { best = j; break; }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) best = min(best, __shfl_xor(best, o, WAVE));
    if (lane == 0) found[wave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        int k = min(min(found[0], found[1]), min(found[2], found[3]));
        out[row] = (unsigned)(k == 0x7fffffff ? V - 1 : k);
    }
}
