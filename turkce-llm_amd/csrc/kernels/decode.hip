// decode.hip -- KV-cache decode on MI355X.
//
// The reference generates by recomputing the whole window each step
// (training/generate.c:186-212: lm_forward over the context, then
// sample_next on the last row).  Here every layer keeps its rotated keys and
// its values in a cache, [B][H][ctx][hd] per layer, so a step costs one
// token's projections plus one pass over the cached keys/values -- an HBM
// bound pass (decode attention reads ctx*hd*8 bytes per head and sequence).
//
// Kernels (the step itself is in decode_fused.hip):
//   k_cache_fill        prefill: copy K, V of a [B*len, 3D] qkv into the cache
//   k_argmax_hist       greedy generation: pick -> next ids and history
//   k_gather_rows       last prompt row of every sequence
//   k_sample_rows       sample_next (generate.c:57-73) on the device
#include "common.h"

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

// Greedy pick per row (argmax_finish's rule, as k_argmax_rows), written
// both as the next step's input ids[row] and into hist[row*hist_ld + step]
// with step = *pos_dev - pos_base, so generation needs no host round trip.
#define ARGMAX_THREADS 1024
#define ARGMAX_UNROLL 8
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
        // ARGMAX_UNROLL float4s per thread in flight at once (loads from
        // clamped valid addresses first, then the compares in index order)
        constexpr int U = ARGMAX_UNROLL;
        const int nq = V >> 2;
        for (int q0 = threadIdx.x; q0 < nq; q0 += U * ARGMAX_THREADS) {
            f32x4 v[U];
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int q = q0 + u * ARGMAX_THREADS;
                v[u] = *(const f32x4*)(z + 4 * (q < nq ? q : q0));
            }
#pragma unroll
            for (int u = 0; u < U; u++) {
                const int q = q0 + u * ARGMAX_THREADS;
                if (q < nq) {
#pragma unroll
                    for (int e = 0; e < 4; e++)
                        if (v[u][e] > best) { best = v[u][e]; idx = 4 * q + e; }
                }
            }
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
