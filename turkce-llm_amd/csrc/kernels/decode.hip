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
//   k_sample_exp        sample_next's exponentials, spread over the GPU
//   k_sample_rows       sample_next (generate.c:57-73) on the device
//   k_sample_hist       sampled generation: pick -> next ids and history
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

// (float)dec_m_exp(x) -- m_expf's bits -- without the series' fifteen
// divisions where that is safe.  For x in [-110, 0] (every sampling input,
// (z - max) / temperature with temperature > 0, above float underflow):
// y = 2^k p(r), x = k ln2 + r with a two-part ln2 and |r| <= ln2/2, p the
// degree-14 Taylor polynomial in Horner form (coefficients 1/n!): relative
// error below 1e-14.  m_exp's own result is within 3e-14 of exp(x) there: its
// r = x - fl(k ln2_f64) carries at most 159 * 2.3e-17 + 2^-53 * 128 of
// absolute error (the subtraction is exact by Sterbenz for |x| >= 0.7), its
// series under 15 roundings.  So when y lies farther than 4e-13 y from the
// midpoint between the float it rounds to and that float's neighbour on y's
// side, m_exp(x) rounds to the same float; otherwise (about one input in
// 10^5) the series itself is evaluated.  Below -110 both give 0 (exp(-110)
// is far under half the smallest float); NaN and positive inputs take the
// series.
__device__ float sample_expf(float xf) {
#pragma clang fp contract(off)
    const double x = (double)xf;
    if (!(x >= -110.0 && x <= 0.0)) return x < -110.0 ? 0.0f : (float)dec_m_exp(x);
    const double LN2_HI = 0.69314718055994529, LN2_LO = 2.3190468138462996e-17;
    const double k = __builtin_rint(x * 1.4426950408889634);
    double r = __builtin_fma(-k, LN2_HI, x);
    r = __builtin_fma(-k, LN2_LO, r);
    const double c[15] = {1.0, 1.0, 0.5, 1.6666666666666666e-1, 4.1666666666666664e-2, 8.3333333333333332e-3,
                          1.3888888888888889e-3, 1.9841269841269841e-4, 2.4801587301587302e-5,
                          2.7557319223985893e-6, 2.7557319223985888e-7, 2.5052108385441720e-8,
                          2.0876756987868100e-9, 1.6059043836821613e-10, 1.1470745597729725e-11};
    double pp = c[14];
#pragma unroll
    for (int n = 13; n >= 0; n--) pp = __builtin_fma(pp, r, c[n]);
    const double y = __builtin_ldexp(pp, (int)k);
    const float f = (float)y;
    const double fd = (double)f;
    const int fb = __float_as_int(f);
    const double nb = y >= fd ? (double)__int_as_float(fb + 1) : (double)__int_as_float(fb > 0 ? fb - 1 : 0);
    const double mid = 0.5 * (fd + nb);
    if (__builtin_fabs(y - mid) > 4e-13 * y) return f;
    return (float)dec_m_exp(x);
}

// ---- sample_next (training/generate.c:57-73) on the device.  Per row:
//   max_v = max_j z_j;  e_j = m_expf((z_j - max_v) / temperature)   (f32)
//   total = sum_j (f64)e_j  and  c_j = sum_{i<=j} (f64)e_i, both sequential
//   r = u * total (u = pcg_uniform);  pick = first j with c_j >= r, else V-1
// The sequential f64 sums are what fix the pick; computing them on one thread
// is a 31,769-long chain of dependent adds.  The kernel finds the pick from
// prefix sums formed in parallel instead (each thread's contiguous chunk in
// order, then the chunk sums scanned across lanes and waves), and proves that
// the sequential sums give the same pick.  Every term is >= 0, so for any
// order of summation a sum whose terms each pass through at most d roundings
// is within d 2^-53 / (1 - d 2^-53) of the exact sum S (relative):
//   sequential c_j:  d <= j, and c_j is non-decreasing (fl is monotone);
//   parallel P_j:    d <= 2C + 6 + 16 (the chunk twice, the lane scan, the
//                    wave totals; C columns a thread);
//   r = fl(u fl(total)) and r' = fl(u P_V): within (V + 2C + 24) 2^-53 of
//   u S_V.
// With j* the first index whose P_j reaches r', the sequential pick is j*
// when P_j* (1 - g_j*) >= r' + E_r and P_{j*-1} (1 + g_{j*-1}) < r' - E_r,
// g_j = (j + 2C + 200) 2^-52 and E_r = (V + 2C + 200) 2^-52 r' (generous
// versions of the bounds above).  When a row's margin is smaller than that
// (about one row in 10^6 at V = 31,769), or its sums are not finite (a
// temperature of 0 or NaN logits), the row falls back to the sequential sums
// on one thread, exactly as the reference computes them.  fallback_all = 1
// takes the sequential path for every row (for tests of the two paths).
//
// The exponentials (the reference's f64 Taylor m_expf) are formed first by
// k_sample_exp over SAMPLE_CHUNKS workgroups per row, so a batch of 64 rows
// fills the GPU, into the per-row scratch e.  The pick then takes one
// 1024-thread block per row (k_sample_rows / k_sample_hist); its thread t
// owns the contiguous columns [t*C, t*C + C), C = ceil(V / 1024) rounded up
// to a multiple of 4 (e rows have the logits' stride), and prefix holds the
// sequential fallback's c_j.
#define SAMPLE_THREADS 1024
#define SAMPLE_CHUNKS 8

// e[row][j] = m_expf((z_j - max_v) / temperature) for the columns of chunk
// blockIdx.y of row blockIdx.x (each workgroup forms the row's max itself:
// the value of a max does not depend on the order, for rows without NaN).
// Workgroup i goes to XCD i % 8, so with the row as the x index (64 rows, a
// multiple of 8) a row's chunks share one XCD's L2 for those reads.
extern "C" __global__ void __launch_bounds__(SAMPLE_THREADS)
k_sample_exp(const float* __restrict__ logits, int ld, int V, float temperature, float* __restrict__ e) {
    // e rows have the logits' stride ld (a multiple of 4), for 16-byte reads
    constexpr int NW = SAMPLE_THREADS / 64;
    __shared__ float red[NW];
    const int row = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float* z = logits + (long long)row * ld;
    float mx = -INFINITY;
    // float4 reads, 8 in flight per thread (clamped addresses, masked after)
    const int nq = V >> 2;
    for (int q0 = t; q0 < nq; q0 += 8 * SAMPLE_THREADS) {
        f32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int q = q0 + u * SAMPLE_THREADS;
            v[u] = *(const f32x4*)(z + 4 * (q < nq ? q : q0));
        }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (q0 + u * SAMPLE_THREADS < nq) mx = fmaxf(fmaxf(mx, fmaxf(v[u][0], v[u][1])), fmaxf(v[u][2], v[u][3]));
    }
    for (int j = 4 * nq + t; j < V; j += SAMPLE_THREADS) mx = fmaxf(mx, z[j]);
    mx = wave_max(mx);
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < NW; w++) mx = fmaxf(mx, red[w]);
    const int cw = (V + SAMPLE_CHUNKS - 1) / SAMPLE_CHUNKS;
    const int c0 = blockIdx.y * cw, c1 = min(c0 + cw, V);
    float* er = e + (long long)row * ld;
    for (int j = c0 + t; j < c1; j += SAMPLE_THREADS) er[j] = sample_expf((z[j] - mx) / temperature);
}

// The pick of one row from its e (block-wide; every thread returns it).
// (inlined: as a called function it would need a stack, i.e. scratch memory
// that the runtime sets up on the kernel's first launch)
__device__ __forceinline__ int sample_row(int V, double u, const float* __restrict__ er, double* __restrict__ pr,
                                          int fallback_all) {
#pragma clang fp contract(off)
    constexpr int NW = SAMPLE_THREADS / 64;
    __shared__ double wsum[NW];
    __shared__ int cand[NW];
    __shared__ int result;
    __shared__ double total_s;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    // thread t: columns [j0, j0 + C), C a multiple of 4 (er is 16-byte aligned)
    const int C = ((V + SAMPLE_THREADS - 1) / SAMPLE_THREADS + 3) & ~3;
    const int j0 = t * C;
    // one batch of 8 float4 loads in flight (clamped valid addresses; columns
    // >= V count as 0)
    auto load8 = [&](int q0, f32x4 (&v)[8]) {
#pragma unroll
        for (int u8 = 0; u8 < 8; u8++) {
            const int jj = j0 + q0 + 4 * u8;
            v[u8] = *(const f32x4*)(er + (jj < V && q0 + 4 * u8 < C ? jj : 0));
        }
    };
    double cs = 0.0;
    for (int q0 = 0; q0 < C; q0 += 32) {
        f32x4 v[8];
        load8(q0, v);
#pragma unroll
        for (int u8 = 0; u8 < 8; u8++)
#pragma unroll
            for (int c4 = 0; c4 < 4; c4++) {
                const int q = q0 + 4 * u8 + c4;
                if (q < C && j0 + q < V) cs += (double)v[u8][c4];
            }
    }
    // exclusive scan of the chunk sums: inclusive within the wave by lane
    // shuffles, then the wave totals in wave order through LDS
    double inc = cs;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double prev = __shfl_up(inc, o, WAVE);
        if (lane >= o) inc = prev + inc;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    double tot = 0.0, wbase = 0.0;
#pragma unroll
    for (int w = 0; w < NW; w++) {
        if (w == wave) wbase = tot;
        tot += wsum[w];
    }
    double base = wbase + __shfl_up(inc, 1, WAVE);
    if (lane == 0) base = wbase;
    const bool finite = tot == tot && tot < INFINITY && tot > 0.0;
    const double rr = u * tot;
    // the first column whose parallel prefix reaches r'
    int found = 0x7fffffff;
    double s_at = 0.0, s_before = 0.0;
    if (finite && !fallback_all && base + cs >= rr) {
        double P = base;
        for (int q0 = 0; q0 < C && found == 0x7fffffff; q0 += 32) {
            f32x4 v[8];
            load8(q0, v);
#pragma unroll
            for (int u8 = 0; u8 < 8; u8++)
#pragma unroll
                for (int c4 = 0; c4 < 4; c4++) {
                    const int q = q0 + 4 * u8 + c4, jj = j0 + q;
                    if (found == 0x7fffffff && q < C && jj < V) {
                        const double Pn = P + (double)v[u8][c4];
                        if (Pn >= rr) {
                            found = jj;
                            s_at = Pn;
                            s_before = P;
                        }
                        P = Pn;
                    }
                }
        }
    }
    int m = found;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) m = min(m, __shfl_xor(m, o, WAVE));
    if (lane == 0) cand[wave] = m;
    __syncthreads();
    m = cand[0];
#pragma unroll
    for (int w = 1; w < NW; w++) m = min(m, cand[w]);
    if (t == 0) result = -1;
    __syncthreads();
    if (found != 0x7fffffff && found == m) {
        const double eps = 0x1p-52, slack = (double)(2 * C + 200);
        const double Er = ((double)V + slack) * eps * rr;
        bool ok = s_at - ((double)m + slack) * eps * s_at >= rr + Er;
        if (m > 0) ok = ok && s_before + ((double)m + slack) * eps * s_before < rr - Er;
        if (ok) result = m;
    }
    __syncthreads();
    if (result >= 0) return result;
    // fallback: the reference's sequential sums, one thread
    if (t == 0) {
        double c = 0.0;
        for (int j = 0; j < V; j++) {
            c += (double)er[j];
            pr[j] = c;
        }
        total_s = c;
    }
    __syncthreads();
    const double r = u * total_s;
    int best = 0x7fffffff;
    for (int j = t; j < V; j += SAMPLE_THREADS)
        if (pr[j] >= r) { best = j; break; }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) best = min(best, __shfl_xor(best, o, WAVE));
    if (lane == 0) cand[wave] = best;
    __syncthreads();
    best = cand[0];
#pragma unroll
    for (int w = 1; w < NW; w++) best = min(best, cand[w]);
    return best == 0x7fffffff ? V - 1 : best;
}

// One block per row, after k_sample_exp: out[row] = sample_next's pick with
// u[row].  e and prefix are per-row scratch ([rows][V] floats / doubles).
extern "C" __global__ void __launch_bounds__(SAMPLE_THREADS)
k_sample_rows(int V, int ld, const double* __restrict__ u, const float* __restrict__ e, double* __restrict__ prefix,
              unsigned* __restrict__ out, int fallback_all) {
    const int row = blockIdx.x;
    const int k = sample_row(V, u[row], e + (long long)row * ld, prefix + (long long)row * V, fallback_all);
    if (threadIdx.x == 0) out[row] = (unsigned)k;
}

// Sampled generation: the pick of step s = *pos_dev - pos_base uses
// u_all[s * rows + row], and goes to the next step's ids[row] and to
// hist[row * hist_ld + s], as k_argmax_hist does for greedy picks.
extern "C" __global__ void __launch_bounds__(SAMPLE_THREADS)
k_sample_hist(int V, int ld, const double* __restrict__ u_all, const float* __restrict__ e,
              double* __restrict__ prefix, unsigned* __restrict__ ids, unsigned* __restrict__ hist, int hist_ld,
              const int* __restrict__ pos_dev, int pos_base, int fallback_all) {
    const int row = blockIdx.x;
    const int s = *pos_dev - pos_base;
    const int k = sample_row(V, u_all[(long long)s * gridDim.x + row], e + (long long)row * ld,
                             prefix + (long long)row * V, fallback_all);
    if (threadIdx.x == 0) {
        ids[row] = (unsigned)k;
        hist[(long long)row * hist_ld + s] = (unsigned)k;
    }
}
