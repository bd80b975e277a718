// rowops.hip -- HBM-bound row and elementwise kernels of the training step.
//
// Counterparts of the reference's non-GEMM kernels (train_kernels.cu:498-800),
// laid out for wave64: one wavefront per row for the D=384 row reductions,
// float4 accesses where rows are 16-byte aligned, and fixed-order
// reductions everywhere (no atomics), so reruns are bit-identical.
#include "common.h"

// ---------------------------------------------------------------- embedding
// x[n, :] = E[ids[n], :]  (train_kernels.cu:724-730). Bit-exact gather.
extern "C" __global__ void __launch_bounds__(256)
k_embed_fwd(const float* __restrict__ E, const unsigned* __restrict__ ids, float* __restrict__ x, int rows, int D) {
    if ((D & 3) == 0) {
        long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;   // float4 index
        int q = D >> 2;
        if (i >= (long long)rows * q) return;
        long long n = i / q;
        int j = (int)(i - n * q);
        ((f32x4*)x)[i] = ((const f32x4*)E)[(long long)ids[n] * q + j];
    } else {
        long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
        if (i >= (long long)rows * D) return;
        long long n = i / D;
        int j = (int)(i - n * D);
        x[i] = E[(long long)ids[n] * D + j];
    }
}

// dE[tok, j] += sum of dx[n, j] over the rows n holding tok, in ascending n
// (embedding.c:4-15, train_kernels.cu:736-740).  The host groups rows by token
// (stable counting sort): order[] lists row indices, segment s covers
// order[seg_start[s] .. seg_start[s+1]) and belongs to token seg_tok[s].
// One thread per (segment, column): no two threads touch the same output.
extern "C" __global__ void __launch_bounds__(256)
k_embed_bwd(const float* __restrict__ dx, const unsigned* __restrict__ order, const unsigned* __restrict__ seg_start,
            const unsigned* __restrict__ seg_tok, int nseg, float* __restrict__ dE, int D) {
    int s = blockIdx.x;
    int j = blockIdx.y * blockDim.x + threadIdx.x;
    if (s >= nseg || j >= D) return;
    float* dst = dE + (long long)seg_tok[s] * D + j;
    float acc = *dst;
    unsigned e = seg_start[s + 1];
    for (unsigned k = seg_start[s]; k < e; k++) acc += dx[(long long)order[k] * D + j];
    *dst = acc;
}

// ---------------------------------------------------------------- RMSNorm
// out = (x * r) * w with r = 1/sqrt(mean(x^2) + eps), r saved per row
// (tensor.c:217-234, train_kernels.cu:535-547).  One wavefront per row;
// sqrt in f64 then rounded, as the reference does.
extern "C" __global__ void __launch_bounds__(256)
k_rmsnorm_fwd(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ out,
              float* __restrict__ rinv, int rows, int cols, float eps) {
    int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + (long long)row * cols;
    float* orow = out + (long long)row * cols;
    if ((cols & 3) == 0 && cols <= 1024) {
        // the row in registers: float4 chunks q = lane + 64*i
        const int c4 = cols >> 2;
        f32x4 v[4];
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = lane + 64 * i;
            v[i] = q < c4 ? *(const f32x4*)(xr + 4 * q) : f32x4{0.f, 0.f, 0.f, 0.f};
            ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
        }
        ss = wave_sum(ss);
        float r = 1.0f / (float)sqrt((double)(ss / (float)cols + eps));
        if (lane == 0) rinv[row] = r;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = lane + 64 * i;
            if (q < c4) {
                f32x4 wv = *(const f32x4*)(w + 4 * q);
                f32x4 o;
#pragma unroll
                for (int e = 0; e < 4; e++) o[e] = v[i][e] * r * wv[e];
                *(f32x4*)(orow + 4 * q) = o;
            }
        }
        return;
    }
    float ss = 0.f;
    for (int i = lane; i < cols; i += 64) ss += xr[i] * xr[i];
    ss = wave_sum(ss);
    float ms = ss / (float)cols;
    float r = 1.0f / (float)sqrt((double)(ms + eps));
    if (lane == 0) rinv[row] = r;
    for (int i = lane; i < cols; i += 64) orow[i] = xr[i] * r * w[i];
}

// dx = dxin + (w*r*dy - (r^3/cols)*x*S), S = sum(dy*w*x)  (model_ops.c:89-117,
// train_kernels.cu:552-569: the reference adds into dx in place; here the
// incoming gradient dxin is a separate buffer, or zero when dxin is null).
// The weight gradient dy*x*r is reduced over the block's RMS_ROWS rows in
// row order and written as one partial row per block; k_colsum_final adds
// the partials in block order.
#define RMS_ROWS 16
extern "C" __global__ void __launch_bounds__(256)
k_rmsnorm_bwd(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ rinv,
              const float* __restrict__ dy, const float* __restrict__ dxin, float* __restrict__ dx,
              float* __restrict__ wpart, int rows, int cols) {
    extern __shared__ float part[];   // [4][cols]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r0 = blockIdx.x * RMS_ROWS;
    float* mine = part + wave * cols;
    // wave `wave` handles rows r0 + wave*RMS_ROWS/4 .. in order
    if ((cols & 3) == 0 && cols <= 1024) {
        // rows in registers, float4 chunks q = lane + 64*i; the dy*x*r
        // partial of the wave's rows accumulates in registers in row order
        const int c4 = cols >> 2;
        f32x4 wv[4], acc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = lane + 64 * i;
            wv[i] = q < c4 ? *(const f32x4*)(w + 4 * q) : f32x4{0.f, 0.f, 0.f, 0.f};
            acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int rr = 0; rr < RMS_ROWS / 4; rr++) {
            const int row = r0 + wave * (RMS_ROWS / 4) + rr;
            if (row >= rows) break;
            const float* xr = x + (long long)row * cols;
            const float* d = dy + (long long)row * cols;
            const float* gi = dxin + (long long)row * cols;
            float* g = dx + (long long)row * cols;
            f32x4 xv[4], dv[4], gv[4];
            float S = 0.f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = lane + 64 * i;
                const bool ok = q < c4;
                xv[i] = ok ? *(const f32x4*)(xr + 4 * q) : f32x4{0.f, 0.f, 0.f, 0.f};
                dv[i] = ok ? *(const f32x4*)(d + 4 * q) : f32x4{0.f, 0.f, 0.f, 0.f};
                gv[i] = ok && dxin ? *(const f32x4*)(gi + 4 * q) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int e = 0; e < 4; e++) S += dv[i][e] * wv[i][e] * xv[i][e];
            }
            S = wave_sum(S);
            const float r = rinv[row];
            const float c = r * r * r / (float)cols;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int q = lane + 64 * i;
                if (q < c4) {
                    f32x4 o;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        o[e] = gv[i][e] + (wv[i][e] * r * dv[i][e] - c * xv[i][e] * S);
                        acc[i][e] += dv[i][e] * xv[i][e] * r;
                    }
                    *(f32x4*)(g + 4 * q) = o;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int q = lane + 64 * i;
            if (q < c4) *(f32x4*)(mine + 4 * q) = acc[i];
        }
    } else {
        for (int i = lane; i < cols; i += 64) mine[i] = 0.f;
        for (int rr = 0; rr < RMS_ROWS / 4; rr++) {
            int row = r0 + wave * (RMS_ROWS / 4) + rr;
            if (row >= rows) break;
            const float* xr = x + (long long)row * cols;
            const float* d = dy + (long long)row * cols;
            const float* gi = dxin + (long long)row * cols;
            float* g = dx + (long long)row * cols;
            float r = rinv[row];
            float r3 = r * r * r;
            float S = 0.f;
            for (int i = lane; i < cols; i += 64) S += d[i] * w[i] * xr[i];
            S = wave_sum(S);
            float c = r3 / (float)cols;
            for (int j = lane; j < cols; j += 64) {
                g[j] = (dxin ? gi[j] : 0.f) + (w[j] * r * d[j] - c * xr[j] * S);
                mine[j] += d[j] * xr[j] * r;
            }
        }
    }
    __syncthreads();
    for (int j = threadIdx.x; j < cols; j += 256) {
        float s = part[j];
        s += part[cols + j];
        s += part[2 * cols + j];
        s += part[3 * cols + j];
        wpart[(long long)blockIdx.x * cols + j] = s;
    }
}

// ---------------------------------------------------------------- RMSNorm, 16 lanes per row
// The same two kernels for rows of cols % 4 == 0, cols <= 64 * NQ floats:
// 16 lanes per row, 4 rows per wave, 16 rows per 256-thread block, lane s
// of a row holding its float4 chunks s, s + 16, ... (NQ of them, chosen per
// model so that no load is wasted).  Every load of a row is issued before
// any arithmetic, from a clamped (valid) address, and masked afterwards:
// one memory latency per row instead of one per dependent step.  The
// row's reductions are 16-lane butterflies.
__device__ __forceinline__ float rms_sum16(float v) {
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) v += __shfl_xor(v, m, WAVE);
    return v;
}

template <int NQ>
__device__ __forceinline__ void rmsnorm_fwd_q(const float* __restrict__ x, const float* __restrict__ w,
                                              float* __restrict__ out, float* __restrict__ rinv, int rows,
                                              int cols, float eps) {
    const int lane = threadIdx.x & 63, sl = lane & 15;
    int row = blockIdx.x * 16 + (threadIdx.x >> 6) * 4 + (lane >> 4);
    const bool rv = row < rows;
    if (!rv) row = rows - 1;
    const int c4 = cols >> 2;
    const float* xr = x + (long long)row * cols;
    f32x4 v[NQ], wv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int q = sl + 16 * i, qc = q < c4 ? q : 0;
        v[i] = *(const f32x4*)(xr + 4 * qc);
        wv[i] = *(const f32x4*)(w + 4 * qc);
    }
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; i++)
        if (sl + 16 * i < c4) ss += v[i][0] * v[i][0] + v[i][1] * v[i][1] + v[i][2] * v[i][2] + v[i][3] * v[i][3];
    ss = rms_sum16(ss);
    const float r = 1.0f / (float)sqrt((double)(ss / (float)cols + eps));
    if (rv && sl == 0) rinv[row] = r;
    float* orow = out + (long long)row * cols;
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int q = sl + 16 * i;
        if (rv && q < c4) {
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; e++) o[e] = v[i][e] * r * wv[i][e];
            *(f32x4*)(orow + 4 * q) = o;
        }
    }
}

// Backward as k_rmsnorm_bwd; the weight-gradient partial of a wave's four
// rows is added across them by butterfly (rows (0+1)+(2+3)), and the four
// waves' partials in wave order, into the block's partial row.
template <int NQ>
__device__ __forceinline__ void rmsnorm_bwd_q(const float* __restrict__ x, const float* __restrict__ w,
                                              const float* __restrict__ rinv, const float* __restrict__ dy,
                                              const float* __restrict__ dxin, float* __restrict__ dx,
                                              float* __restrict__ wpart, int rows, int cols) {
    extern __shared__ float part[];   // [4][cols]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, sl = lane & 15;
    int row = blockIdx.x * 16 + wave * 4 + (lane >> 4);
    const bool rv = row < rows;
    if (!rv) row = rows - 1;
    const int c4 = cols >> 2;
    const long long ro = (long long)row * cols;
    f32x4 wv[NQ], xv[NQ], dv[NQ], gv[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int q = sl + 16 * i, qc = q < c4 ? q : 0;
        wv[i] = *(const f32x4*)(w + 4 * qc);
        xv[i] = *(const f32x4*)(x + ro + 4 * qc);
        dv[i] = *(const f32x4*)(dy + ro + 4 * qc);
        gv[i] = dxin ? *(const f32x4*)(dxin + ro + 4 * qc) : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const float r = rinv[row];
    float S = 0.f;
#pragma unroll
    for (int i = 0; i < NQ; i++)
        if (sl + 16 * i < c4)
#pragma unroll
            for (int e = 0; e < 4; e++) S += dv[i][e] * wv[i][e] * xv[i][e];
    S = rms_sum16(S);
    const float c = r * r * r / (float)cols;
    float* g = dx + ro;
#pragma unroll
    for (int i = 0; i < NQ; i++) {
        const int q = sl + 16 * i;
        const bool ok = q < c4;
        f32x4 o, a;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            o[e] = gv[i][e] + (wv[i][e] * r * dv[i][e] - c * xv[i][e] * S);
            a[e] = (rv && ok) ? dv[i][e] * xv[i][e] * r : 0.f;
        }
        if (rv && ok) *(f32x4*)(g + 4 * q) = o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            a[e] += __shfl_xor(a[e], 16, WAVE);
            a[e] += __shfl_xor(a[e], 32, WAVE);
        }
        if (lane < 16 && ok) *(f32x4*)(part + wave * cols + 4 * q) = a;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < cols; j += 256)
        wpart[(long long)blockIdx.x * cols + j] = ((part[j] + part[cols + j]) + part[2 * cols + j]) + part[3 * cols + j];
}

#define RMS_Q_KERNELS(NQ)                                                                                      \
    extern "C" __global__ void __launch_bounds__(256)                                                          \
    k_rmsnorm_fwd_q##NQ(const float* x, const float* w, float* out, float* rinv, int rows, int cols, float eps) { \
        rmsnorm_fwd_q<NQ>(x, w, out, rinv, rows, cols, eps);                                                 \
    }                                                                                                          \
    extern "C" __global__ void __launch_bounds__(256)                                                          \
    k_rmsnorm_bwd_q##NQ(const float* x, const float* w, const float* rinv, const float* dy, const float* dxin, \
                        float* dx, float* wpart, int rows, int cols) {                                          \
        rmsnorm_bwd_q<NQ>(x, w, rinv, dy, dxin, dx, wpart, rows, cols);                                      \
    }
RMS_Q_KERNELS(1)
RMS_Q_KERNELS(2)
RMS_Q_KERNELS(4)
RMS_Q_KERNELS(6)
RMS_Q_KERNELS(8)
RMS_Q_KERNELS(16)

// ---------------------------------------------------------------- column sums
// out[c] (+)= sum over b of partial[b, c] (the RMSNorm weight gradient's
// per-block partials), over the partial rows of row group blockIdx.y
// (rows [y*group_rows, min(nb, (y+1)*group_rows)) -> row y of out).  A block
// covers 64 columns; its 4 wavefronts each add a contiguous quarter of the
// group's rows in order, and the four quarter sums are added in order.
// Loads are issued 16 at a time ahead of their (ordered) additions.  The
// host runs it twice -- 16-row groups over many blocks, then the group sums
// in group order -- so the reduction fills the GPU and keeps a fixed order.
extern "C" __global__ void __launch_bounds__(256)
k_colsum_final(const float* __restrict__ partial, int nb, int cols, float* __restrict__ out, int accumulate,
               int group_rows) {
    __shared__ float red[4][64];
    const int cl = threadIdx.x & 63, q = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl;
    const int g0 = blockIdx.y * group_rows;
    int gn = nb - g0;
    if (gn > group_rows) gn = group_rows;
    partial += (long long)g0 * cols;
    out += (long long)blockIdx.y * cols;
    const int per = (gn + 3) / 4;
    const int b0 = q * per;
    int b1 = b0 + per;
    if (b1 > gn) b1 = gn;
    float s = 0.f;
    if (c < cols) {
        const float* src = partial + c;
        int b = b0;
        for (; b + 16 <= b1; b += 16) {
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; k++) v[k] = src[(long long)(b + k) * cols];
#pragma unroll
            for (int k = 0; k < 16; k++) s += v[k];
        }
        for (; b < b1; b++) s += src[(long long)b * cols];
    }
    red[q][cl] = s;
    __syncthreads();
    if (q == 0 && c < cols) {
        float v = ((red[0][cl] + red[1][cl]) + red[2][cl]) + red[3][cl];
        out[c] = accumulate ? out[c] + v : v;
    }
}

// ---------------------------------------------------------------- SwiGLU
// h = (g * sigmoid(g)) * u over gu = [gate | up] (feedforward.c:146-150).
extern "C" __global__ void __launch_bounds__(256)
k_swiglu_fwd(const float* __restrict__ gu, float* __restrict__ h, int rows, int F) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if ((F & 3) == 0) {   // one float4 of h per thread
        const int q = F >> 2;
        if (i >= (long long)rows * q) return;
        long long n = i / q;
        int j = (int)(i - n * q) * 4;
        f32x4 g = *(const f32x4*)(gu + n * 2 * F + j), u = *(const f32x4*)(gu + n * 2 * F + F + j);
        f32x4 o;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float sg = 1.0f / (1.0f + expf(-g[e]));
            o[e] = (g[e] * sg) * u[e];
        }
        *(f32x4*)(h + n * F + j) = o;
        return;
    }
    if (i >= (long long)rows * F) return;
    long long n = i / F;
    int j = (int)(i - n * F);
    float g = gu[n * 2 * F + j], u = gu[n * 2 * F + F + j];
    float sg = 1.0f / (1.0f + expf(-g));
    h[i] = (g * sg) * u;
}

// Gradients of h = silu(g)*u in the reference autograd order (node.c:81-96,
// 217-226): du = dh*silu; dg = (dh*u)*sg + ((dh*u)*g)*(sg*(1-sg)).
extern "C" __global__ void __launch_bounds__(256)
k_swiglu_bwd(const float* __restrict__ gu, const float* __restrict__ dh, float* __restrict__ dgu, int rows, int F) {
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if ((F & 3) == 0) {   // one float4 of dh per thread
        const int q = F >> 2;
        if (i >= (long long)rows * q) return;
        long long n = i / q;
        int j = (int)(i - n * q) * 4;
        f32x4 g = *(const f32x4*)(gu + n * 2 * F + j), u = *(const f32x4*)(gu + n * 2 * F + F + j);
        f32x4 d = *(const f32x4*)(dh + n * F + j);
        f32x4 dg, du;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float sg = 1.0f / (1.0f + expf(-g[e]));
            float silu_g = d[e] * u[e];
            dg[e] = silu_g * sg + (silu_g * g[e]) * (sg * (1.0f - sg));
            du[e] = d[e] * (g[e] * sg);
        }
        *(f32x4*)(dgu + n * 2 * F + j) = dg;
        *(f32x4*)(dgu + n * 2 * F + F + j) = du;
        return;
    }
    if (i >= (long long)rows * F) return;
    long long n = i / F;
    int j = (int)(i - n * F);
    float g = gu[n * 2 * F + j], u = gu[n * 2 * F + F + j];
    float sg = 1.0f / (1.0f + expf(-g));
    float d = dh[i];
    float silu_g = d * u;
    float gate = silu_g * sg + (silu_g * g) * (sg * (1.0f - sg));
    dgu[n * 2 * F + j] = gate;
    dgu[n * 2 * F + F + j] = d * (g * sg);
}

// ---------------------------------------------------------------- cross-entropy
// One 256-thread block per row of logits [rows, ld] (V valid columns):
//   loss_rows[n] = log(sum exp(z - max)) + max - z[t]      (loss.c:76-104)
//   z <- (softmax(z) - onehot(t)) * grad_scale  if write_grad (loss.c:55-74)
// The max/sum pass is an online (max, scaled-sum) reduction per thread,
// combined across the block in fixed order.
__device__ __forceinline__ void ms_combine(float& m, float& s, float m2, float s2) {
    if (m2 > m) { s = s * expf(m - m2) + s2; m = m2; }
    else if (m2 != -INFINITY) { s = s + s2 * expf(m2 - m); }
}

extern "C" __global__ void __launch_bounds__(256)
k_cross_entropy(float* __restrict__ logits, int ld, const unsigned* __restrict__ targets,
                float* __restrict__ loss_rows, int V, float grad_scale, int write_grad,
                const float* __restrict__ stats, int nst, const float* __restrict__ zt_rows) {
    __shared__ float sm[4], ss[4];
    const long long row = blockIdx.x;
    float* z = logits + row * ld;
    const bool vec = ((ld & 3) == 0);
    float m = -INFINITY, s = 0.f;
    const float L2E = 1.4426950408889634f;
    if (stats) {
        // the LM-head GEMM left (max, sum) per column block of the row:
        // combine them in a fixed order instead of re-reading the logits
        const float* st = stats + 2 * row * nst;
        for (int q = threadIdx.x; q < nst; q += 256) ms_combine(m, s, st[2 * q], st[2 * q + 1]);
    } else if (vec) {
        // per float4: one rescale to the new running max, then four
        // exponentials (exp2 of log2e-scaled differences, one instruction)
        const int nq = (V + 3) >> 2;
        for (int q = threadIdx.x; q < nq; q += 256) {
            f32x4 v = ((const f32x4*)z)[q];
#pragma unroll
            for (int e = 0; e < 4; e++)
                if (4 * q + e >= V) v[e] = -INFINITY;
            const float nm = fmaxf(fmaxf(m, fmaxf(v[0], v[1])), fmaxf(v[2], v[3]));
            s = s * exp2f((m - nm) * L2E) + ((exp2f((v[0] - nm) * L2E) + exp2f((v[1] - nm) * L2E)) +
                                             (exp2f((v[2] - nm) * L2E) + exp2f((v[3] - nm) * L2E)));
            m = nm;
        }
    } else {
        for (int j = threadIdx.x; j < V; j += 256) {
            float x = z[j];
            if (x > m) { s = s * expf(m - x) + 1.f; m = x; }
            else s += expf(x - m);
        }
    }
    // wave-level fixed-order combine
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        float m2 = __shfl_xor(m, o, WAVE), s2 = __shfl_xor(s, o, WAVE);
        float mn = fmaxf(m, m2);
        float a = (m == -INFINITY) ? 0.f : s * expf(m - mn);
        float b = (m2 == -INFINITY) ? 0.f : s2 * expf(m2 - mn);
        m = mn; s = a + b;
    }
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) { sm[wave] = m; ss[wave] = s; }
    __syncthreads();
    float M = sm[0], S = ss[0];
    for (int w = 1; w < 4; w++) ms_combine(M, S, sm[w], ss[w]);
    // zt_rows (with stats, no gradient): the LM-head GEMM left each row's
    // target logit and never wrote the logits.  The loss is stored before
    // the barrier: the target logit's load then has to complete before the
    // other waves start overwriting the row with the gradient.  (With the
    // store after the barrier, the compiler turned the uniform load into a
    // scalar load and sank it below the barrier into thread 0's branch, so it
    // could read the target's gradient instead of its logit.)
    const unsigned t = targets[row];
    if (threadIdx.x == 0) {
        const float zt = zt_rows ? zt_rows[row] : z[t];
        loss_rows[row] = (float)log((double)S) + M - zt;
    }
    __syncthreads();
    if (!write_grad) return;
    float inv = 1.0f / S;
    if (vec) {
        const int nq = ld >> 2;
        for (int q = threadIdx.x; q < nq; q += 256) {
            f32x4 v = ((f32x4*)z)[q];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                int j = 4 * q + e;
                float p = (j < V) ? exp2f((v[e] - M) * L2E) * inv : 0.f;
                if (j == (int)t) p -= 1.0f;
                v[e] = p * grad_scale;
            }
            ((f32x4*)z)[q] = v;
        }
    } else {
        for (int j = threadIdx.x; j < V; j += 256) {
            float p = expf(z[j] - M) * inv;
            if (j == (int)t) p -= 1.0f;
            z[j] = p * grad_scale;
        }
    }
}

// Greedy pick per row: first index of the row maximum (ties -> lowest index),
// NaN and all -inf rows as argmax_finish says.
extern "C" __global__ void __launch_bounds__(256)
k_argmax_rows(const float* __restrict__ logits, int ld, int V, unsigned* __restrict__ out) {
    __shared__ float bv[4];
    __shared__ int bi[4];
    const float* z = logits + (long long)blockIdx.x * ld;
    float best = -INFINITY;
    int idx = ARGMAX_NONE;
    for (int j = threadIdx.x; j < V; j += 256) {
        float v = z[j];
        if (v > best) { best = v; idx = j; }
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
        for (int w = 1; w < 4; w++)
            if (bv[w] > b || (bv[w] == b && bi[w] < k)) { b = bv[w]; k = bi[w]; }
        out[blockIdx.x] = (unsigned)argmax_finish(z, k);
    }
}

// ---------------------------------------------------------------- grad norm
// Per-block partial sums of squares over a fixed 1024x256 grid-stride layout
// (train_kernels.cu:777-784); the host adds the partials in f64 in order.
// Each thread's sum runs over its elements in index order; the loads of 16
// consecutive strides are issued together ahead of their adds.
extern "C" __global__ void __launch_bounds__(256)
k_sumsq_partial(const float* __restrict__ x, long long n, float* __restrict__ partial) {
    __shared__ float ws[4];
    constexpr int U = 16;
    const long long stride = (long long)gridDim.x * blockDim.x;
    long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    float s = 0.f;
    for (; i + (U - 1) * stride < n; i += U * stride) {
        float v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = x[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; u++) s += v[u] * v[u];
    }
    for (; i < n; i += stride) s += x[i] * x[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = ((ws[0] + ws[1]) + ws[2]) + ws[3];
}

// ---------------------------------------------------------------- Adam / AdamW
// adam_update_one (adam.c:80-95) with the clip scale of k_adam
// (train_kernels.cu:787-800).  wd != 0 adds decoupled weight decay:
// p -= lr*m_hat/(sqrt(v_hat)+eps) + (lr*wd)*p; wd = 0 is exactly Adam.
// Contraction is off so each operation rounds as the CPU path does.
__device__ __forceinline__ void adam_one(float& p, float g, float& m, float& v, float lr, float b1, float b2,
                                         float eps, float bc1, float bc2, float gs, float lrwd) {
#pragma clang fp contract(off)
    float gi = g * gs;
    float mi = b1 * m + (1.0f - b1) * gi;
    float vi = b2 * v + (1.0f - b2) * gi * gi;
    m = mi;
    v = vi;
    float mh = mi / bc1;
    float vh = vi / bc2;
    float upd = lr * mh / (__builtin_sqrtf(vh) + eps);
    if (lrwd != 0.f) upd = upd + lrwd * p;
    p = p - upd;
}

__device__ __forceinline__ void adam_body(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m,
                                          float* __restrict__ v, long long n, float lr, float b1, float b2, float eps,
                                          float bc1, float bc2, float grad_scale, float lrwd) {
    long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    long long nq = n >> 2;
    if (q < nq) {
        f32x4 pp = ((f32x4*)p)[q], gg = ((const f32x4*)g)[q], mm = ((f32x4*)m)[q], vv = ((f32x4*)v)[q];
#pragma unroll
        for (int e = 0; e < 4; e++) {
            float a = pp[e], b = mm[e], c = vv[e];
            adam_one(a, gg[e], b, c, lr, b1, b2, eps, bc1, bc2, grad_scale, lrwd);
            pp[e] = a; mm[e] = b; vv[e] = c;
        }
        ((f32x4*)p)[q] = pp; ((f32x4*)m)[q] = mm; ((f32x4*)v)[q] = vv;
    }
    long long tail = nq * 4 + q;
    if (q < (n & 3)) {
        float a = p[tail], b = m[tail], c = v[tail];
        adam_one(a, g[tail], b, c, lr, b1, b2, eps, bc1, bc2, grad_scale, lrwd);
        p[tail] = a; m[tail] = b; v[tail] = c;
    }
}

extern "C" __global__ void __launch_bounds__(256)
k_adam(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m, float* __restrict__ v, long long n,
       float lr, float b1, float b2, float eps, float bc1, float bc2, float grad_scale, float lrwd) {
    adam_body(p, g, m, v, n, lr, b1, b2, eps, bc1, bc2, grad_scale, lrwd);
}

// Same step with the gradient scale read from device memory (the clip scale
// k_norm_clip leaves there), so a queued training step needs no host value.
extern "C" __global__ void __launch_bounds__(256)
k_adam_ds(float* __restrict__ p, const float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
          long long n, float lr, float b1, float b2, float eps, float bc1, float bc2,
          const float* __restrict__ grad_scale, float lrwd) {
    adam_body(p, g, m, v, n, lr, b1, b2, eps, bc1, bc2, *grad_scale, lrwd);
}

// ------------------------------------------------------- queued driver steps
// mean_loss (model/gpu_train.c:478-487) on the device: sequence b's T row
// losses are added in order in f32 and divided by T, then the B means are
// added in order and divided by B -- the host function's operation sequence.
// acc != 0 adds the result onto *out (the validation sum over batches,
// training/train_lm_gpu.c:241-253); otherwise it is stored.  One workgroup:
// up to 256 sequences at a time, each summed by one thread from column
// chunks that the whole workgroup stages in LDS with coalesced loads.
#define LOSS_MEAN_CHUNK 4096
extern "C" __global__ void __launch_bounds__(256)
k_loss_mean(const float* __restrict__ rows, int B, int T, float* __restrict__ out, int acc) {
#pragma clang fp contract(off)
    __shared__ float buf[LOSS_MEAN_CHUNK];
    __shared__ float means[256];
    float total = 0.f;   // thread 0: the in-order sum of the sequence means
    for (int b0 = 0; b0 < B; b0 += 256) {
        const int nb = B - b0 < 256 ? B - b0 : 256;
        const int tc = LOSS_MEAN_CHUNK / nb;
        float s = 0.f;
        for (int t0 = 0; t0 < T; t0 += tc) {
            const int w = T - t0 < tc ? T - t0 : tc;
            __syncthreads();
            for (int e = threadIdx.x; e < nb * w; e += 256) {
                const int r = e / w, c = e - r * w;
                buf[e] = rows[(long long)(b0 + r) * T + t0 + c];
            }
            __syncthreads();
            if ((int)threadIdx.x < nb) {
                // in order; 16 LDS reads in flight ahead of their adds
                const float* q = buf + threadIdx.x * w;
                int c = 0;
                for (; c + 16 <= w; c += 16) {
                    float v[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) v[u] = q[c + u];
#pragma unroll
                    for (int u = 0; u < 16; u++) s += v[u];
                }
                for (; c < w; c++) s += q[c];
            }
        }
        if ((int)threadIdx.x < nb) means[threadIdx.x] = s / (float)T;
        __syncthreads();
        if (threadIdx.x == 0)
            for (int b = 0; b < nb; b++) total += means[b];
    }
    if (threadIdx.x == 0) {
        const float mean = total / (float)B;
        *out = (acc ? *out : 0.0f) + mean;
    }
}

// m_sqrt (runtime/mathlib.c:56-83), the reference's own method: x = m*2^e
// with m in [1,2), e made even, six Newton steps y = (y + m/y)/2 from
// m/2 + 1/2, then y*2^(e/2) through the exponent field (no denormals).
__device__ double ref_sqrt64(double x) {
#pragma clang fp contract(off)
    if (x < 0.0) return __longlong_as_double(0x7FF8000000000000ll);
    const unsigned long long b = (unsigned long long)__double_as_longlong(x);
    const int ex = (int)((b >> 52) & 0x7FF);
    if (x == 0.0 || ex == 0x7FF) return x;
    int e = ex - 1023;
    double m = __longlong_as_double((long long)((b & 0xFFFFFFFFFFFFFull) | (1023ull << 52)));
    if (e & 1) { m *= 2.0; e -= 1; }
    double y = m * 0.5 + 0.5;
    for (int i = 0; i < 6; i++) y = 0.5 * (y + m / y);
    const unsigned long long yb = (unsigned long long)__double_as_longlong(y);
    const long long ne = (long long)((yb >> 52) & 0x7FF) + e / 2;
    if (ne >= 0x7FF) return __longlong_as_double(0x7FF0000000000000ll);
    if (ne <= 0) return 0.0;
    return __longlong_as_double((long long)((yb & 0x800FFFFFFFFFFFFFull) | ((unsigned long long)ne << 52)));
}

// Grad norm (model/gpu_train.c:502-512: the fixed-grid partial sums added in
// block order in f64, then m_sqrt) and the driver's clip scale
// (training/train_lm_gpu.c:218-220: clip/norm in f64, rounded to f32, when
// the norm exceeds clip; 1 otherwise; clip <= 0 never clips).  The
// workgroup stages the partials in LDS; thread 0 adds them in order.
#define NORM_CLIP_CHUNK 4096
extern "C" __global__ void __launch_bounds__(256) k_norm_clip(const float* __restrict__ partial, int n, double clip,
                                                             double* __restrict__ norm_out,
                                                             float* __restrict__ scale_out) {
#pragma clang fp contract(off)
    __shared__ float buf[NORM_CLIP_CHUNK];
    double ss = 0.0;
    for (int i0 = 0; i0 < n; i0 += NORM_CLIP_CHUNK) {
        const int w = n - i0 < NORM_CLIP_CHUNK ? n - i0 : NORM_CLIP_CHUNK;
        __syncthreads();
        for (int e = threadIdx.x; e < w; e += blockDim.x) buf[e] = partial[i0 + e];
        __syncthreads();
        if (threadIdx.x == 0) {
            int e = 0;
            for (; e + 16 <= w; e += 16) {
                float v[16];
#pragma unroll
                for (int u = 0; u < 16; u++) v[u] = buf[e + u];
#pragma unroll
                for (int u = 0; u < 16; u++) ss += (double)v[u];
            }
            for (; e < w; e++) ss += (double)buf[e];
        }
    }
    if (threadIdx.x != 0) return;
    const double nrm = ref_sqrt64(ss);
    *norm_out = nrm;
    *scale_out = (clip > 0.0 && nrm > clip) ? (float)(clip / nrm) : 1.0f;
}

// Element-wise ref_sqrt64 of n values (lets a host test compare the device
// restatement with the host runtime's m_sqrt).
extern "C" __global__ void k_ref_sqrt64(const double* __restrict__ x, double* __restrict__ y, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) y[i] = ref_sqrt64(x[i]);
}
