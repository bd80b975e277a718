/* trlm_oracle.c -- TEST INFRASTRUCTURE ONLY (see trlm_oracle.h).
 *
 * A clean-room CPU restatement of the fp32 CPU path of turkce-llm: the
 * maths and PRNG of runtime/, the model of model/, the autograd order of
 * autograd/node.c and the data-parallel averaging of training/.  It exists
 * to check the HIP path; the product never links it.
 *
 * Faithfulness rules followed throughout:
 *   - fp32 arithmetic in the reference's evaluation order (no FMA
 *     contraction: built with -ffp-contract=off on a target without FMA);
 *   - every dot product is summed sequentially from 0.0f in ascending index
 *     order, as tensor_matmul2d does (tensor/tensor.c:351-373);
 *   - gradients are accumulated with "+=" into zeroed buffers in the order
 *     the reference's topological backward visits the nodes
 *     (autograd/node.c:290-318).
 * Loop orders are rearranged for speed only where the per-element sequence
 * of fp32 operations stays identical (e.g. i-k-j matmul).  Masked attention
 * entries are skipped: the reference's exp(-1e9 - max) is exactly 0
 * (runtime/mathlib.c:142), so they contribute exact zeros.
 */
#include "trlm_oracle.h"

#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ======================= mathlib (runtime/mathlib.c) ======================= */

#define OR_PI 3.14159265358979323846
#define OR_LN2 0.69314718055994530942

static uint64_t f64_to_bits(double x) { uint64_t u; memcpy(&u, &x, 8); return u; }
static double bits_to_f64(uint64_t u) { double x; memcpy(&x, &u, 8); return x; }

static int is_nan64(double x) {
    uint64_t b = f64_to_bits(x);
    return ((b >> 52) & 0x7FF) == 0x7FF && (b & 0x000FFFFFFFFFFFFFull) != 0;
}
static int is_inf64(double x) {
    uint64_t b = f64_to_bits(x);
    return ((b >> 52) & 0x7FF) == 0x7FF && (b & 0x000FFFFFFFFFFFFFull) == 0;
}
static double pos_inf(void) { return bits_to_f64(0x7FF0000000000000ull); }
static double neg_inf(void) { return bits_to_f64(0xFFF0000000000000ull); }
static double qnan(void) { return bits_to_f64(0x7FF8000000000000ull); }

/* x = m * 2^e with m in [1,2) (mathlib.c:82-89). */
static double frac_exp(double x, int* e) {
    uint64_t b = f64_to_bits(x);
    *e = (int)((b >> 52) & 0x7FF) - 1023;
    return bits_to_f64((b & 0x000FFFFFFFFFFFFFull) | (1023ull << 52));
}

/* x * 2^e by exponent arithmetic, flushing to 0 / inf (mathlib.c:91-104). */
static double mul_pow2(double x, int e) {
    if (x == 0.0) return 0.0;
    uint64_t b = f64_to_bits(x);
    uint64_t s = b & 0x8000000000000000ull;
    int64_t ne = (int64_t)((b >> 52) & 0x7FF) + e;
    if (ne >= 0x7FF) return s ? neg_inf() : pos_inf();
    if (ne <= 0) return s ? -0.0 : 0.0;
    return bits_to_f64(s | ((uint64_t)ne << 52) | (b & 0x000FFFFFFFFFFFFFull));
}

/* Newton iteration on the mantissa, 6 steps from m/2+1/2 (mathlib.c:108-135). */
double or_m_sqrt(double x) {
    if (x < 0.0) return qnan();
    if (x == 0.0 || is_nan64(x) || is_inf64(x)) return x;
    int e;
    double m = frac_exp(x, &e);
    if (e & 1) { m *= 2.0; e -= 1; }
    double y = m * 0.5 + 0.5;
    for (int i = 0; i < 6; i++) y = 0.5 * (y + m / y);
    return mul_pow2(y, e / 2);
}

/* Round-to-nearest k = x/ln2, Taylor series of exp(r) (mathlib.c:139-158). */
double or_m_exp(double x) {
    if (is_nan64(x)) return x;
    if (x > 709.782712893384) return pos_inf();
    if (x < -745.1332191019412) return 0.0;
    double kf = x / OR_LN2;
    int64_t k = (int64_t)(kf + (kf >= 0.0 ? 0.5 : -0.5));
    double r = x - (double)k * OR_LN2;
    double term = 1.0, acc = 1.0;
    for (int n = 1; n < 40; n++) {
        term *= r / (double)n;
        acc += term;
        if (term < 1e-18 && term > -1e-18) break;
    }
    return mul_pow2(acc, (int)k);
}

/* atanh series of z = (m-1)/(m+1), m folded into [sqrt2/2, sqrt2) (mathlib.c:162-186). */
double or_m_log(double x) {
    if (is_nan64(x) || x < 0.0) return qnan();
    if (x == 0.0) return neg_inf();
    if (is_inf64(x)) return x;
    int e;
    double m = frac_exp(x, &e);
    if (m > 1.4142135623730951) { m *= 0.5; e += 1; }
    double z = (m - 1.0) / (m + 1.0);
    double z2 = z * z;
    double term = z, acc = z;
    for (int n = 3; n < 60; n += 2) {
        term *= z2;
        double add = term / (double)n;
        acc += add;
        if (add < 1e-18 && add > -1e-18) break;
    }
    return 2.0 * acc + (double)e * OR_LN2;
}

/* exp(e*log(b)) with the integer-exponent sign rule (mathlib.c:194-207). */
double or_m_pow(double b, double e) {
    if (e == 0.0) return 1.0;
    if (b == 0.0) return e > 0.0 ? 0.0 : pos_inf();
    if (b < 0.0) {
        if (e != (double)(int64_t)e) return qnan();
        double mag = or_m_exp(e * or_m_log(-b));
        return (((int64_t)e) % 2 != 0) ? -mag : mag;
    }
    return or_m_exp(e * or_m_log(b));
}

static double sin_series(double t) {   /* mathlib.c:215-225 */
    double t2 = t * t, term = t, acc = t;
    for (int n = 1; n < 20; n++) {
        term *= -t2 / (double)((2 * n) * (2 * n + 1));
        acc += term;
        if (term < 1e-18 && term > -1e-18) break;
    }
    return acc;
}

static double cos_series(double t) {   /* mathlib.c:227-237 */
    double t2 = t * t, term = 1.0, acc = 1.0;
    for (int n = 1; n < 20; n++) {
        term *= -t2 / (double)((2 * n - 1) * (2 * n));
        acc += term;
        if (term < 1e-18 && term > -1e-18) break;
    }
    return acc;
}

/* quadrant reduction by round(x / (pi/2)) (mathlib.c:240-248). */
static double quarter_turns(double x, int* quad) {
    const double half_pi = OR_PI / 2.0;
    double qf = x / half_pi;
    int64_t q = (int64_t)(qf + (qf >= 0.0 ? 0.5 : -0.5));
    double core = x - (double)q * half_pi;
    int64_t r = q % 4;
    if (r < 0) r += 4;
    *quad = (int)r;
    return core;
}

double or_m_sin(double x) {            /* mathlib.c:250-260 */
    if (is_nan64(x) || is_inf64(x)) return qnan();
    int q;
    double c = quarter_turns(x, &q);
    if (q == 0) return sin_series(c);
    if (q == 1) return cos_series(c);
    if (q == 2) return -sin_series(c);
    return -cos_series(c);
}

double or_m_cos(double x) {            /* mathlib.c:262-272 */
    if (is_nan64(x) || is_inf64(x)) return qnan();
    int q;
    double c = quarter_turns(x, &q);
    if (q == 0) return cos_series(c);
    if (q == 1) return -sin_series(c);
    if (q == 2) return -cos_series(c);
    return sin_series(c);
}

/* f32 wrappers round the f64 result once (mathlib.c:290-296). */
float or_m_sqrtf(float x) { return (float)or_m_sqrt((double)x); }
float or_m_expf(float x) { return (float)or_m_exp((double)x); }
float or_m_logf(float x) { return (float)or_m_log((double)x); }
float or_m_powf(float b, float e) { return (float)or_m_pow((double)b, (double)e); }
float or_m_sinf(float x) { return (float)or_m_sin((double)x); }
float or_m_cosf(float x) { return (float)or_m_cos((double)x); }

/* training/lr_schedule.c:6-15: warmup (step+1)/W of peak, then
 * min + (peak-min) * (1 + cos(pi*p))/2 in f64 with p clamped to 1. */
float or_lr_warmup_cosine(uint64_t step, uint64_t warmup, uint64_t total, float peak, float min_lr) {
    if (warmup > 0 && step < warmup) return peak * (float)(step + 1) / (float)warmup;
    if (total <= warmup) return min_lr;
    double p = (double)(step - warmup) / (double)(total - warmup);
    if (p > 1.0) p = 1.0;
    double c = 0.5 * (1.0 + or_m_cos(3.14159265358979323846 * p));
    return (float)((double)min_lr + ((double)peak - (double)min_lr) * c);
}

/* ======================= PCG32 (runtime/prng.c) ======================= */

uint32_t or_pcg_next_u32(OrPcg* r) {     /* prng.c:10-17, pcg_setseq_64_xsh_rr_32 */
    uint64_t old = r->state;
    r->state = old * 6364136223846793005ull + r->inc;
    uint32_t xs = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    uint32_t rot = (uint32_t)(old >> 59u);
    return (xs >> rot) | (xs << ((32u - rot) & 31u));
}

void or_pcg_seed(OrPcg* r, uint64_t initstate, uint64_t initseq) {   /* prng.c:19-31 */
    r->state = 0;
    r->inc = (initseq << 1u) | 1u;
    r->has_cached = 0;
    r->cached = 0.0;
    or_pcg_next_u32(r);
    r->state += initstate;
    or_pcg_next_u32(r);
}

static double pcg_unit(OrPcg* r) { return (double)or_pcg_next_u32(r) * (1.0 / 4294967296.0); }

/* rejection sampling on 64-bit draws (prng.c:51-70). */
int64_t or_pcg_range_i64(OrPcg* r, int64_t lo, int64_t hi) {
    uint64_t range = (uint64_t)(hi - lo);
    if (range == 0) return lo;
    uint64_t threshold = (uint64_t)(-(int64_t)range) % range;
    uint64_t v;
    do {
        uint64_t a = or_pcg_next_u32(r);
        uint64_t b = or_pcg_next_u32(r);
        v = (a << 32) | b;
    } while (v < threshold);
    return lo + (int64_t)(v % range);
}

/* Box-Muller with the second value cached (prng.c:72-94). */
double or_pcg_gaussian(OrPcg* r, double mean, double stddev) {
    double z;
    if (r->has_cached) {
        r->has_cached = 0;
        z = r->cached;
    } else {
        double u1 = pcg_unit(r);
        if (u1 <= 0.0) u1 = 1.0 / 4294967296.0;
        double u2 = pcg_unit(r);
        double rad = or_m_sqrt(-2.0 * or_m_log(u1));
        double th = 2.0 * OR_PI * u2;
        r->cached = rad * or_m_sin(th);
        r->has_cached = 1;
        z = rad * or_m_cos(th);
    }
    return mean + stddev * z;
}

/* ======================= model layout / init ======================= */

enum { K_AN = 0, K_WQKV, K_BQKV, K_WO, K_BO, K_FN, K_WGU, K_BGU, K_WD, K_BD };

uint32_t or_num_params(const OrCfg* c) { return 10u * c->L + 2u; }

/* lm_collect_params order (lm_model.c:134-148). */
uint64_t or_param_layout(const OrCfg* c, uint64_t* offsets, uint64_t* numels) {
    uint64_t D = c->D, F = c->F, n = 0, off = 0;
    uint64_t sizes[10] = { D, D * 3 * D, 3 * D, D * D, D, D, D * 2 * F, 2 * F, F * D, D };
    offsets[n] = off; numels[n] = (uint64_t)c->V * D; off += numels[n]; n++;
    for (uint32_t l = 0; l < c->L; l++)
        for (int k = 0; k < 10; k++) { offsets[n] = off; numels[n] = sizes[k]; off += sizes[k]; n++; }
    offsets[n] = off; numels[n] = D; off += D; n++;
    return off;
}

static void fill_gauss(OrPcg* r, float* dst, uint64_t n) {
    for (uint64_t i = 0; i < n; i++) dst[i] = (float)or_pcg_gaussian(r, 0.0, (double)0.02f);
}
static void fill_const(float* dst, uint64_t n, float v) { for (uint64_t i = 0; i < n; i++) dst[i] = v; }

/* lm_init draw order: embedding, then per layer w_qkv, wo, w_gate_up,
 * w_down; biases 0, norm weights 1 (lm_model.c:57-110). */
void or_lm_init(const OrCfg* c, uint64_t seed_a, uint64_t seed_b, float* params) {
    uint64_t off[10 * 64 + 2], num[10 * 64 + 2];
    or_param_layout(c, off, num);
    OrPcg r;
    or_pcg_seed(&r, seed_a, seed_b);
    fill_gauss(&r, params + off[0], num[0]);
    for (uint32_t l = 0; l < c->L; l++) {
        uint32_t b = 1 + 10 * l;
        fill_const(params + off[b + K_AN], num[b + K_AN], 1.0f);
        fill_gauss(&r, params + off[b + K_WQKV], num[b + K_WQKV]);
        fill_const(params + off[b + K_BQKV], num[b + K_BQKV], 0.0f);
        fill_gauss(&r, params + off[b + K_WO], num[b + K_WO]);
        fill_const(params + off[b + K_BO], num[b + K_BO], 0.0f);
        fill_const(params + off[b + K_FN], num[b + K_FN], 1.0f);
        fill_gauss(&r, params + off[b + K_WGU], num[b + K_WGU]);
        fill_const(params + off[b + K_BGU], num[b + K_BGU], 0.0f);
        fill_gauss(&r, params + off[b + K_WD], num[b + K_WD]);
        fill_const(params + off[b + K_BD], num[b + K_BD], 0.0f);
    }
    fill_const(params + off[1 + 10 * c->L], c->D, 1.0f);
}

/* theta_k = base^(-2k/hd), angle = pos*theta (model/rope.c:4-18). */
void or_rope_tables(uint32_t T, uint32_t hd, float* cos_t, float* sin_t) {
    uint32_t half = hd / 2;
    for (uint32_t p = 0; p < T; p++)
        for (uint32_t k = 0; k < half; k++) {
            float ex = -(2.0f * (float)k) / (float)hd;
            float th = or_m_powf(10000.0f, ex);
            float ang = (float)p * th;
            cos_t[(uint64_t)p * half + k] = or_m_cosf(ang);
            sin_t[(uint64_t)p * half + k] = or_m_sinf(ang);
        }
}

/* window of sequence w: pcg_seed(seed_base*1000003+w, 99+w) (gpu_train.c:296-307,
 * data_parallel.c:110-114). */
void or_sample_batch(const uint32_t* tokens, uint64_t num_tokens, uint32_t T, uint32_t B,
                     uint64_t seed_base, uint32_t* ids, uint32_t* tgt) {
    int64_t max_start = (int64_t)(num_tokens - T - 1);
    for (uint32_t w = 0; w < B; w++) {
        OrPcg r;
        or_pcg_seed(&r, seed_base * 1000003ull + w, 99ull + w);
        int64_t s = or_pcg_range_i64(&r, 0, max_start);
        for (uint32_t t = 0; t < T; t++) {
            ids[(uint64_t)w * T + t] = tokens[s + t];
            tgt[(uint64_t)w * T + t] = tokens[s + t + 1];
        }
    }
}

uint32_t or_argmax(const float* row, uint32_t n) {
    uint32_t best = 0;
    for (uint32_t j = 1; j < n; j++) if (row[j] > row[best]) best = j;
    return best;
}

/* sample_next (training/generate.c:57-73): max of the row; e_j =
 * m_expf((z_j - max) / temperature) summed in f64 in index order;
 * r = pcg_uniform * sum (prng.c:33-36); the first j whose running f64 sum
 * reaches r, else n - 1. */
uint32_t or_sample_next(const float* logits, uint32_t n, float temperature, OrPcg* rng, float* scratch) {
    float mx = logits[0];
    for (uint32_t j = 1; j < n; j++) if (logits[j] > mx) mx = logits[j];
    double sum = 0.0;
    for (uint32_t j = 0; j < n; j++) {
        float e = or_m_expf((logits[j] - mx) / temperature);
        scratch[j] = e;
        sum += (double)e;
    }
    double r = (double)or_pcg_next_u32(rng) * (1.0 / 4294967296.0) * sum;
    double c = 0.0;
    for (uint32_t j = 0; j < n; j++) {
        c += (double)scratch[j];
        if (c >= r) return j;
    }
    return n - 1;
}

/* ======================= dense kernels ======================= */

/* C[M,N] (+)= A @ B where B rows are contiguous (row stride ldb).  Each
 * C[i][j] is 0.0f followed by "+= a[i][k]*b[k][j]" for k ascending -- the
 * per-element order of tensor_matmul2d (tensor.c:359-371), with the j loop
 * innermost so the compiler can vectorise across independent elements. */
static void mm_rows(uint32_t M, uint32_t N, uint32_t K, const float* A, int64_t a_rs, int64_t a_cs,
                    const float* Bm, int64_t ldb, float* C, int64_t ldc) {
    for (uint32_t i = 0; i < M; i++) {
        float* c = C + (int64_t)i * ldc;
        for (uint32_t j = 0; j < N; j++) c[j] = 0.0f;
        for (uint32_t k = 0; k < K; k++) {
            float a = A[(int64_t)i * a_rs + (int64_t)k * a_cs];
            const float* b = Bm + (int64_t)k * ldb;
            for (uint32_t j = 0; j < N; j++) c[j] += a * b[j];
        }
    }
}

/* Out[r][c] = In[c][r], exact copy. */
static void transpose_copy(uint32_t rows_in, uint32_t cols_in, const float* In, int64_t ld_in, float* Out) {
    for (uint32_t r = 0; r < rows_in; r++)
        for (uint32_t c = 0; c < cols_in; c++) Out[(int64_t)c * rows_in + r] = In[(int64_t)r * ld_in + c];
}

void or_matmul(uint32_t M, uint32_t N, uint32_t K, const float* A, int64_t a_rs, int64_t a_cs,
               const float* Bm, int64_t b_rs, int64_t b_cs, float* C) {
    if (b_cs == 1) { mm_rows(M, N, K, A, a_rs, a_cs, Bm, b_rs, C, N); return; }
    float* tmp = (float*)malloc((size_t)K * N * sizeof(float));
    for (uint32_t k = 0; k < K; k++)
        for (uint32_t j = 0; j < N; j++) tmp[(uint64_t)k * N + j] = Bm[(int64_t)k * b_rs + (int64_t)j * b_cs];
    mm_rows(M, N, K, A, a_rs, a_cs, tmp, N, C, N);
    free(tmp);
}

/* tensor_rmsnorm (tensor.c:217-234): r = 1/sqrtf(mean(x^2)+eps), y = x*r*w. */
static float rms_inv(const float* x, uint32_t n, float eps) {
    float ss = 0.0f;
    for (uint32_t i = 0; i < n; i++) ss += x[i] * x[i];
    float ms = ss / (float)n;
    return 1.0f / or_m_sqrtf(ms + eps);
}

static void rmsnorm_fwd(const float* x, const float* w, float* y, uint32_t rows, uint32_t n, float eps) {
    for (uint32_t o = 0; o < rows; o++) {
        const float* xr = x + (uint64_t)o * n;
        float r = rms_inv(xr, n, eps);
        float* yr = y + (uint64_t)o * n;
        for (uint32_t i = 0; i < n; i++) yr[i] = xr[i] * r * w[i];
    }
}

/* backward_rmsnorm (model_ops.c:89-117): dx += w*r*dy - (r^3/n)*x*S, dw += dy*x*r. */
static void rmsnorm_bwd(const float* x, const float* w, const float* dy, float* dx, float* dw,
                        uint32_t rows, uint32_t n, float eps) {
    for (uint32_t o = 0; o < rows; o++) {
        const float* xr = x + (uint64_t)o * n;
        const float* d = dy + (uint64_t)o * n;
        float* g = dx + (uint64_t)o * n;
        float r = rms_inv(xr, n, eps);
        float r3 = r * r * r;
        float S = 0.0f;
        for (uint32_t i = 0; i < n; i++) S += d[i] * w[i] * xr[i];
        for (uint32_t j = 0; j < n; j++) {
            g[j] += w[j] * r * d[j] - (r3 / (float)n) * xr[j] * S;
            dw[j] += d[j] * xr[j] * r;
        }
    }
}

/* backward_add_bias (model_ops.c:44-59): db[j] += g[i][j], rows in order. */
static void bias_grad(const float* g, float* db, uint32_t rows, uint32_t cols) {
    for (uint32_t i = 0; i < rows; i++)
        for (uint32_t j = 0; j < cols; j++) db[j] += g[(uint64_t)i * cols + j];
}

/* ======================= per-sequence model ======================= */

typedef struct Seq {
    const OrCfg* c;
    uint32_t T;
    const float* P;           /* flat params */
    uint64_t off[10 * 64 + 2];
    float* cosT; float* sinT;  /* [T, hd/2] */
    /* saved activations, per layer */
    float **x_in, **n1, **qkv, **Qr, **Kr, **Pm, **att, **x2, **n2, **gu, **sg, **silu, **h;
    float* x_fin; float* nf; float* logits;   /* logits: [T,V] then dlogits */
    float* tmpT;  /* scratch for transposed weights */
} Seq;

static void* xcalloc(uint64_t n) { return calloc((size_t)n, sizeof(float)); }

static void seq_alloc(Seq* s, const OrCfg* c, uint32_t T, const float* P, const float* cosT, const float* sinT) {
    s->c = c; s->T = T; s->P = P;
    uint64_t num[10 * 64 + 2];
    or_param_layout(c, s->off, num);
    s->cosT = (float*)cosT; s->sinT = (float*)sinT;
    uint64_t D = c->D, F = c->F, H = c->H, L = c->L, V = c->V;
    float*** all[] = { &s->x_in, &s->n1, &s->qkv, &s->Qr, &s->Kr, &s->Pm, &s->att, &s->x2, &s->n2, &s->gu, &s->sg, &s->silu, &s->h };
    uint64_t sz[] = { T * D, T * D, T * 3 * D, T * D, T * D, H * (uint64_t)T * T, T * D, T * D, T * D, T * 2 * F, T * F, T * F, T * F };
    for (int a = 0; a < 13; a++) {
        *all[a] = (float**)calloc(L, sizeof(float*));
        for (uint64_t l = 0; l < L; l++) (*all[a])[l] = (float*)xcalloc(sz[a]);
    }
    s->x_fin = (float*)xcalloc(T * D);
    s->nf = (float*)xcalloc(T * D);
    s->logits = (float*)xcalloc((uint64_t)T * V);
    uint64_t big = V * D;
    if (2 * F * D > big) big = 2 * F * D;
    if (3 * D * D > big) big = 3 * D * D;
    s->tmpT = (float*)xcalloc(big);
}

static void seq_free(Seq* s) {
    float** all[] = { s->x_in, s->n1, s->qkv, s->Qr, s->Kr, s->Pm, s->att, s->x2, s->n2, s->gu, s->sg, s->silu, s->h };
    for (int a = 0; a < 13; a++) { for (uint32_t l = 0; l < s->c->L; l++) free(all[a][l]); free(all[a]); }
    free(s->x_fin); free(s->nf); free(s->logits); free(s->tmpT);
}

#define PRM(s, l, k) ((s)->P + (s)->off[1 + 10 * (l) + (k)])

/* C = A[rows, K] @ W[K, N] + b  (node_add_bias(node_matmul2d(...)),
 * attention.c:72, feedforward.c:145,152). */
static void linear(const float* A, const float* W, const float* b, float* C, uint32_t rows, uint32_t K, uint32_t N) {
    mm_rows(rows, N, K, A, K, 1, W, N, C, N);
    for (uint32_t i = 0; i < rows; i++)
        for (uint32_t j = 0; j < N; j++) C[(uint64_t)i * N + j] = C[(uint64_t)i * N + j] + b[j];
}

/* tensor_rope (rope.c:20-40) on a column slice. */
static void rope_fwd(const float* x, int64_t ldx, float* y, uint32_t T, uint32_t hd, const float* ct, const float* st) {
    uint32_t half = hd / 2;
    for (uint32_t p = 0; p < T; p++)
        for (uint32_t k = 0; k < half; k++) {
            float x0 = x[(int64_t)p * ldx + 2 * k], x1 = x[(int64_t)p * ldx + 2 * k + 1];
            float c = ct[(uint64_t)p * half + k], s = st[(uint64_t)p * half + k];
            y[(uint64_t)p * hd + 2 * k] = x0 * c - x1 * s;
            y[(uint64_t)p * hd + 2 * k + 1] = x0 * s + x1 * c;
        }
}

static void seq_forward(Seq* s, const uint32_t* ids) {
    const OrCfg* c = s->c;
    uint32_t T = s->T, D = c->D, H = c->H, F = c->F, V = c->V, hd = D / H;
    const float* E = s->P + s->off[0];
    float scale = 1.0f / or_m_sqrtf((float)hd);
    float* x = s->x_in[0];
    for (uint32_t i = 0; i < T; i++) memcpy(x + (uint64_t)i * D, E + (uint64_t)ids[i] * D, D * sizeof(float));
    float* S = (float*)xcalloc(T);
    for (uint32_t l = 0; l < c->L; l++) {
        x = s->x_in[l];
        rmsnorm_fwd(x, PRM(s, l, K_AN), s->n1[l], T, D, c->eps);
        linear(s->n1[l], PRM(s, l, K_WQKV), PRM(s, l, K_BQKV), s->qkv[l], T, D, 3 * D);
        float* att = s->att[l];
        for (uint32_t h = 0; h < H; h++) {
            float* Q = s->Qr[l] + (uint64_t)h * T * hd;
            float* K = s->Kr[l] + (uint64_t)h * T * hd;
            const float* Vv = s->qkv[l] + 2 * D + h * hd;
            rope_fwd(s->qkv[l] + h * hd, 3 * D, Q, T, hd, s->cosT, s->sinT);
            rope_fwd(s->qkv[l] + D + h * hd, 3 * D, K, T, hd, s->cosT, s->sinT);
            float* Pm = s->Pm[l] + (uint64_t)h * T * T;
            for (uint32_t i = 0; i < T; i++) {
                /* scores = (q.k)*scale + mask, softmax (attention.c:101-105,
                 * tensor.c:192-215); entries j > i are exactly 0. */
                for (uint32_t j = 0; j <= i; j++) {
                    float acc = 0.0f;
                    for (uint32_t k = 0; k < hd; k++) acc += Q[(uint64_t)i * hd + k] * K[(uint64_t)j * hd + k];
                    S[j] = acc * scale + 0.0f;
                }
                float mx = S[0];
                for (uint32_t j = 1; j <= i; j++) if (S[j] > mx) mx = S[j];
                float sum = 0.0f;
                float* prow = Pm + (uint64_t)i * T;
                for (uint32_t j = 0; j <= i; j++) { float e = or_m_expf(S[j] - mx); prow[j] = e; sum += e; }
                for (uint32_t j = 0; j <= i; j++) prow[j] /= sum;
                for (uint32_t j = i + 1; j < T; j++) prow[j] = 0.0f;
                /* head_out = P @ V (attention.c:106) */
                float* o = att + (uint64_t)i * D + h * hd;
                for (uint32_t k = 0; k < hd; k++) o[k] = 0.0f;
                for (uint32_t j = 0; j <= i; j++) {
                    float p = prow[j];
                    const float* vr = Vv + (uint64_t)j * 3 * D;
                    for (uint32_t k = 0; k < hd; k++) o[k] += p * vr[k];
                }
            }
        }
        float* ao = s->x2[l];   /* attn_out, then x2 = x + attn_out */
        linear(att, PRM(s, l, K_WO), PRM(s, l, K_BO), ao, T, D, D);
        for (uint64_t i = 0; i < (uint64_t)T * D; i++) ao[i] = x[i] + ao[i];
        rmsnorm_fwd(s->x2[l], PRM(s, l, K_FN), s->n2[l], T, D, c->eps);
        linear(s->n2[l], PRM(s, l, K_WGU), PRM(s, l, K_BGU), s->gu[l], T, D, 2 * F);
        for (uint32_t i = 0; i < T; i++)
            for (uint32_t j = 0; j < F; j++) {   /* feedforward.c:146-150 */
                float g = s->gu[l][(uint64_t)i * 2 * F + j], u = s->gu[l][(uint64_t)i * 2 * F + F + j];
                float sg = 1.0f / (1.0f + or_m_expf(-g));
                float si = g * sg;
                s->sg[l][(uint64_t)i * F + j] = sg;
                s->silu[l][(uint64_t)i * F + j] = si;
                s->h[l][(uint64_t)i * F + j] = si * u;
            }
        float* xo = (l + 1 < c->L) ? s->x_in[l + 1] : s->x_fin;
        linear(s->h[l], PRM(s, l, K_WD), PRM(s, l, K_BD), xo, T, F, D);
        for (uint64_t i = 0; i < (uint64_t)T * D; i++) xo[i] = s->x2[l][i] + xo[i];
    }
    free(S);
    rmsnorm_fwd(s->x_fin, s->P + s->off[1 + 10 * c->L], s->nf, T, D, c->eps);
    /* logits = nf @ E^T (lm_model.c:128-130) */
    transpose_copy(V, D, E, D, s->tmpT);
    mm_rows(T, V, D, s->nf, D, 1, s->tmpT, V, s->logits, V);
}

/* node_cross_entropy_loss (loss.c:76-104) and its backward (loss.c:55-74):
 * logits are replaced by dlogits = (softmax - onehot) * (1/T). */
static float seq_ce(Seq* s, const uint32_t* tgt, float* loss_rows) {
    uint32_t T = s->T, V = s->c->V;
    float total = 0.0f, scale = 1.0f / (float)T;
    for (uint32_t i = 0; i < T; i++) {
        float* row = s->logits + (uint64_t)i * V;
        float mx = row[0];
        for (uint32_t j = 1; j < V; j++) if (row[j] > mx) mx = row[j];
        float sum = 0.0f;
        float* e = s->tmpT;
        for (uint32_t j = 0; j < V; j++) { e[j] = or_m_expf(row[j] - mx); sum += e[j]; }
        uint32_t t = tgt[i];
        float li = (or_m_logf(sum) + mx) - row[t];
        if (loss_rows) loss_rows[i] = li;
        total += li;
        for (uint32_t j = 0; j < V; j++) {
            float g = e[j] / sum;
            if (j == t) g -= 1.0f;
            row[j] = 0.0f + g * scale;
        }
    }
    return total / (float)T;
}

/* Backward of one sequence into zeroed grads G (autograd/node.c order). */
static void seq_backward(Seq* s, const uint32_t* ids, float* G) {
    const OrCfg* c = s->c;
    uint32_t T = s->T, D = c->D, H = c->H, F = c->F, V = c->V, hd = D / H, half = hd / 2;
    const float* E = s->P + s->off[0];
    float* dE = G + s->off[0];
    float scale = 1.0f / or_m_sqrtf((float)hd);
    float* dl = s->logits;
    float* dx = (float*)xcalloc((uint64_t)T * D);
    float* dn = (float*)xcalloc((uint64_t)T * D);
    float* gx2 = (float*)xcalloc((uint64_t)T * D);
    float* datt = (float*)xcalloc((uint64_t)T * D);
    float* dqkv = (float*)xcalloc((uint64_t)T * 3 * D);
    float* dh = (float*)xcalloc((uint64_t)T * F);
    float* dgu = (float*)xcalloc((uint64_t)T * 2 * F);
    uint64_t tmp_n = (uint64_t)D * V;
    if ((uint64_t)D * 3 * D > tmp_n) tmp_n = (uint64_t)D * 3 * D;
    if ((uint64_t)D * 2 * F > tmp_n) tmp_n = (uint64_t)D * 2 * F;
    if ((uint64_t)T * hd > tmp_n) tmp_n = (uint64_t)T * hd;
    float* tmp = (float*)xcalloc(tmp_n);
    float* dP = (float*)xcalloc(T);
    float* dS = (float*)xcalloc((uint64_t)T * T);
    float* dQ = (float*)xcalloc((uint64_t)T * hd);
    float* dK = (float*)xcalloc((uint64_t)T * hd);

    /* head: dnf = dl @ E; dE = (nf^T @ dl)^T  (node.c:116-127 via the transpose node) */
    mm_rows(T, D, V, dl, V, 1, E, D, dn, D);
    mm_rows(D, V, T, s->nf, 1, D, dl, V, tmp, V);          /* [D, V] */
    for (uint32_t d = 0; d < D; d++)
        for (uint32_t v = 0; v < V; v++) dE[(uint64_t)v * D + d] += tmp[(uint64_t)d * V + v];
    rmsnorm_bwd(s->x_fin, s->P + s->off[1 + 10 * c->L], dn, dx, G + s->off[1 + 10 * c->L], T, D, c->eps);

    for (int li = (int)c->L - 1; li >= 0; li--) {
        uint32_t l = (uint32_t)li;
        float* Gl = G + s->off[1 + 10 * l];
        (void)Gl;
#define GRD(k) (G + s->off[1 + 10 * l + (k)])
        /* x3 = x2 + ffn_out: gx2 = 0 + g3 */
        for (uint64_t i = 0; i < (uint64_t)T * D; i++) gx2[i] = 0.0f + dx[i];
        bias_grad(dx, GRD(K_BD), T, D);
        transpose_copy(F, D, PRM(s, l, K_WD), D, s->tmpT);       /* Wd^T [D, F] */
        mm_rows(T, F, D, dx, D, 1, s->tmpT, F, dh, F);           /* dh = g3 @ Wd^T */
        mm_rows(F, D, T, s->h[l], 1, F, dx, D, tmp, D);          /* Wd.grad = h^T @ g3 */
        for (uint64_t i = 0; i < (uint64_t)F * D; i++) GRD(K_WD)[i] += tmp[i];
        for (uint32_t i = 0; i < T; i++)
            for (uint32_t j = 0; j < F; j++) {
                uint64_t a = (uint64_t)i * F + j, b2 = (uint64_t)i * 2 * F;
                float g = s->gu[l][b2 + j], u = s->gu[l][b2 + F + j];
                float sg = s->sg[l][a], si = s->silu[l][a], d = dh[a];
                float silu_g = 0.0f + d * u;
                float up_g = 0.0f + d * si;
                float gate_g = 0.0f + silu_g * sg;
                float sg_g = 0.0f + silu_g * g;
                float local = sg * (1.0f - sg);
                gate_g += sg_g * local;
                dgu[b2 + j] = gate_g;
                dgu[b2 + F + j] = up_g;
            }
        bias_grad(dgu, GRD(K_BGU), T, 2 * F);
        transpose_copy(D, 2 * F, PRM(s, l, K_WGU), 2 * F, s->tmpT);   /* [2F, D] */
        mm_rows(T, D, 2 * F, dgu, 2 * F, 1, s->tmpT, D, dn, D);
        mm_rows(D, 2 * F, T, s->n2[l], 1, D, dgu, 2 * F, tmp, 2 * F);
        for (uint64_t i = 0; i < (uint64_t)D * 2 * F; i++) GRD(K_WGU)[i] += tmp[i];
        rmsnorm_bwd(s->x2[l], PRM(s, l, K_FN), dn, gx2, GRD(K_FN), T, D, c->eps);
        /* x2 = x + attn_out: gx = 0 + gx2 */
        for (uint64_t i = 0; i < (uint64_t)T * D; i++) dx[i] = 0.0f + gx2[i];
        bias_grad(gx2, GRD(K_BO), T, D);
        transpose_copy(D, D, PRM(s, l, K_WO), D, s->tmpT);
        mm_rows(T, D, D, gx2, D, 1, s->tmpT, D, datt, D);
        mm_rows(D, D, T, s->att[l], 1, D, gx2, D, tmp, D);
        for (uint64_t i = 0; i < (uint64_t)D * D; i++) GRD(K_WO)[i] += tmp[i];
        for (uint32_t h = 0; h < H; h++) {
            const float* Q = s->Qr[l] + (uint64_t)h * T * hd;
            const float* K = s->Kr[l] + (uint64_t)h * T * hd;
            const float* Vv = s->qkv[l] + 2 * D + h * hd;
            const float* Pm = s->Pm[l] + (uint64_t)h * T * T;
            for (uint64_t i = 0; i < (uint64_t)T * hd; i++) { dQ[i] = 0.0f; dK[i] = 0.0f; }
            float* dV = tmp;   /* [T, hd] */
            for (uint64_t i = 0; i < (uint64_t)T * hd; i++) dV[i] = 0.0f;
            for (uint32_t i = 0; i < T; i++) {
                const float* dO = datt + (uint64_t)i * D + h * hd;
                const float* prow = Pm + (uint64_t)i * T;
                /* dP = dO @ V^T; softmax backward (node.c:258-276); scale (node.c:100-103) */
                for (uint32_t j = 0; j <= i; j++) {
                    float acc = 0.0f;
                    const float* vr = Vv + (uint64_t)j * 3 * D;
                    for (uint32_t k = 0; k < hd; k++) acc += dO[k] * vr[k];
                    dP[j] = acc;
                }
                float dot = 0.0f;
                for (uint32_t j = 0; j <= i; j++) dot += dP[j] * prow[j];
                float* ds = dS + (uint64_t)i * T;
                for (uint32_t j = 0; j <= i; j++) ds[j] = 0.0f + (0.0f + prow[j] * (dP[j] - dot)) * scale;
                /* dQ = dS @ K */
                float* dq = dQ + (uint64_t)i * hd;
                for (uint32_t j = 0; j <= i; j++) {
                    float w = ds[j];
                    const float* kr = K + (uint64_t)j * hd;
                    for (uint32_t k = 0; k < hd; k++) dq[k] += w * kr[k];
                }
            }
            /* dK = (Q^T @ dS)^T and dV = P^T @ dO: rows i ascending for each j */
            for (uint32_t i = 0; i < T; i++) {
                const float* qr = Q + (uint64_t)i * hd;
                const float* dO = datt + (uint64_t)i * D + h * hd;
                const float* ds = dS + (uint64_t)i * T;
                const float* prow = Pm + (uint64_t)i * T;
                for (uint32_t j = 0; j <= i; j++) {
                    float w = ds[j], p = prow[j];
                    float* dk = dK + (uint64_t)j * hd;
                    float* dv = dV + (uint64_t)j * hd;
                    for (uint32_t k = 0; k < hd; k++) { dk[k] += qr[k] * w; dv[k] += p * dO[k]; }
                }
            }
            /* RoPE backward (model_ops.c:130-155) into dqkv columns */
            for (uint32_t p = 0; p < T; p++) {
                float* row = dqkv + (uint64_t)p * 3 * D;
                for (uint32_t k = 0; k < half; k++) {
                    float cc = s->cosT[(uint64_t)p * half + k], ss = s->sinT[(uint64_t)p * half + k];
                    float a0 = dQ[(uint64_t)p * hd + 2 * k], a1 = dQ[(uint64_t)p * hd + 2 * k + 1];
                    row[h * hd + 2 * k] = 0.0f + (a0 * cc + a1 * ss);
                    row[h * hd + 2 * k + 1] = 0.0f + (-a0 * ss + a1 * cc);
                    float b0 = dK[(uint64_t)p * hd + 2 * k], b1 = dK[(uint64_t)p * hd + 2 * k + 1];
                    row[D + h * hd + 2 * k] = 0.0f + (b0 * cc + b1 * ss);
                    row[D + h * hd + 2 * k + 1] = 0.0f + (-b0 * ss + b1 * cc);
                }
                for (uint32_t k = 0; k < hd; k++) row[2 * D + h * hd + k] = 0.0f + dV[(uint64_t)p * hd + k];
            }
        }
        bias_grad(dqkv, GRD(K_BQKV), T, 3 * D);
        transpose_copy(D, 3 * D, PRM(s, l, K_WQKV), 3 * D, s->tmpT);  /* [3D, D] */
        mm_rows(T, D, 3 * D, dqkv, 3 * D, 1, s->tmpT, D, dn, D);
        mm_rows(D, 3 * D, T, s->n1[l], 1, D, dqkv, 3 * D, tmp, 3 * D);
        for (uint64_t i = 0; i < (uint64_t)D * 3 * D; i++) GRD(K_WQKV)[i] += tmp[i];
        rmsnorm_bwd(s->x_in[l], PRM(s, l, K_AN), dn, dx, GRD(K_AN), T, D, c->eps);
#undef GRD
    }
    /* backward_embedding (embedding.c:4-15) */
    for (uint32_t i = 0; i < T; i++)
        for (uint32_t j = 0; j < D; j++) dE[(uint64_t)ids[i] * D + j] += dx[(uint64_t)i * D + j];
    free(dx); free(dn); free(gx2); free(datt); free(dqkv); free(dh); free(dgu); free(tmp);
    free(dP); free(dS); free(dQ); free(dK);
}

/* ======================= batch drivers (threads) ======================= */

typedef struct Job {
    const OrCfg* c; const float* P; const uint32_t* ids; const uint32_t* tgt;
    uint32_t B, T, first, stride;
    float* logits_out;          /* forward-only mode */
    float* grads;               /* [B][total] per-sequence grads, or NULL */
    float* losses;              /* [B] */
    float* loss_rows;           /* [B*T] or NULL */
    uint64_t total;
    const float* cosT; const float* sinT;
} Job;

static void* job_run(void* arg) {
    Job* j = (Job*)arg;
    for (uint32_t w = j->first; w < j->B; w += j->stride) {
        Seq s;
        seq_alloc(&s, j->c, j->T, j->P, j->cosT, j->sinT);
        const uint32_t* ids = j->ids + (uint64_t)w * j->T;
        seq_forward(&s, ids);
        if (j->logits_out) {
            memcpy(j->logits_out + (uint64_t)w * j->T * j->c->V, s.logits, (uint64_t)j->T * j->c->V * sizeof(float));
        } else {
            j->losses[w] = seq_ce(&s, j->tgt + (uint64_t)w * j->T, j->loss_rows ? j->loss_rows + (uint64_t)w * j->T : NULL);
            if (j->grads) seq_backward(&s, ids, j->grads + (uint64_t)w * j->total);
        }
        seq_free(&s);
    }
    return NULL;
}

static void run_jobs(Job* proto, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if ((uint32_t)nthreads > proto->B) nthreads = (int)proto->B;
    pthread_t th[64];
    Job jobs[64];
    for (int t = 0; t < nthreads; t++) {
        jobs[t] = *proto;
        jobs[t].first = (uint32_t)t;
        jobs[t].stride = (uint32_t)nthreads;
        pthread_create(&th[t], NULL, job_run, &jobs[t]);
    }
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
}

void or_forward_logits(const OrCfg* c, const float* params, const uint32_t* ids, uint32_t B, uint32_t T,
                       float* logits, int nthreads) {
    uint32_t hd = c->D / c->H;
    float* ct = (float*)xcalloc((uint64_t)T * hd / 2);
    float* st = (float*)xcalloc((uint64_t)T * hd / 2);
    or_rope_tables(T, hd, ct, st);
    Job j; memset(&j, 0, sizeof(j));
    j.c = c; j.P = params; j.ids = ids; j.B = B; j.T = T; j.logits_out = logits; j.cosT = ct; j.sinT = st;
    run_jobs(&j, nthreads);
    free(ct); free(st);
}

/* data_parallel_step (data_parallel.c:139-199): per-sequence grads summed in
 * worker order onto zero, then scaled by 1/B; loss = sum(loss_w)/B. */
float or_forward_backward(const OrCfg* c, const float* params, const uint32_t* ids, const uint32_t* tgt,
                          uint32_t B, uint32_t T, float* grads, float* loss_rows, int nthreads) {
    uint64_t off[10 * 64 + 2], num[10 * 64 + 2];
    uint64_t total = or_param_layout(c, off, num);
    uint32_t hd = c->D / c->H;
    float* ct = (float*)xcalloc((uint64_t)T * hd / 2);
    float* st = (float*)xcalloc((uint64_t)T * hd / 2);
    or_rope_tables(T, hd, ct, st);
    float* per = grads ? (float*)xcalloc((uint64_t)B * total) : NULL;
    float* losses = (float*)xcalloc(B);
    Job j; memset(&j, 0, sizeof(j));
    j.c = c; j.P = params; j.ids = ids; j.tgt = tgt; j.B = B; j.T = T; j.grads = per; j.losses = losses;
    j.loss_rows = loss_rows; j.total = total; j.cosT = ct; j.sinT = st;
    run_jobs(&j, nthreads);
    if (grads) {
        float inv = 1.0f / (float)B;
        for (uint64_t k = 0; k < total; k++) grads[k] = 0.0f;
        for (uint32_t w = 0; w < B; w++) {
            const float* src = per + (uint64_t)w * total;
            for (uint64_t k = 0; k < total; k++) grads[k] += src[k];
        }
        for (uint64_t k = 0; k < total; k++) grads[k] *= inv;
    }
    float ls = 0.0f;
    for (uint32_t w = 0; w < B; w++) ls += losses[w];
    free(per); free(losses); free(ct); free(st);
    return ls / (float)B;
}

/* adam_update_one (adam.c:80-95), with the GPU path's grad_scale
 * (train_kernels.cu:792) and, when wd != 0, the decoupled decay term
 * p -= lr*wd*p folded into the same subtraction. */
void or_adam_step(float* p, const float* g, float* m, float* v, uint64_t n, uint64_t t,
                  float lr, float b1, float b2, float eps, float wd, float grad_scale) {
    float bc1 = 1.0f - or_m_powf(b1, (float)t);
    float bc2 = 1.0f - or_m_powf(b2, (float)t);
    for (uint64_t j = 0; j < n; j++) {
        float gj = g[j] * grad_scale;
        m[j] = b1 * m[j] + (1.0f - b1) * gj;
        v[j] = b2 * v[j] + (1.0f - b2) * gj * gj;
        float mh = m[j] / bc1;
        float vh = v[j] / bc2;
        float upd = lr * mh / (or_m_sqrtf(vh) + eps);
        if (wd != 0.0f) upd = upd + (lr * wd) * p[j];
        p[j] -= upd;
    }
}
