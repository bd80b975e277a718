/* trlm_host.c -- standalone host runtime for the GPU path (libtrlm_host.so).
 *
 * The GPU entry points call a small part of the reference's host runtime:
 * allocation from an Allocator, tensor views, graph nodes, PCG32, scalar
 * maths and the RoPE tables.  In a drop-in build those symbols come from the
 * reference's own objects and this library is not linked.  Standalone (the
 * tests, bench.py) it provides them with the same behaviour:
 *   - maths and PCG follow the reference's algorithms step for step, because
 *     their bits feed the model (RoPE tables, Adam bias correction, batch
 *     sampling): runtime/mathlib.c:82-296, runtime/prng.c:10-94;
 *   - the Allocator is a simple bump arena over one mmap reservation (the
 *     reference adds a free list, runtime/memory.c:159-240; this path never
 *     needs to reuse freed blocks);
 *   - tensor and node helpers follow tensor/tensor.c and autograd/node.c.
 */
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#include "trlm_host.h"

/* ---------------- Allocator ---------------- */

Allocator allocator_create(u64 reserve_size) {
    Allocator a;
    memset(&a, 0, sizeof(a));
    void* p = mmap(NULL, reserve_size, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS | MAP_NORESERVE, -1, 0);
    a.backing.base = (p == MAP_FAILED) ? NULL : (u8*)p;
    a.backing.reserved = reserve_size;
    a.backing.committed = reserve_size;
    a.backing.used = 0;
    return a;
}

void* allocator_alloc(Allocator* a, u64 size) {
    u64 at = (a->backing.used + 63u) & ~63ull;
    if (!a->backing.base || at + size > a->backing.reserved) {
        fprintf(stderr, "[MEMORY ERROR] arena reservation exceeded: need %llu bytes, reserved %llu\n",
                (unsigned long long)(at + size), (unsigned long long)a->backing.reserved);
        fflush(stderr);
        _exit(1);
    }
    a->backing.used = at + size;
    return a->backing.base + at;
}

void allocator_free(Allocator* a, void* ptr) { (void)a; (void)ptr; }

void allocator_destroy(Allocator* a) {
    if (a->backing.base) munmap(a->backing.base, a->backing.reserved);
    memset(a, 0, sizeof(*a));
}

/* ---------------- Tensor (tensor/tensor.c) ---------------- */

static void row_major_strides(const u64* shape, u32 ndim, i64* st) {
    i64 acc = 1;
    for (i32 d = (i32)ndim - 1; d >= 0; d--) { st[d] = acc; acc *= (i64)shape[d]; }
}

Tensor tensor_create(Allocator* alloc, const u64* shape, u32 ndim) {
    Tensor t;
    memset(&t, 0, sizeof(t));
    t.ndim = ndim;
    t.numel = 1;
    for (u32 d = 0; d < ndim; d++) { t.shape[d] = shape[d]; t.numel *= shape[d]; }
    row_major_strides(t.shape, ndim, t.strides);
    t.data = (f32*)allocator_alloc(alloc, t.numel * sizeof(f32));
    t.owns_data = TRUE;
    return t;
}

bool32 tensor_is_contiguous(const Tensor* t) {
    i64 st[TENSOR_MAX_DIMS];
    row_major_strides(t->shape, t->ndim, st);
    for (u32 d = 0; d < t->ndim; d++) if (t->strides[d] != st[d]) return FALSE;
    return TRUE;
}

Tensor tensor_transpose(const Tensor* src, u32 dim0, u32 dim1) {
    Tensor o = *src;
    o.owns_data = FALSE;
    u64 s = o.shape[dim0]; o.shape[dim0] = o.shape[dim1]; o.shape[dim1] = s;
    i64 t = o.strides[dim0]; o.strides[dim0] = o.strides[dim1]; o.strides[dim1] = t;
    return o;
}

static u64 offset_of(const Tensor* t, u64 flat) {
    i64 off = 0;
    for (i32 d = (i32)t->ndim - 1; d >= 0; d--) {
        off += (i64)(flat % t->shape[d]) * t->strides[d];
        flat /= t->shape[d];
    }
    return (u64)off;
}

Tensor tensor_contiguous(Allocator* alloc, const Tensor* src) {
    Tensor o = tensor_create(alloc, src->shape, src->ndim);
    for (u64 i = 0; i < o.numel; i++) o.data[i] = src->data[offset_of(src, i)];
    return o;
}

/* dst += src element-wise in flat order (tensor.c:329-349). */
void tensor_add_inplace(Tensor* dst, const Tensor* src) {
    for (u64 i = 0; i < dst->numel; i++) dst->data[offset_of(dst, i)] += src->data[offset_of(src, i)];
}

/* ---------------- Node (autograd/node.c) ---------------- */

static Node* make_node(Allocator* alloc, Tensor value, bool32 requires_grad) {
    Node* n = (Node*)allocator_alloc(alloc, sizeof(Node));
    memset(n, 0, sizeof(Node));
    n->value = value;
    n->grad = tensor_create(alloc, value.shape, value.ndim);
    memset(n->grad.data, 0, n->grad.numel * sizeof(f32));
    n->requires_grad = requires_grad;
    return n;
}

Node* node_leaf(Allocator* alloc, Tensor value, bool32 requires_grad) { return make_node(alloc, value, requires_grad); }
Node* node_make_custom(Allocator* alloc, Tensor value, bool32 requires_grad) {
    return make_node(alloc, value, requires_grad);
}

/* Post-order DFS from the loss, then backward_fn in reverse (node.c:288-318). */
static void visit(Node* n, Node*** list, u64* count, u64* cap) {
    if (!n || n->visited) return;
    n->visited = TRUE;
    for (u32 i = 0; i < n->num_parents; i++) visit(n->parents[i], list, count, cap);
    if (*count == *cap) {
        *cap = *cap ? *cap * 2 : 256;
        *list = (Node**)realloc(*list, *cap * sizeof(Node*));
    }
    (*list)[(*count)++] = n;
}

void backward(Allocator* alloc, Node* loss) {
    Node** list = NULL;
    u64 count = 0, cap = 0;
    visit(loss, &list, &count, &cap);
    loss->grad.data[0] = 1.0f;
    for (u64 i = count; i-- > 0;) if (list[i]->backward_fn) list[i]->backward_fn(list[i], alloc);
    for (u64 i = 0; i < count; i++) list[i]->visited = FALSE;
    free(list);
}

/* ---------------- scalar maths (runtime/mathlib.c) ---------------- */

typedef union { f64 f; u64 u; } Bits64;

#define LN2 0.69314718055994530942
#define PI 3.14159265358979323846
#define MANT 0x000FFFFFFFFFFFFFull

static int nan64(f64 x) { Bits64 b; b.f = x; return ((b.u >> 52) & 0x7FF) == 0x7FF && (b.u & MANT); }
static int inf64(f64 x) { Bits64 b; b.f = x; return ((b.u >> 52) & 0x7FF) == 0x7FF && !(b.u & MANT); }
static f64 make64(u64 u) { Bits64 b; b.u = u; return b.f; }

/* mantissa in [1,2) and unbiased exponent */
static f64 mant_exp(f64 x, i32* e) {
    Bits64 b; b.f = x;
    *e = (i32)((b.u >> 52) & 0x7FF) - 1023;
    return make64((b.u & MANT) | (1023ull << 52));
}

/* x * 2^e through the exponent field; no denormals (mathlib.c:91-104) */
static f64 scale_pow2(f64 x, i32 e) {
    if (x == 0.0) return 0.0;
    Bits64 b; b.f = x;
    u64 sign = b.u & 0x8000000000000000ull;
    i64 ne = (i64)((b.u >> 52) & 0x7FF) + e;
    if (ne >= 0x7FF) return make64(sign | 0x7FF0000000000000ull);
    if (ne <= 0) return sign ? -0.0 : 0.0;
    return make64(sign | ((u64)ne << 52) | (b.u & MANT));
}

f64 m_sqrt(f64 x) {
    if (x < 0.0) return make64(0x7FF8000000000000ull);
    if (x == 0.0 || nan64(x) || inf64(x)) return x;
    i32 e;
    f64 m = mant_exp(x, &e);
    if (e & 1) { m *= 2.0; e -= 1; }
    f64 y = m * 0.5 + 0.5;
    for (i32 i = 0; i < 6; i++) y = 0.5 * (y + m / y);
    return scale_pow2(y, e / 2);
}

f64 m_exp(f64 x) {
    if (nan64(x)) return x;
    if (x > 709.782712893384) return make64(0x7FF0000000000000ull);
    if (x < -745.1332191019412) return 0.0;
    f64 q = x / LN2;
    i64 k = (i64)(q + (q >= 0.0 ? 0.5 : -0.5));
    f64 r = x - (f64)k * LN2;
    f64 term = 1.0, sum = 1.0;
    for (i32 n = 1; n < 40; n++) {
        term *= r / (f64)n;
        sum += term;
        if (term < 1e-18 && term > -1e-18) break;
    }
    return scale_pow2(sum, (i32)k);
}

f64 m_log(f64 x) {
    if (nan64(x) || x < 0.0) return make64(0x7FF8000000000000ull);
    if (x == 0.0) return make64(0xFFF0000000000000ull);
    if (inf64(x)) return x;
    i32 e;
    f64 m = mant_exp(x, &e);
    if (m > 1.4142135623730951) { m *= 0.5; e += 1; }
    f64 z = (m - 1.0) / (m + 1.0), z2 = z * z, term = z, sum = z;
    for (i32 n = 3; n < 60; n += 2) {
        term *= z2;
        f64 add = term / (f64)n;
        sum += add;
        if (add < 1e-18 && add > -1e-18) break;
    }
    return 2.0 * sum + (f64)e * LN2;
}

f64 m_pow(f64 base, f64 exponent) {
    if (exponent == 0.0) return 1.0;
    if (base == 0.0) return exponent > 0.0 ? 0.0 : make64(0x7FF0000000000000ull);
    if (base < 0.0) {
        if (exponent != (f64)(i64)exponent) return make64(0x7FF8000000000000ull);
        f64 mag = m_exp(exponent * m_log(-base));
        return ((i64)exponent % 2 != 0) ? -mag : mag;
    }
    return m_exp(exponent * m_log(base));
}

static f64 taylor_sin(f64 t) {
    f64 t2 = t * t, term = t, sum = t;
    for (i32 n = 1; n < 20; n++) {
        term *= -t2 / (f64)((2 * n) * (2 * n + 1));
        sum += term;
        if (term < 1e-18 && term > -1e-18) break;
    }
    return sum;
}

static f64 taylor_cos(f64 t) {
    f64 t2 = t * t, term = 1.0, sum = 1.0;
    for (i32 n = 1; n < 20; n++) {
        term *= -t2 / (f64)((2 * n - 1) * (2 * n));
        sum += term;
        if (term < 1e-18 && term > -1e-18) break;
    }
    return sum;
}

static f64 reduce_half_pi(f64 x, i32* quadrant) {
    const f64 hp = PI / 2.0;
    f64 q = x / hp;
    i64 k = (i64)(q + (q >= 0.0 ? 0.5 : -0.5));
    f64 core = x - (f64)k * hp;
    i64 r = k % 4;
    *quadrant = (i32)(r < 0 ? r + 4 : r);
    return core;
}

f64 m_sin(f64 x) {
    if (nan64(x) || inf64(x)) return make64(0x7FF8000000000000ull);
    i32 q;
    f64 c = reduce_half_pi(x, &q);
    switch (q) { case 0: return taylor_sin(c); case 1: return taylor_cos(c); case 2: return -taylor_sin(c); default: return -taylor_cos(c); }
}

f64 m_cos(f64 x) {
    if (nan64(x) || inf64(x)) return make64(0x7FF8000000000000ull);
    i32 q;
    f64 c = reduce_half_pi(x, &q);
    switch (q) { case 0: return taylor_cos(c); case 1: return -taylor_sin(c); case 2: return -taylor_cos(c); default: return taylor_sin(c); }
}

f32 m_sqrtf(f32 x) { return (f32)m_sqrt((f64)x); }
f32 m_powf(f32 b, f32 e) { return (f32)m_pow((f64)b, (f64)e); }
f32 m_sinf(f32 x) { return (f32)m_sin((f64)x); }
f32 m_cosf(f32 x) { return (f32)m_cos((f64)x); }

/* ---------------- PCG32 (runtime/prng.c) ---------------- */

u32 pcg_next_u32(PCGState* rng) {
    u64 s = rng->state;
    rng->state = s * 6364136223846793005ull + rng->inc;
    u32 x = (u32)(((s >> 18u) ^ s) >> 27u);
    u32 rot = (u32)(s >> 59u);
    return (x >> rot) | (x << ((32u - rot) & 31u));
}

PCGState pcg_seed(u64 initstate, u64 initseq) {
    PCGState r;
    memset(&r, 0, sizeof(r));
    r.inc = (initseq << 1u) | 1u;
    pcg_next_u32(&r);
    r.state += initstate;
    pcg_next_u32(&r);
    return r;
}

i64 pcg_range_i64(PCGState* rng, i64 lo, i64 hi) {
    u64 range = (u64)(hi - lo);
    if (range == 0) return lo;
    u64 threshold = (u64)(-(i64)range) % range;
    u64 v;
    do {
        u64 hi32 = pcg_next_u32(rng);
        v = (hi32 << 32) | (u64)pcg_next_u32(rng);
    } while (v < threshold);
    return lo + (i64)(v % range);
}

f64 pcg_gaussian(PCGState* rng, f64 mean, f64 stddev) {
    f64 z;
    if (rng->has_cached_gaussian) {
        rng->has_cached_gaussian = FALSE;
        z = rng->cached_gaussian;
    } else {
        f64 u1 = (f64)pcg_next_u32(rng) * (1.0 / 4294967296.0);
        if (u1 <= 0.0) u1 = 1.0 / 4294967296.0;
        f64 u2 = (f64)pcg_next_u32(rng) * (1.0 / 4294967296.0);
        f64 r = m_sqrt(-2.0 * m_log(u1));
        f64 th = 2.0 * PI * u2;
        z = r * m_cos(th);
        rng->cached_gaussian = r * m_sin(th);
        rng->has_cached_gaussian = TRUE;
    }
    return mean + stddev * z;
}

/* ---------------- RoPE tables (model/rope.c:4-18) ---------------- */

void rope_build_tables(Tensor* cos_out, Tensor* sin_out, u64 seq_len, u64 head_dim, f32 base) {
    u64 half = head_dim / 2;
    for (u64 pos = 0; pos < seq_len; pos++)
        for (u64 k = 0; k < half; k++) {
            f32 ex = -(2.0f * (f32)k) / (f32)head_dim;
            f32 ang = (f32)pos * m_powf(base, ex);
            i64 off = (i64)pos * cos_out->strides[0] + (i64)k * cos_out->strides[1];
            cos_out->data[off] = m_cosf(ang);
            sin_out->data[off] = m_sinf(ang);
        }
}

/* ---------------- layout report ---------------- */

/* sizeof / offsetof of the boundary structures, so a binding written in
 * another language (the tests' ctypes mirror) can check its layout. */
void trlm_host_layout(u64* out) {
    out[0] = sizeof(Tensor);
    out[1] = sizeof(Node);
    out[2] = offsetof(Node, backward_fn);
    out[3] = offsetof(Node, aux_ptr);
    out[4] = sizeof(LMModel);
    out[5] = offsetof(LMModel, final_norm_w);
    out[6] = offsetof(LMModel, eps);
    out[7] = sizeof(AdamOptimizer);
    out[8] = offsetof(AdamOptimizer, t);
    out[9] = sizeof(Allocator);
    out[10] = sizeof(PCGState);
    out[11] = offsetof(Tensor, numel);
}
