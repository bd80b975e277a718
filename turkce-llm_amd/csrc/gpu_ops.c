/* gpu_ops.c -- node_matmul2d_gpu on the MFMA GEMM (see include/gpu_ops.h).
 *
 * Same contract as the reference's model/gpu_ops.c: an autograd node whose
 * forward A@B and backward dA += dC@B^T, dB += A^T@dC run on the GPU, with
 * host round-trips by API design and gradient accumulation on the host
 * (gpu_ops.c:224-235).  Differences, all MI355X-side:
 *   - an operand that is a transposed view of a contiguous tensor (the tied
 *     head's embed_table^T, every B^T / A^T of the backward) is uploaded as
 *     stored and handed to the GEMM as a transposed layout; the reference
 *     makes a contiguous host copy first (gpu_ops.c:182-183);
 *   - row-major views with a wider row stride (column slices) are uploaded
 *     with one pitched copy and used with their leading dimension;
 *   - each slot owns a stream and grow-only device buffers (as the
 *     reference's persistent buffers, gpu_ops.c:85-108);
 *   - operands inside a range the caller pinned (gpu_ops_pin, trlm_ext.h:
 *     weights that stay fixed while generate/chat run) are read from a
 *     device copy made once per GPU, with the view's own leading dimension,
 *     instead of being uploaded on every call.
 */
#include <pthread.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <time.h>
#include <unistd.h>

#include "gpu_ops.h"
#include "trlm_ext.h"

#define MAX_GPU_CONTEXTS 32

typedef struct Slot {
    HipCtx ctx;
    TrlmGemm* gemm;
    hipDeviceptr_t buf[3];
    u64 cap[3];
    void* stage;        /* pinned host staging for results (grow-only) */
    u64 stage_cap;
} Slot;

static Slot g_slots[MAX_GPU_CONTEXTS];

/* Pinned host ranges and their device copies (one per device, made on first
 * use there by the slot that needed it). */
#define MAX_PINS 4096
#define MAX_PIN_DEVICES 16
typedef struct Pin {
    const f32* data;
    u64 count;
    hipDeviceptr_t dev[MAX_PIN_DEVICES];
    u32 owner[MAX_PIN_DEVICES];     /* slot whose context allocated dev[d] */
} Pin;
static Pin g_pins[MAX_PINS];
static u32 g_num_pins = 0;
static pthread_mutex_t g_pin_mutex = PTHREAD_MUTEX_INITIALIZER;
static u32 g_num_worker_slots = 0;
static int g_initialized = 0;
static pthread_mutex_t g_slot0_mutex = PTHREAD_MUTEX_INITIALIZER;
static pthread_mutex_t g_debug_mutex = PTHREAD_MUTEX_INITIALIZER;
static _Thread_local i32 g_tls_worker_id = -1;
static f64 g_debug_seconds = 0.0;
static u32 g_debug_calls = 0;

static f64 now_seconds(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (f64)ts.tv_sec + (f64)ts.tv_nsec * 1e-9;
}

void gpu_ops_debug_stats(f64* out_total_seconds, u32* out_call_count) {
    pthread_mutex_lock(&g_debug_mutex);
    *out_total_seconds = g_debug_seconds;
    *out_call_count = g_debug_calls;
    pthread_mutex_unlock(&g_debug_mutex);
}

void gpu_ops_debug_reset(void) {
    pthread_mutex_lock(&g_debug_mutex);
    g_debug_seconds = 0.0;
    g_debug_calls = 0;
    pthread_mutex_unlock(&g_debug_mutex);
}

static void slot_init(u32 s, Allocator* scratch, const char* path, i32 device) {
    memset(&g_slots[s], 0, sizeof(Slot));
    g_slots[s].ctx = hip_init_on_device(scratch, path, device);
    hip_set_current(&g_slots[s].ctx);
    g_slots[s].gemm = trlm_gemm_create(&g_slots[s].ctx);
}

void gpu_ops_init(Allocator* scratch, const char* ptx_path) {
    slot_init(0, scratch, ptx_path, 0);
    g_initialized = 1;
}

/* One slot per worker, spread round-robin over the visible devices
 * (gpu_ops.c:140-160). */
void gpu_ops_init_workers(Allocator* scratch, const char* ptx_path, u32 num_workers) {
    if (num_workers > MAX_GPU_CONTEXTS - 1) num_workers = MAX_GPU_CONTEXTS - 1;
    i32 ndev = hip_device_count();
    if (ndev < 1) ndev = 1;
    for (u32 i = 0; i < num_workers; i++) slot_init(1 + i, scratch, ptx_path, (i32)(i % (u32)ndev));
    g_num_worker_slots = num_workers;
}

void gpu_ops_set_worker_id(i32 worker_id) { g_tls_worker_id = worker_id; }

static void slot_release(u32 s) {
    hip_set_current(&g_slots[s].ctx);
    if (g_slots[s].stage) {
        hipHostFree(g_slots[s].stage);
        g_slots[s].stage = NULL;
        g_slots[s].stage_cap = 0;
    }
    trlm_gemm_destroy(g_slots[s].gemm);
    g_slots[s].gemm = NULL;
    hip_shutdown(&g_slots[s].ctx);
}

void gpu_ops_pin(const f32* data, u64 count) {
    if (!data || count == 0) return;
    pthread_mutex_lock(&g_pin_mutex);
    if (g_num_pins == MAX_PINS) {
        fprintf(stderr, "[HIP ERROR] gpu_ops: more than %d pinned ranges\n", MAX_PINS);
        fflush(stderr);
        _exit(1);
    }
    Pin* p = &g_pins[g_num_pins++];
    memset(p, 0, sizeof(*p));
    p->data = data;
    p->count = count;
    pthread_mutex_unlock(&g_pin_mutex);
}

void gpu_ops_unpin_all(void) {
    pthread_mutex_lock(&g_pin_mutex);
    for (u32 i = 0; i < g_num_pins; i++)
        for (u32 d = 0; d < MAX_PIN_DEVICES; d++)
            if (g_pins[i].dev[d]) {
                hip_set_current(&g_slots[g_pins[i].owner[d]].ctx);
                hip_free(g_pins[i].dev[d]);
            }
    g_num_pins = 0;
    pthread_mutex_unlock(&g_pin_mutex);
}

/* Device address of a view lying wholly inside a pinned range, on the
 * current slot's device (copying the range there on first use); 0 when the
 * view is not pinned. */
static hipDeviceptr_t pinned_view(u32 slot, const f32* data, u64 extent) {
    hipDeviceptr_t out = 0;
    pthread_mutex_lock(&g_pin_mutex);
    for (u32 i = 0; i < g_num_pins; i++) {
        Pin* p = &g_pins[i];
        if (data < p->data || data + extent > p->data + p->count) continue;
        i32 d = g_slots[slot].ctx.device;
        if (d < 0 || d >= MAX_PIN_DEVICES) break;
        if (!p->dev[d]) {
            p->dev[d] = hip_alloc(p->count * sizeof(f32));
            p->owner[d] = slot;
            hip_h2d(p->dev[d], p->data, p->count * sizeof(f32));
        }
        out = (hipDeviceptr_t)((char*)p->dev[d] + (u64)(data - p->data) * sizeof(f32));
        break;
    }
    pthread_mutex_unlock(&g_pin_mutex);
    return out;
}

void gpu_ops_shutdown(void) {
    if (!g_initialized) return;
    gpu_ops_unpin_all();
    slot_release(0);
    for (u32 i = 0; i < g_num_worker_slots; i++) slot_release(1 + i);
    g_num_worker_slots = 0;
    g_initialized = 0;
}

static hipDeviceptr_t slot_buf(Slot* s, u32 which, u64 bytes) {
    if (s->cap[which] < bytes) {
        if (s->cap[which] > 0) hip_free(s->buf[which]);
        s->buf[which] = hip_alloc(bytes);
        s->cap[which] = bytes;
    }
    return s->buf[which];
}

/* A result goes to the caller's tensor through the slot's pinned staging
 * buffer: the DMA runs at pinned-memory speed, and the copy into the
 * tensor -- freshly carved arena pages, each faulted in on first touch --
 * is split over up to D2H_THREADS host threads, which take their page
 * faults in parallel.  Small results are copied directly. */
#define D2H_THREADS 8
#define D2H_MIN_PART (1ull << 20)
typedef struct CopyPart { u8* dst; const u8* src; u64 n; } CopyPart;

static void* copy_part(void* arg) {
    CopyPart* c = (CopyPart*)arg;
    memcpy(c->dst, c->src, c->n);
    return NULL;
}

static void d2h_result(Slot* s, f32* dst, hipDeviceptr_t src, u64 bytes) {
    if (bytes < 2 * D2H_MIN_PART) {
        hip_d2h(dst, src, bytes);
        return;
    }
    if (s->stage_cap < bytes) {
        if (s->stage) hipHostFree(s->stage);
        s->stage = NULL;
        hipError_t r = hipHostMalloc(&s->stage, bytes, hipHostMallocDefault);
        if (r != hipSuccess) {
            fprintf(stderr, "[HIP ERROR] gpu_ops: hipHostMalloc of %llu bytes -> %s\n", (unsigned long long)bytes,
                    hipGetErrorName(r));
            _exit(1);
        }
        s->stage_cap = bytes;
    }
    hipError_t r = hipMemcpyDtoHAsync(s->stage, src, bytes, s->ctx.stream);
    if (r == hipSuccess) r = hipStreamSynchronize(s->ctx.stream);
    if (r != hipSuccess) {
        fprintf(stderr, "[HIP ERROR] gpu_ops: result download -> %s\n", hipGetErrorName(r));
        _exit(1);
    }
    u64 nt = bytes / D2H_MIN_PART;
    if (nt > D2H_THREADS) nt = D2H_THREADS;
    const u64 per = ((bytes + nt - 1) / nt + 63) & ~63ull;
    CopyPart parts[D2H_THREADS];
    pthread_t th[D2H_THREADS];
    int started[D2H_THREADS];
    for (u64 i = 0; i < nt; i++) {
        const u64 off = i * per < bytes ? i * per : bytes;
        parts[i].dst = (u8*)dst + off;
        parts[i].src = (const u8*)s->stage + off;
        parts[i].n = (off + per < bytes ? off + per : bytes) - off;
        started[i] = i > 0 && pthread_create(&th[i], NULL, copy_part, &parts[i]) == 0;
    }
    copy_part(&parts[0]);
    for (u64 i = 1; i < nt; i++) {
        if (started[i]) pthread_join(th[i], NULL);
        else copy_part(&parts[i]);
    }
}

/* How a 2-D view is laid out in host memory. */
typedef struct View {
    int trans;          /* 0: element (r,c) at data[r*ld + c]; 1: at data[c*ld + r] */
    u64 ld;
    const f32* data;
    Tensor packed;      /* host copy when the view has neither form */
} View;

static View classify(Allocator* alloc, const Tensor* t) {
    View v;
    memset(&v, 0, sizeof(v));
    u64 rows = t->shape[0], cols = t->shape[1];
    if (t->strides[1] == 1 && (u64)t->strides[0] >= cols) {
        v.trans = 0; v.ld = (u64)t->strides[0]; v.data = t->data;
    } else if (t->strides[0] == 1 && (u64)t->strides[1] >= rows) {
        v.trans = 1; v.ld = (u64)t->strides[1]; v.data = t->data;
    } else {
        v.packed = tensor_contiguous(alloc, t);
        v.trans = 0; v.ld = cols; v.data = v.packed.data;
    }
    if (rows <= 1 && !v.trans) v.ld = cols;
    if (cols <= 1 && v.trans) v.ld = rows;
    return v;
}

/* A view's operand on the device: its pinned copy when it lies in a pinned
 * range (leading dimension as stored on the host), otherwise an upload into
 * the slot's packed buffer `which` (leading dimension = the stored row
 * length).  Returns the device pointer; *ld receives the leading dimension. */
static hipDeviceptr_t upload_view(u32 slot, Slot* s, u32 which, const View* v, u64 rows, u64 cols, u64* ld) {
    u64 srow = v->trans ? rows : cols;      /* stored row length */
    u64 nrow = v->trans ? cols : rows;      /* stored row count  */
    if (!v->packed.data && nrow > 0 && srow > 0) {
        hipDeviceptr_t pin = pinned_view(slot, v->data, (nrow - 1) * v->ld + srow);
        if (pin) {
            *ld = v->ld;
            return pin;
        }
    }
    *ld = srow;
    hipDeviceptr_t d = slot_buf(s, which, nrow * srow * sizeof(f32));
    if (v->ld == srow) {
        hip_h2d(d, v->data, nrow * srow * sizeof(f32));
    } else {
        hipError_t r = hipMemcpy2DAsync(d, srow * sizeof(f32), v->data, v->ld * sizeof(f32), srow * sizeof(f32),
                                        nrow, hipMemcpyHostToDevice, s->ctx.stream);
        if (r != hipSuccess) {
            fprintf(stderr, "[HIP ERROR] gpu_ops: pitched upload -> %s\n", hipGetErrorName(r));
            _exit(1);
        }
        hip_sync();
    }
    return d;
}

static Tensor gpu_matmul(Allocator* alloc, const Tensor* a, const Tensor* b) {
    f64 t0 = now_seconds();
    u64 M = a->shape[0], K = a->shape[1], N = b->shape[1];
    u64 out_shape[2] = { M, N };
    Tensor out = tensor_create(alloc, out_shape, 2);
    View va = classify(alloc, a), vb = classify(alloc, b);

    i32 wid = g_tls_worker_id;
    int own = (wid >= 0 && (u32)wid < g_num_worker_slots);
    u32 slot = own ? (u32)(1 + wid) : 0;
    if (!own) pthread_mutex_lock(&g_slot0_mutex);
    Slot* s = &g_slots[slot];
    hip_set_current(&s->ctx);

    u64 lda, ldb;
    hipDeviceptr_t da = upload_view(slot, s, 0, &va, M, K, &lda);
    hipDeviceptr_t db = upload_view(slot, s, 1, &vb, K, N, &ldb);
    hipDeviceptr_t dc = slot_buf(s, 2, (M * N > 0 ? M * N : 1) * sizeof(f32));
    trlm_gemm(s->gemm, va.trans, vb.trans, da, db, dc, (i32)M, (i32)N, (i32)K, (i32)lda, (i32)ldb,
              (i32)N, 1, 0, 0, 0, 1.0f, 0.0f, NULL, NULL, (i32)N);
    d2h_result(s, out.data, dc, M * N * sizeof(f32));

    if (!own) pthread_mutex_unlock(&g_slot0_mutex);
    pthread_mutex_lock(&g_debug_mutex);
    g_debug_seconds += now_seconds() - t0;
    g_debug_calls++;
    pthread_mutex_unlock(&g_debug_mutex);
    return out;
}

/* dA += dC @ B^T ; dB += A^T @ dC  (gpu_ops.c:224-235) */
static void backward_matmul2d_gpu(Node* self, Allocator* alloc) {
    Node* a = self->parents[0];
    Node* b = self->parents[1];
    Tensor bt = tensor_transpose(&b->value, 0, 1);
    Tensor da = gpu_matmul(alloc, &self->grad, &bt);
    tensor_add_inplace(&a->grad, &da);
    Tensor at = tensor_transpose(&a->value, 0, 1);
    Tensor db = gpu_matmul(alloc, &at, &self->grad);
    tensor_add_inplace(&b->grad, &db);
}

Node* node_matmul2d_gpu(Allocator* alloc, Node* a, Node* b) {
    Tensor v = gpu_matmul(alloc, &a->value, &b->value);
    Node* n = node_make_custom(alloc, v, TRUE);
    n->parents[0] = a;
    n->parents[1] = b;
    n->num_parents = 2;
    n->backward_fn = backward_matmul2d_gpu;
    return n;
}
