/* hip_backend.c -- HIP module-API backend (see include/hip_backend.h).
 *
 * Role of cuda/cuda_backend.c (cuda_backend.c:15-161): fatal error check,
 * kernel image load, allocation, synchronous copies and launch helpers.
 */
#include "hip_backend.h"

#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

struct HipAllocList {
    pthread_mutex_t lock;
    void** ptrs;
    u64 count;
    u64 cap;
    void* image;   /* the loaded code object's bytes, owned until hip_shutdown */
};

struct HipSide {
    hipStream_t stream;
    hipEvent_t fork, join;
    hipEvent_t mark[HIP_SIDE_MARKS];
    i32 active;
};

static _Thread_local HipCtx* tls_ctx = NULL;

static void fatal_exit(void) {
    fflush(stdout);
    fflush(stderr);
    _exit(1);
}

/* Same convention as the reference (cuda_backend.c:23-34): name what failed,
 * the error's name and description, and end the process. */
static void check(hipError_t r, const char* what) {
    if (r != hipSuccess) {
        fprintf(stderr, "[HIP ERROR] %s -> %s: %s\n", what, hipGetErrorName(r), hipGetErrorString(r));
        fatal_exit();
    }
}

/* The code object is read into memory the context owns and keeps until
 * hip_shutdown has unloaded the module: the HSA loader may keep referring to
 * the bytes a code object was loaded from (a reader created from memory
 * must outlive the loaded object), so they must not live in an arena the
 * caller may reset or free while the module is loaded. */
static void* read_image(const char* path, u64* out_size) {
    FILE* f = fopen(path, "rb");
    if (!f) {
        fprintf(stderr, "[HIP ERROR] cannot open kernel image: %s\n", path);
        fatal_exit();
    }
    fseek(f, 0, SEEK_END);
    long size = ftell(f);
    fseek(f, 0, SEEK_SET);
    u8* buf = (u8*)malloc((size_t)size + 1);
    if (!buf) {
        fprintf(stderr, "[HIP ERROR] out of host memory for kernel image: %s\n", path);
        fatal_exit();
    }
    size_t got = fread(buf, 1, (size_t)size, f);
    fclose(f);
    if (got != (size_t)size) {
        fprintf(stderr, "[HIP ERROR] short read of kernel image: %s\n", path);
        fatal_exit();
    }
    buf[size] = 0;
    *out_size = (u64)size;
    return buf;
}

HipCtx hip_init_on_device(Allocator* scratch, const char* image_path, i32 device_index) {
    HipCtx c;
    memset(&c, 0, sizeof(c));
    i32 count = 0;
    check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (count < 1) {
        fprintf(stderr, "[HIP ERROR] no HIP device found\n");
        fatal_exit();
    }
    if (device_index < 0 || device_index >= count) {
        fprintf(stderr, "[HIP ERROR] device index %d exceeds the %d visible devices\n", device_index, count);
        fatal_exit();
    }
    c.device = device_index;
    check(hipSetDevice(device_index), "hipSetDevice");
    (void)scratch;   /* the reference reads the image into it; here the context owns the bytes */
    u64 size;
    void* image = read_image(image_path, &size);
    check(hipModuleLoadData(&c.module, image), "hipModuleLoadData");
    check(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    c.allocs = (HipAllocList*)calloc(1, sizeof(HipAllocList));
    pthread_mutex_init(&c.allocs->lock, NULL);
    c.allocs->image = image;
    return c;
}

HipCtx hip_init(Allocator* scratch, const char* image_path) {
    return hip_init_on_device(scratch, image_path, 0);
}

i32 hip_device_count(void) {
    i32 count = 0;
    check(hipGetDeviceCount(&count), "hipGetDeviceCount");
    return count;
}

void hip_shutdown(HipCtx* c) {
    if (!c->allocs) return;
    check(hipSetDevice(c->device), "hipSetDevice");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->side) check(hipStreamSynchronize(c->side->stream), "hipStreamSynchronize");
    for (u64 i = 0; i < c->allocs->count; i++)
        if (c->allocs->ptrs[i]) check(hipFree(c->allocs->ptrs[i]), "hipFree");
    void* image = c->allocs->image;
    free(c->allocs->ptrs);
    pthread_mutex_destroy(&c->allocs->lock);
    free(c->allocs);
    c->allocs = NULL;
    if (c->side) {
        check(hipStreamSynchronize(c->side->stream), "hipStreamSynchronize");
        for (i32 i = 0; i < HIP_SIDE_MARKS; i++) check(hipEventDestroy(c->side->mark[i]), "hipEventDestroy");
        check(hipEventDestroy(c->side->fork), "hipEventDestroy");
        check(hipEventDestroy(c->side->join), "hipEventDestroy");
        check(hipStreamDestroy(c->side->stream), "hipStreamDestroy");
        free(c->side);
        c->side = NULL;
    }
    check(hipStreamDestroy(c->stream), "hipStreamDestroy");
    check(hipModuleUnload(c->module), "hipModuleUnload");
    free(image);
    if (tls_ctx == c) tls_ctx = NULL;
}

void hip_set_current(HipCtx* c) {
    check(hipSetDevice(c->device), "hipSetDevice");
    tls_ctx = c;
}

static HipCtx* current(const char* what) {
    if (!tls_ctx) {
        fprintf(stderr, "[HIP ERROR] %s: no context is current on this thread\n", what);
        fatal_exit();
    }
    return tls_ctx;
}

hipStream_t hip_current_stream(void) { return current("hip_current_stream")->stream; }

u32 hip_cu_count(void) {
    int n = 0;
    check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, current("hip_cu_count")->device),
          "hipDeviceGetAttribute(multiprocessor count)");
    return (u32)n;
}

u32 hip_blocks_per_cu(hipFunction_t f, u32 block_threads) {
    int n = 0;
    check(hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, (int)block_threads, 0),
          "hipModuleOccupancyMaxActiveBlocksPerMultiprocessor");
    return (u32)n;
}

hipFunction_t hip_get_kernel(HipCtx* c, const char* name) {
    hipFunction_t f;
    hipError_t r = hipModuleGetFunction(&f, c->module, name);
    if (r != hipSuccess) {
        fprintf(stderr, "[HIP ERROR] hipModuleGetFunction(%s) -> %s: %s\n", name, hipGetErrorName(r),
                hipGetErrorString(r));
        fatal_exit();
    }
    return f;
}

hipDeviceptr_t hip_alloc(u64 bytes) {
    HipCtx* c = current("hip_alloc");
    void* p = NULL;
    check(hipMalloc(&p, bytes ? bytes : 4), "hipMalloc");
    HipAllocList* l = c->allocs;
    pthread_mutex_lock(&l->lock);
    if (l->count == l->cap) {
        l->cap = l->cap ? l->cap * 2 : 256;
        l->ptrs = (void**)realloc(l->ptrs, l->cap * sizeof(void*));
    }
    l->ptrs[l->count++] = p;
    pthread_mutex_unlock(&l->lock);
    return p;
}

void hip_free(hipDeviceptr_t p) {
    HipCtx* c = current("hip_free");
    HipAllocList* l = c->allocs;
    pthread_mutex_lock(&l->lock);
    for (u64 i = l->count; i-- > 0;) {
        if (l->ptrs[i] == p) { l->ptrs[i] = l->ptrs[--l->count]; break; }
    }
    pthread_mutex_unlock(&l->lock);
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->side) check(hipStreamSynchronize(c->side->stream), "hipStreamSynchronize");
    check(hipFree(p), "hipFree");
}

void hip_h2d(hipDeviceptr_t dst, const void* src, u64 bytes) {
    HipCtx* c = current("hip_h2d");
    check(hipMemcpyHtoDAsync(dst, (void*)src, bytes, c->stream), "hipMemcpyHtoDAsync");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

void hip_d2h(void* dst, hipDeviceptr_t src, u64 bytes) {
    HipCtx* c = current("hip_d2h");
    check(hipMemcpyDtoHAsync(dst, src, bytes, c->stream), "hipMemcpyDtoHAsync");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
}

void hip_launch(hipFunction_t f, u32 gx, u32 gy, u32 gz, u32 bx, u32 by, u32 bz, u32 shared_bytes,
                void** params) {
    HipCtx* c = current("hip_launch");
    if (gx == 0 || gy == 0 || gz == 0) return;
    hipStream_t st = (c->side && c->side->active) ? c->side->stream : c->stream;
    check(hipModuleLaunchKernel(f, gx, gy, gz, bx, by, bz, shared_bytes, st, params, NULL),
          "hipModuleLaunchKernel");
}

static int side_serial;

void hip_side_serial(i32 on) { side_serial = on != 0; }

void hip_side_begin(void) {
    HipCtx* c = current("hip_side_begin");
    if (side_serial) return;
    if (!c->side) {
        HipSide* s = (HipSide*)calloc(1, sizeof(HipSide));
        check(hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
        check(hipEventCreateWithFlags(&s->fork, hipEventDisableTiming), "hipEventCreateWithFlags");
        check(hipEventCreateWithFlags(&s->join, hipEventDisableTiming), "hipEventCreateWithFlags");
        for (i32 i = 0; i < HIP_SIDE_MARKS; i++)
            check(hipEventCreateWithFlags(&s->mark[i], hipEventDisableTiming), "hipEventCreateWithFlags");
        c->side = s;
    }
    check(hipEventRecord(c->side->fork, c->stream), "hipEventRecord");
    check(hipStreamWaitEvent(c->side->stream, c->side->fork, 0), "hipStreamWaitEvent");
    c->side->active = 1;
}

static void check_mark(i32 mark, const char* what) {
    if (mark < 0 || mark >= HIP_SIDE_MARKS) {
        fprintf(stderr, "[HIP ERROR] %s: side mark %d out of range\n", what, mark);
        fatal_exit();
    }
}

void hip_side_end(i32 mark) {
    HipCtx* c = current("hip_side_end");
    check_mark(mark, "hip_side_end");
    if (side_serial) return;
    if (!c->side || !c->side->active) {
        fprintf(stderr, "[HIP ERROR] hip_side_end without hip_side_begin\n");
        fatal_exit();
    }
    check(hipEventRecord(c->side->mark[mark], c->side->stream), "hipEventRecord");
    c->side->active = 0;
}

void hip_main_wait(i32 mark) {
    HipCtx* c = current("hip_main_wait");
    check_mark(mark, "hip_main_wait");
    if (side_serial || !c->side) return;   /* no side stream, or nothing queued on it */
    check(hipStreamWaitEvent(c->stream, c->side->mark[mark], 0), "hipStreamWaitEvent");
}

void hip_side_join(void) {
    HipCtx* c = current("hip_side_join");
    if (!c->side) return;
    check(hipEventRecord(c->side->join, c->side->stream), "hipEventRecord");
    check(hipStreamWaitEvent(c->stream, c->side->join, 0), "hipStreamWaitEvent");
}

#define BLOCK_1D 256u

void hip_launch_1d(hipFunction_t f, u32 n, void** params) {
    hip_launch(f, (n + BLOCK_1D - 1) / BLOCK_1D, 1, 1, BLOCK_1D, 1, 1, 0, params);
}

void hip_launch_1d_shared(hipFunction_t f, u32 n, u32 block_size, u32 shared_bytes, void** params) {
    hip_launch(f, (n + block_size - 1) / block_size, 1, 1, block_size, 1, 1, shared_bytes, params);
}

#define BLOCK_2D 16u

void hip_launch_2d(hipFunction_t f, u32 rows, u32 cols, void** params) {
    hip_launch(f, (cols + BLOCK_2D - 1) / BLOCK_2D, (rows + BLOCK_2D - 1) / BLOCK_2D, 1, BLOCK_2D, BLOCK_2D, 1,
               0, params);
}

void hip_memset_zero(hipDeviceptr_t p, u64 bytes) {
    HipCtx* c = current("hip_memset_zero");
    check(hipMemsetD8Async(p, 0, bytes, c->stream), "hipMemsetD8Async");
}

void hip_sync(void) {
    HipCtx* c = current("hip_sync");
    check(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    if (c->side) check(hipStreamSynchronize(c->side->stream), "hipStreamSynchronize");
}
