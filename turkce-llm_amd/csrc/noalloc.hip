// noalloc.hip -- trlm_gemm_noalloc: the raw GEMM (trlm_gemm) for callers that
// cannot allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc).
//
// trlm_gemm's split-K plans write raw partials to a workspace that the GEMM
// engine allocates on first need (hip_alloc, grow-only).  This variant runs
// the same plan and the same kernels with that workspace in `scratch`, a
// fixed 32 MiB device array of this library: every GPU the library runs on
// holds one copy, from set-up until the process ends.  Its device address on
// each device is resolved once, at set-up (trlm_gemm_create), with the device
// current, and only that address is handed to kernels or copies; the array's
// name is host-side only.
//
// A plan whose partials exceed the scratch runs with the most splits whose
// partials fit (one split needs none), as trlm_gemm forced to that count.
// Every split writes its whole slab of partials before the ordered
// reduction reads it, so nothing in scratch needs clearing between calls.
// All calls on one GPU share its scratch: calls that overlap in time on one
// GPU (other streams, other contexts, other threads) race.
#include <hip/hip_runtime.h>
#include <pthread.h>
#include <stdio.h>
#include <unistd.h>

#include "gpu_internal.h"

#define TRLM_SCRATCH_BYTES (32ull << 20)
#define TRLM_MAX_DEVICES 64

static __device__ __align__(256) float scratch[TRLM_SCRATCH_BYTES / sizeof(float)];

static void* scratch_dev[TRLM_MAX_DEVICES];
static pthread_mutex_t scratch_lock = PTHREAD_MUTEX_INITIALIZER;

static void noalloc_fatal(const char* what, hipError_t r) {
    fprintf(stderr, "[HIP ERROR] %s -> %s: %s\n", what, hipGetErrorName(r), hipGetErrorString(r));
    fflush(stderr);
    _exit(1);
}

extern "C" void trlm_noalloc_setup(i32 device) {
    if (device < 0 || device >= TRLM_MAX_DEVICES) {
        fprintf(stderr, "[HIP ERROR] trlm_noalloc_setup: device %d outside 0..%d\n", device, TRLM_MAX_DEVICES - 1);
        fflush(stderr);
        _exit(1);
    }
    pthread_mutex_lock(&scratch_lock);
    if (!scratch_dev[device]) {
        int prev = 0;
        hipError_t r = hipGetDevice(&prev);
        if (r != hipSuccess) noalloc_fatal("hipGetDevice", r);
        if (prev != device && (r = hipSetDevice(device)) != hipSuccess) noalloc_fatal("hipSetDevice", r);
        void* ptr = NULL;
        r = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (r != hipSuccess || !ptr) noalloc_fatal("hipGetSymbolAddress(scratch)", r);
        scratch_dev[device] = ptr;
        if (prev != device && (r = hipSetDevice(prev)) != hipSuccess) noalloc_fatal("hipSetDevice", r);
    }
    pthread_mutex_unlock(&scratch_lock);
}

extern "C" i32 trlm_gemm_noalloc(TrlmGemm* e, i32 trans_a, i32 trans_b, hipDeviceptr_t A, hipDeviceptr_t B,
                                 hipDeviceptr_t C, i32 M, i32 N, i32 K, i32 lda, i32 ldb, i32 ldc, u32 batch, i64 sA,
                                 i64 sB, i64 sC, f32 alpha, f32 beta, hipDeviceptr_t bias, hipDeviceptr_t resid,
                                 i32 ldr) {
    // The scratch copy is the one of the engine's device, and its kernels
    // must run there: a thread that made another device current is refused.
    const i32 device = trlm_gemm_device(e);
    int cur = -1;
    hipError_t r = hipGetDevice(&cur);
    if (r != hipSuccess) noalloc_fatal("hipGetDevice", r);
    if (cur != device) {
        fprintf(stderr,
                "trlm_gemm_noalloc: refused, nothing launched: the engine belongs to device %d, device %d is current\n",
                device, cur);
        fflush(stderr);
        return -1;
    }
    pthread_mutex_lock(&scratch_lock);
    void* ws = (device >= 0 && device < TRLM_MAX_DEVICES) ? scratch_dev[device] : NULL;
    pthread_mutex_unlock(&scratch_lock);
    if (!ws) {
        fprintf(stderr, "[HIP ERROR] trlm_gemm_noalloc: no scratch address for device %d\n", device);
        fflush(stderr);
        _exit(1);
    }
    return trlm_gemm_ws(e, trans_a, trans_b, A, B, C, M, N, K, lda, ldb, ldc, batch, sA, sB, sC, alpha, beta, bias,
                        resid, ldr, NULL, (hipDeviceptr_t)ws, TRLM_SCRATCH_BYTES / sizeof(float));
}
