/* hip_backend.h -- thin HIP module-API backend for gfx950 code objects.
 *
 * Takes the role of the reference's CUDA Driver-API backend
 * (cuda/cuda_backend.h:9-65, cuda/driver_api.h): a context loads one kernel
 * image, kernels are looked up by name and launched with a `void**` argument
 * array, memory is allocated/copied synchronously, and any failure prints a
 * diagnostic and ends the process with _exit(1) (cuda_backend.c:15-34).
 *
 * MI355X-specific choices:
 *   - the image is a gfx950 code object (.hsaco from hipcc --genco), loaded
 *     with hipModuleLoadData: no JIT step, unlike the reference's PTX;
 *   - every context owns one HIP stream at default priority; launches and
 *     copies go to the stream of the context made current on the calling
 *     thread (hip_set_current), and the blocking helpers synchronise it, so
 *     callers see the reference's in-order, synchronous behaviour;
 *   - HIP has no context destroy that frees memory, so a context records
 *     the buffers allocated while it is current and hip_shutdown frees them.
 */
#ifndef HIP_BACKEND_H
#define HIP_BACKEND_H

#ifndef __HIP_PLATFORM_AMD__
#define __HIP_PLATFORM_AMD__
#endif
#include <hip/hip_runtime_api.h>

#include "trlm_host.h"

typedef struct HipAllocList HipAllocList;
typedef struct HipSide HipSide;

typedef struct HipCtx {
    i32 device;
    hipModule_t module;
    hipStream_t stream;
    HipAllocList* allocs;
    HipSide* side;   /* second stream (hip_side_begin), created on first use */
} HipCtx;

#ifdef __cplusplus
extern "C" {
#endif

/* cuda_init / cuda_init_on_device (cuda_backend.h:19,29). image_path names a
 * gfx950 code object.  The context reads it into memory of its own and keeps
 * it until hip_shutdown (the loader may refer to it while the module is
 * loaded); `scratch`, where the reference reads its PTX, is not used. */
HipCtx hip_init(Allocator* scratch, const char* image_path);
HipCtx hip_init_on_device(Allocator* scratch, const char* image_path, i32 device_index);
i32 hip_device_count(void);                                   /* cuda_backend.h:32 */
void hip_shutdown(HipCtx* c);                                 /* cuda_backend.h:34 */
void hip_set_current(HipCtx* c);                              /* cuda_backend.h:40 */
hipFunction_t hip_get_kernel(HipCtx* c, const char* name);    /* cuda_backend.h:42 */

hipDeviceptr_t hip_alloc(u64 bytes);                          /* cuda_backend.h:44-47 */
void hip_free(hipDeviceptr_t p);
void hip_h2d(hipDeviceptr_t dst, const void* src, u64 bytes);
void hip_d2h(void* dst, hipDeviceptr_t src, u64 bytes);

void hip_launch_1d(hipFunction_t f, u32 n, void** params);    /* cuda_backend.h:50-60 */
void hip_launch_2d(hipFunction_t f, u32 rows, u32 cols, void** params);
void hip_launch_1d_shared(hipFunction_t f, u32 n, u32 block_size, u32 shared_bytes, void** params);
void hip_launch(hipFunction_t f, u32 gx, u32 gy, u32 gz, u32 bx, u32 by, u32 bz, u32 shared_bytes,
                void** params);
void hip_memset_zero(hipDeviceptr_t p, u64 bytes);            /* cuda_backend.h:63 */
void hip_sync(void);                                          /* cuda_backend.h:65 */

/* The stream of the context current on this thread (for event timing). */
hipStream_t hip_current_stream(void);

/* Not in the reference's backend: the compute units of the current
 * context's device, and how many workgroups of block_threads threads of
 * kernel f one compute unit holds at once (the attention forward places its
 * jobs by them). */
u32 hip_cu_count(void);
u32 hip_blocks_per_cu(hipFunction_t f, u32 block_threads);

/* Overlap within one context (not in the reference's backend): a second
 * stream at default priority.  hip_side_begin() sends the current context's
 * later launches to it, ordered after everything already queued on the main
 * stream; hip_side_end(mark) sends launches back to the main stream and
 * records mark (0..HIP_SIDE_MARKS-1) on the side stream; hip_main_wait(mark)
 * makes the main stream wait for the side work up to that mark (a mark never
 * recorded is already reached); hip_side_join() makes it wait for all side
 * work queued so far.  hip_sync and hip_free also wait for the side stream. */
#define HIP_SIDE_MARKS 8
void hip_side_begin(void);
/* hip_side_serial(1): until hip_side_serial(0), in every context of the
 * process, side sections run on the main stream in the order they are
 * issued and marks / waits / joins are no-ops -- the same work as one stream
 * (for checking the overlap).  Call between operations, not inside one. */
void hip_side_serial(i32 on);
void hip_side_end(i32 mark);
void hip_main_wait(i32 mark);
void hip_side_join(void);

#ifdef __cplusplus
}
#endif

#endif /* HIP_BACKEND_H */
