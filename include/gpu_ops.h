/* gpu_ops.h -- autograd matmul node computed on the GPU (hybrid CPU path).
 *
 * Drop-in for the reference's model/gpu_ops.h: prototypes byte-identical to
 * model/gpu_ops.h:23-60.  `ptx_path` names the gfx950 kernel image instead of
 * a PTX file.  Forward and both backward products run on the MFMA GEMM;
 * transposed operands (e.g. the tied LM head's embed_table^T) are passed to
 * the GEMM as transposed layouts instead of being copied on the host.
 *
 * Threading as in the reference (gpu_ops.c:18-21,127-152): slot 0 is shared
 * behind a mutex; gpu_ops_init_workers gives each worker its own slot (own
 * stream and device buffers) selected by a thread-local worker id.
 */
#ifndef MODEL_GPU_OPS_H
#define MODEL_GPU_OPS_H

#include "trlm_host.h"

#ifdef __cplusplus
extern "C" {
#endif

void gpu_ops_init(Allocator* scratch, const char* ptx_path);
void gpu_ops_shutdown(void);
void gpu_ops_init_workers(Allocator* scratch, const char* ptx_path, u32 num_workers);
void gpu_ops_set_worker_id(i32 worker_id);
Node* node_matmul2d_gpu(Allocator* alloc, Node* a, Node* b);
void gpu_ops_debug_stats(f64* out_total_seconds, u32* out_call_count);
void gpu_ops_debug_reset(void);

#ifdef __cplusplus
}
#endif

#endif /* MODEL_GPU_OPS_H */
