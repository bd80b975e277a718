// trlm_kernels.hip -- the single gfx950 code object of the GPU path.
// Built with: hipcc --genco --offload-arch=gfx950 -O3
//             -Xclang -target-feature -Xclang -packed-fp32-ops
#include "gemm.hip"
#include "rowops.hip"
#include "attention.hip"
#include "decode.hip"
#include "decode_fused.hip"
