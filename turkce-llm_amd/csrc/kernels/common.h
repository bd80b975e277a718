// common.h -- shared device helpers for the gfx950 kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

#define WAVE 64

// Fixed-order butterfly reductions across the 64 lanes of a wavefront.  The
// xor pattern is fixed, so every lane ends with the same, reproducible value.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, WAVE));
    return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, WAVE);
    return v;
}

// Greedy pick of one row, the rule of the reference's max scan
// (generate.c:57-58: best starts at index 0 and moves only to a strictly
// greater value).  Threads collect (value, index) with a strict > from
// (-inf, ARGMAX_NONE), and reductions keep the larger value, the lower index
// on ties, so NaNs are never picked; the result is then 0 when row[0] is NaN
// (no value compares greater than it) or when nothing exceeded -inf.  Every
// pick is a valid index, whatever the row holds.
#define ARGMAX_NONE 0x7fffffff
__device__ __forceinline__ int argmax_finish(const float* row, int idx) {
    const float z0 = row[0];
    return (z0 != z0 || idx == ARGMAX_NONE) ? 0 : idx;
}
