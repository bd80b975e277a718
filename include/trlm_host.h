/* trlm_host.h -- host-side types that appear in the trainer's C signatures.
 *
 * The GPU path's entry points (gpu_train.h, gpu_ops.h) take the reference's
 * host structures by pointer, so these definitions are layout-compatible
 * with the reference's own:
 *   u8..f64 / bool32        runtime/types.h:9-29
 *   Arena / Allocator       runtime/memory.h:56-86
 *   Tensor                  tensor/tensor.h:18-27
 *   Node                    autograd/node.h:23-46
 *   PCGState                runtime/prng.h:17-22
 *   Attention/FeedForward/BlockWeights, LMModel
 *                           model/attention.h:18-21, feedforward.h:13-16,
 *                           transformer_block.h:12-17, lm_model.h:12-23
 *   AdamOptimizer           training/adam.h:13-20
 *
 * The functions declared at the bottom are the host runtime the GPU path
 * calls (allocation, tensor views, RoPE tables, PCG, scalar maths).  In a
 * drop-in build they resolve to the reference's own objects; standalone they
 * come from libtrlm_host.so (turkce-llm_amd/csrc/host/trlm_host.c).
 *
 * Installed in the reference tree (this header beside model/lm_model.h, as
 * the drop-in puts it), the definitions come from the reference's own
 * headers instead, so the reference's callers, which include those headers
 * too, see each type defined once.  TRLM_STANDALONE_TYPES forces the
 * definitions below.
 */
#ifndef TRLM_HOST_H
#define TRLM_HOST_H

#if !defined(TRLM_STANDALONE_TYPES) && __has_include("lm_model.h") && __has_include("../runtime/types.h") && \
    __has_include("../training/adam.h")
#define TRLM_HOST_FROM_REFERENCE 1
#include "../runtime/types.h"
#include "../runtime/memory.h"
#include "../runtime/prng.h"
#include "../runtime/mathlib.h"
#include "../tensor/tensor.h"
#include "../autograd/node.h"
#include "lm_model.h"
#include "rope.h"
#include "../training/adam.h"
#else

typedef unsigned char      u8;
typedef unsigned short     u16;
typedef unsigned int       u32;
typedef unsigned long long u64;
typedef signed char        i8;
typedef signed short       i16;
typedef signed int         i32;
typedef signed long long   i64;
typedef float  f32;
typedef double f64;
typedef u64 usize;
typedef i64 isize;
typedef u32 bool32;
#ifndef TRUE
#define TRUE  1
#define FALSE 0
#endif
#define NULL_PTR ((void*)0)

typedef struct Arena {
    u8* base;
    u64 reserved;
    u64 committed;
    u64 used;
} Arena;

typedef struct FreeBlock FreeBlock;

typedef struct Allocator {
    Arena backing;
    FreeBlock* free_list;
    FreeBlock* last_phys;
} Allocator;

#define TENSOR_MAX_DIMS 6

typedef struct Tensor {
    f32* data;
    u64  shape[TENSOR_MAX_DIMS];
    i64  strides[TENSOR_MAX_DIMS];   /* in elements */
    u32  ndim;
    u64  numel;
    bool32 owns_data;
} Tensor;

#define NODE_MAX_PARENTS 3

typedef struct Node Node;
struct Node {
    Tensor value;
    Tensor grad;
    bool32 requires_grad;
    Node* parents[NODE_MAX_PARENTS];
    u32 num_parents;
    void (*backward_fn)(Node* self, Allocator* alloc);
    bool32 visited;
    u32 aux_dim0;
    u32 aux_dim1;
    f32 aux_scalar;
    const void* aux_ptr;
};

typedef struct PCGState {
    u64 state;
    u64 inc;
    bool32 has_cached_gaussian;
    f64 cached_gaussian;
} PCGState;

typedef struct AttentionWeights {
    Node* w_qkv; Node* b_qkv;   /* [D, 3D], [3D] */
    Node* wo; Node* bo;         /* [D, D],  [D]  */
} AttentionWeights;

typedef struct FeedForwardWeights {
    Node* w_gate_up; Node* b_gate_up;   /* [D, 2F], [2F]: gate | up */
    Node* w_down; Node* b_down;         /* [F, D],  [D] */
} FeedForwardWeights;

typedef struct BlockWeights {
    Node* attn_norm_w;
    AttentionWeights attn;
    Node* ffn_norm_w;
    FeedForwardWeights ffn;
} BlockWeights;

#define LM_MAX_LAYERS 32

typedef struct LMModel {
    Node* embed_table;   /* [V, D], tied output projection */
    BlockWeights blocks[LM_MAX_LAYERS];
    Node* final_norm_w;
    u32 num_layers;
    u32 num_heads;
    u32 d_model;
    u32 vocab_size;
    f32 eps;
} LMModel;

typedef struct AdamOptimizer {
    Node** params;
    Tensor* m;
    Tensor* v;
    u32 num_params;
    u64 t;
    f32 lr, beta1, beta2, eps;
} AdamOptimizer;

#ifdef __cplusplus
extern "C" {
#endif

/* allocation (runtime/memory.h:88-91) */
Allocator allocator_create(u64 reserve_size);
void* allocator_alloc(Allocator* a, u64 size);
void  allocator_free(Allocator* a, void* ptr);
void  allocator_destroy(Allocator* a);

/* tensors and graph nodes (tensor/tensor.h:32-79, autograd/node.h:48-74) */
Tensor tensor_create(Allocator* alloc, const u64* shape, u32 ndim);
bool32 tensor_is_contiguous(const Tensor* t);
Tensor tensor_transpose(const Tensor* src, u32 dim0, u32 dim1);
Tensor tensor_contiguous(Allocator* alloc, const Tensor* src);
void tensor_add_inplace(Tensor* dst, const Tensor* src);
Node* node_leaf(Allocator* alloc, Tensor value, bool32 requires_grad);
Node* node_make_custom(Allocator* alloc, Tensor value, bool32 requires_grad);
void backward(Allocator* alloc, Node* loss);

/* PCG32 (runtime/prng.h:26-44) and scalar maths (runtime/mathlib.h:35-50) */
PCGState pcg_seed(u64 initstate, u64 initseq);
u32 pcg_next_u32(PCGState* rng);
i64 pcg_range_i64(PCGState* rng, i64 lo, i64 hi);
f64 pcg_gaussian(PCGState* rng, f64 mean, f64 stddev);
f64 m_sqrt(f64 x);
f64 m_exp(f64 x);
f64 m_log(f64 x);
f64 m_pow(f64 base, f64 exponent);
f64 m_sin(f64 x);
f64 m_cos(f64 x);
f32 m_sqrtf(f32 x);
f32 m_powf(f32 base, f32 exponent);
f32 m_sinf(f32 x);
f32 m_cosf(f32 x);

/* RoPE tables [seq_len, head_dim/2] (model/rope.h:10) */
void rope_build_tables(Tensor* cos_out, Tensor* sin_out, u64 seq_len, u64 head_dim, f32 base);

#ifdef __cplusplus
}
#endif

#endif /* types from the reference's headers */
#endif /* TRLM_HOST_H */
