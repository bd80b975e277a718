#!/usr/bin/env bash
# dropin.sh -- TEST INFRASTRUCTURE ONLY: the drop-in binding, built for real.
#
# Builds every program of the reference (scripts/build_all.sh:24-40 compiles
# each main against all non-main objects) the way a maintainer binds this
# library to the reference, from the reference's sources where they lie:
#   - an overlay of the reference tree (real directories, a symlink per file,
#     in a temporary directory outside this repository) in which
#     model/gpu_train.h and model/gpu_ops.h are this build's headers and
#     model/ also holds hip_backend.h, trlm_host.h and trlm_ext.h;
#   - model/gpu_train.c, model/gpu_ops.c and cuda/cuda_backend.c left out of
#     the objects; programs linked with libtrlm_hip.so and libamdhip64
#     instead of -lcuda;
#   - the reference's flags (-Wall -Wextra -std=c11 -O2 -pthread -I.), plus
#     -D_DEFAULT_SOURCE, which glibc needs for MAP_ANONYMOUS under -std=c11
#     (runtime/memory.c:33), as oracle/Makefile adds it.
# tests/test_cuda.c is the one program not built: it drives the CUDA backend
# itself (cuda/cuda_backend.h) and the reference's test-only kernels.
# Outputs: oracle/_ref/dropin/<dir>_<program> (never committed), and
# oracle/_ref/dropin/layout.txt, sizeof/offsetof of the host types from the
# reference's own headers.  Usage: oracle/dropin.sh [reference root]
set -euo pipefail
REF=${1:-/root/reference}
HERE=$(cd "$(dirname "$0")" && pwd)
ROOT=$(dirname "$HERE")
LIBDIR=$ROOT/turkce-llm_amd
ROCM=${ROCM_PATH:-/opt/rocm}
OUT=$HERE/_ref/dropin
[ -f "$LIBDIR/libtrlm_hip.so" ] || { echo "libtrlm_hip.so not built" >&2; exit 2; }
TREE=$(mktemp -d "${TMPDIR:-/tmp}/trlm_dropin.XXXXXX")
trap 'rm -rf "$TREE"' EXIT

cp -rs "$REF/." "$TREE/"
for h in gpu_train.h gpu_ops.h; do rm -f "$TREE/model/$h"; done
for h in gpu_train.h gpu_ops.h hip_backend.h trlm_host.h trlm_ext.h; do cp "$ROOT/include/$h" "$TREE/model/$h"; done

CFLAGS=(-Wall -Wextra -std=c11 -O2 -pthread -I. -D_DEFAULT_SOURCE -I"$ROCM/include")
mkdir -p "$OUT" "$TREE/.obj"
cd "$TREE"
OBJS=()
MAINS=()
while IFS= read -r f; do
    case "$f" in
        model/gpu_train.c|model/gpu_ops.c|cuda/*) continue ;;
    esac
    if grep -q 'int main' "$f"; then MAINS+=("$f"); continue; fi
    o=".obj/$(echo "$f" | tr / _).o"
    gcc "${CFLAGS[@]}" -c "$f" -o "$o"
    OBJS+=("$o")
done < <(find . -name '*.c' -not -path './.obj/*' | sed 's|^\./||' | sort)

built=0
for f in "${MAINS[@]}"; do
    [ "$f" = tests/test_cuda.c ] && continue
    name=$(echo "${f%.c}" | tr / _)
    gcc "${CFLAGS[@]}" "$f" "${OBJS[@]}" -o "$OUT/$name" -L"$LIBDIR" -ltrlm_hip -Wl,-rpath,"$LIBDIR" \
        -L"$ROCM/lib" -lamdhip64 -Wl,-rpath,"$ROCM/lib"
    built=$((built + 1))
done

# host-type layout from the reference's own headers (compared with
# trlm_host.h's definitions by tests/test_abi.py)
cat > .obj/layout.c <<'EOF'
#include <stddef.h>
#include <stdio.h>
#include "runtime/types.h"
#include "runtime/memory.h"
#include "runtime/prng.h"
#include "tensor/tensor.h"
#include "autograd/node.h"
#include "model/lm_model.h"
#include "training/adam.h"
#define S(T) printf(#T " %zu\n", sizeof(T))
#define O(T, m) printf(#T "." #m " %zu\n", offsetof(T, m))
int main(void) {
    S(Arena); S(Allocator); S(Tensor); S(Node); S(PCGState); S(AttentionWeights); S(FeedForwardWeights);
    S(BlockWeights); S(LMModel); S(AdamOptimizer);
    O(Allocator, free_list); O(Tensor, strides); O(Tensor, ndim); O(Tensor, numel); O(Tensor, owns_data);
    O(Node, grad); O(Node, requires_grad); O(Node, parents); O(Node, num_parents); O(Node, backward_fn);
    O(Node, visited); O(Node, aux_dim0); O(Node, aux_scalar); O(Node, aux_ptr);
    O(PCGState, has_cached_gaussian); O(PCGState, cached_gaussian);
    O(BlockWeights, attn); O(BlockWeights, ffn_norm_w); O(BlockWeights, ffn);
    O(LMModel, blocks); O(LMModel, final_norm_w); O(LMModel, num_layers); O(LMModel, vocab_size); O(LMModel, eps);
    O(AdamOptimizer, m); O(AdamOptimizer, v); O(AdamOptimizer, num_params); O(AdamOptimizer, t);
    O(AdamOptimizer, lr); O(AdamOptimizer, eps);
    return 0;
}
EOF
gcc -std=c11 -I. .obj/layout.c -o .obj/layout
.obj/layout > "$OUT/layout.txt"
echo "dropin: ${#OBJS[@]} reference objects, $built programs linked against libtrlm_hip.so -> $OUT"
