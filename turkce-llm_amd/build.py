"""Build the MI355X GPU path in-tree.

Outputs (next to this file, git-ignored, shipped to the GPU box as built):
  trlm_kernels.hsaco  gfx950 code object with every kernel (hipcc --genco)
  libtrlm_hip.so      the drop-in C library: hip_backend.c, trlm_gemm.c,
                      gpu_train.c, gpu_decode.c, checkpoint.c, train_loop.c,
                      gpu_ops.c (gcc, HIP runtime API)
  libtrlm_host.so     standalone host runtime (allocator, tensors, nodes,
                      PCG, scalar maths, RoPE tables) for use without the
                      reference's own runtime objects
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
INC = os.path.join(ROOT, "include")
CSRC = os.path.join(HERE, "csrc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HSACO = os.path.join(HERE, "trlm_kernels.hsaco")
LIB_HIP = os.path.join(HERE, "libtrlm_hip.so")
LIB_HOST = os.path.join(HERE, "libtrlm_host.so")
NOALLOC_O = os.path.join(HERE, "noalloc.o")

# Packed-fp32 VALU ops are disabled for all device code: some of their forms
# have given wrong results on the target boxes, without any error.
HIPCC_FLAGS = ["--genco", "--offload-arch=gfx950", "-O3", "-Xclang", "-target-feature", "-Xclang",
               "-packed-fp32-ops"]
CFLAGS = ["-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter", "-D_DEFAULT_SOURCE",
          "-D__HIP_PLATFORM_AMD__", "-I" + INC, "-I" + os.path.join(ROCM, "include")]


def _run(cmd):
    print("  " + " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build_kernels():
    src = os.path.join(CSRC, "kernels", "trlm_kernels.hip")
    _run([os.path.join(ROCM, "bin", "hipcc")] + HIPCC_FLAGS + [src, "-o", HSACO])


def build_host():
    _run(["gcc"] + CFLAGS + ["-shared", os.path.join(CSRC, "host", "trlm_host.c"), "-o", LIB_HOST])


def build_hip_lib():
    srcs = [os.path.join(CSRC, f) for f in ("hip_backend.c", "trlm_gemm.c", "gpu_train.c", "gpu_decode.c", "checkpoint.c",
                                            "train_loop.c", "gpu_ops.c")]
    # noalloc.hip holds the no-allocation GEMM's scratch array (a __device__
    # global of this library, not of the kernel image) and its entry point.
    _run([os.path.join(ROCM, "bin", "hipcc"), "-c", "-fPIC", "--offload-arch=gfx950", "-O3", "-Xclang",
          "-target-feature", "-Xclang", "-packed-fp32-ops", "-I" + INC, os.path.join(CSRC, "noalloc.hip"),
          "-o", NOALLOC_O])
    # Host-runtime symbols (allocator_alloc, tensor_*, pcg_*, m_*, rope_build_tables)
    # stay undefined: the reference's objects or libtrlm_host.so provide them.
    _run(["gcc"] + CFLAGS + ["-shared"] + srcs + [NOALLOC_O] +
         ["-o", LIB_HIP, "-L" + os.path.join(ROCM, "lib"), "-Wl,-rpath," + os.path.join(ROCM, "lib"),
          "-lamdhip64", "-pthread"])


def build_all():
    build_kernels()
    build_host()
    build_hip_lib()


if __name__ == "__main__":
    build_all()
    sys.exit(0)
