"""The reference's own GPU test programs, run on MI355X against this build.

oracle/dropin.sh (run in the build container, where /root/reference
exists) compiles the reference's programs from their own sources against
include/ installed as model/gpu_train.h / model/gpu_ops.h and links them with
libtrlm_hip.so; the binaries sit in oracle/_ref/dropin/.  Each program below
is run unchanged in a directory whose cuda/kernels.ptx and
cuda/train_kernels.ptx -- the image paths the programs pass to
gpu_ops_init / gpu_trainer_create -- are this build's gfx950 code object.
A program passes when it exits 0 (each counts its own failed checks and
returns 1 on any).

  tests/test_gpu_train.c    trainer vs data_parallel_step on the CPU path
                            (off-grid, T=1024, and the real model with the
                            gpu_ops hybrid path as the CPU side): loss,
                            gradients, determinism, eval == fb, grad norm,
                            Adam, upload/download, scaled Adam
  tests/test_gpu_ops.c      node_matmul2d_gpu forward/backward vs the CPU
  tests/test_lm_model_gpu.c lm_forward with GPU layers vs the CPU
  tests/test_batched_lm.c   batched lm_forward on the GPU path
  tests/test_data_parallel.c data_parallel_step with 8 worker threads on
                            the gpu_ops worker slots vs one thread
  tests/test_resume.c       training resumed from a checkpoint with the
                            gpu_ops worker slots equals the uninterrupted run
"""
import os
import subprocess
import time

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "oracle", "_ref", "dropin")
PROGRAMS = ["tests_test_gpu_ops", "tests_test_lm_model_gpu", "tests_test_batched_lm", "tests_test_gpu_train",
            "tests_test_data_parallel", "tests_test_resume"]


@pytest.mark.parametrize("prog", PROGRAMS)
def test_reference_program_passes(trlm, tmp_path, prog):
    exe = os.path.join(BIN, prog)
    if not os.path.exists(exe):
        pytest.skip("oracle/dropin.sh has not been run (needs the reference tree)")
    (tmp_path / "cuda").mkdir()
    for name in ("kernels.ptx", "train_kernels.ptx"):
        os.symlink(trlm.KERNELS, tmp_path / "cuda" / name)
    print("running %s" % prog, flush=True)
    t0 = time.time()
    r = subprocess.run(["timeout", "-k", "10", "100", exe], cwd=tmp_path, capture_output=True, text=True)
    dt = time.time() - t0
    print(r.stdout[-4000:])
    print(r.stderr[-2000:])
    print("%s: exit %d in %.1f s" % (prog, r.returncode, dt))
    assert r.returncode == 0, (prog, r.returncode)
