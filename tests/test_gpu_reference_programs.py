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

and the reference's GPU training driver itself (training/train_lm_gpu.c),
resumed for its last three steps and compared bit for bit with this
library's queued driver loop.
"""
import os
import subprocess
import time

import numpy as np
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


def test_reference_training_driver_last_steps(trlm, orc, tmp_path):
    """The reference's own GPU training driver (training/train_lm_gpu.c),
    unchanged and linked against this library, at its own shape: the real
    model, 14 sequences x 1024 tokens per step, its lr schedule (warmup 1000,
    cosine to step 70,000, 6e-4 -> 6e-5), clipping at 1.0 and Adam (0.9,
    0.999, 1e-8).  Resumed from a TRLM checkpoint at t = 69,997 (:147-171),
    it runs the last three steps on a synthetic corpus, the validation
    windows (:226-244) and the best and final checkpoint saves, and exits.
    Its final checkpoint -- parameters, Adam moments and t -- equals, bit for
    bit, this library's queued driver loop (gpu_trainer_train_steps) run from
    the same checkpoint over the same steps; its printed validation loss
    equals gpu_trainer_eval_windows' to the three decimals it prints."""
    import re
    exe = os.path.join(BIN, "training_train_lm_gpu")
    if not os.path.exists(exe):
        pytest.skip("oracle/dropin.sh has not been run (needs the reference tree)")
    V, D, H, L, F, B, T = 31769, 384, 6, 12, 1024, 14, 1024
    first, total = 69997, 70000
    model = orc.Model(V, D, H, L, F)
    shapes = model.shapes()
    params = model.init(1337, 1)
    n = params.size
    rng = np.random.default_rng(69997)   # Adam moments of the resumed state (any seeded values)
    m0 = (1e-3 * rng.standard_normal(n)).astype(np.float32)
    v0 = np.square(1e-3 * rng.standard_normal(n)).astype(np.float32)
    tokens = orc.random_tokens(200000, V, 4242, 11, hi_exclusive=V)
    val_tokens = tokens.size * 10 // 1000
    train_tokens = tokens.size - val_tokens
    for d in ("cuda", "data/raw", "checkpoints"):
        (tmp_path / d).mkdir(parents=True)
    os.symlink(trlm.KERNELS, tmp_path / "cuda" / "train_kernels.ptx")
    tokens.tofile(tmp_path / "data" / "raw" / "wikipedia_tokens.bin")
    start = tmp_path / "checkpoints" / "lm_wiki_faz3_latest.bin"
    start.write_bytes(orc.trlm_bytes(shapes, params, m0, v0, first))

    print("running training_train_lm_gpu from step %d" % first, flush=True)
    r = subprocess.run(["timeout", "-k", "10", "120", exe], cwd=tmp_path, capture_output=True, text=True)
    print(r.stdout[-3000:])
    print(r.stderr[-2000:])
    assert r.returncode == 0, r.returncode
    got = orc.trlm_parse((tmp_path / "checkpoints" / "lm_wiki_faz3_final.bin").read_bytes(), shapes, True)
    assert got is not None
    gp, gm, gv, gt = got
    assert gt == total
    best = (tmp_path / "checkpoints" / "lm_wiki_faz3_best.bin").read_bytes()
    assert best == (tmp_path / "checkpoints" / "lm_wiki_faz3_final.bin").read_bytes()
    val_printed = float(re.search(r"val_kayip=([0-9.]+)", r.stdout).group(1))

    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    adam = trlm.Adam(hm, 6e-4, 0.9, 0.999, 1e-8)
    try:
        assert tr.checkpoint_load(str(start), adam)
        s = trlm.TrlmSchedule()
        s.warmup_steps, s.total_steps, s.peak_lr, s.min_lr = 1000, total, 6e-4, 6e-5
        s.grad_clip, s.weight_decay, s.seed_base = 1.0, 0.0, 2026
        losses, norms, lrs = tr.train_steps(adam, tokens[:train_tokens], s, first, total - first)
        val = float(tr.eval_windows(tokens, train_tokens, val_tokens, 8))
        wp = tr.download(adam)
        wm, wv, wt = adam.flat("m"), adam.flat("v"), int(adam.opt.t)
    finally:
        tr.destroy()
        hm.close()
    print("driver steps %d..%d: losses %s, grad norms %s; validation loss %.6f (printed %.3f)"
          % (first, total - 1, losses, norms, val, val_printed))
    assert np.isfinite(losses).all()
    assert wt == gt
    assert np.array_equal(wp.view(np.uint32), gp.view(np.uint32))
    assert np.array_equal(wm.view(np.uint32), gm.view(np.uint32))
    assert np.array_equal(wv.view(np.uint32), gv.view(np.uint32))
    assert abs(val - val_printed) <= 0.0005 + 1e-6, (val, val_printed)
