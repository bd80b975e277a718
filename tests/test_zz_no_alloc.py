"""trlm_gemm_noalloc: the raw GEMM with its split-K partials in the library's
fixed 32 MiB scratch array instead of an allocated workspace.

Through the C ABI:
  - two calls in a row -- a weight-gradient shape that takes split-K
    (384x1152x8192 TN: 7 splits, 12.4 MB of partials), then a smaller
    decode-sized one with the full epilogue (64 rows, alpha, beta*C, bias,
    residual) -- each equal to trlm_gemm's result on the same inputs bit for
    bit (same plan, same kernels), with the device's free memory unchanged;
  - the scratch boundary: with 8 splits forced on both engines, a
    1024x1024 product whose partials fill exactly 32 MiB runs with its 8
    splits, and a 1028x1024 one (32 MiB + 128 KiB) runs with the 7 splits
    that fit, each equal bit for bit to trlm_gemm forced to that split count;
  - the full-size LM-head dX (8192x384x31769 NN, planned with 8 splits,
    100.7 MB of partials) runs with the 2 splits that fit, equal to
    trlm_gemm forced to 2 splits.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _hip_runtime():
    """The HIP runtime this process already loaded (with libtrlm_hip.so)."""
    with open("/proc/self/maps") as fh:
        paths = {line.split()[-1] for line in fh if "libamdhip64.so" in line}
    assert len(paths) == 1, paths
    return C.CDLL(paths.pop())


def _free_bytes():
    hip = _hip_runtime()
    free, total = C.c_size_t(0), C.c_size_t(0)
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return free.value


def _case(rng, ta, tb, M, N, K, epilogue):
    A = rng.standard_normal((K, M) if ta else (M, K)).astype(np.float32)
    B = (0.02 * rng.standard_normal((N, K) if tb else (K, N))).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32) if epilogue else None
    resid = rng.standard_normal((M, N)).astype(np.float32) if epilogue else None
    return dict(ta=ta, tb=tb, M=M, N=N, K=K, A=A, B=B, C0=C0, bias=bias, resid=resid,
                alpha=0.5 if epilogue else 1.0, beta=1.0 if epilogue else 0.0)


def _upload(dev, c):
    up = {k: dev.upload(c[k]) for k in ("A", "B")}
    up["bias"] = dev.upload(c["bias"]) if c["bias"] is not None else None
    up["resid"] = dev.upload(c["resid"]) if c["resid"] is not None else None
    return up


def _lds(c):
    return c["A"].shape[1], c["B"].shape[1]


def test_noalloc_equals_trlm_gemm_two_calls(trlm):
    rng = np.random.default_rng(7)
    cases = [_case(rng, 1, 0, 384, 1152, 8192, False), _case(rng, 0, 0, 64, 1152, 384, True)]
    ref = trlm.Device()       # trlm_gemm (allocating engine) on its own context
    dev = trlm.Device()       # trlm_gemm_noalloc on a fresh engine
    try:
        want, plans = [], []
        for c in cases:
            ref.current()
            up = _upload(ref, c)
            dC = ref.upload(c["C0"])
            lda, ldb = _lds(c)
            ref.matmul(c["ta"], c["tb"], up["A"], up["B"], dC, c["M"], c["N"], c["K"], lda, ldb, c["N"],
                       alpha=c["alpha"], beta=c["beta"], bias=up["bias"], resid=up["resid"], ldr=c["N"])
            want.append(ref.download(dC, (c["M"], c["N"])))
            plans.append(ref.last_variant())
        # both take split-K (use the scratch), the second call's partials fewer
        assert plans[0][1] > 1 and plans[1][1] > 1, plans
        assert plans[1][1] * cases[1]["M"] * cases[1]["N"] < plans[0][1] * cases[0]["M"] * cases[0]["N"], plans
        dev.current()
        bufs = []
        for c in cases:
            up = _upload(dev, c)
            up["C"] = dev.upload(c["C0"])
            bufs.append(up)
        dev.sync()
        before = _free_bytes()
        for c, up in zip(cases, bufs):
            lda, ldb = _lds(c)
            rc = dev.matmul_noalloc(c["ta"], c["tb"], up["A"], up["B"], up["C"], c["M"], c["N"], c["K"], lda, ldb,
                                    c["N"], alpha=c["alpha"], beta=c["beta"], bias=up["bias"], resid=up["resid"],
                                    ldr=c["N"])
            assert rc == 0
        dev.sync()
        after = _free_bytes()
        got = [dev.download(up["C"], (c["M"], c["N"])) for c, up in zip(cases, bufs)]
        assert [dev.last_variant()] == [plans[1]]
    finally:
        dev.close()
        ref.close()
    assert after == before, (before, after)
    for g, w in zip(got, want):
        assert np.array_equal(g.view(np.uint32), w.view(np.uint32))


def _pair_run(trlm, c, splits_ref):
    """trlm_gemm with splits_ref forced, and trlm_gemm_noalloc with the
    engine's own plan (forced splits given as c['force']), on fresh
    contexts; returns (want, got, ref plan, noalloc plan, free before,
    free after)."""
    ref, dev = trlm.Device(), trlm.Device()
    try:
        ref.current()
        ref.force(None, splits_ref)
        up = _upload(ref, c)
        dC = ref.upload(c["C0"])
        lda, ldb = _lds(c)
        ref.matmul(c["ta"], c["tb"], up["A"], up["B"], dC, c["M"], c["N"], c["K"], lda, ldb, c["N"])
        want = ref.download(dC, (c["M"], c["N"]))
        plan_ref = ref.last_variant()
        dev.current()
        dev.force(None, c["force"])
        up = _upload(dev, c)
        dC = dev.upload(c["C0"])
        dev.sync()
        before = _free_bytes()
        rc = dev.matmul_noalloc(c["ta"], c["tb"], up["A"], up["B"], dC, c["M"], c["N"], c["K"], lda, ldb, c["N"])
        dev.sync()
        after = _free_bytes()
        assert rc == 0
        got = dev.download(dC, (c["M"], c["N"]))
        plan = dev.last_variant()
    finally:
        dev.close()
        ref.close()
    return want, got, plan_ref, plan, before, after


@pytest.mark.parametrize("M,fit", [(1024, 8), (1028, 7)])
def test_noalloc_scratch_boundary(trlm, M, fit):
    rng = np.random.default_rng(11)
    c = _case(rng, 1, 0, M, 1024, 2048, False)
    c["force"] = 8
    assert (8 * M * 1024 <= (32 << 20) // 4) == (fit == 8)
    want, got, plan_ref, plan, before, after = _pair_run(trlm, c, fit)
    assert plan_ref[1] == fit and plan == plan_ref, (plan_ref, plan)
    assert after == before, (before, after)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_noalloc_caps_the_lm_head_dx(trlm):
    M, V, D, ldv = 8192, 31769, 384, 31772   # the trainer's logits rows are padded to 16 bytes
    rng = np.random.default_rng(5)
    c = dict(ta=0, tb=0, M=M, N=D, K=V, A=rng.standard_normal((M, ldv), dtype=np.float32) * np.float32(1e-4),
             B=rng.standard_normal((V, D), dtype=np.float32) * np.float32(0.02), C0=np.zeros((M, D), np.float32),
             bias=None, resid=None, force=0)
    _, hip = trlm.libs()
    sp = C.c_int32(0)
    hip.trlm_gemm_plan(0, 0, M, D, V, 1, C.byref(sp))
    assert sp.value * M * D * 4 > (32 << 20), sp.value   # the plan's own partials do not fit
    want, got, plan_ref, plan, before, after = _pair_run(trlm, c, 2)
    assert plan_ref[1] == 2 and plan == plan_ref, (plan_ref, plan)
    assert after == before, (before, after)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
