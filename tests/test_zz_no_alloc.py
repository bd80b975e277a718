"""trlm_gemm_noalloc: the raw GEMM with its split-K partials in the library's
fixed 32 MiB scratch array instead of an allocated workspace.

Through the C ABI, two calls in a row -- a weight-gradient shape whose
split-K plan fills most of the scratch (384x1152x8192 TN, 16 splits,
28.4 MB), then a smaller decode-sized one with the full epilogue (64 rows,
alpha, beta*C, bias, residual) -- each equal to trlm_gemm's result on the
same inputs bit for bit (same plan, same kernels), with the device's free
memory unchanged across both calls; and a shape whose plan needs more than
the scratch (the full LM-head dX, 100.7 MB) is refused with -1 and leaves C
untouched.
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


def test_noalloc_refuses_plans_beyond_the_scratch(trlm):
    M, V, D, ld = 8192, 31769, 384, 31772
    dev = trlm.Device()
    try:
        dG = dev.empty(M * ld * 4)          # full-size operands: nothing may be read even if launched
        dE = dev.empty(V * D * 4)
        C0 = np.full((M, D), 3.0, np.float32)
        dC = dev.upload(C0)
        rc = dev.matmul_noalloc(0, 0, dG, dE, dC, M, D, V, ld, D, D)
        dev.sync()
        got = dev.download(dC, (M, D))
    finally:
        dev.close()
    assert rc == -1
    assert np.array_equal(got, C0)
