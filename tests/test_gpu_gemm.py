"""fp32 MFMA GEMM parity through the C ABI (trlm_gemm), against fp64 numpy.

Covers the reference's GEMM contract (train_kernels.cu:97-193,226-329;
gpu_train.c:42-118): NN / NT / TN layouts, batched strides, alpha/beta,
bias and residual epilogues, off-grid shapes (M, N, K not multiples of the
tiles), unaligned leading dimensions (scalar-load variants), split-K, and the
model's real shapes at M = B*T = 8192.  Tolerance: max |C - C64| <= 1e-4 *
max |C64| per output (the north star's fp32 bar), except exact cases.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev(trlm):
    d = trlm.Device()
    yield d
    d.close()


def stored(op_mat, trans):
    """The array as it is stored for a given op(): A^T is stored for trans."""
    return np.ascontiguousarray(op_mat.T if trans else op_mat)


def run_gemm(dev, A, B, ta, tb, alpha=1.0, beta=0.0, C0=None, bias=None, resid=None, pad=0):
    """C = alpha*A@B (+beta*C0) (+bias) (+resid) with A [M,K], B [K,N] given as
    op() values; stored transposed when ta/tb.  pad widens leading dims."""
    M, K = A.shape
    N = B.shape[1]
    As, Bs = stored(A, ta), stored(B, tb)
    if pad:
        As = np.pad(As, ((0, 0), (0, pad)))
        Bs = np.pad(Bs, ((0, 0), (0, pad)))
    lda, ldb = As.shape[1], Bs.shape[1]
    dA, dB = dev.upload(As.astype(np.float32)), dev.upload(Bs.astype(np.float32))
    c_init = np.zeros((M, N), np.float32) if C0 is None else C0.astype(np.float32)
    dC = dev.upload(c_init)
    dbias = dev.upload(bias.astype(np.float32)) if bias is not None else None
    dres = dev.upload(resid.astype(np.float32)) if resid is not None else None
    dev.matmul(ta, tb, dA, dB, dC, M, N, K, lda, ldb, N, alpha=alpha, beta=beta, bias=dbias, resid=dres, ldr=N)
    out = dev.download(dC, (M, N))
    variant = dev.last_variant()
    for p in (dA, dB, dC, dbias, dres):
        if p is not None:
            dev.free(p)
    return out, variant


def ref64(A, B, alpha=1.0, beta=0.0, C0=None, bias=None, resid=None):
    r = alpha * (A.astype(np.float64) @ B.astype(np.float64))
    if beta != 0.0:
        r = r + beta * C0
    if bias is not None:
        r = r + bias
    if resid is not None:
        r = resid + r
    return r


TILES = ["256x128", "128x256", "128x128", "128x128_k32", "64x128", "64x128_k32", "64x64", "64x64_k32"]


def close(got, want, tol=1e-4):
    scale = max(np.abs(want).max(), 1e-30)
    err = np.abs(got.astype(np.float64) - want).max()
    return err <= tol * scale, err / scale


def test_mfma_lane_layout(trlm, dev):
    """The operand/result lane layout every GEMM and attention kernel
    assumes for v_mfma_f32_32x32x2f32, checked exactly with small integers."""
    hip = dev.hip
    rng = np.random.default_rng(0)
    a = rng.integers(-4, 5, 64).astype(np.float32)
    b = rng.integers(-4, 5, 64).astype(np.float32)
    da, db, dout = dev.upload(a), dev.upload(b), dev.empty(64 * 16 * 4)
    f = hip.hip_get_kernel(C.byref(dev.ctx), b"k_mfma_layout_probe")
    pa, pb, po = C.c_void_p(da), C.c_void_p(db), C.c_void_p(dout)
    args = (C.c_void_p * 3)(C.addressof(pa), C.addressof(pb), C.addressof(po))
    hip.hip_launch(f, 1, 1, 1, 64, 1, 1, 0, args)
    out = dev.download(dout, (64, 16))
    A = np.zeros((32, 2)); B = np.zeros((2, 32))
    for l in range(64):
        A[l % 32, l // 32] = a[l]
        B[l // 32, l % 32] = b[l]
    D = A @ B
    want = np.zeros((64, 16))
    for l in range(64):
        for r in range(16):
            want[l, r] = D[8 * (r // 4) + 4 * (l // 32) + r % 4, l % 32]
    for p in (da, db, dout):
        dev.free(p)
    assert np.array_equal(out, want)


def test_mfma16_lane_layout(trlm, dev):
    """The lane layout the fused decode GEMMs (decode_fused.hip) assume for
    v_mfma_f32_16x16x4f32: lane l holds A[l % 16][l / 16] and B[l / 16][l % 16];
    result register r of lane l is D[4 (l / 16) + r][l % 16].  Exact with
    small integers."""
    hip = dev.hip
    rng = np.random.default_rng(1)
    a = rng.integers(-4, 5, 64).astype(np.float32)
    b = rng.integers(-4, 5, 64).astype(np.float32)
    da, db, dout = dev.upload(a), dev.upload(b), dev.empty(64 * 4 * 4)
    f = hip.hip_get_kernel(C.byref(dev.ctx), b"k_mfma16_layout_probe")
    pa, pb, po = C.c_void_p(da), C.c_void_p(db), C.c_void_p(dout)
    args = (C.c_void_p * 3)(C.addressof(pa), C.addressof(pb), C.addressof(po))
    hip.hip_launch(f, 1, 1, 1, 64, 1, 1, 0, args)
    out = dev.download(dout, (64, 4))
    A = np.zeros((16, 4)); B = np.zeros((4, 16))
    for l in range(64):
        A[l % 16, l // 16] = a[l]
        B[l // 16, l % 16] = b[l]
    D = A @ B
    want = np.zeros((64, 4))
    for l in range(64):
        for r in range(4):
            want[l, r] = D[4 * (l // 16) + r, l % 16]
    for p in (da, db, dout):
        dev.free(p)
    assert np.array_equal(out, want)


SMALL = [  # M, N, K
    (1, 1, 1), (4, 5, 3), (12, 150, 32), (65, 33, 17), (64, 64, 64), (127, 129, 130),
    (200, 96, 48), (31, 1000, 40), (128, 128, 16), (300, 200, 600), (96, 160, 1200),
]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("M,N,K", SMALL)
def test_gemm_offgrid(dev, M, N, K, ta, tb):
    rng = np.random.default_rng(M * 7 + N * 13 + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    got, var = run_gemm(dev, A, B, ta, tb)
    ok, rel = close(got, ref64(A, B))
    assert ok, (var, rel)


RAGGED_ALIGNED = [  # M, N, K: odd sizes, leading dims rounded up to 4
    (301, 203, 605), (130, 70, 5001), (257, 129, 47), (8, 1031, 333),
]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("M,N,K", RAGGED_ALIGNED)
def test_gemm_ragged_aligned_nan_padding(dev, M, N, K, ta, tb):
    """Edge tiles of the aligned kernels run the unchecked loop with their
    out-of-range rows/columns redirected, and a partial last k step runs
    guarded.  The stored rows are padded to a multiple of 4 with NaN: any
    padding element that reached a stored output would show."""
    rng = np.random.default_rng(M + 3 * N + 7 * K + ta + 2 * tb)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)

    def padded(x):
        w = (x.shape[1] + 3) // 4 * 4
        out = np.full((x.shape[0], w), np.nan, np.float32)
        out[:, :x.shape[1]] = x
        return out

    As, Bs = padded(stored(A, ta)), padded(stored(B, tb))
    dA, dB = dev.upload(As), dev.upload(Bs)
    dC = dev.upload(np.zeros((M, N), np.float32))
    dev.matmul(ta, tb, dA, dB, dC, M, N, K, As.shape[1], Bs.shape[1], N)
    got = dev.download(dC, (M, N))
    var = dev.last_variant()
    for x in (dA, dB, dC):
        dev.free(x)
    assert "_u" not in var[0], var          # the aligned kernels ran
    assert np.isfinite(got).all(), var
    ok, rel = close(got, ref64(A, B))
    assert ok, (var, rel)


def test_gemm_small_integers_exact(dev):
    """test_cuda.c:55-94's case (4x3 @ 3x5 of small exact values): exact."""
    A = np.array([(i % 7) - 3.0 for i in range(12)], np.float32).reshape(4, 3)
    B = np.array([(i % 5) * 0.5 for i in range(15)], np.float32).reshape(3, 5)
    for ta, tb in [(0, 0), (0, 1), (1, 0)]:
        got, _ = run_gemm(dev, A, B, ta, tb)
        assert np.array_equal(got, (A.astype(np.float64) @ B).astype(np.float32))


@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_gemm_epilogue_terms_bitwise(dev, tile, ta, tb):
    """Each epilogue term alone and bias with the residual, on every forced
    tile variant and split count, off-grid (edge tiles in M and N): with the
    accumulation fixed by the forced plan, C must equal, bit for bit, the
    plain product P = alpha*acc plus the term in fp32 (P + bias, resid + P,
    P + C0 at beta 1, resid + (P + bias)).  The aligned operands take the
    transposed LDS store, so this pins its row / column / term wiring; P
    itself is checked against fp64."""
    rng = np.random.default_rng(11 + len(tile) + 3 * ta + 7 * tb)
    M, N, K = 300, 260, 1000
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    try:
        for splits in (1, 3):
            dev.force(tile, splits)
            P, var = run_gemm(dev, A, B, ta, tb, alpha=0.5)
            assert var == ("k_gemm_%s_%s" % (["nn", "nt", "tn"][ta * 2 + tb], tile), splits), var
            ok, rel = close(P, ref64(A, B, 0.5))
            assert ok, (var, rel)
            cases = [(dict(bias=bias), P + bias), (dict(resid=resid), resid + P),
                     (dict(beta=1.0, C0=C0), P + C0), (dict(bias=bias, resid=resid), resid + (P + bias))]
            for kw, want in cases:
                got, _ = run_gemm(dev, A, B, ta, tb, alpha=0.5, **kw)
                assert np.array_equal(got.view(np.uint32), want.astype(np.float32).view(np.uint32)), (var, sorted(kw))
    finally:
        dev.force(None)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_gemm_epilogue(dev, ta, tb):
    rng = np.random.default_rng(5)
    M, N, K = 257, 190, 96
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    got, _ = run_gemm(dev, A, B, ta, tb, alpha=0.5, beta=1.0, C0=C0, bias=bias, resid=resid)
    ok, rel = close(got, ref64(A, B, 0.5, 1.0, C0, bias, resid))
    assert ok, rel


def test_gemm_unaligned_leading_dims(dev):
    rng = np.random.default_rng(9)
    M, N, K = 71, 45, 33   # with pad=2 every stored row length is odd
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    for ta, tb in [(0, 0), (0, 1), (1, 0)]:
        got, var = run_gemm(dev, A, B, ta, tb, pad=2)
        assert var[0].endswith("_u")
        ok, rel = close(got, ref64(A, B))
        assert ok, (var, rel)


@pytest.mark.parametrize("M,N,K", [(384, 384, 8192), (100, 68, 4000), (1024, 384, 8192), (700, 132, 2048)])
def test_gemm_split_k(dev, M, N, K):
    """Long-K weight-gradient shapes take the split-K path; partials are
    reduced in split order, so two runs are bit-identical."""
    rng = np.random.default_rng(M + K)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    got, var = run_gemm(dev, A, B, 1, 0)
    assert var[1] > 1, var
    ok, rel = close(got, ref64(A, B))
    assert ok, (var, rel)
    again, _ = run_gemm(dev, A, B, 1, 0)
    assert np.array_equal(got.view(np.uint32), again.view(np.uint32))


def test_gemm_batched(dev):
    rng = np.random.default_rng(11)
    bt, M, N, K = 5, 70, 50, 40
    A = rng.standard_normal((bt, M, K)).astype(np.float32)
    B = rng.standard_normal((bt, K, N)).astype(np.float32)
    dA, dB, dC = dev.upload(A), dev.upload(B), dev.empty(bt * M * N * 4)
    dev.matmul(0, 0, dA, dB, dC, M, N, K, K, N, N, batch=bt, sA=M * K, sB=K * N, sC=M * N)
    got = dev.download(dC, (bt, M, N))
    for p in (dA, dB, dC):
        dev.free(p)
    want = np.einsum("bmk,bkn->bmn", A.astype(np.float64), B.astype(np.float64))
    ok, rel = close(got, want)
    assert ok, rel


MODEL = [  # name, M, N, K, ta, tb (row-major as the trainer lays them out)
    ("qkv_fwd", 8192, 1152, 384, 0, 0),
    ("attn_out_fwd", 8192, 384, 384, 0, 0),
    ("gate_up_fwd", 8192, 2048, 384, 0, 0),
    ("down_fwd", 8192, 384, 1024, 0, 0),
    ("qkv_dx", 8192, 384, 1152, 0, 1),
    ("attn_out_dx", 8192, 384, 384, 0, 1),
    ("gate_up_dx", 8192, 384, 2048, 0, 1),
    ("down_dx", 8192, 1024, 384, 0, 1),
    ("qkv_dw", 384, 1152, 8192, 1, 0),
    ("attn_out_dw", 384, 384, 8192, 1, 0),
    ("gate_up_dw", 384, 2048, 8192, 1, 0),
    ("down_dw", 1024, 384, 8192, 1, 0),
]


@pytest.mark.parametrize("name,M,N,K,ta,tb", MODEL)
def test_gemm_model_shapes(dev, name, M, N, K, ta, tb):
    rng = np.random.default_rng(len(name))
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = (0.02 * rng.standard_normal((K, N))).astype(np.float32)
    got, var = run_gemm(dev, A, B, ta, tb)
    ok, rel = close(got, ref64(A, B))
    print("%s %s split %d: max err / max|C| = %.2e" % (name, var[0], var[1], rel))
    assert ok, (name, var, rel)


def test_gemm_lm_head_rows(dev):
    """LM head NT [8192,384] x E[31769,384]^T, checked on a row sample."""
    rng = np.random.default_rng(3)
    M, N, K = 8192, 31769, 384
    A = rng.standard_normal((M, K)).astype(np.float32)
    E = (0.02 * rng.standard_normal((N, K))).astype(np.float32)
    ldc = (N + 3) // 4 * 4
    dA, dE, dC = dev.upload(A), dev.upload(E), dev.empty(M * ldc * 4)
    dev.matmul(0, 1, dA, dE, dC, M, N, K, K, K, ldc)
    got = dev.download(dC, (M, ldc))[:, :N]
    for p in (dA, dE, dC):
        dev.free(p)
    rows = rng.choice(M, 64, replace=False)
    want = A[rows].astype(np.float64) @ E.T.astype(np.float64)
    ok, rel = close(got[rows], want)
    assert ok, rel


def test_gemm_lm_head_backward_rows(dev):
    """The LM head's two backward GEMMs at full size, in the trainer's layout
    (logit rows padded to ld = 31772), checked against fp64 on samples:
    dX = dlogits [8192, 31769] . E [31769, 384] (NN, K = 31769, split-K)
    on 64 rows, and dW = dlogits^T . nf [31769, 8192] x [8192, 384] (TN,
    M = 31769) on 64 rows, including the last one."""
    rng = np.random.default_rng(21)
    M, V, D, ld = 8192, 31769, 384, 31772
    G = np.zeros((M, ld), np.float32)
    G[:, :V] = rng.standard_normal((M, V), dtype=np.float32)
    G[:, V:] = np.float32("nan")                  # padding columns are never read
    E = (0.02 * rng.standard_normal((V, D))).astype(np.float32)
    nf = rng.standard_normal((M, D)).astype(np.float32)
    dG, dE, dnf = dev.upload(G), dev.upload(E), dev.upload(nf)
    dX, dW = dev.empty(M * D * 4), dev.empty(V * D * 4)
    try:
        dev.matmul(0, 0, dG, dE, dX, M, D, V, ld, D, D)
        var_x = dev.last_variant()
        dev.matmul(1, 0, dG, dnf, dW, V, D, M, ld, D, D)
        var_w = dev.last_variant()
        gx = dev.download(dX, (M, D))
        gw = dev.download(dW, (V, D))
    finally:
        for p in (dG, dE, dnf, dX, dW):
            dev.free(p)
    rows = np.sort(rng.choice(M, 64, replace=False))
    ok, rel = close(gx[rows], G[rows, :V].astype(np.float64) @ E.astype(np.float64))
    print("lm_head_dx %s split %d: %.2e" % (var_x[0], var_x[1], rel))
    assert ok, (var_x, rel)
    assert var_x[1] > 1, var_x
    wrows = np.sort(np.concatenate([rng.choice(V - 1, 63, replace=False), [V - 1]]))
    ok, rel = close(gw[wrows], G[:, wrows].T.astype(np.float64) @ nf.astype(np.float64))
    print("lm_head_dw %s split %d: %.2e" % (var_w[0], var_w[1], rel))
    assert ok, (var_w, rel)



@pytest.mark.parametrize("tile", TILES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_gemm_every_tile_variant(dev, tile, ta, tb):
    """Each aligned tile variant, forced, on an off-grid shape (M, N not
    tile multiples, K not a multiple of the k step) with the full epilogue,
    then with a forced split-K; the selection is restored afterwards."""
    rng = np.random.default_rng(len(tile) * 3 + ta + 2 * tb)
    M, N, K = 300, 260, 1000
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    C0 = rng.standard_normal((M, N)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    resid = rng.standard_normal((M, N)).astype(np.float32)
    try:
        for splits in (1, 3):
            dev.force(tile, splits)
            got, var = run_gemm(dev, A, B, ta, tb, alpha=0.5, beta=1.0, C0=C0, bias=bias, resid=resid)
            assert var == ("k_gemm_%s_%s" % (["nn", "nt", "tn"][ta * 2 + tb], tile), splits), var
            ok, rel = close(got, ref64(A, B, 0.5, 1.0, C0, bias, resid))
            assert ok, (var, rel)
    finally:
        dev.force(None)


@pytest.mark.parametrize("splits", [1, 2, 5, 8, 13])
def test_splitk_reduce4_equals_scalar_reduce(trlm, dev, splits):
    """k_gemm_splitk_reduce4 (four columns per thread, taken when every operand
    is 16-byte aligned) against k_gemm_splitk_reduce on the same partials:
    same bits for every epilogue term and for the column-sum row (row M of
    the partials), with split counts on both sides of its 4-wide load loop."""
    import ctypes as C
    _, hip = trlm.libs()
    rng = np.random.default_rng(splits)
    M, N, ldc, ldr = 37, 388, 392, 396
    rows = M + 1
    W = rng.standard_normal((splits, rows, N)).astype(np.float32)
    C0 = rng.standard_normal((M, ldc)).astype(np.float32)
    bias = rng.standard_normal(N).astype(np.float32)
    resid = rng.standard_normal((M, ldr)).astype(np.float32)
    dW, dbias, dres = dev.upload(W), dev.upload(bias), dev.upload(resid)
    fs = hip.hip_get_kernel(C.byref(dev.ctx), b"k_gemm_splitk_reduce")
    f4 = hip.hip_get_kernel(C.byref(dev.ctx), b"k_gemm_splitk_reduce4")
    try:
        for alpha, beta, use_b, use_r in [(1.0, 0.0, False, False), (0.5, 0.0, True, False), (0.5, 0.0, False, True),
                                          (0.5, 1.0, True, False), (0.75, 0.0, True, True)]:
            outs = []
            for f, nthreads in ((fs, rows * N), (f4, rows * N // 4)):
                dC, dcs = dev.upload(C0), dev.empty(N * 4)
                a = [C.c_void_p(dW), C.c_int32(splits), C.c_int64(rows * N), C.c_void_p(dC), C.c_int32(M),
                     C.c_int32(N), C.c_int32(ldc), C.c_float(alpha), C.c_float(beta),
                     C.c_void_p(dbias if use_b else None), C.c_void_p(dres if use_r else None), C.c_int32(ldr),
                     C.c_void_p(dcs)]
                args = (C.c_void_p * len(a))(*[C.addressof(x) for x in a])
                hip.hip_launch(f, (nthreads + 255) // 256, 1, 1, 256, 1, 1, 0, args)
                outs.append((dev.download(dC, (M, ldc)), dev.download(dcs, N)))
                dev.free(dC)
                dev.free(dcs)
            (cs, ss), (c4, s4) = outs
            assert np.array_equal(cs.view(np.uint32), c4.view(np.uint32)), (alpha, beta, use_b, use_r)
            assert np.array_equal(ss.view(np.uint32), s4.view(np.uint32))
            want = alpha * W[:, :M, :].astype(np.float64).sum(0)
            if beta:
                want = want + beta * C0[:, :N]
            if use_b:
                want = want + bias
            if use_r:
                want = resid[:, :N] + want
            assert np.abs(c4[:, :N] - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
            assert np.array_equal(c4[:, N:], C0[:, N:])   # columns past N untouched
    finally:
        for p in (dW, dbias, dres):
            dev.free(p)



@pytest.mark.parametrize("tile", ["128x128", "128x128_k32", "256x128", "64x128_k32", "64x64_k32"])
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1)])
def test_gemm_store_paths_agree(dev, tile, ta, tb):
    """With the accumulation fixed by the forced plan, the epilogue's two
    store paths give the same bits: ldc a multiple of 4 takes the store
    through LDS, an odd ldc the per-element path (both map the interleaved
    fragments' rows and columns, for the NN / TN kernels that use them),
    with alpha alone, bias + residual, and beta * C.  Columns past N are not
    touched."""
    rng = np.random.default_rng(17 + len(tile) + 3 * ta + tb)
    M, N, K = 300, 260, 200
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    As, Bs = stored(A, ta), stored(B, tb)
    bias = rng.standard_normal(N).astype(np.float32)
    dA, dB, db = dev.upload(As), dev.upload(Bs), dev.upload(bias)
    try:
        dev.force(tile, 1)
        for terms in ("alpha", "bias_resid", "beta"):
            outs = []
            for ldc in (N, N + 3):
                C0 = rng.standard_normal((M, ldc)).astype(np.float32) if not outs else outs_c0_pad(outs[0][1], ldc)
                R0 = C0.copy()
                dC, dR = dev.upload(C0), dev.upload(R0)
                kw = {}
                if terms == "bias_resid":
                    kw = dict(bias=db, resid=dR, ldr=ldc)
                elif terms == "beta":
                    kw = dict(beta=1.0)
                dev.matmul(ta, tb, dA, dB, dC, M, N, K, As.shape[1], Bs.shape[1], ldc, alpha=0.5, **kw)
                assert dev.last_variant() == ("k_gemm_%s_%s" % (["nn", "nt", "tn"][ta * 2 + tb], tile), 1)
                got = dev.download(dC, (M, ldc))
                outs.append((got, C0))
                dev.free(dC)
                dev.free(dR)
            (g0, c0), (g1, c1) = outs
            assert np.array_equal(g0[:, :N].view(np.uint32), g1[:, :N].view(np.uint32)), terms
            assert np.array_equal(g1[:, N:], c1[:, N:])
            want = ref64(A, B, 0.5, 1.0 if terms == "beta" else 0.0, c0[:, :N],
                         bias if terms == "bias_resid" else None, c0[:, :N] if terms == "bias_resid" else None)
            ok, rel = close(g0[:, :N], want)
            assert ok, (terms, rel)
    finally:
        dev.force(None)
        for p in (dA, dB, db):
            dev.free(p)


def outs_c0_pad(c0, ldc):
    """The first run's initial C (and residual) widened to ldc columns, so
    both runs add the same values."""
    out = np.zeros((c0.shape[0], ldc), np.float32)
    out[:, :c0.shape[1]] = c0[:, :min(c0.shape[1], ldc)]
    out[:, c0.shape[1]:] = 7.0
    return out
