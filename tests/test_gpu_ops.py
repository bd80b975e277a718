"""node_matmul2d_gpu (model/gpu_ops.h) through the C ABI -- the hybrid path's
GPU matmul node, as tests/test_gpu_ops.c and test_cuda.c exercise it.

  - forward equals the reference-order CPU matmul within 1e-4 of max|C|
    (test_gpu_ops.c:25-50 used 1e-2 absolute), including the tied LM head's
    transposed operand (embed_table^T) and a column-slice view, which the
    GPU path consumes without host copies;
  - backward: dA += dC B^T and dB += A^T dC accumulate onto existing grads;
  - central-difference gradient check on a 2x3 @ 3x2 product
    (test_gpu_ops.c:52-104);
  - per-worker slots from several threads (gpu_ops_init_workers +
    gpu_ops_set_worker_id) give the same results; debug counters count calls;
  - pinned operands (gpu_ops_pin, additive): a product over pinned weights,
    plain or as the head's transposed view, is bit-identical to the unpinned
    product; the pinned copy is what is read (changing the host values after
    pinning leaves the result unchanged until gpu_ops_unpin_all); a view that
    reaches past a pinned range is uploaded as before; worker slots on the
    same device share the copy.
"""
import ctypes as C
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ops(trlm):
    host, hip = trlm.libs()
    alloc = host.allocator_create(1 << 32)
    hip.gpu_ops_init(C.byref(alloc), trlm.KERNELS.encode())
    hip.gpu_ops_init_workers(C.byref(alloc), trlm.KERNELS.encode(), 3)
    yield host, hip, alloc
    hip.gpu_ops_shutdown()
    host.allocator_destroy(C.byref(alloc))


def leaf(trlm, host, alloc, arr):
    arr = np.ascontiguousarray(arr, np.float32)
    sh = (C.c_uint64 * arr.ndim)(*arr.shape)
    t = host.tensor_create(C.byref(alloc), sh, arr.ndim)
    trlm.tensor_np(t)[:] = arr.ravel()
    return host.node_leaf(C.byref(alloc), t, 1)


def value(trlm, node):
    t = node.contents.value
    return trlm.tensor_np(t).reshape(t.shape[0], t.shape[1]).copy()


def grad(trlm, node):
    t = node.contents.grad
    return trlm.tensor_np(t).reshape(t.shape[0], t.shape[1]).copy()


def run_backward(trlm, alloc, node, dC):
    trlm.tensor_np(node.contents.grad)[:] = np.ascontiguousarray(dC, np.float32).ravel()
    fn = C.CFUNCTYPE(None, trlm.NodeP, C.POINTER(trlm.Allocator))(node.contents.backward_fn)
    fn(node, C.byref(alloc))


@pytest.mark.parametrize("M,K,N", [(64, 48, 32), (4, 3, 5), (257, 384, 190), (128, 384, 1152)])
def test_forward_backward(trlm, orc, ops, M, K, N):
    host, hip, alloc = ops
    rng = np.random.default_rng(M + K + N)
    A = rng.standard_normal((M, K)).astype(np.float32)
    B = rng.standard_normal((K, N)).astype(np.float32)
    na, nb = leaf(trlm, host, alloc, A), leaf(trlm, host, alloc, B)
    # existing gradients must be accumulated onto
    ga0 = rng.standard_normal((M, K)).astype(np.float32)
    gb0 = rng.standard_normal((K, N)).astype(np.float32)
    trlm.tensor_np(na.contents.grad)[:] = ga0.ravel()
    trlm.tensor_np(nb.contents.grad)[:] = gb0.ravel()
    out = hip.node_matmul2d_gpu(C.byref(alloc), na, nb)
    got = value(trlm, out)
    want = orc.matmul(A, B)
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()
    dC = rng.standard_normal((M, N)).astype(np.float32)
    run_backward(trlm, alloc, out, dC)
    da = dC.astype(np.float64) @ B.T.astype(np.float64) + ga0
    db = A.T.astype(np.float64) @ dC.astype(np.float64) + gb0
    assert np.abs(grad(trlm, na) - da).max() <= 1e-4 * np.abs(da).max()
    assert np.abs(grad(trlm, nb) - db).max() <= 1e-4 * np.abs(db).max()


def test_tied_head_transposed_view(trlm, orc, ops):
    """logits = x @ embed_table^T with the transpose passed as a view
    (lm_model.c:128-130)."""
    host, hip, alloc = ops
    rng = np.random.default_rng(1)
    V, D, T = 3001, 384, 37
    x = rng.standard_normal((T, D)).astype(np.float32)
    E = (0.02 * rng.standard_normal((V, D))).astype(np.float32)
    nx, nE = leaf(trlm, host, alloc, x), leaf(trlm, host, alloc, E)
    Et = host.tensor_transpose(C.byref(nE.contents.value), 0, 1)
    nEt = host.node_leaf(C.byref(alloc), Et, 1)
    out = hip.node_matmul2d_gpu(C.byref(alloc), nx, nEt)
    got = value(trlm, out)
    want = orc.matmul(x, np.ascontiguousarray(E.T))
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


def test_column_slice_view(trlm, orc, ops):
    """A [rows, cols] view into a wider row-major tensor (node_slice_cols)."""
    host, hip, alloc = ops
    rng = np.random.default_rng(2)
    big = rng.standard_normal((40, 96)).astype(np.float32)
    W = rng.standard_normal((32, 24)).astype(np.float32)
    nbig, nW = leaf(trlm, host, alloc, big), leaf(trlm, host, alloc, W)
    view = trlm.Tensor.from_buffer_copy(nbig.contents.value)
    view.shape[1] = 32
    view.numel = 40 * 32
    view.data = C.cast(C.addressof(nbig.contents.value.data.contents) + 4 * 32, C.POINTER(C.c_float))
    nv = host.node_leaf(C.byref(alloc), view, 1)
    out = hip.node_matmul2d_gpu(C.byref(alloc), nv, nW)
    want = orc.matmul(np.ascontiguousarray(big[:, 32:64]), W)
    assert np.abs(value(trlm, out) - want).max() <= 1e-4 * np.abs(want).max()


def test_central_difference(trlm, ops):
    host, hip, alloc = ops
    rng = np.random.default_rng(3)
    a0 = rng.standard_normal((2, 3)).astype(np.float32)
    b0 = rng.standard_normal((3, 2)).astype(np.float32)

    def loss(a, b):
        na, nb = leaf(trlm, host, alloc, a), leaf(trlm, host, alloc, b)
        return float(value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), na, nb)).sum())

    na, nb = leaf(trlm, host, alloc, a0), leaf(trlm, host, alloc, b0)
    out = hip.node_matmul2d_gpu(C.byref(alloc), na, nb)
    run_backward(trlm, alloc, out, np.ones((2, 2), np.float32))
    ga, gb = grad(trlm, na), grad(trlm, nb)
    eps = 1e-2
    for arr, g, which in ((a0, ga, 0), (b0, gb, 1)):
        for idx in np.ndindex(arr.shape):
            p, m = arr.copy(), arr.copy()
            p[idx] += eps
            m[idx] -= eps
            lp = loss(p, b0) if which == 0 else loss(a0, p)
            lm = loss(m, b0) if which == 0 else loss(a0, m)
            num = (lp - lm) / (2 * eps)
            assert abs(num - g[idx]) <= 0.03 + 0.05 * abs(num)


def test_worker_slots_from_threads(trlm, orc, ops):
    host, hip, alloc = ops
    rng = np.random.default_rng(4)
    mats = [(rng.standard_normal((100, 64)).astype(np.float32), rng.standard_normal((64, 80)).astype(np.float32))
            for _ in range(3)]
    nodes = [(leaf(trlm, host, alloc, a), leaf(trlm, host, alloc, b)) for a, b in mats]
    results = [None] * 3
    hip.gpu_ops_debug_reset()
    lock = threading.Lock()

    def work(i):
        hip.gpu_ops_set_worker_id(i)
        a, b = nodes[i]
        with lock:   # the shared Allocator is not thread-safe; the GPU slots are
            out = hip.node_matmul2d_gpu(C.byref(alloc), a, b)
        results[i] = value(trlm, out)

    th = [threading.Thread(target=work, args=(i,)) for i in range(3)]
    for t in th:
        t.start()
    for t in th:
        t.join()
    for (a, b), r in zip(mats, results):
        want = orc.matmul(a, b)
        assert np.abs(r - want).max() <= 1e-4 * np.abs(want).max()
    secs, calls = C.c_double(), C.c_uint32()
    hip.gpu_ops_debug_stats(C.byref(secs), C.byref(calls))
    assert calls.value == 3 and secs.value > 0.0


def _data_ptr(node):
    return C.cast(node.contents.value.data, C.c_void_p).value


def test_pinned_operands(trlm, orc, ops):
    host, hip, alloc = ops
    rng = np.random.default_rng(9)
    V, D, T = 2003, 384, 5
    x = rng.standard_normal((T, D)).astype(np.float32)
    E = (0.02 * rng.standard_normal((V, D))).astype(np.float32)
    W = rng.standard_normal((D, 640)).astype(np.float32)
    nx, nE, nW = leaf(trlm, host, alloc, x), leaf(trlm, host, alloc, E), leaf(trlm, host, alloc, W)
    Et = host.tensor_transpose(C.byref(nE.contents.value), 0, 1)
    nEt = host.node_leaf(C.byref(alloc), Et, 1)
    head0 = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nEt))
    proj0 = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nW))
    try:
        hip.gpu_ops_pin(_data_ptr(nE), V * D)
        hip.gpu_ops_pin(_data_ptr(nW), D * 640)
        head1 = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nEt))
        proj1 = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nW))
        assert np.array_equal(head0.view(np.uint32), head1.view(np.uint32))
        assert np.array_equal(proj0.view(np.uint32), proj1.view(np.uint32))
        # the device copy is what is read: host changes are not seen while pinned
        trlm.tensor_np(nW.contents.value)[:] *= 2.0
        proj2 = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nW))
        assert np.array_equal(proj0.view(np.uint32), proj2.view(np.uint32))
        # a view past the pinned range (here: rows 0..D of a longer buffer
        # whose pin covers only half of it) is uploaded as before
        hip.gpu_ops_unpin_all()
        hip.gpu_ops_pin(_data_ptr(nW), (D // 2) * 640)
        proj3 = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nW))
        want3 = orc.matmul(x, 2.0 * W)
        assert np.abs(proj3 - want3).max() <= 1e-4 * np.abs(want3).max()
        # worker slots read the pinned copy too
        hip.gpu_ops_unpin_all()
        hip.gpu_ops_pin(_data_ptr(nE), V * D)
        outs = [None] * 3
        lock = threading.Lock()

        def work(i):
            hip.gpu_ops_set_worker_id(i)
            with lock:
                outs[i] = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nEt))

        th = [threading.Thread(target=work, args=(i,)) for i in range(3)]
        for t in th:
            t.start()
        for t in th:
            t.join()
        for o in outs:
            assert np.array_equal(o.view(np.uint32), head0.view(np.uint32))
    finally:
        hip.gpu_ops_unpin_all()
        hip.gpu_ops_set_worker_id(-1)
    # unpinned again: the doubled host values are read
    proj4 = value(trlm, hip.node_matmul2d_gpu(C.byref(alloc), nx, nW))
    want4 = orc.matmul(x, 2.0 * W)
    assert np.abs(proj4 - want4).max() <= 1e-4 * np.abs(want4).max()
