"""Forward-only entry points: logits, mean cross-entropy without destroying
the logits, and greedy argmax (BASELINE configs 1 and 3; additive API).

Config 1 is the reference's own CPU-runnable case: the real architecture,
lm_init(pcg_seed(1337,1)), B=1, T=128, ids pcg_range_i64(0, 31769) from
pcg_seed(4242,7).  Logits within 1e-4 of max|logits|; the GPU argmax kernel
must equal the host argmax of the same logits bit for bit (first index of
the maximum), and the oracle's next token whenever its top-2 margin exceeds
the logit tolerance.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def real_model(trlm, orc):
    model = orc.Model(31769, 384, 6, 12, 1024)
    params = model.init(1337, 1)
    hm = trlm.HostModel(31769, 384, 6, 12, 1024, params)
    yield model, params, hm
    hm.close()


def host_argmax(logits):
    return np.argmax(logits, axis=1).astype(np.uint32)   # first index of the max


def test_config1_logits_and_greedy(trlm, orc, real_model):
    model, params, hm = real_model
    ids = orc.random_tokens(128, 31769, 4242, 7, hi_exclusive=31769)
    want = model.forward_logits(params, ids, 1, 128)
    tr = trlm.Trainer(hm, 1, 128)
    try:
        got = tr.forward_logits(ids)
        am = tr.greedy_argmax()
    finally:
        tr.destroy()
    scale = np.abs(want).max()
    err = np.abs(got.astype(np.float64) - want).max() / scale
    assert err <= 1e-4, err
    assert np.array_equal(am, host_argmax(got))
    ref_next = host_argmax(want)
    top2 = np.sort(want, axis=1)[:, -2:]
    clear = (top2[:, 1] - top2[:, 0]) > 4e-4 * scale
    assert np.array_equal(am[clear], ref_next[clear])
    print("config1: logits rel err %.3e, next token %d (oracle %d)" % (err, am[-1], ref_next[-1]))


@pytest.mark.parametrize("V", [700, 2000, 5003])
def test_training_loss_equals_forward_loss(trlm, orc, V):
    """The loss forward_backward returns equals the forward-only loss bit for
    bit, five times in a row, at vocabularies where every wave of the
    cross-entropy's row writes gradient values in its first pass (V > 1024
    columns, and V % 4 != 0 for the per-element path): the row's target
    logit must be read before any of them overwrites it."""
    D, H, L, F, T, B = 32, 2, 1, 32, 64, 8
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    toks = orc.random_tokens(4000, V)
    ids, tgt = orc.sample_batch(toks, T, B, 31)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    try:
        want = np.float32(tr.forward_loss_logits(ids, tgt, want_logits=False)[0])
        got = [np.float32(tr.forward_backward(ids, tgt)) for _ in range(5)]
    finally:
        tr.destroy()
        hm.close()
    cpu_loss, _, _ = model.forward_backward(params, ids, tgt, B, T, want_grads=False)
    assert abs(float(want) - cpu_loss) <= 1e-4 * abs(cpu_loss)
    assert all(g.view(np.uint32) == want.view(np.uint32) for g in got), (want, got)


@pytest.mark.parametrize("V,D,H,L,F,T,B", [(50, 32, 2, 2, 48, 12, 5), (500, 64, 2, 2, 128, 256, 3),
                                           # config 3's B8 T1024 rows at the real width, every logit compared
                                           (2000, 384, 6, 2, 1024, 1024, 8)])
def test_forward_loss_keeps_logits(trlm, orc, V, D, H, L, F, T, B):
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    toks = orc.random_tokens(8000, V)
    ids, tgt = orc.sample_batch(toks, T, B, 77)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    try:
        loss, logits = tr.forward_loss_logits(ids, tgt)
        ev = tr.eval_loss(ids, tgt)
        logits2 = tr.forward_logits(ids)
        am = tr.greedy_argmax()
    finally:
        tr.destroy()
        hm.close()
    want = model.forward_logits(params, ids, B, T)
    cpu_loss, _, _ = model.forward_backward(params, ids, tgt, B, T, want_grads=False)
    assert np.float32(loss).view(np.uint32) == np.float32(ev).view(np.uint32)
    assert abs(loss - cpu_loss) <= 1e-4 * abs(cpu_loss)
    assert np.array_equal(logits.view(np.uint32), logits2.view(np.uint32))
    assert np.abs(logits - want).max() <= 1e-4 * np.abs(want).max()
    assert np.array_equal(am, host_argmax(logits2))


def test_attention_placement_table_keeps_bits(trlm, orc, monkeypatch):
    """At B8 T1024 with 6 heads (48 x 16 forward attention jobs) the trainer
    gives the attention forward its balanced placement table; the logits
    equal, bit for bit, those of a trainer that keeps the kernel's own order
    (TRLM_ATTN_SNAKE=1, read at creation)."""
    V, D, H, L, F, T, B = 300, 384, 6, 1, 128, 1024, 8
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    ids = orc.random_tokens(B * T, V, 4242, 13, hi_exclusive=V)
    got = []
    for snake in ("0", "1"):
        monkeypatch.setenv("TRLM_ATTN_SNAKE", snake)
        hm = trlm.HostModel(V, D, H, L, F, params)
        tr = trlm.Trainer(hm, B, T)
        try:
            got.append(tr.forward_logits(ids))
        finally:
            tr.destroy()
            hm.close()
    assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))


GEMM_TILES = [None, "256x128", "128x256", "128x128", "128x128_k32", "64x128", "64x128_k32", "64x64", "64x64_k32"]


@pytest.mark.parametrize("V,D,H,T,B", [(50, 32, 2, 12, 5), (1001, 32, 2, 64, 3), (31769, 64, 4, 128, 2)])
def test_eval_loss_without_logits(trlm, orc, V, D, H, T, B):
    """eval_loss never writes the logits: the LM-head GEMM leaves the row
    statistics and each row's target logit.  Its loss must equal, bit for
    bit, the loss forward_loss_logits computes from stored logits, for
    targets on tile and wave-column edges, the first and the last column --
    with the plan's own tile and with each tile variant forced on the
    trainer's GEMM engine, so that every variant's statistics and
    target-logit epilogue (and its no-store path) is checked."""
    L, F = 2, 2 * D
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    toks = orc.random_tokens(20000, V)
    ids, tgt = orc.sample_batch(toks, T, B, 91)
    edges = [c for c in (0, 1, 31, 32, 63, 64, 65, 127, 128, 255, 256, V - 2, V - 1) if 0 <= c < V]
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    try:
        for tile in GEMM_TILES:
            tr.force_gemm(tile)
            for k, targets in enumerate([tgt, np.zeros_like(tgt), np.full_like(tgt, V - 1),
                                         np.resize(np.array(edges, np.uint32), tgt.size)]):
                loss, _ = tr.forward_loss_logits(ids, targets, want_logits=False)
                ev = tr.eval_loss(ids, targets)
                head = tr.gemm_last_variant()[0]   # the LM head is the forward's last GEMM
                assert head.startswith("k_gemm_nt_"), head
                if tile is not None:
                    assert head == "k_gemm_nt_" + tile, (tile, head)
                assert np.float32(loss).view(np.uint32) == np.float32(ev).view(np.uint32), (tile, k, loss, ev)
        tr.force_gemm(None)
        cpu_loss, _, _ = model.forward_backward(params, ids, tgt, B, T, want_grads=False)
        ev = tr.eval_loss(ids, tgt)
        assert abs(ev - cpu_loss) <= 1e-4 * abs(cpu_loss)
    finally:
        tr.destroy()
        hm.close()


def test_argmax_ties_pick_lowest_index(trlm):
    """Rows with repeated maxima: the kernel must return the first index."""
    _, hip = trlm.libs()
    import ctypes as C
    dev = trlm.Device()
    try:
        rows, V = 7, 1000
        z = np.zeros((rows, V), np.float32)
        spots = [(0, [5, 900]), (1, [0, 999]), (2, [255, 256, 511]), (3, [998, 999]), (4, [10]), (5, [700, 3]),
                 (6, list(range(0, 1000, 37)))]
        for r, cols in spots:
            z[r, cols] = 3.0
        dz, dout = dev.upload(z), dev.empty(rows * 4)
        f = hip.hip_get_kernel(C.byref(dev.ctx), b"k_argmax_rows")
        pz, po = C.c_void_p(dz), C.c_void_p(dout)
        ld, vv = C.c_int32(V), C.c_int32(V)
        args = (C.c_void_p * 4)(C.addressof(pz), C.addressof(ld), C.addressof(vv), C.addressof(po))
        hip.hip_launch(f, rows, 1, 1, 256, 1, 1, 0, args)
        out = dev.download(dout, rows, np.uint32)
        assert list(out) == [min(c) for _, c in spots]
    finally:
        dev.close()
