"""Token gathers bit for bit, and the greedy pick's rule on NaN / -inf rows.

north_star asks for bit-exact token gathers and greedy argmax:
  - the embedding gather (k_embed_fwd, train_kernels.cu:724-730), launched
    as trlm_embed_rows -- the host function the trainer's forward and every
    decode step call -- launches it, at the real vocabulary: x == E[ids] bit
    for bit, ids including 0, V-1 and repeats, for D % 4 == 0 (16-byte path)
    and D % 4 != 0;
  - the decode prefill's last-row gather (k_gather_rows, launched as
    gpu_decoder_prefill launches it) bit for bit;
  - greedy picks (k_argmax_rows behind gpu_trainer_greedy_argmax and
    gpu_decoder_greedy; k_argmax_hist behind gpu_decoder_generate_greedy)
    equal or_argmax, the reference's max-scan rule (generate.c:57-58), on rows
    with a NaN at index 0, NaNs elsewhere, all NaN and all -inf, directly and
    through models whose weights hold NaNs; every pick is below V.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _orc_argmax(orc, rows):
    L = orc.lib()
    return np.array([L.or_argmax(np.ascontiguousarray(r, np.float32), r.size) for r in rows], np.uint32)


@pytest.mark.parametrize("V,D,rows", [(31769, 384, 8192), (31769, 384, 333), (50, 18, 777)])
def test_embedding_gather_bit_exact(trlm, orc, V, D, rows):
    """k_embed_fwd launched as trlm_embed_rows launches it (16-byte path when
    D % 4 == 0: one float4 per thread, else one float; 256 threads per
    block) on the real model's lm_init embedding (V 31769, D 384) and an
    odd width."""
    model = orc.Model(V, D, 2 if D % 2 == 0 and (D // 2) % 2 == 0 else 1, 1, 24)
    E = model.init(1337, 1)[:V * D].reshape(V, D)
    rng = np.random.default_rng(11 + rows)
    ids = rng.integers(0, V, rows).astype(np.uint32)
    ids[:6] = [0, V - 1, 0, V - 1, 5 % V, 5 % V]
    dev = trlm.Device()
    try:
        dE, dids, dx = dev.upload(E), dev.upload(ids), dev.empty(rows * D * 4)
        f = dev.hip.hip_get_kernel(C.byref(dev.ctx), b"k_embed_fwd")
        vals = [C.c_void_p(dE), C.c_void_p(dids), C.c_void_p(dx), C.c_int32(rows), C.c_int32(D)]
        args = (C.c_void_p * len(vals))(*[C.addressof(v) for v in vals])
        work = rows * D // 4 if D % 4 == 0 else rows * D
        dev.hip.hip_launch(f, (work + 255) // 256, 1, 1, 256, 1, 1, 0, args)
        x = dev.download(dx, (rows, D))
    finally:
        dev.close()
    assert np.array_equal(x.view(np.uint32), E[ids].view(np.uint32))


def test_prefill_last_row_gather_bit_exact(trlm):
    """k_gather_rows as gpu_decoder_prefill launches it: row b of the output
    is row b*len + len-1 of the [batch*len, D] input."""
    dev = trlm.Device()
    try:
        B, ln, D = 64, 128, 384
        src = np.random.default_rng(2).standard_normal((B * ln, D)).astype(np.float32)
        src[3, 5] = np.float32("nan")      # bits of any value, NaN included, move unchanged
        dsrc, ddst = dev.upload(src), dev.empty(B * D * 4)
        f = dev.hip.hip_get_kernel(C.byref(dev.ctx), b"k_gather_rows")
        vals = [C.c_void_p(dsrc), C.c_int32(D), C.c_int32(ln), C.c_int32(ln - 1), C.c_int32(D), C.c_int32(B),
                C.c_void_p(ddst)]
        args = (C.c_void_p * len(vals))(*[C.addressof(v) for v in vals])
        dev.hip.hip_launch(f, (B * D + 255) // 256, 1, 1, 256, 1, 1, 0, args)
        got = dev.download(ddst, (B, D))
    finally:
        dev.close()
    want = src.reshape(B, ln, D)[:, -1, :]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _special_rows(V):
    nan, inf = np.float32("nan"), np.float32("inf")
    rng = np.random.default_rng(4)
    rows = rng.standard_normal((10, V)).astype(np.float32)
    rows[0, 0] = nan                              # NaN at index 0 -> 0
    rows[1, :] = nan                              # all NaN -> 0
    rows[2, :] = -inf                             # all -inf -> 0
    rows[3, 1::3] = nan                           # NaNs elsewhere are never picked
    rows[4, :] = -inf
    rows[4, V - 1] = -1e30                        # the only finite value, last index
    rows[5, :] = -inf
    rows[5, 1::2] = nan                           # -inf and NaN only -> 0
    rows[6, V // 2] = inf                         # +inf is a maximum like any other
    rows[7, [7, V - 2]] = 50.0                    # ties -> first
    rows[8, :] = 1.0
    rows[8, 0] = nan                              # NaN first, everything else equal
    rows[9, :] = 0.0                              # all equal -> 0
    return rows


@pytest.mark.parametrize("V,ld", [(31769, 31772), (1000, 1000), (37, 37)])
def test_argmax_kernels_nan_rule(trlm, orc, V, ld):
    rows = _special_rows(V)
    want = _orc_argmax(orc, rows)
    assert want[0] == 0 and want[1] == 0 and want[2] == 0 and want[4] == V - 1 and want[5] == 0
    assert want[6] == V // 2 and want[7] == 7 and want[8] == 0 and want[9] == 0
    assert not np.isnan(rows[3, want[3]])
    n = rows.shape[0]
    padded = np.full((n, ld), np.float32(7e30))   # padding columns are never read
    padded[:, :V] = rows
    dev = trlm.Device()
    try:
        dz = dev.upload(padded)
        dout, dids, dhist, dpos = dev.empty(n * 4), dev.empty(n * 4), dev.empty(n * 4 * 3), dev.upload(
            np.array([5], np.int32))
        f = dev.hip.hip_get_kernel(C.byref(dev.ctx), b"k_argmax_rows")
        vals = [C.c_void_p(dz), C.c_int32(ld), C.c_int32(V), C.c_void_p(dout)]
        args = (C.c_void_p * 4)(*[C.addressof(v) for v in vals])
        dev.hip.hip_launch(f, n, 1, 1, 256, 1, 1, 0, args)
        g = dev.hip.hip_get_kernel(C.byref(dev.ctx), b"k_argmax_hist")
        vals2 = [C.c_void_p(dz), C.c_int32(ld), C.c_int32(V), C.c_void_p(dids), C.c_void_p(dhist), C.c_int32(3),
                 C.c_void_p(dpos), C.c_int32(4)]
        args2 = (C.c_void_p * len(vals2))(*[C.addressof(v) for v in vals2])
        dev.hip.hip_launch(g, n, 1, 1, 1024, 1, 1, 0, args2)
        got = dev.download(dout, n, np.uint32)
        got_ids = dev.download(dids, n, np.uint32)
        hist = dev.download(dhist, (n, 3), np.uint32)
    finally:
        dev.close()
    assert np.array_equal(got, want), (got, want)
    assert np.array_equal(got_ids, want)
    assert np.array_equal(hist[:, 1], want)       # step = *pos - base = 1
    assert not hist[:, 0].any() and not hist[:, 2].any()


@pytest.mark.parametrize("where", ["embed_row0", "embed_row7", "final_norm"])
def test_greedy_on_nan_weights(trlm, orc, where):
    """A model whose weights hold NaNs (a diverged checkpoint): the trainer's
    and the decoder's greedy picks equal or_argmax of their own logits, and
    generate_greedy feeds only valid ids back (all picks < V)."""
    V, D, H, L, F, B, T = 61, 32, 2, 2, 48, 3, 9
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    if where == "embed_row0":
        params[0:D] = np.nan
    elif where == "embed_row7":
        params[7 * D:8 * D] = np.nan
    else:
        params[-D:] = np.nan
    prompt = orc.random_tokens(B * T, V, 4242, 9)
    prompt[prompt == 7] = 8
    prompt[prompt == 0] = 1
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    dec = trlm.Decoder(tr, B, T + 6)
    try:
        logits = tr.forward_logits(prompt)
        am = tr.greedy_argmax()
        assert np.array_equal(am, _orc_argmax(orc, logits)), where
        dec.prefill(prompt.reshape(B, T))
        for s in range(3):
            lg = dec.logits()
            pick = dec.greedy()
            assert np.array_equal(pick, _orc_argmax(orc, lg)), (where, s)
            assert (pick < V).all()
            dec.step(pick)
        out = dec.generate_greedy(prompt.reshape(B, T), 6)
        assert (out < V).all()
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()
    if where != "embed_row7":
        assert not am.any() and not out.any()     # every row has NaN at index 0 or is all NaN
