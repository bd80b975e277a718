"""The queued training driver loop (gpu_trainer_train_steps,
gpu_trainer_eval_windows) against the reference driver's call sequence.

The reference's loop body (training/train_lm_gpu.c:212-223) is: lr from
lr_warmup_cosine, gpu_trainer_sample_batch with seed 2026 + step,
forward_backward, grad_norm, clip scale = (f32)(clip / norm) when norm > clip
else 1, adam_step_scaled.  Run step by step through those public entry
points (each itself pinned to the oracle in test_gpu_train.py) with the
reference's own schedule (oracle restatement, pinned to oracle/_ref), that
sequence is the checker: the queued loop must give the same losses, norms
and learning rates and leave the same parameters, Adam moments and t, bit
for bit -- across two calls (resume at first_step > 0) and with AdamW.  The
validation windows (train_lm_gpu.c:241-258) are checked the same way, and
the device restatement of m_sqrt (the norm's square root) against the host
runtime's m_sqrt on 4096 values.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V, D, H, L, F, B, T = 61, 32, 2, 2, 48, 3, 16


def make(trlm, orc, seed=1337):
    model = orc.Model(V, D, H, L, F)
    params = model.init(seed, 1)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    adam = trlm.Adam(hm, 3e-4, 0.9, 0.95, 1e-8)
    tr.upload(adam)
    return hm, tr, adam


def schedule(trlm, wd, clip):
    s = trlm.TrlmSchedule()
    s.warmup_steps, s.total_steps, s.peak_lr, s.min_lr = 2, 8, 3e-3, 3e-4
    s.grad_clip, s.weight_decay, s.seed_base = clip, wd, 2026
    return s


def manual_steps(trlm, orc, tr, adam, tokens, s, first, n):
    _, hip = trlm.libs()
    ids = np.zeros(B * T, np.uint32)
    tgt = np.zeros(B * T, np.uint32)
    out = []
    for step in range(first, first + n):
        lr = orc.lr_warmup_cosine(step, s.warmup_steps, s.total_steps, s.peak_lr, s.min_lr)
        adam.opt.lr = float(lr)
        hip.gpu_trainer_sample_batch(tokens, len(tokens), T, B, s.seed_base + step, ids, tgt)
        loss = np.float32(tr.forward_backward(ids, tgt))
        norm = tr.grad_norm()
        scale = np.float32(s.grad_clip / norm) if (s.grad_clip > 0 and norm > s.grad_clip) else np.float32(1.0)
        if s.weight_decay == 0:
            tr.adam_step(adam, float(scale))
        else:
            tr.adamw_step(adam, s.weight_decay, float(scale))
        out.append((loss, norm, lr))
    return out


def state(tr, adam, hm):
    p = tr.download(adam)
    return p.copy(), adam.flat("m"), adam.flat("v"), adam.opt.t


@pytest.mark.parametrize("wd,clip", [(0.0, 0.25), (0.1, 0.25), (0.0, 0.0)])
def test_train_steps_equal_driver_sequence(trlm, orc, wd, clip):
    tokens = orc.random_tokens(5000, V)
    s = schedule(trlm, wd, clip)
    hm1, tr1, ad1 = make(trlm, orc)
    hm2, tr2, ad2 = make(trlm, orc)
    try:
        l1, n1, r1 = tr1.train_steps(ad1, tokens, s, 0, 3)
        l2, n2, r2 = tr1.train_steps(ad1, tokens, s, 3, 4)
        got = list(zip(np.concatenate([l1, l2]), np.concatenate([n1, n2]), np.concatenate([r1, r2])))
        want = manual_steps(trlm, orc, tr2, ad2, tokens, s, 0, 7)
        clipped = 0
        for i, ((gl, gn, gr), (wl, wn, wr)) in enumerate(zip(got, want)):
            assert np.float32(gl).view(np.uint32) == np.float32(wl).view(np.uint32), (i, gl, wl)
            assert float(gn).hex() == float(wn).hex(), (i, gn, wn)
            assert np.float32(gr).view(np.uint32) == np.float32(wr).view(np.uint32), (i, gr, wr)
            clipped += clip > 0 and wn > clip
        if clip > 0:
            assert clipped > 0, "the schedule never clipped: the test would not cover the clip scale"
        a, b = state(tr1, ad1, hm1), state(tr2, ad2, hm2)
        for x, y in zip(a[:3], b[:3]):
            assert np.array_equal(x.view(np.uint32), y.view(np.uint32))
        assert a[3] == b[3] == 7
        assert np.float32(ad1.opt.lr) == np.float32(ad2.opt.lr)
        print("train_steps wd=%g clip=%g: losses %s" % (wd, clip, np.round([g[0] for g in got], 4)))
    finally:
        for tr, hm in ((tr1, hm1), (tr2, hm2)):
            tr.destroy()
            hm.close()


def test_eval_windows_equal_driver_sequence(trlm, orc):
    tokens = orc.random_tokens(6000, V)
    train_tokens, val_tokens, val_batches = 4000, 2000, 5
    hm, tr, adam = make(trlm, orc)
    try:
        got = tr.eval_windows(tokens, train_tokens, val_tokens, val_batches)
        stride = (val_tokens - T - 1) // (val_batches * B)
        val_sum = np.float32(0.0)
        for vb in range(val_batches):
            ids = np.zeros(B * T, np.uint32)
            tgt = np.zeros(B * T, np.uint32)
            for w in range(B):
                start = train_tokens + (vb * B + w) * stride
                ids[w * T:(w + 1) * T] = tokens[start:start + T]
                tgt[w * T:(w + 1) * T] = tokens[start + 1:start + T + 1]
            val_sum = np.float32(val_sum + np.float32(tr.eval_loss(ids, tgt)))
        want = np.float32(val_sum / np.float32(val_batches))
        assert np.float32(got).view(np.uint32) == want.view(np.uint32), (got, want)
    finally:
        tr.destroy()
        hm.close()


def test_device_sqrt_equals_m_sqrt(trlm):
    host, hip = trlm.libs()
    dev = trlm.Device()
    try:
        rng = np.random.default_rng(5)
        x = np.ldexp(rng.uniform(1.0, 2.0, 4000), rng.integers(-1000, 1000, 4000)).astype(np.float64)
        special = [0.0, -0.0, 1.0, 2.0, 4.0, 0.25, 1e-300, 1e300, 2.0 ** -1022, 5e-324, float("inf"), 9.0, 1e-8]
        x = np.concatenate([x, np.array(special, np.float64)])
        n = x.size
        px, py = dev.upload(x), dev.empty(n * 8)
        f = hip.hip_get_kernel(C.byref(dev.ctx), b"k_ref_sqrt64")
        a_x, a_y, a_n = C.c_void_p(px), C.c_void_p(py), C.c_int(n)
        args = (C.c_void_p * 3)(C.cast(C.pointer(a_x), C.c_void_p), C.cast(C.pointer(a_y), C.c_void_p),
                                C.cast(C.pointer(a_n), C.c_void_p))
        hip.hip_launch(f, (n + 255) // 256, 1, 1, 256, 1, 1, 0, args)
        got = dev.download(py, (n,), np.float64)
        want = np.array([host.m_sqrt(float(v)) for v in x], np.float64)
        assert np.array_equal(got.view(np.uint64), want.view(np.uint64))
        dev.free(px)
        dev.free(py)
    finally:
        dev.close()
