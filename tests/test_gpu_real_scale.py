"""Parity at the benchmark's real sizes.

1. The real model (V31769 D384 H6 L12 F1024) at T=1024, B=2, against the
   reference's own CPU path (oracle/_ref, frozen by
   tests/golden/make_golden.py t1024): loss within 1e-4 relative; logits rows
   (first, second and last positions of both sequences) within 1e-4 of
   max|logits|; every gradient tensor on 256 seeded entries within
   compare_tensor's bar (1e-4*max|want| + 1e-4*|want|,
   test_gpu_train.c:53-66), and its max|g|, sum g and sum |g| within what
   that per-element bar allows.  Per-tensor max-abs errors are reported.
2. Config 5 at its real shape: batch 64, 128-token prompts from
   pcg_seed(4242,9), greedy generation to a context of 1024 (896 picks).
   generate_greedy equals the step-by-step loop (prefill, greedy, step) bit
   for bit; at contexts 128..1023 (both sides of every 256-key chunk
   boundary) the step path's logits equal a fresh prefill of the whole
   context -- the trainer's full forward (trlm_forward_hidden) at the last
   position -- within 1e-4 of max|logits|, and each pick is or_argmax of the
   step path's logits.
"""
import hashlib
import os

import numpy as np
import pytest

from conftest import parity_report

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = 1e-4


@pytest.fixture(scope="module")
def real(trlm, orc):
    model = orc.Model(31769, 384, 6, 12, 1024)
    params = model.init(1337, 1)
    hm = trlm.HostModel(31769, 384, 6, 12, 1024, params)
    yield model, params, hm
    hm.close()


def test_real_model_t1024_against_reference(trlm, real):
    model, params, hm = real
    fx = dict(np.load(os.path.join(GOLDEN, "ref_real_t1024.npz")))
    assert hashlib.sha256(params.view(np.uint8)).hexdigest() == str(fx["params_sha256"])
    B, T, V = 2, 1024, model.V
    tr = trlm.Trainer(hm, B, T)
    try:
        loss = tr.forward_backward(fx["ids"], fx["tgt"])
        got = tr.grads()
        logits = tr.forward_logits(fx["ids"]).reshape(B, T, V)
    finally:
        tr.destroy()
    want_loss = float(fx["loss"])
    rows = [("loss", abs(loss - want_loss), abs(want_loss))]
    assert abs(loss - want_loss) <= TOL * abs(want_loss), (loss, want_loss)
    lg = np.stack([logits[b, t] for b, t in fx["logit_rows"]])
    lerr = float(np.abs(lg.astype(np.float64) - fx["logits"]).max())
    lmax = float(np.abs(fx["logits"]).max())
    rows.append(("logits", lerr, lmax))
    assert lerr <= TOL * lmax, (lerr, lmax)
    failures = []
    for i, (name, g) in enumerate(zip(model.names(), model.split(got))):
        g = g.ravel().astype(np.float64)
        idx, want = fx["grad_idx"][i], fx["grad_val"][i].astype(np.float64)
        wmax = float(fx["grad_max"][i])
        diff = np.abs(g[idx] - want)
        rows.append((name, float(diff.max()), wmax))
        if (diff > TOL * wmax + TOL * np.abs(want) + 1e-12).any():
            failures.append((name, "samples", float(diff.max() / wmax)))
        # what the per-element bar allows for the whole tensor
        slack = TOL * (g.size * wmax + float(fx["grad_abs"][i])) + 1e-9
        if abs(np.abs(g).max() - wmax) > TOL * wmax + 1e-12:
            failures.append((name, "max", float(np.abs(g).max()), wmax))
        if abs(g.sum() - float(fx["grad_sum"][i])) > slack:
            failures.append((name, "sum", float(g.sum()), float(fx["grad_sum"][i])))
        if abs(np.abs(g).sum() - float(fx["grad_abs"][i])) > slack:
            failures.append((name, "abs sum", float(np.abs(g).sum()), float(fx["grad_abs"][i])))
    parity_report("real_t1024_b2", rows)
    assert not failures, failures


def test_config5_real_shape_decode(trlm, orc, real):
    model, params, hm = real
    B, P, CTX = 64, 128, 1024
    S = CTX - P
    prompt = orc.random_tokens(B * P, model.V, 4242, 9, hi_exclusive=model.V).reshape(B, P)
    checks = [0, 1, 127, 128, 129, 383, 384, 639, 640, 895]   # pick s is made at context P + s
    L = orc.lib()
    tr = trlm.Trainer(hm, 1, 8)
    dec = trlm.Decoder(tr, B, CTX)
    full = trlm.Decoder(tr, B, CTX)
    rows = []
    try:
        gen = dec.generate_greedy(prompt, S)
        assert (gen < model.V).all()
        dec.prefill(prompt)
        step_logits = {}
        for s in range(S):
            if s in checks:
                step_logits[s] = dec.logits()
            pick = dec.greedy()
            assert np.array_equal(pick, gen[:, s]), s
            if s + 1 < S:
                dec.step(pick)
        for s in checks:
            ctx = np.concatenate([prompt, gen[:, :s]], axis=1)
            full.prefill(ctx)
            want = full.logits()
            got = step_logits[s]
            err = float(np.abs(got.astype(np.float64) - want).max())
            scale = float(np.abs(want).max())
            rows.append(("ctx %d" % (P + s), err, scale))
            assert err <= TOL * scale, (s, err, scale)
            picks = np.array([L.or_argmax(np.ascontiguousarray(r), model.V) for r in got], np.uint32)
            assert np.array_equal(picks, gen[:, s]), s
    finally:
        full.destroy()
        dec.destroy()
        tr.destroy()
    parity_report("decode_config5", rows, header="context  max|step-full|  max|full|  ratio")
