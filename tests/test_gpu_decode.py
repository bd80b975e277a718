"""KV-cache decode (additive API) through the C ABI.

The reference generates by recomputing the full window each step and reading
the last row (training/generate.c:186-212).  Within the context (no window
slide) that last row is what the decoder must produce, so:
  - after the prefill and after every step, the decoder's logits equal the
    oracle's full forward over the whole context at its last position, within
    1e-4 of max|logits| (head_dim 16, 32, 64; contexts crossing the
    256-key chunks of the decode attention; batches 2 to 65; d_model up to
    512; d_ff not a multiple of 16);
  - greedy picks are the first maximum of those logits; generate_greedy
    equals prefill + greedy + step by hand, bit for bit;
  - sampling follows sample_next (generate.c:57-73) bit for bit: the oracle's
    restatement, run on the decoder's own logits with the same PCG streams,
    picks the same tokens and leaves the streams in the same state, both on
    the kernel's parallel exact-prefix path and on its sequential path, at
    the real vocabulary and temperatures 0.05 to 2 (and 0); sampled
    generation on the device equals the per-token loop;
  - at the real architecture (V 31769, D 384, L 12) the decoder equals the
    GPU trainer's full forward (itself pinned to the oracle) at the last
    position, within 1e-4; and at config 5's own shape (batch 64, 128-token
    prompts, 8 teacher-forced steps) it equals the oracle's forward on four
    of the sequences at every position, within 1e-4.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def rel_err(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())


def last_rows(orc, model, params, ctx, B):
    """Oracle logits of the last position of each sequence, ctx [B, T]."""
    T = ctx.shape[1]
    full = model.forward_logits(params, np.ascontiguousarray(ctx, np.uint32).ravel(), B, T)
    return full.reshape(B, T, -1)[:, -1, :]


@pytest.mark.parametrize("V,D,H,L,F,B,P,S", [
    (61, 32, 2, 2, 48, 3, 5, 6),       # head_dim 16
    (97, 64, 2, 2, 96, 2, 9, 5),       # head_dim 32
    (83, 128, 2, 2, 160, 2, 7, 4),     # head_dim 64
    (71, 128, 2, 1, 64, 2, 250, 12),   # keys cross the 256-key chunk boundary
    (53, 32, 2, 1, 32, 65, 3, 2),      # batch 65
    (59, 96, 6, 2, 64, 3, 6, 4),       # six heads, odd batch: a workgroup with one sequence
    (61, 192, 12, 2, 96, 3, 5, 4),     # twelve heads of 16
    (67, 512, 8, 1, 100, 3, 5, 4),     # d_model 512 (64 projection rows per wave, k_dec_head_k32), d_ff 100
    (61, 448, 7, 2, 36, 2, 6, 4),      # d_model 448, seven heads; d_ff 36: partial 16-column blocks
])
def test_decode_equals_full_recompute(trlm, orc, V, D, H, L, F, B, P, S):
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    prompt = orc.random_tokens(B * P, V, 4242, 9).reshape(B, P)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    dec = trlm.Decoder(tr, B, P + S + 1)
    try:
        dec.prefill(prompt)
        ctx = prompt.copy()
        worst = 0.0
        for s in range(S + 1):
            got = dec.logits()
            want = last_rows(orc, model, params, ctx, B)
            err = rel_err(got, want)
            worst = max(worst, err)
            assert err <= 1e-4, (s, err)
            nxt = dec.greedy()
            assert np.array_equal(nxt, np.argmax(got, axis=1).astype(np.uint32))
            assert dec.length() == ctx.shape[1]
            if s < S:
                dec.step(nxt)
                ctx = np.concatenate([ctx, nxt[:, None]], axis=1)
        print("decode V%d D%d P%d S%d: worst rel err %.2e" % (V, D, P, S, worst))
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()


def test_generate_greedy_matches_manual_loop(trlm, orc):
    V, D, H, L, F, B, P, S = 67, 64, 2, 2, 96, 3, 6, 7
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    prompt = orc.random_tokens(B * P, V, 4242, 9).reshape(B, P)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    d1 = trlm.Decoder(tr, B, P + S)
    d2 = trlm.Decoder(tr, B, P + S)
    try:
        gen = d1.generate_greedy(prompt, S)
        d2.prefill(prompt)
        manual = []
        for s in range(S):
            nxt = d2.greedy()
            manual.append(nxt)
            if s + 1 < S:
                d2.step(nxt)
        assert np.array_equal(gen, np.stack(manual, axis=1))
    finally:
        d1.destroy()
        d2.destroy()
        tr.destroy()
        hm.close()


def test_sampling_follows_sample_next(trlm, orc):
    V, D, H, L, F, B, P = 113, 64, 2, 2, 96, 4, 5
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    prompt = orc.random_tokens(B * P, V, 4242, 9).reshape(B, P)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    dec = trlm.Decoder(tr, B, P + 10)
    rngs = (trlm.PCGState * B)(*[trlm.libs()[0].pcg_seed(4242, 7 + b) for b in range(B)])
    mirror = [orc.pcg_stream(4242, 7 + b) for b in range(B)]
    try:
        dec.prefill(prompt)
        for step in range(8):
            logits = dec.logits()
            for temp in (0.85,):
                got = dec.sample(rngs, temp)
                want = [orc.sample_next(logits[b], temp, mirror[b]) for b in range(B)]
                assert list(got) == want, (step, list(got), want)
                for b in range(B):
                    assert rngs[b].state == mirror[b].state and rngs[b].inc == mirror[b].inc
            dec.step(got)
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()


def test_generate_sampled_matches_manual_loop(trlm, orc):
    """gpu_decoder_generate_sampled draws every uniform up front and samples
    on the device: the same picks as prefill + (sample, step) per token, bit
    for bit, and the PCG streams end in the same state."""
    V, D, H, L, F, B, P, S = 97, 64, 2, 2, 96, 3, 6, 9
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    prompt = orc.random_tokens(B * P, V, 4242, 9).reshape(B, P)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    d1 = trlm.Decoder(tr, B, P + S)
    d2 = trlm.Decoder(tr, B, P + S)
    seed = lambda: (trlm.PCGState * B)(*[trlm.libs()[0].pcg_seed(4242, 7 + b) for b in range(B)])
    r1, r2 = seed(), seed()
    try:
        gen = d1.generate_sampled(prompt, S, r1, 0.85)
        d2.prefill(prompt)
        manual = []
        for s in range(S):
            nxt = d2.sample(r2, 0.85)
            manual.append(nxt)
            if s + 1 < S:
                d2.step(nxt)
        assert np.array_equal(gen, np.stack(manual, axis=1)), (gen, np.stack(manual, axis=1))
        for b in range(B):
            assert r1[b].state == r2[b].state and r1[b].inc == r2[b].inc
    finally:
        d1.destroy()
        d2.destroy()
        tr.destroy()
        hm.close()


@pytest.mark.parametrize("temp", [0.85, 0.05, 2.0, 0.0])
def test_sampling_parallel_decision_equals_sequential_sums(trlm, orc, temp, monkeypatch):
    """At the real vocabulary (V 31,769), batch 64: the kernel's parallel
    exact-prefix decision picks what the reference's sequential f64 sums pick
    -- the same kernel forced onto its sequential path
    (TRLM_SAMPLE_SEQUENTIAL=1) and the oracle's sample_next on the same
    logits and PCG streams -- for three decode positions; temperature 0.05
    spreads the probabilities over hundreds of binades (most terms far below
    the running sum's rounding), 0 makes every sum NaN (the reference then
    returns the last index)."""
    V, D, H, L, F, B, P = 31769, 64, 2, 1, 64, 64, 4
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    params[:V * D] *= np.float32(20.0)    # the tied head's rows: logits of a few units, not ~0.2
    prompt = orc.random_tokens(B * P, V, 4242, 9).reshape(B, P)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    dec = trlm.Decoder(tr, B, P + 4)
    seeds = lambda: (trlm.PCGState * B)(*[trlm.libs()[0].pcg_seed(99, b) for b in range(B)])
    ra, rb = seeds(), seeds()
    mirror = [orc.pcg_stream(99, b) for b in range(B)]
    try:
        dec.prefill(prompt)
        for step in range(3):
            logits = dec.logits()
            fast = dec.sample(ra, temp)
            monkeypatch.setenv("TRLM_SAMPLE_SEQUENTIAL", "1")
            seq = dec.sample(rb, temp)
            monkeypatch.delenv("TRLM_SAMPLE_SEQUENTIAL")
            want = [orc.sample_next(logits[b], temp, mirror[b]) for b in range(B)]
            assert list(seq) == want, (step, list(seq), want)
            assert list(fast) == want, (step, list(fast), want)
            dec.step(fast)
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()


@pytest.mark.parametrize("temp", [1.0, 0.37])
def test_sample_exponentials_equal_m_expf(trlm, orc, temp):
    """k_sample_exp's e_j = m_expf((z_j - max) / temperature) bit for bit
    against the oracle's m_expf (the reference's f64 Taylor series), over
    64 rows x 31,769 inputs spanning [-120, 0]: both sides of the -110
    cut-off and of float underflow (exp(x) ~ 2^-150), exact 0, and inputs
    whose exp lies within 1e-13 of a midpoint between two floats (where the
    kernel evaluates the series itself instead of its fast polynomial)."""
    import ctypes as C
    rows, V = 64, 31769
    ld = (V + 3) // 4 * 4
    rng = np.random.default_rng(3)
    z = rng.uniform(-120.0 * temp, 0.0, size=(rows, V)).astype(np.float32)
    z[:, 0] = 0.0                                          # the row max
    specials = np.array([-0.0, -1e-30, -110.0, -109.99999, -110.00001, -103.2789, -103.9721, -104.5, -87.33655,
                         -0.6931472, -0.34657359, -745.2, -1e-7], np.float32)
    z[0, 1:1 + specials.size] = specials * np.float32(temp)
    # inputs whose exp is within 1e-13 (relative) of a float rounding midpoint
    cand = rng.uniform(-103.0, 0.0, size=4_000_000)
    cand = cand.astype(np.float32).astype(np.float64)
    y = np.exp(cand)
    f = y.astype(np.float32).astype(np.float64)
    up = np.nextafter(y.astype(np.float32), np.float32(np.inf)).astype(np.float64)
    dn = np.nextafter(y.astype(np.float32), np.float32(0)).astype(np.float64)
    mid = np.where(y >= f, 0.5 * (f + up), 0.5 * (f + dn))
    near = cand[np.abs(y - mid) < 1e-13 * y].astype(np.float32)
    assert near.size >= 3, near.size
    z[1, 1:1 + near.size] = near * np.float32(temp)
    x = ((z - z.max(axis=1, keepdims=True)) / np.float32(temp)).astype(np.float32)
    m_expf = orc.lib().or_m_expf
    want = np.array([[m_expf(float(v)) for v in row] for row in x[:2]], np.float32)
    pad = np.zeros((rows, ld), np.float32)
    pad[:, :V] = z
    _, hip = trlm.libs()
    dev = trlm.Device()
    try:
        dz, de = dev.upload(pad), dev.empty(rows * ld * 4)
        f_ = hip.hip_get_kernel(C.byref(dev.ctx), b"k_sample_exp")
        pz, pe = C.c_void_p(dz), C.c_void_p(de)
        cl, cv, ct = C.c_int32(ld), C.c_int32(V), C.c_float(temp)
        args = (C.c_void_p * 5)(C.addressof(pz), C.addressof(cl), C.addressof(cv), C.addressof(ct), C.addressof(pe))
        hip.hip_launch(f_, rows, 8, 1, 1024, 1, 1, 0, args)
        got = dev.download(de, (rows, ld))[:, :V]
    finally:
        dev.close()
    assert np.array_equal(got[:2].view(np.uint32), want.view(np.uint32))
    # the other rows: the same function, checked on a seeded sample of columns
    idx = rng.integers(0, V, size=4000)
    for r in range(2, rows, 7):
        w = np.array([m_expf(float(v)) for v in x[r, idx]], np.float32)
        assert np.array_equal(got[r, idx].view(np.uint32), w.view(np.uint32)), r
    print("near-midpoint inputs: %d" % near.size)


def test_real_architecture_against_gpu_full_forward(trlm, orc):
    """V 31769, D 384, H 6, L 12, F 1024: batch 4, prompt 100, 3 steps; the
    decoder's logits at the last position equal the trainer's full forward
    (B=4, T=len) within 1e-4 of max|logits|."""
    V, D, H, L, F, B, P, S = 31769, 384, 6, 12, 1024, 4, 100, 3
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    prompt = orc.random_tokens(B * P, V, 4242, 9).reshape(B, P)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    dec = trlm.Decoder(tr, B, P + S + 1)
    try:
        dec.prefill(prompt)
        ctx = prompt.copy()
        for s in range(S + 1):
            got = dec.logits()
            full = trlm.Trainer(hm, B, ctx.shape[1])
            try:
                want = full.forward_logits(ctx.ravel()).reshape(B, ctx.shape[1], V)[:, -1, :]
            finally:
                full.destroy()
            err = rel_err(got, want)
            assert err <= 1e-4, (s, err)
            nxt = dec.greedy()
            if s < S:
                dec.step(nxt)
                ctx = np.concatenate([ctx, nxt[:, None]], axis=1)
        print("real-scale decode: last rel err %.2e" % err)
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()


def test_config5_shape_against_oracle(trlm, orc):
    """Config 5's shape (the real model, batch 64, 128-token prompts) against
    the oracle itself: 8 teacher-forced steps, so every step's context is
    known in advance and one oracle forward over the whole 136 tokens gives
    the reference logits of every position (attention is causal).  Four of
    the 64 sequences are compared -- the two sequence pairs that share the
    first and last attention workgroups -- after the prefill and after each
    step, within 1e-4 of max|logits|; each greedy pick is the first maximum
    of the decoder's own logits."""
    V, D, H, L, F, B, P, S = 31769, 384, 6, 12, 1024, 64, 128, 8
    sel = np.array([0, 1, 62, 63])
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    ctx = orc.random_tokens(B * (P + S), V, 4242, 9, hi_exclusive=V).reshape(B, P + S)
    want = model.forward_logits(params, np.ascontiguousarray(ctx[sel]).ravel(), len(sel), P + S)
    want = want.reshape(len(sel), P + S, V)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    dec = trlm.Decoder(tr, B, P + S + 1)
    try:
        dec.prefill(np.ascontiguousarray(ctx[:, :P]))
        worst = 0.0
        for s in range(S + 1):
            got = dec.logits()
            assert dec.length() == P + s
            err = rel_err(got[sel], want[:, P + s - 1, :])
            worst = max(worst, err)
            assert err <= 1e-4, (s, err)
            assert np.array_equal(dec.greedy(), np.argmax(got, axis=1).astype(np.uint32))
            if s < S:
                dec.step(np.ascontiguousarray(ctx[:, P + s]))
        print("config-5 shape against the oracle: worst rel err %.2e over %d positions" % (worst, S + 1))
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()


def test_replayed_steps_survive_training_and_new_prompts(trlm, orc):
    """Steps after the first replay a captured step.  Interleaving a training
    step of the same trainer (its GEMM workspace grows), and a second prefill
    with a new prompt, must leave later steps exact: every step is checked
    against the oracle's full recompute."""
    V, D, H, L, F, B, P = 89, 64, 2, 2, 96, 3, 6
    model = orc.Model(V, D, H, L, F)
    params = model.init(1337, 1)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 4, 64)
    dec = trlm.Decoder(tr, B, 32)
    toks = orc.random_tokens(4000, V)
    ids_t, tgt_t = orc.sample_batch(toks, 64, 4, 5)
    try:
        for trial in range(2):
            prompt = orc.random_tokens(B * P, V, 4242, 20 + trial).reshape(B, P)
            dec.prefill(prompt)
            ctx = prompt.copy()
            for s in range(5):
                want = last_rows(orc, model, params, ctx, B)
                assert rel_err(dec.logits(), want) <= 1e-4, (trial, s)
                nxt = dec.greedy()
                dec.step(nxt)
                ctx = np.concatenate([ctx, nxt[:, None]], axis=1)
                if s == 2:
                    tr.forward_backward(ids_t, tgt_t)   # no optimizer step: weights unchanged
            want = last_rows(orc, model, params, ctx, B)
            assert rel_err(dec.logits(), want) <= 1e-4, (trial, "last")
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()
