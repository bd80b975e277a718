"""TRLM v1 checkpoints straight from / to the GPU trainer (additive API;
the reference's training/checkpoint.c format and rules, pinned on the CPU
against the reference's own checkpoint_save / checkpoint_load by
tests/test_oracle.py::test_checkpoint_*):
  - a save after training steps is byte-identical to what checkpoint_save
    writes for the downloaded parameters and Adam state (oracle
    restatement of the format);
  - a load restores device parameters, Adam m / v and t bit for bit, and
    refreshes the host mirror;
  - resume: save after 2 steps, load into a fresh trainer, 2 more steps on
    both -> identical parameters and Adam state (test_resume.c's property);
  - invalid files (truncated, other shapes, optimizer state missing) are
    rejected and change nothing; a failed save leaves the old file intact.
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

V, D, H, L, F, B, T = 97, 64, 2, 2, 96, 3, 16


def setup(trlm, orc, seed=1337):
    model = orc.Model(V, D, H, L, F)
    params = model.init(seed, 1)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    adam = trlm.Adam(hm, 3e-3, 0.9, 0.95, 1e-8)
    return model, params, hm, tr, adam


def train(tr, adam, orc, steps, seed):
    toks = orc.random_tokens(4000, V)
    for s in range(steps):
        ids, tgt = orc.sample_batch(toks, T, B, seed + s)
        tr.forward_backward(ids, tgt)
        tr.adamw_step(adam, 0.1)


def state(tr, adam):
    p = tr.download(adam)
    return p.copy(), adam.flat("m"), adam.flat("v"), adam.opt.t


def same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_save_matches_reference_format(trlm, orc, tmp_path):
    model, _, hm, tr, adam = setup(trlm, orc)
    try:
        train(tr, adam, orc, 2, 100)
        path = str(tmp_path / "a.trlm")
        assert tr.checkpoint_save(path, adam)
        p, m, v, t = state(tr, adam)
        assert t == 2
        assert open(path, "rb").read() == orc.trlm_bytes(model.shapes(), p, m, v, t)
        nopt = str(tmp_path / "b.trlm")
        assert tr.checkpoint_save(nopt)
        assert open(nopt, "rb").read() == orc.trlm_bytes(model.shapes(), p)
        assert not os.path.exists(path + ".tmp")
    finally:
        tr.destroy()
        hm.close()


def test_load_restores_device_and_mirror(trlm, orc, tmp_path):
    model, _, hm, tr, adam = setup(trlm, orc)
    rng = np.random.default_rng(9)
    n = sum(int(np.prod(s)) for s in model.shapes())
    p = rng.standard_normal(n).astype(np.float32)
    m = rng.standard_normal(n).astype(np.float32)
    v = rng.random(n).astype(np.float32)
    path = str(tmp_path / "r.trlm")
    open(path, "wb").write(orc.trlm_bytes(model.shapes(), p, m, v, 77))
    try:
        assert tr.checkpoint_load(path, adam)
        assert adam.opt.t == 77
        assert same_bits(hm.values(), p)                  # host mirror
        assert same_bits(adam.flat("m"), m) and same_bits(adam.flat("v"), v)
        hm.set_values(np.zeros(n, np.float32))
        adam.set_flat("m", np.zeros(n, np.float32))
        got_p, got_m, got_v, _ = state(tr, adam)          # device
        assert same_bits(got_p, p) and same_bits(got_m, m) and same_bits(got_v, v)
    finally:
        tr.destroy()
        hm.close()


def test_resume_is_bit_identical(trlm, orc, tmp_path):
    _, _, hm, tr, adam = setup(trlm, orc)
    _, _, hm2, tr2, adam2 = setup(trlm, orc, seed=4242)
    path = str(tmp_path / "resume.trlm")
    try:
        train(tr, adam, orc, 2, 200)
        assert tr.checkpoint_save(path, adam)
        train(tr, adam, orc, 2, 300)
        assert tr2.checkpoint_load(path, adam2)
        train(tr2, adam2, orc, 2, 300)
        a, b = state(tr, adam), state(tr2, adam2)
        for x, y in zip(a[:3], b[:3]):
            assert same_bits(x, y)
        assert a[3] == b[3] == 4
    finally:
        tr.destroy()
        tr2.destroy()
        hm.close()
        hm2.close()


@pytest.mark.parametrize("case", ["truncated", "shape", "no_opt"])
def test_invalid_files_change_nothing(trlm, orc, tmp_path, case):
    model, params, hm, tr, adam = setup(trlm, orc)
    n = params.size
    rng = np.random.default_rng(1)
    other = rng.standard_normal(n).astype(np.float32)
    good = orc.trlm_bytes(model.shapes(), other, other, other, 5)
    if case == "truncated":
        data = good[:-3]
    elif case == "shape":
        bad = orc.Model(V + 1, D, H, L, F)
        data = orc.trlm_bytes(bad.shapes(), np.zeros(sum(int(np.prod(s)) for s in bad.shapes()), np.float32))
    else:
        data = orc.trlm_bytes(model.shapes(), other)
    path = str(tmp_path / "bad.trlm")
    open(path, "wb").write(data)
    try:
        before = state(tr, adam)
        assert not tr.checkpoint_load(path, adam)
        after = state(tr, adam)
        for x, y in zip(before[:3], after[:3]):
            assert same_bits(x, y)
        assert same_bits(hm.values(), params)
        assert after[3] == before[3]
        # a save that cannot be written leaves nothing behind
        assert not tr.checkpoint_save(str(tmp_path / "missing_dir" / "x.trlm"), adam)
    finally:
        tr.destroy()
        hm.close()
