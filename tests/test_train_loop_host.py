"""The driver loop's learning-rate schedule (training/lr_schedule.c:6-15),
host-side, no GPU.

Pins: the oracle's restatement against the reference's own known answers
(tests/test_lr_schedule.c:21-34, same tolerance and monotonicity checks) and
bit for bit against the reference's lr_warmup_cosine compiled into
oracle/_ref; the library's trlm_lr_warmup_cosine (a host function of the C
ABI, used by gpu_trainer_train_steps) bit for bit against the oracle.
"""
import numpy as np
import pytest

PEAK, MIN, W, TOT = np.float32(6e-4), np.float32(6e-5), 1000, 70000


def near(a, b):
    a, b = np.float32(a), np.float32(b)
    return abs(float(a) - float(b)) <= 1e-6 * abs(float(b)) + 1e-12


def test_schedule_known_answers(orc):
    lr = lambda s: orc.lr_warmup_cosine(s, W, TOT, PEAK, MIN)
    assert near(lr(0), PEAK / np.float32(1000.0))
    assert near(lr(499), PEAK * np.float32(0.5))
    assert near(lr(W - 1), PEAK)
    assert near(lr(W), PEAK)
    assert near(lr(W + (TOT - W) // 2), np.float32(0.5) * (PEAK + MIN))
    assert near(lr(TOT), MIN)
    assert near(lr(TOT + 5000), MIN)
    up = [lr(s) for s in range(W)]
    assert all(b > a for a, b in zip(up, up[1:]))
    down = [lr(s) for s in range(W, TOT + 1, 7)]
    assert all(b <= a + 1e-12 for a, b in zip(down, down[1:]))
    # degenerate schedules: no warmup starts at peak; total <= warmup holds min
    assert orc.lr_warmup_cosine(0, 0, 100, PEAK, MIN) == PEAK
    assert orc.lr_warmup_cosine(5, 10, 10, PEAK, MIN) == PEAK * np.float32(6) / np.float32(10)
    assert orc.lr_warmup_cosine(12, 10, 10, PEAK, MIN) == MIN


def test_schedule_matches_reference(orc):
    if not orc.reference_available():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    ref = orc.Reference()
    for (w, tot, first, n) in [(W, TOT, 0, 3000), (W, TOT, TOT - 1500, 3000), (0, 500, 0, 600), (30, 30, 0, 60),
                               (2, 8, 0, 12)]:
        want = ref.lr_schedule(first, n, w, tot, PEAK, MIN)
        got = np.array([orc.lr_warmup_cosine(first + i, w, tot, PEAK, MIN) for i in range(n)], np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (w, tot, first)


def test_library_schedule_matches_oracle(trlm, orc):
    _, hip = trlm.libs()
    for (w, tot) in [(W, TOT), (0, 500), (2, 8), (30, 30)]:
        for s in list(range(0, 40)) + list(range(w, min(tot + 50, w + 4000), 13)):
            got = np.float32(hip.trlm_lr_warmup_cosine(s, w, tot, PEAK, MIN))
            want = orc.lr_warmup_cosine(s, w, tot, PEAK, MIN)
            assert got.view(np.uint32) == want.view(np.uint32), (w, tot, s)
