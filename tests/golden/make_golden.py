"""Write the golden fixtures of tests/golden/ from the reference's own CPU
path, compiled from /root/reference into oracle/_ref (oracle/Makefile).

Run in the build container (where /root/reference exists):
    python tests/golden/make_golden.py           (a few minutes)
    python tests/golden/make_golden.py t1024     (ref_real_t1024.npz, ~15 min)
Outputs (data only: inputs and the reference's outputs):
  ref_small.npz     off-grid model V50 D32 H2 L2 F48 T12 B5: lm_init params,
                    token ids/targets, logits, loss, averaged gradients, and
                    one Adam step (the first case of test_gpu_train.c)
  ref_scalars.json  scalar maths and PCG outputs at fixed points, SHA-256 of
                    the real model's lm_init bits and of RoPE tables, the
                    real-scale (V31769 D384 H6 L12 F1024 T128 B4) loss with
                    per-tensor gradient sums, and SHA-256 of the batches the
                    reference's gpu_trainer_sample_batch (model/gpu_train.c:
                    296-307) draws for SAMPLE_CASES
  ref_real_t1024.npz  the real model (V31769 D384 H6 L12 F1024, lm_init
                    pcg_seed(1337,1)) at T=1024 B=2 (windows of the 200,000
                    token stream, seed 2026): loss, logits rows (sequence,
                    position) in LOGIT_ROWS, and per gradient tensor max|g|,
                    sum g (f64), sum |g| (f64) and GRAD_SAMPLES seeded entries
Every token window below comes from the reference's own sampler.
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402

MATH_POINTS = {
    "sqrt": [4.0, 2.0, 0.25, 1e6, 3.3e-7, 123456.789],
    "exp": [0.0, 1.0, -1.0, 10.0, -10.0, -87.3, 0.3466, 5.5e-3],
    "log": [1.0, 2.718281828459045, 2.0, 100.0, 31769.0, 1.000001, 0.001],
    "sin": [0.0, 0.5235987755982988, 1.234, 100.0, -7.5, 1023.0],
    "cos": [0.0, 1.0471975511965976, 1.234, 100.0, -7.5, 1023.0],
}
POW_POINTS = [(2.0, 10.0), (2.0, 0.5), (-2.0, 3.0), (0.9, 7.0), (0.999, 3.0), (10000.0, -0.03125)]
F32_POINTS = {"sqrtf": [2.0, 64.0, 1e-5, 0.3], "expf": [1.0, -3.25, -60.0], "logf": [31769.0, 1.5],
              "sinf": [0.5235988, 1023.0], "cosf": [0.5235988, 1023.0]}
# (num_tokens, vocab, token seed a, token seed b, T, B, seed_base): the
# fixtures' own windows, the config-4 stream at seeds 2026 + step, and edges
# (max_start = 0 and 1, seed_base * 1000003 wrapping past 2^64).
SAMPLE_CASES = [
    (4000, 50, 4242, 7, 12, 5, 2026),
    (200000, 31769, 4242, 7, 128, 4, 2026),
    (200000, 31769, 4242, 7, 1024, 8, 2026),
    (200000, 31769, 4242, 7, 1024, 8, 2027),
    (200000, 31769, 4242, 7, 1024, 8, 2028),
    (5000, 300, 1, 2, 50, 6, 9),
    (13, 50, 3, 3, 12, 3, 7),
    (14, 50, 3, 3, 12, 9, 8),
    (70000, 1000, 5, 6, 333, 17, (1 << 63) + 12345),
]

WHICH = {"sqrt": 0, "exp": 1, "log": 2, "pow": 3, "sin": 4, "cos": 5,
         "sqrtf": 10, "expf": 11, "logf": 12, "powf": 13, "sinf": 14, "cosf": 15}


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).view(np.uint8)).hexdigest()


LOGIT_ROWS = [(0, 0), (0, 1), (0, 1023), (1, 511), (1, 1023)]
GRAD_SAMPLES = 256


def t1024():
    oracle.build(with_ref=True)
    ref = oracle.Reference()
    real = oracle.Model(31769, 384, 6, 12, 1024)
    p = ref.lm_init(real, 1337, 1)
    toks = oracle.random_tokens(200000, 31769)
    T, B = 1024, 2
    ids, tgt = ref.sample_batch(toks, T, B, 2026)
    loss, grads = ref.forward_backward(real, p, ids, tgt, B, T, nthreads=B)
    logits = ref.forward_logits(real, p, ids, B, T, nthreads=B).reshape(B, T, -1)
    rows = np.stack([logits[b, t] for b, t in LOGIT_ROWS])
    rng = np.random.default_rng(1024)
    gmax, gsum, gabs, gidx, gval = [], [], [], [], []
    for g in real.split(grads):
        g = g.ravel()
        gmax.append(np.abs(g).max())
        gsum.append(g.astype(np.float64).sum())
        gabs.append(np.abs(g).astype(np.float64).sum())
        idx = np.sort(rng.choice(g.size, min(GRAD_SAMPLES, g.size), replace=False))
        idx = np.pad(idx, (0, GRAD_SAMPLES - idx.size), constant_values=idx[-1])
        gidx.append(idx)
        gval.append(g[idx])
    np.savez_compressed(os.path.join(HERE, "ref_real_t1024.npz"), ids=ids, tgt=tgt, loss=np.float32(loss),
                        logit_rows=np.array(LOGIT_ROWS, np.int32), logits=rows,
                        grad_max=np.array(gmax, np.float32), grad_sum=np.array(gsum), grad_abs=np.array(gabs),
                        grad_idx=np.array(gidx, np.int64), grad_val=np.array(gval, np.float32),
                        params_sha256=np.array(sha(p)))
    print("wrote ref_real_t1024.npz: loss", float(loss))


def main():
    oracle.build(with_ref=True)
    ref = oracle.Reference()
    out = {}
    # scalar maths, as float64 bit patterns (hex)
    m = {}
    for name, pts in MATH_POINTS.items():
        m[name] = [[x, float(ref.h.refh_m(WHICH[name], x, 0.0)).hex()] for x in pts]
    m["pow"] = [[a, b, float(ref.h.refh_m(3, a, b)).hex()] for a, b in POW_POINTS]
    m["powf"] = [[a, b, float(ref.h.refh_m(13, a, b)).hex()] for a, b in POW_POINTS]
    for name, pts in F32_POINTS.items():
        m[name] = [[x, float(ref.h.refh_m(WHICH[name], x, 0.0)).hex()] for x in pts]
    out["math"] = m
    # PCG32 streams
    u = np.zeros(8, np.uint32)
    ref.h.refh_pcg_u32(42, 54, 8, u)
    out["pcg_u32_42_54"] = [int(x) for x in u]
    r = np.zeros(16, np.int64)
    ref.h.refh_pcg_range(4242, 7, 0, 31768, 16, r)
    out["pcg_range_4242_7_0_31768"] = [int(x) for x in r]
    g = np.zeros(8, np.float64)
    ref.h.refh_pcg_gauss(1337, 1, 8, g)
    out["pcg_gauss_1337_1"] = [float(x).hex() for x in g]
    # RoPE tables
    for T, hd in [(128, 64), (1024, 64), (12, 16)]:
        c = np.zeros((T, hd // 2), np.float32)
        s = np.zeros((T, hd // 2), np.float32)
        ref.h.refh_rope_tables(T, hd, c, s)
        out["rope_%d_%d" % (T, hd)] = [sha(c), sha(s)]
    # real model: init hash and the real-scale case of test_gpu_train.c
    real = oracle.Model(31769, 384, 6, 12, 1024)
    p = ref.lm_init(real, 1337, 1)
    out["real_init_sha256"] = sha(p)
    out["real_num_params"] = int(real.total)
    toks = oracle.random_tokens(200000, 31769)
    ids, tgt = ref.sample_batch(toks, 128, 4, 2026)
    out["real_ids_sha256"] = sha(ids)
    loss, grads = ref.forward_backward(real, p, ids, tgt, 4, 128)
    out["real_loss_hex"] = float(loss).hex()
    out["real_grad_tensor_sums"] = [float(x.astype(np.float64).sum()).hex() for x in real.split(grads)]
    out["real_grad_sha256"] = sha(grads)
    # the reference's batch sampler
    sb = []
    for n, V, sa, sbb, T, B, seed in SAMPLE_CASES:
        toks = oracle.random_tokens(n, V, sa, sbb)
        i, t = ref.sample_batch(toks, T, B, seed)
        sb.append([n, V, sa, sbb, T, B, seed, sha(i), sha(t)])
    out["sample_batch"] = sb
    with open(os.path.join(HERE, "ref_scalars.json"), "w") as fh:
        json.dump(out, fh, indent=1, sort_keys=True)

    # small off-grid case, full arrays
    small = oracle.Model(50, 32, 2, 2, 48)
    ps = ref.lm_init(small, 1337, 1)
    toks = oracle.random_tokens(4000, 50)
    ids, tgt = ref.sample_batch(toks, 12, 5, 2026)
    logits = ref.forward_logits(small, ps, ids, 5, 12)
    loss, grads = ref.forward_backward(small, ps, ids, tgt, 5, 12)
    pa, ma, va = ps.copy(), np.zeros_like(ps), np.zeros_like(ps)
    ref.adam_step(small, pa, grads, ma, va, 0, 3e-4, 0.9, 0.999, 1e-8)
    np.savez_compressed(os.path.join(HERE, "ref_small.npz"), params=ps, ids=ids, tgt=tgt, logits=logits,
                        loss=np.float32(loss), grads=grads, adam_p=pa, adam_m=ma, adam_v=va)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    if len(sys.argv) > 1 and sys.argv[1] == "t1024":
        t1024()
    else:
        main()
