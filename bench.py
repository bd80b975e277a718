"""bench.py -- MI355X GPU matmul path of turkce-llm, one JSON line.

Headline (BASELINE.json metric, configs[1]): the fp32 GEMM sweep at the
model's real shapes with M = B*T = 8192 -- QKV, attention-out, gate/up
(fused, N = 2F), down and the 31,769-wide tied LM head, each as forward
(NN, LM head NT), dX (NT / NN for the head) and dW (TN).  One "step" is one
pass over all fifteen GEMMs with operands resident in HBM.  value = sweep
FLOPs / sweep time (TFLOP/s), against the 157.3 TFLOP/s FP32-MFMA peak.

Also reported (same run, same library): forward tokens/s (config 3: B=8,
T=1024, forward + mean cross-entropy) and training tokens/s (config 4:
forward, CE, full backward and AdamW with lr 3e-4, betas 0.9/0.95,
eps 1e-8, wd 0.1), with random-init weights of the real architecture.

roofline: the LM-head forward GEMM (the largest single kernel), algorithmic
2*M*N*K FLOPs per launch divided by its average launch time measured here
with HIP events on the library's stream.

cpu_baseline: the reference's own CPU matmul (tensor_matmul2d, built from
/root/reference into oracle/_ref) on the sweep's whole QKV forward GEMM, its
rows split over 8 host threads; falls back to the oracle restatement when
oracle/_ref was not built.
cpu_model: the reference's CPU forward (config 3) and training step
(config 4) at B=8, T=1024 on 8 host threads, one sequence each, as
training/data_parallel.c runs it, from one transformer block at T=1024 and
16 rows of the head timed at that shape and scaled to the 12 layers and
1024 rows (cpu_model_baseline); gpu_vs_cpu_forward / gpu_vs_cpu_train are
the GPU's rates over these.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_FP32_MFMA = 157.3   # TFLOP/s, MI355X dense FP32 matrix
PEAK_HBM = 8000.0        # GB/s
V, D, H, L, F = 31769, 384, 6, 12, 1024
B, T = 8, 1024
M = B * T
METRIC = "GEMM TFLOP/s (% FP32-MFMA peak); fwd+train tokens/s, 33.5M LM, B8 T1024"

# name, forward N, K   (forward: [M,K] x [K,N])
SHAPES = [("qkv", 3 * D, D), ("attn_out", D, D), ("gate_up", 2 * F, D), ("down", D, F), ("lm_head", V, D)]


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def load_trlm():
    import importlib.util
    spec = importlib.util.spec_from_file_location("trlm_amd", os.path.join(ROOT, "turkce-llm_amd", "trlm.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["trlm_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


class Sweep:
    """Device operands of the fifteen GEMMs and their launches."""

    def __init__(self, trlm, dev, M=M):
        self.dev = dev
        rng = np.random.default_rng(2026)
        self.items = []
        self.bufs = []
        for name, N, K in SHAPES:
            ldn = (N + 3) // 4 * 4
            X = rng.standard_normal((M, K), dtype=np.float32)                 # activations N(0,1)
            if name == "lm_head":
                W = (0.02 * rng.standard_normal((N, K), dtype=np.float32))   # E [V, D]
            else:
                W = (0.02 * rng.standard_normal((K, N), dtype=np.float32))   # W [K, N]
            dY = rng.standard_normal((M, ldn), dtype=np.float32)
            dX, dW, dWb = dev.upload(X), dev.upload(W), dev.upload(dY)
            dOut = dev.empty(M * ldn * 4)
            dGX = dev.empty(M * K * 4)
            dGW = dev.empty(N * K * 4)
            self.bufs += [dX, dW, dWb, dOut, dGX, dGW]
            fl = 2.0 * M * N * K
            if name == "lm_head":
                # logits = X @ E^T (NT); dX = dY @ E (NN, K = V); dE = dY^T @ X (TN, K = M)
                self.items.append((name + "_fwd", fl, (0, 1, dX, dW, dOut, M, N, K, K, K, ldn)))
                self.items.append((name + "_dx", fl, (0, 0, dWb, dW, dGX, M, K, N, ldn, K, K)))
                self.items.append((name + "_dw", fl, (1, 0, dWb, dX, dGW, N, K, M, ldn, K, K)))
            else:
                # Y = X @ W (NN); dX = dY @ W^T (NT); dW = X^T @ dY (TN, K = M)
                self.items.append((name + "_fwd", fl, (0, 0, dX, dW, dOut, M, N, K, K, N, ldn)))
                self.items.append((name + "_dx", fl, (0, 1, dWb, dW, dGX, M, K, N, ldn, N, K)))
                self.items.append((name + "_dw", fl, (1, 0, dX, dWb, dGW, K, N, M, K, ldn, N)))
        self.flops = sum(f for _, f, _ in self.items)

    def run(self, item):
        ta, tb, A, Bm, Cm, m, n, k, lda, ldb, ldc = item[2]
        self.dev.matmul(ta, tb, A, Bm, Cm, m, n, k, lda, ldb, ldc)

    def step(self):
        for it in self.items:
            self.run(it)

    def close(self):
        for p in self.bufs:
            self.dev.free(p)


def time_events(hip, fn, reps):
    from ctypes import byref
    import trlm_amd
    t = trlm_amd.TrlmTimer()
    hip.trlm_timer_create(byref(t))
    hip.trlm_timer_start(byref(t))
    for _ in range(reps):
        fn()
    ms = hip.trlm_timer_stop_ms(byref(t))
    hip.trlm_timer_destroy(byref(t))
    return ms / reps


def model_params(rng):
    """Random-init weights of the real architecture (lm_init's layout and
    scales: matrices N(0, 0.02), biases 0, norm weights 1)."""
    parts = [0.02 * rng.standard_normal(V * D, dtype=np.float32)]
    for _ in range(L):
        parts += [np.ones(D, np.float32), 0.02 * rng.standard_normal(D * 3 * D, dtype=np.float32),
                  np.zeros(3 * D, np.float32), 0.02 * rng.standard_normal(D * D, dtype=np.float32),
                  np.zeros(D, np.float32), np.ones(D, np.float32),
                  0.02 * rng.standard_normal(D * 2 * F, dtype=np.float32), np.zeros(2 * F, np.float32),
                  0.02 * rng.standard_normal(F * D, dtype=np.float32), np.zeros(D, np.float32)]
    parts.append(np.ones(D, np.float32))
    return np.concatenate(parts).astype(np.float32)


def model_benchmarks(trlm, steps, warmup):
    rng = np.random.default_rng(7)
    params = model_params(rng)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, B, T)
    adam = trlm.Adam(hm, 3e-4, 0.9, 0.95, 1e-8)
    ids = rng.integers(0, V, M, dtype=np.uint32)
    tgt = rng.integers(0, V, M, dtype=np.uint32)
    out = {}
    try:
        for _ in range(warmup):
            tr.eval_loss(ids, tgt)
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = tr.eval_loss(ids, tgt)
        fwd = (time.perf_counter() - t0) / steps
        for _ in range(warmup):
            tr.forward_backward(ids, tgt)
            tr.adamw_step(adam, 0.1)
        t0 = time.perf_counter()
        for _ in range(steps):
            loss = tr.forward_backward(ids, tgt)
            tr.adamw_step(adam, 0.1)
        trn = (time.perf_counter() - t0) / steps
        out = {"fwd_ms": fwd * 1e3, "fwd_tokens_per_s": M / fwd, "train_ms": trn * 1e3,
               "train_tokens_per_s": M / trn, "train_loss_last": float(loss),
               "fwd_tflops_algorithmic": 625.16e9 / fwd / 1e12, "train_tflops_algorithmic": 1875.5e9 / trn / 1e12}
        out.update(driver_benchmarks(trlm, tr, adam, rng, steps, warmup))
    finally:
        tr.destroy()
        hm.close()
    return out


def driver_benchmarks(trlm, tr, adam, rng, steps, warmup):
    """The reference driver's full step (train_lm_gpu.c:212-223: schedule,
    sampled batch, forward/backward, grad norm, clip, AdamW) at B8 T1024 on
    a synthetic 4M-token stream: as the reference's call sequence (host
    waits inside every call) and queued (gpu_trainer_train_steps)."""
    _, hip = trlm.libs()
    tokens = rng.integers(0, V, 1 << 22, dtype=np.uint32)
    s = trlm.TrlmSchedule()
    s.warmup_steps, s.total_steps, s.peak_lr, s.min_lr = 100, 10000, 6e-4, 6e-5
    s.grad_clip, s.weight_decay, s.seed_base = 1.0, 0.1, 2026
    ids = np.zeros(M, np.uint32)
    tgt = np.zeros(M, np.uint32)

    def sequence(first, n):
        for step in range(first, first + n):
            adam.opt.lr = hip.trlm_lr_warmup_cosine(step, s.warmup_steps, s.total_steps, s.peak_lr, s.min_lr)
            hip.gpu_trainer_sample_batch(tokens, tokens.size, T, B, s.seed_base + step, ids, tgt)
            tr.forward_backward(ids, tgt)
            norm = tr.grad_norm()
            tr.adamw_step(adam, s.weight_decay, (s.grad_clip / norm) if norm > s.grad_clip else 1.0)

    sequence(0, warmup)
    t0 = time.perf_counter()
    sequence(warmup, steps)
    seq = (time.perf_counter() - t0) / steps
    tr.train_steps(adam, tokens, s, 0, warmup)
    t0 = time.perf_counter()
    losses, _, _ = tr.train_steps(adam, tokens, s, warmup, steps)
    queued = (time.perf_counter() - t0) / steps
    return {"driver_step_ms": queued * 1e3, "driver_tokens_per_s": M / queued,
            "driver_step_ms_call_sequence": seq * 1e3, "driver_loss_last": float(losses[-1])}


def hybrid_benchmarks(trlm, reps=10):
    """The hybrid path's tied LM head as generate.c runs it each token
    (lm_forward over a 128-token window: node_matmul2d_gpu of x [128, D] by
    the transposed view of E [V, D]), with E uploaded on every call (the
    reference's behaviour) and with E pinned (gpu_ops_pin)."""
    import ctypes as C
    host, hip = trlm.libs()
    alloc = host.allocator_create(1 << 31)
    hip.gpu_ops_init(C.byref(alloc), trlm.KERNELS.encode())
    rng = np.random.default_rng(13)
    Tw = 128

    def leaf(arr):
        sh = (C.c_uint64 * 2)(*arr.shape)
        t = host.tensor_create(C.byref(alloc), sh, 2)
        trlm.tensor_np(t)[:] = arr.ravel()
        return host.node_leaf(C.byref(alloc), t, 1)

    try:
        nx = leaf(rng.standard_normal((Tw, D)).astype(np.float32))
        nE = leaf((0.02 * rng.standard_normal((V, D))).astype(np.float32))
        nEt = host.node_leaf(C.byref(alloc), host.tensor_transpose(C.byref(nE.contents.value), 0, 1), 1)
        out = {}
        for key in ("hybrid_head_ms", "hybrid_head_ms_pinned"):
            if key.endswith("pinned"):
                hip.gpu_ops_pin(C.cast(nE.contents.value.data, C.c_void_p).value, V * D)
            hip.node_matmul2d_gpu(C.byref(alloc), nx, nEt)
            t0 = time.perf_counter()
            for _ in range(reps):
                hip.node_matmul2d_gpu(C.byref(alloc), nx, nEt)
            out[key] = (time.perf_counter() - t0) / reps * 1e3
        out["hybrid_head_config"] = "node_matmul2d_gpu [128,384] x E^T [384,31769] view, logits to host"
        return out
    finally:
        hip.gpu_ops_shutdown()
        host.allocator_destroy(C.byref(alloc))


DEC_B, DEC_PROMPT, DEC_CTX = 64, 128, 1024
DEC_TEMP = 0.85   # generate.c:54 TEMPERATURE


def decode_benchmark(trlm):
    """Config 5: 64 sequences, 128-token prompts (ids pcg_range_i64(0, V) from
    pcg_seed(4242, 9)), greedy KV-cache decode to context 1024: 896 new tokens
    per sequence (prefill + 895 steps), random-init weights of the real
    architecture.  Bytes per step = all weights (133.96 MB) + the K and V
    cache read by the step (64*12*2*ctx*384*4 B).  The same generation
    sampled (sample_next at temperature 0.85, one PCG stream per sequence) is
    timed as decode_sampled_*."""
    host, _ = trlm.libs()
    import ctypes as C
    rng = np.random.default_rng(11)
    params = model_params(rng)
    pcg = host.pcg_seed(4242, 9)
    prompt = np.array([host.pcg_range_i64(C.byref(pcg), 0, V) for _ in range(DEC_B * DEC_PROMPT)],
                      np.uint32).reshape(DEC_B, DEC_PROMPT)
    hm = trlm.HostModel(V, D, H, L, F, params)
    tr = trlm.Trainer(hm, 1, 8)
    dec = trlm.Decoder(tr, DEC_B, DEC_CTX)
    try:
        dec.generate_greedy(prompt, 16)       # warm-up (kernels, workspaces, prefill buffers)
        steps = DEC_CTX - DEC_PROMPT
        t0 = time.perf_counter()
        dec.generate_greedy(prompt, steps)
        dt = time.perf_counter() - t0
        # sampled generation (the reference's generate.c: sample_next at TEMPERATURE 0.85), one PCG
        # stream per sequence, pcg_seed(4242, 7 + b) (the reference's single stream is (4242, 7))
        rngs = (trlm.PCGState * DEC_B)(*[host.pcg_seed(4242, 7 + b) for b in range(DEC_B)])
        dec.generate_sampled(prompt, 16, rngs, DEC_TEMP)
        rngs = (trlm.PCGState * DEC_B)(*[host.pcg_seed(4242, 7 + b) for b in range(DEC_B)])
        t0 = time.perf_counter()
        dec.generate_sampled(prompt, steps, rngs, DEC_TEMP)
        dts = time.perf_counter() - t0
    finally:
        dec.destroy()
        tr.destroy()
        hm.close()
    weights = 4.0 * (V * D + L * (2 * D + 3 * D * D + 3 * D + D * D + D + 2 * D * F + 2 * F + F * D + D) + D)
    kv = sum(DEC_B * L * 2 * n * D * 4.0 for n in range(DEC_PROMPT + 1, DEC_CTX + 1))
    total = weights * (steps - 1) + kv - DEC_B * L * 2 * DEC_CTX * D * 4.0
    tokens = DEC_B * steps
    return {"decode_tokens_per_s": tokens / dt, "decode_ms_per_token": dt * 1e3 / steps,
            "decode_gbps": total / dt / 1e9, "decode_total_s": dt,
            "decode_sampled_tokens_per_s": tokens / dts, "decode_sampled_ms_per_token": dts * 1e3 / steps,
            "decode_sampled_temperature": DEC_TEMP,
            "decode_config": "batch %d, prompt %d, greedy to context %d (%d steps)" % (
                DEC_B, DEC_PROMPT, DEC_CTX, steps - 1)}


CPU_THREADS = 8        # one per sequence of the B=8 batch, as data_parallel_step runs it
CPU_HEAD_ROWS = 16     # rows of the timed head piece; every head row costs the same


def host_cpu():
    """nproc, the cores this process may run on, and the CPU model name."""
    model = "?"
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    model = ln.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)), "model": model}


def cpu_baseline():
    """The reference's tensor_matmul2d on the whole QKV forward GEMM of the
    sweep (8192x1152x384), its rows split over CPU_THREADS concurrent threads,
    each running the reference's single-threaded loop on its share (the
    reference parallelises over sequences, one thread each); the oracle's
    reference-order matmul on one thread when oracle/_ref was not built."""
    import oracle
    rng = np.random.default_rng(1)
    K, N = D, 3 * D
    Wq = (0.02 * rng.standard_normal((K, N))).astype(np.float32)
    X = rng.standard_normal((M, K)).astype(np.float32)
    if oracle.reference_available():
        out = np.zeros((M, N), np.float32)
        dt = oracle.Reference().h.refh_time_matmul_threads(M, N, K, X, Wq, out, CPU_THREADS)
        rows, cores, kind = M, CPU_THREADS, "reference"
        what = "tensor_matmul2d (oracle/_ref), rows split over %d threads" % cores
    else:
        rows, cores, kind = 512, 1, "port"
        t0 = time.perf_counter()
        oracle.matmul(X[:rows], Wq)
        dt = time.perf_counter() - t0
        what = "the oracle's reference-order matmul, 1 thread"
    tflops = 2.0 * rows * N * K / dt / 1e12
    return {"value": tflops, "unit": "TFLOP/s", "cores": cores, "kind": kind,
            "sample": "QKV forward GEMM %dx%dx%d through %s, %.1f s" % (rows, N, K, what, dt)}


def cpu_model_baseline():
    """Config 3 (forward + CE) and config 4 (training step) of the
    reference's CPU path at B=8, T=1024, from pieces timed at that shape
    (oracle/ref_harness.c refh_time_pieces): CPU_THREADS concurrent threads,
    one sequence each, run one transformer_block over T=1024 rows (forward,
    then backward) and the embedding + final RMSNorm + tied head + CE over
    CPU_HEAD_ROWS rows (forward, then backward); adam_step_parallel is timed
    over the whole model.  A step is then 12 * block + (T / rows) * head
    (+ Adam), since the 12 blocks are identical and a head row's cost does
    not depend on T.  Needs oracle/_ref (None without it)."""
    import oracle
    if not oracle.reference_available():
        return None
    ref = oracle.Reference()
    model = oracle.Model(V, D, H, L, F)
    params = ref.lm_init(model)
    tok = oracle.random_tokens(4 * CPU_THREADS * T + T + 2, V)
    ids, tgt = oracle.sample_batch(tok, T, CPU_THREADS, 2026)
    out = np.zeros(4)
    t0 = time.perf_counter()
    rc = ref.h.refh_time_pieces(C.byref(model.cfg), params, ids, tgt, T, CPU_HEAD_ROWS, CPU_THREADS, out)
    if rc != 0:
        raise RuntimeError("refh_time_pieces failed: %d" % rc)
    grads = (1e-3 * np.random.default_rng(3).standard_normal(model.total)).astype(np.float32)
    adam = ref.h.refh_time_adam(C.byref(model.cfg), params.copy(), grads, CPU_THREADS)
    wall = time.perf_counter() - t0
    scale = T / CPU_HEAD_ROWS
    fwd_s = L * out[0] + scale * out[2]
    step_s = L * out[1] + scale * out[3] + adam
    tokens = CPU_THREADS * T
    return {"fwd_tokens_per_s": tokens / fwd_s, "train_tokens_per_s": tokens / step_s,
            "fwd_s": fwd_s, "step_s": step_s, "threads": CPU_THREADS, "kind": "reference",
            "pieces_s": {"block_fwd": out[0], "block_fwd_bwd": out[1], "head_fwd": out[2],
                         "head_fwd_bwd": out[3], "adam": adam},
            "sample": ("reference CPU path (oracle/_ref), %d threads, one T=%d sequence each: one transformer_block "
                       "fwd / fwd+bwd at T=%d and embedding+final norm+tied head+CE fwd / fwd+bwd on %d rows, "
                       "timed together; step = %d x block + %d x head (+ adam_step_parallel over all %d "
                       "parameters); %.0f s of wall" % (CPU_THREADS, T, T, CPU_HEAD_ROWS, L, int(scale),
                                                        model.total, wall))}


def summarize_profile(path):
    """Print per-kernel statistics from a rocprofv3 run (--kernel-trace
    --output-format csv): one line per (kernel, grid) so that the LM-head
    dispatches of the NT GEMM stand apart from the other NT shapes."""
    import csv
    import glob
    files = glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True)
    if not files:
        sys.exit("no *kernel_trace.csv under %s" % path)
    groups = {}
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = r.get("Kernel_Name") or r.get("kernel_name")
                dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                grid = (r.get("Grid_Size_X") or r.get("Grid_Size", "?"), r.get("Grid_Size_Y", ""),
                        r.get("Grid_Size_Z", ""))
                key = (name, "x".join(g for g in grid if g))
                groups.setdefault(key, []).append(dur)
    total = sum(sum(v) for v in groups.values())
    print("%-36s %-22s %7s %12s %12s %7s" % ("kernel", "grid (work-items)", "calls", "total_us", "avg_us", "pct"))
    for (name, grid), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        print("%-36s %-22s %7d %12.1f %12.2f %6.2f%%" % (name[:36], grid, len(v), sum(v) / 1e3,
                                                          sum(v) / len(v) / 1e3, 100.0 * sum(v) / total))


TILES = ["256x128", "128x256", "128x128", "128x128_k32", "64x128", "64x128_k32", "64x64", "64x64_k32"]


def tune(trlm, hip, reps, out_path=None):
    """Time every aligned tile variant and split-K factor on the sweep GEMMs
    (at M = B*T and at two smaller row counts) and print them, fastest
    first; the automatic choice is marked '*'.  out_path: all timings as
    JSON lines {name, M, N, K, layout, variant, splits, ms, tflops, auto}."""
    dev = trlm.Device()
    fh = open(out_path, "w") if out_path else None
    for m_rows in (M, 2048, 512):
        sweep = Sweep(trlm, dev, m_rows)
        for it in sweep.items:
            sweep.run(it)
            auto = "%s/split%d" % dev.last_variant()
            ta, tb, _, _, _, m, n, k = it[2][:8]
            rows = []
            for tile in TILES:
                for sp in [1, 2, 3, 4, 6, 8, 12, 16, 24, 32]:
                    if sp > 1 and k // sp < 256:
                        continue
                    dev.force(tile, sp)
                    sweep.run(it)
                    dev.sync()
                    ms = time_events(hip, lambda: sweep.run(it), reps)
                    name, got_sp = dev.last_variant()
                    rows.append((it[1] / (ms * 1e-3) / 1e12, "%s/split%d" % (name, got_sp), ms))
                    if fh:
                        fh.write(json.dumps({"name": it[0], "M": m, "N": n, "K": k, "layout": [ta, tb],
                                             "variant": name, "splits": got_sp, "ms": ms,
                                             "tflops": rows[-1][0], "auto": rows[-1][1] == auto}) + "\n")
            dev.force(None)
            rows.sort(reverse=True)
            print("%s M=%d  (auto %s)" % (it[0], m_rows, auto), flush=True)
            for tf, name, ms in rows[:4]:
                print("   %7.1f TF  %8.4f ms  %s%s" % (tf, ms, name, " *" if name == auto else ""), flush=True)
            a = [r for r in rows if r[1] == auto]
            if a and a[0] not in rows[:4]:
                print("   %7.1f TF  %8.4f ms  %s *" % (a[0][0], a[0][2], auto), flush=True)
        sweep.close()
    if fh:
        fh.close()
    dev.close()


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "lm_head_fwd_hbm_traffic.txt")
PROBE_COPY_BYTES = 512 << 20


def traffic_probe(trlm):
    """Dispatches for the HBM-traffic counter passes: three device copies of
    PROBE_COPY_BYTES (the calibration: a plain copy reads and writes exactly
    that many bytes), then three LM-head forward GEMMs of the sweep."""
    _, hip = trlm.libs()
    rt = C.CDLL("libamdhip64.so")
    rt.hipMemcpyDtoD.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    dev = trlm.Device()
    sweep = Sweep(trlm, dev)
    src, dst = dev.empty(PROBE_COPY_BYTES), dev.empty(PROBE_COPY_BYTES)
    dev.sync()
    for _ in range(3):
        assert rt.hipMemcpyDtoD(dst, src, PROBE_COPY_BYTES) == 0
    head = [it for it in sweep.items if it[0] == "lm_head_fwd"][0]
    for _ in range(3):
        sweep.run(head)
    dev.sync()
    print("probe: 3 copies of %d bytes, 3 x %s" % (PROBE_COPY_BYTES, "%s/split%d" % dev.last_variant()), flush=True)
    dev.free(src)
    dev.free(dst)
    sweep.close()
    dev.close()


def counter_probe(trlm, phase):
    """Dispatches for the per-kernel counter tables (profiles/
    kernel_counters_*.txt): three calibration copies of PROBE_COPY_BYTES,
    then
      train:  config 4 with every side section on the main stream
              (hip_side_serial: no contention between overlapped kernels) --
              two training steps (forward, CE, backward, AdamW) and one
              forward;
      decode: config 5's step kernels at context ~1000 -- a 1000-token
              prefill of 64 sequences and 4 eager decode steps, greedy,
              then the same sampled at temperature 0.85."""
    host, hip = trlm.libs()
    rt = C.CDLL("libamdhip64.so")
    rt.hipMemcpyDtoD.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
    dev = trlm.Device()
    src, dst = dev.empty(PROBE_COPY_BYTES), dev.empty(PROBE_COPY_BYTES)
    dev.sync()
    for _ in range(3):
        assert rt.hipMemcpyDtoD(dst, src, PROBE_COPY_BYTES) == 0
    dev.sync()
    dev.free(src)
    dev.free(dst)
    dev.close()
    rng = np.random.default_rng(7)
    params = model_params(rng)
    hm = trlm.HostModel(V, D, H, L, F, params)
    try:
        if phase == "train":
            tr = trlm.Trainer(hm, B, T)
            adam = trlm.Adam(hm, 3e-4, 0.9, 0.95, 1e-8)
            ids = rng.integers(0, V, M, dtype=np.uint32)
            tgt = rng.integers(0, V, M, dtype=np.uint32)
            hip.hip_side_serial(1)
            try:
                for _ in range(2):
                    tr.forward_backward(ids, tgt)
                    tr.adamw_step(adam, 0.1)
                tr.eval_loss(ids, tgt)
                hip.hip_sync()
            finally:
                hip.hip_side_serial(0)
                tr.destroy()
        else:
            os.environ["TRLM_DECODE_EAGER"] = "1"   # kernel tracers cannot follow graph replays here
            tr = trlm.Trainer(hm, 1, 8)
            dec = trlm.Decoder(tr, DEC_B, DEC_CTX)
            try:
                prompt = rng.integers(0, V, DEC_B * 1000, dtype=np.uint32).reshape(DEC_B, 1000)
                dec.generate_greedy(prompt, 5)
                rngs = (trlm.PCGState * DEC_B)(*[host.pcg_seed(4242, 7 + b) for b in range(DEC_B)])
                dec.generate_sampled(prompt, 5, rngs, DEC_TEMP)
            finally:
                dec.destroy()
                tr.destroy()
    finally:
        hm.close()
    print("counter probe (%s) done" % phase, flush=True)


TILE_DIMS = {"256x128": (256, 128), "128x256": (128, 256), "128x128": (128, 128), "128x128_k32": (128, 128),
             "64x128": (64, 128), "64x128_k32": (64, 128), "64x64": (64, 64), "64x64_k32": (64, 64)}


def gemm_roles():
    """(kernel, total work-items) -> role for the B8 T1024 training step's
    GEMMs (and their split-K reductions), from the engine's own plan
    (trlm_gemm_plan); launches are tiles x 256 work-items x splits."""
    _, hip = load_trlm().libs()
    shapes = [("QKV fwd", 0, 0, M, 3 * D, D), ("attn-out fwd", 0, 0, M, D, D), ("gate_up fwd", 0, 0, M, 2 * F, D),
              ("down fwd", 0, 0, M, D, F), ("LM-head fwd", 0, 1, M, V, D), ("QKV dX", 0, 1, M, D, 3 * D),
              ("attn-out dX", 0, 1, M, D, D), ("gate_up dX", 0, 1, M, D, 2 * F), ("down dX", 0, 1, M, F, D),
              ("LM-head dX", 0, 0, M, D, V), ("QKV dW", 1, 0, D, 3 * D, M), ("attn-out dW", 1, 0, D, D, M),
              ("gate_up dW", 1, 0, D, 2 * F, M), ("down dW", 1, 0, F, D, M), ("LM-head dW", 1, 0, V, D, M)]
    roles = {}
    sp = C.c_int32()
    for role, ta, tb, m, n, k in shapes:
        name = hip.trlm_gemm_plan(ta, tb, m, n, k, 1, C.byref(sp)).decode()
        bm, bn = TILE_DIMS[name.split("_", 3)[3]]
        splits = sp.value if role not in ("QKV fwd", "LM-head fwd") else 1   # RoPE / row statistics: no split
        grid = -(-m // bm) * -(-n // bn) * 256 * splits
        roles.setdefault((name[:40], str(grid)), []).append(role)
        if splits > 1:
            for rows in (m, m + 1):   # the weight gradients' partials carry the bias sums in an extra row
                g2 = -(-(rows * n) // 256) * 256
                roles.setdefault(("k_gemm_splitk_reduce", str(g2)), []).append(role + " reduce")
                g4 = -(-(rows * n // 4) // 256) * 256   # four columns per thread (aligned operands)
                roles.setdefault(("k_gemm_splitk_reduce4", str(g4)), []).append(role + " reduce")
    attn_grid = B * H * -(-T // 64) * 256
    for k in ("k_attn_fwd_hd64", "k_attn_bwd_dkv_hd64", "k_attn_bwd_dq_hd64"):
        roles[(k, str(attn_grid))] = ["B8 T1024"]
    return {k: " / ".join(sorted(set(v))) for k, v in roles.items()}


def counter_summary(phase, trace_dir, busy_dir, fetch_dir, write_dir):
    """Per-kernel table from a --kernel-trace run and three --pmc runs of
    --counter-probe PHASE: average duration; matrix-core use = SQ_VALU_MFMA_
    BUSY_CYCLES / (1024 SIMDs x kernel cycles), kernel cycles = SQ_CYCLES /
    32 shader engines; HBM bytes = FETCH_SIZE and WRITE_SIZE scaled by the
    factors that make the calibration copies read their true size, and the
    GB/s they give over the kernel's average duration.  The decode table
    lists the step's kernels only (not the prefill's)."""
    import csv
    import glob

    def rows(d, pat):
        for f in glob.glob(os.path.join(d, "**", pat), recursive=True):
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    yield r

    def key(r):
        if "Grid_Size_X" in r:   # kernel trace: per dimension
            grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        else:                    # counter collection: total work-items
            grid = int(r["Grid_Size"])
        return (r["Kernel_Name"][:40], str(grid))

    dur = {}
    for r in rows(trace_dir, "*kernel_trace.csv"):
        dur.setdefault(key(r), []).append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    ctr = {}
    for d in (busy_dir, fetch_dir, write_dir):
        per = {}
        for r in rows(d, "*counter_collection.csv"):
            k = (key(r), r["Dispatch_Id"], r["Counter_Name"])
            per[k] = per.get(k, 0.0) + float(r["Counter_Value"])
        for (k, _, c), v in per.items():
            ctr.setdefault(k, {}).setdefault(c, []).append(v)
    # the calibration copies: the copyBuffer dispatches of the largest grid
    # (the others are small staging copies of host uploads)
    copies = [k for k in ctr if "copyBuffer" in k[0]]
    copy = [k for k in copies if int(k[1]) == max(int(c[1]) for c in copies)]
    kib = PROBE_COPY_BYTES / 1024.0
    f_fetch = kib / np.median([v for k in copy for v in ctr[k].get("FETCH_SIZE", [])])
    f_write = kib / np.median([v for k in copy for v in ctr[k].get("WRITE_SIZE", [])])
    roles = gemm_roles() if phase == "train" else {}
    print("calibration: copies of %d B; FETCH_SIZE x %.4f, WRITE_SIZE x %.4f" % (PROBE_COPY_BYTES, f_fetch, f_write))
    print("%-24s %-22s %9s %6s %9s %7s %9s %9s %8s %6s" % ("kernel", "role", "grid", "calls", "avg_us", "mfma%",
                                                          "fetch_MB", "write_MB", "GB/s", "%HBM"))
    for k, v in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        if k not in ctr or "copyBuffer" in k[0]:
            continue
        if phase == "decode" and not (k[0].startswith("k_dec_") or k[0].startswith("k_argmax") or
                                      k[0].startswith("k_sample")):
            continue
        c = {n: float(np.median(x)) for n, x in ctr[k].items()}
        avg = sum(v) / len(v) / 1e3
        busy = c["SQ_VALU_MFMA_BUSY_CYCLES"] / (32.0 * c["SQ_CYCLES"]) if c.get("SQ_CYCLES") else float("nan")
        fb = c.get("FETCH_SIZE", float("nan")) * 1024.0 * f_fetch / 1e6
        wb = c.get("WRITE_SIZE", float("nan")) * 1024.0 * f_write / 1e6
        gbs = (fb + wb) / avg * 1e3   # MB per us -> GB/s
        print("%-24s %-22s %9s %6d %9.2f %6.1f%% %9.2f %9.2f %8.0f %5.1f%%" % (
            k[0].replace("k_gemm_", "gemm_")[:24], roles.get(k, "")[:22], k[1], len(v), avg, 100.0 * busy, fb, wb,
            gbs, 100.0 * gbs / 8000.0))


def traffic_summarize(fetch_dir, write_dir):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the probe's copies and
    LM-head GEMMs; each counter is scaled by the factor that makes it read
    the copy's true size, and the LM head's scaled sum is its HBM traffic."""
    import csv
    import glob

    def per_kernel(d, counter):
        vals = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] != counter:
                    continue
                k = "copy" if "copyBuffer" in r["Kernel_Name"] else (
                    "head" if r["Kernel_Name"].startswith("k_gemm_nt") else None)
                if k:
                    vals.setdefault(k, {}).setdefault(r["Dispatch_Id"], 0.0)
                    vals[k][r["Dispatch_Id"]] += float(r["Counter_Value"])
        return {k: sorted(v.values()) for k, v in vals.items()}

    fe, wr = per_kernel(fetch_dir, "FETCH_SIZE"), per_kernel(write_dir, "WRITE_SIZE")
    kib = PROBE_COPY_BYTES / 1024.0
    f_fetch = kib / np.median(fe["copy"])
    f_write = kib / np.median(wr["copy"])
    head_f = np.median(fe["head"]) * f_fetch * 1024.0
    head_w = np.median(wr["head"]) * f_write * 1024.0
    M_, N_, K_ = M, V, D
    alg = 4.0 * (M_ * K_ + N_ * K_ + M_ * N_)
    print("copy calibration: FETCH_SIZE %.0f KiB -> factor %.4f; WRITE_SIZE %.0f KiB -> factor %.4f (copy of %d B)"
          % (np.median(fe["copy"]), f_fetch, np.median(wr["copy"]), f_write, PROBE_COPY_BYTES))
    print("lm_head_fwd per launch: FETCH %.1f MB, WRITE %.1f MB (scaled)" % (head_f / 1e6, head_w / 1e6))
    print("algorithmic bytes (A + B read once, C written once): %.1f MB" % (alg / 1e6))
    print("traffic_bytes %d" % int(head_f + head_w))


def traffic_bytes():
    """The LM-head forward's measured HBM bytes per launch, from the committed
    counter summary (null when it was not measured)."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes "):
                return int(line.split()[1])
    except OSError:
        pass
    return None


def main():
    if len(sys.argv) > 6 and sys.argv[1] == "--counter-summary":
        counter_summary(*sys.argv[2:7])
        return
    if len(sys.argv) > 3 and sys.argv[1] == "--traffic-summarize":
        traffic_summarize(sys.argv[2], sys.argv[3])
        return
    if len(sys.argv) > 2 and sys.argv[1] == "--summarize":
        summarize_profile(sys.argv[2])
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-model", action="store_true", help="skip the forward/training measurements")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-decode", action="store_true",
                    help="skip the config-5 decode leg (its replayed HIP graph does not run under "
                         "rocprofv3's kernel trace, which ends the process with SIGSEGV)")
    ap.add_argument("--model-only", action="store_true",
                    help="only the B8 T1024 forward/train measurements (for focused profiling); "
                         "prints them as a JSON line without the sweep")
    ap.add_argument("--tune", action="store_true",
                    help="time every GEMM tile variant / split-K factor on the sweep shapes and exit")
    ap.add_argument("--tune-out", default=None, help="with --tune: write every timing as JSON lines here")
    ap.add_argument("--decode-only", action="store_true", help="only the config-5 decode measurement (JSON line)")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="only the dispatches the FETCH_SIZE / WRITE_SIZE counter passes read")
    ap.add_argument("--counter-probe", choices=["train", "decode"], default=None,
                    help="the dispatches of a per-kernel counter table: calibration copies, then config 4 with "
                         "the side stream serialised (train) or config-5 decode steps at context ~1000 (decode)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: every box in this build has one GPU, and the multi-GPU design "
              "(RCCL data parallel over the gpu_ops worker slots) is not implemented. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    trlm = load_trlm()
    _, hip = trlm.libs()
    if args.tune:
        tune(trlm, hip, max(3, args.steps // 2), args.tune_out)
        return
    if args.decode_only:
        print(json.dumps(decode_benchmark(trlm)), flush=True)
        return
    if args.traffic_probe:
        traffic_probe(trlm)
        return
    if args.counter_probe:
        counter_probe(trlm, args.counter_probe)
        return
    if args.model_only:
        print(json.dumps(model_benchmarks(trlm, args.steps, max(6, args.warmup))), flush=True)
        return
    dev = trlm.Device()
    sweep = Sweep(trlm, dev)
    log("sweep: %d GEMMs, %.1f GFLOP per step" % (len(sweep.items), sweep.flops / 1e9))
    for _ in range(args.warmup):
        sweep.step()
    dev.sync()
    total_ms = time_events(hip, sweep.step, args.steps)
    per_gemm = {}
    variants = {}
    for it in sweep.items:
        ms = time_events(hip, lambda it=it: sweep.run(it), max(3, args.steps // 2))
        per_gemm[it[0]] = round(it[1] / (ms * 1e-3) / 1e12, 2)
        sweep.run(it)
        variants[it[0]] = "%s/split%d" % dev.last_variant()
    log("per-GEMM TFLOP/s: %s" % per_gemm)
    # dominant kernel: the LM-head forward GEMM, one launch = one kernel
    head = [it for it in sweep.items if it[0] == "lm_head_fwd"][0]
    head_ms = time_events(hip, lambda: sweep.run(head), max(5, args.steps))
    achieved = head[1] / (head_ms * 1e-3) / 1e12
    sweep.close()
    dev.close()

    value = sweep.flops / (total_ms * 1e-3) / 1e12
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(total_ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "fp32 GEMM sweep at model shapes (configs[1]): QKV, attn-out, gate_up, down, "
                               "LM head x (fwd, dX, dW), M=B*T=8192", "global_batch": B, "seq_len": T,
                   "parallelism": "single-gpu"},
        "pct_fp32_mfma_peak": round(100.0 * value / PEAK_FP32_MFMA, 2),
        "gemm_tflops": per_gemm, "gemm_variant": variants,
        "roofline": {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_MFMA, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP32_MFMA, 4), "traffic": traffic_bytes(),
                     "kernel": "%s (LM head fwd 8192x31769x384 NT)" % variants["lm_head_fwd"],
                     "launch_ms": round(head_ms, 4)},
    }
    if not args.no_model:
        log("model: forward / train at B=%d T=%d" % (B, T))
        # the clocks settle over the first few full-model steps: at least 6 untimed
        line.update({k: (round(v, 3) if isinstance(v, float) else v)
                     for k, v in model_benchmarks(trlm, max(3, args.steps // 2), max(6, args.warmup)).items()})
    if not args.no_model:
        log("hybrid path: tied head per generated token")
        line.update({k: (round(v, 3) if isinstance(v, float) else v) for k, v in hybrid_benchmarks(trlm).items()})
    if not args.no_model and not args.no_decode:
        log("decode: config 5")
        line.update({k: (round(v, 3) if isinstance(v, float) else v) for k, v in decode_benchmark(trlm).items()})
    if not args.no_cpu:
        log("cpu baseline leg: QKV GEMM through the reference's tensor_matmul2d")
        cb = cpu_baseline()
        line["cpu_baseline"] = {"value": cb["value"], "unit": cb["unit"], "cores": cb["cores"], "kind": cb["kind"],
                                "sample": cb["sample"]}
        line["cpu_host"] = host_cpu()
        line["gpu_vs_cpu_gemm"] = round(value / cb["value"], 1)
        if not args.no_model:
            log("cpu baseline: the reference's forward and training step at B=8 T=1024 (about 70 s)")
            ct = cpu_model_baseline()
            if ct is not None:
                line["cpu_model"] = {k: (round(v, 3) if isinstance(v, float) else v) for k, v in ct.items()
                                     if k != "pieces_s"}
                line["cpu_model"]["pieces_s"] = {k: round(v, 3) for k, v in ct["pieces_s"].items()}
                if "fwd_tokens_per_s" in line:
                    line["gpu_vs_cpu_forward"] = round(line["fwd_tokens_per_s"] / ct["fwd_tokens_per_s"], 1)
                if "train_tokens_per_s" in line:
                    line["gpu_vs_cpu_train"] = round(line["train_tokens_per_s"] / ct["train_tokens_per_s"], 1)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
