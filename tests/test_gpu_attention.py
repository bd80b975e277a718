"""The flash-attention kernels on their own, against float64 attention.

The trainer's parity tests reach these kernels only through whole training
steps.  Here k_attn_fwd, k_attn_dvec, k_attn_bwd_dkv and k_attn_bwd_dq are
launched as gpu_train.c launches them (grid (B*H, ceil(T/64)), 256 threads;
D over N*D/4 threads) on random Q, K, V, dO and compared with a float64
restatement of the reference's materialised attention
(train_kernels.cu:631-664: S = QK^T * scale, causal mask, softmax, O = PV;
backward dP = dO V^T, dS = P o (dP - rowsum(dO o O)), dQ = dS K * scale,
dK = dS^T Q * scale, dV = P^T dO).  With RoPE tables the backward stores dQ
and dK through the transpose of the rotation (model_ops.c:130-155), as the
trainer's fused path does.  Shapes: every head dim the kernels are built
for, T off the 64-row grid, T = 1, and a grid of more than 256 workgroups
(a partial second dispatch round of the snake order).  Tolerance per tensor:
|got - want| <= 1e-4 * max|want| + 1e-4 * |want| (test_gpu_train.c:53-66),
for dQ and dK plus 1e-5 times the same products on absolute values (at
T = 1 they are exactly 0 and float32 leaves ~1e-7 of cancellation); the
backward is bit-identical when run twice.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class AttnParams(C.Structure):
    _fields_ = [("qkv", C.c_void_p), ("out", C.c_void_p), ("O", C.c_void_p), ("dO", C.c_void_p),
                ("lse", C.c_void_p), ("dvec", C.c_void_p), ("B", C.c_int), ("T", C.c_int), ("H", C.c_int),
                ("D", C.c_int), ("ldq", C.c_int), ("ldo", C.c_int), ("scale", C.c_float),
                ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p), ("ds", C.c_void_p), ("jobs", C.c_void_p)]


def _reference(qkv, dO, B, T, H, HD, cos, sin):
    D = H * HD
    q64, o64 = qkv.astype(np.float64), dO.astype(np.float64)
    scale = 1.0 / np.sqrt(HD)
    O = np.zeros((B * T, D))
    lse = np.zeros(B * H * T)
    dqkv = np.zeros((B * T, 3 * D))
    mag = np.zeros((B * T, 3 * D))   # the same products on absolute values
    mask = np.triu(np.ones((T, T), bool), 1)
    for b in range(B):
        rows = slice(b * T, (b + 1) * T)
        for h in range(H):
            q = q64[rows, h * HD:(h + 1) * HD]
            k = q64[rows, D + h * HD:D + (h + 1) * HD]
            v = q64[rows, 2 * D + h * HD:2 * D + (h + 1) * HD]
            s = q @ k.T * scale
            s[mask] = -np.inf
            m = s.max(1, keepdims=True)
            e = np.exp(s - m)
            l = e.sum(1, keepdims=True)
            p = e / l
            o = p @ v
            O[rows, h * HD:(h + 1) * HD] = o
            lse[(b * H + h) * T:(b * H + h + 1) * T] = (m[:, 0] + np.log(l[:, 0])) / np.log(2.0)
            do = o64[rows, h * HD:(h + 1) * HD]
            dp = do @ v.T
            ds = p * (dp - (do * o).sum(1, keepdims=True))
            dq, dk, dv = ds @ k * scale, ds.T @ q * scale, p.T @ do
            dsm = p * (np.abs(dp) + np.abs((do * o).sum(1, keepdims=True)))
            dqm, dkm = dsm @ np.abs(k) * scale, dsm.T @ np.abs(q) * scale
            if cos is not None:
                c, sn = cos.astype(np.float64), sin.astype(np.float64)
                for g in (dq, dk):
                    a0, a1 = g[:, 0::2].copy(), g[:, 1::2].copy()
                    g[:, 0::2] = a0 * c + a1 * sn
                    g[:, 1::2] = -a0 * sn + a1 * c
                for g in (dqm, dkm):
                    t = g[:, 0::2] + g[:, 1::2]
                    g[:, 0::2] = t
                    g[:, 1::2] = t
            mag[rows, h * HD:(h + 1) * HD] = dqm
            mag[rows, D + h * HD:D + (h + 1) * HD] = dkm
            dqkv[rows, h * HD:(h + 1) * HD] = dq
            dqkv[rows, D + h * HD:D + (h + 1) * HD] = dk
            dqkv[rows, 2 * D + h * HD:2 * D + (h + 1) * HD] = dv
    return O, lse, dqkv, mag


def _check(name, got, want, mag=None):
    err = np.abs(got.astype(np.float64) - want)
    bound = 1e-4 * np.abs(want).max() + 1e-4 * np.abs(want)
    if mag is not None:
        # dQ and dK come out of dP - rowsum(dO o O), which cancels exactly
        # when a row attends to one key (T = 1): float32 rounding is then
        # measured against the terms' own size
        bound = bound + 1e-5 * mag
    worst = float((err - bound).max())
    print("%-5s max|got-want| %.3e  max|want| %.3e" % (name, float(err.max()), float(np.abs(want).max())))
    assert worst <= 0.0, (name, float(err.max()))


CASES = [
    dict(B=2, H=3, T=200, HD=64, rope=True),
    dict(B=1, H=2, T=64, HD=32, rope=False),
    dict(B=3, H=4, T=77, HD=16, rope=True),
    dict(B=2, H=1, T=1, HD=64, rope=False),
    dict(B=8, H=6, T=384, HD=64, rope=True),    # 288 workgroups
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B%dH%dT%dhd%d%s" % (c["B"], c["H"], c["T"], c["HD"],
                                                                        "rope" if c["rope"] else ""))
def test_attention_kernels_match_float64(trlm, case):
    B, H, T, HD = case["B"], case["H"], case["T"], case["HD"]
    D, N, nqb = H * HD, B * T, (T + 63) // 64
    print("attention case", case, flush=True)
    rng = np.random.default_rng(1000 + T + HD)
    qkv = (0.5 * rng.standard_normal((N, 3 * D))).astype(np.float32)
    dO = rng.standard_normal((N, D)).astype(np.float32)
    cos = sin = None
    if case["rope"]:
        ang = rng.uniform(0.0, 6.3, (T, HD // 2))
        cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    want_O, want_lse, want_d, mag = _reference(qkv, dO, B, T, H, HD, cos, sin)

    dev = trlm.Device()
    try:
        k = lambda n: dev.hip.hip_get_kernel(C.byref(dev.ctx), n.encode())
        dq_, ddo = dev.upload(qkv), dev.upload(dO)
        dOut, dlse, ddv = dev.empty(N * D * 4), dev.empty(B * H * T * 4), dev.empty(B * H * T * 4)
        dds = dev.empty(B * H * nqb * (nqb + 1) // 2 * 4096 * 4)
        dgrad = [dev.empty(N * 3 * D * 4) for _ in range(2)]
        rc = dev.upload(cos) if cos is not None else None
        rs = dev.upload(sin) if sin is not None else None

        def launch(name, p, gx, gy):
            args = (C.c_void_p * 1)(C.cast(C.pointer(p), C.c_void_p))
            dev.hip.hip_launch(k(name), gx, gy, 1, 256, 1, 1, 0, args)

        common = dict(B=B, T=T, H=H, D=D, ldq=3 * D, ldo=D, scale=float(1.0 / np.sqrt(HD)))
        pf = AttnParams(qkv=dq_, out=dOut, lse=dlse, **common)
        launch("k_attn_fwd_hd%d" % HD, pf, B * H, nqb)
        got_O = dev.download(dOut, (N, D))
        got_lse = dev.download(dlse, (B * H * T,))
        grads = []
        for out in dgrad:
            pb = AttnParams(qkv=dq_, out=out, O=dOut, dO=ddo, lse=dlse, dvec=ddv, ds=dds, rope_cos=rc, rope_sin=rs,
                            **common)
            launch("k_attn_dvec_hd%d" % HD, pb, (N * D // 4 + 255) // 256, 1)
            launch("k_attn_bwd_dkv_hd%d" % HD, pb, B * H, nqb)
            launch("k_attn_bwd_dq_hd%d" % HD, pb, B * H, nqb)
            grads.append(dev.download(out, (N, 3 * D)))
    finally:
        dev.close()

    _check("O", got_O, want_O)
    _check("lse", got_lse, want_lse)
    _check("dQ", grads[0][:, :D], want_d[:, :D], mag[:, :D])
    _check("dK", grads[0][:, D:2 * D], want_d[:, D:2 * D], mag[:, D:2 * D])
    _check("dV", grads[0][:, 2 * D:], want_d[:, 2 * D:])
    assert np.array_equal(grads[0].view(np.uint32), grads[1].view(np.uint32))


@pytest.mark.parametrize("B,H,T", [(8, 6, 1024), (2, 3, 200)])
def test_forward_job_placement_keeps_bits(trlm, B, H, T):
    """The forward's job placement (AttnParams.jobs) changes which workgroup
    takes which (query block, head), never what it computes: O and the
    log-sum-exp are the same bits in the kernel's own snake order, with the
    library's balanced table (trlm_attn_job_table; B8 T1024 is its 48-head,
    16-block, 256-unit case) and with a random permutation of the jobs."""
    HD = 64
    D, N, nqb = H * HD, B * T, (T + 63) // 64
    print("job placement case B%d H%d T%d" % (B, H, T), flush=True)
    rng = np.random.default_rng(77 + T)
    qkv = (0.5 * rng.standard_normal((N, 3 * D))).astype(np.float32)
    tables = [None]
    if B * H == 48 and nqb == 16:
        t = (C.c_int32 * (B * H * nqb))()
        assert trlm.libs()[1].trlm_attn_job_table(B * H, nqb, 256, 8, t) == 1
        tables.append(np.frombuffer(t, dtype=np.int32).copy())
    perm = rng.permutation(B * H * nqb)
    tables.append(((perm // (B * H)) << 16 | (perm % (B * H))).astype(np.int32))
    dev = trlm.Device()
    try:
        f = dev.hip.hip_get_kernel(C.byref(dev.ctx), b"k_attn_fwd_hd64")
        dq_ = dev.upload(qkv)
        outs = []
        for tab in tables:
            dOut, dlse = dev.empty(N * D * 4), dev.empty(B * H * T * 4)
            djobs = dev.upload(tab) if tab is not None else None
            p = AttnParams(qkv=dq_, out=dOut, lse=dlse, B=B, T=T, H=H, D=D, ldq=3 * D, ldo=D,
                           scale=float(1.0 / np.sqrt(HD)), jobs=djobs)
            args = (C.c_void_p * 1)(C.cast(C.pointer(p), C.c_void_p))
            dev.hip.hip_launch(f, B * H, nqb, 1, 256, 1, 1, 0, args)
            outs.append((dev.download(dOut, (N, D)), dev.download(dlse, (B * H * T,))))
    finally:
        dev.close()
    for O, lse in outs[1:]:
        assert np.array_equal(O.view(np.uint32), outs[0][0].view(np.uint32))
        assert np.array_equal(lse.view(np.uint32), outs[0][1].view(np.uint32))
