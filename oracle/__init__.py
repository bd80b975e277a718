"""ctypes front end of the CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module.  It loads oracle/liboracle.so (the C restatement of the
reference's fp32 CPU path, trlm_oracle.c) and, when it was built,
oracle/_ref/libtrlm_refh.so (a harness over the reference's own CPU sources,
ref_harness.c).
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libtrlm_ref.so")
REF_HARNESS = os.path.join(HERE, "_ref", "libtrlm_refh.so")

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")
u64p = np.ctypeslib.ndpointer(np.uint64, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")


class Cfg(C.Structure):
    """Model dimensions (V, D, H, L, F, eps) -- layout of OrCfg / RefCfg."""
    _fields_ = [("V", C.c_uint32), ("D", C.c_uint32), ("H", C.c_uint32),
                ("L", C.c_uint32), ("F", C.c_uint32), ("eps", C.c_float)]


class Pcg(C.Structure):
    _fields_ = [("state", C.c_uint64), ("inc", C.c_uint64),
                ("has_cached", C.c_uint32), ("cached", C.c_double)]


def build(ref_root="/root/reference", with_ref=True):
    """Compile liboracle.so, and oracle/_ref when the reference tree exists."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if with_ref and os.path.isdir(ref_root):
        subprocess.run(["make", "-s", "-C", HERE, "ref", "REF=" + ref_root], check=True)


def _load():
    if not os.path.exists(LIB):
        build(with_ref=False)
    lib = C.CDLL(LIB)
    cfgp = C.POINTER(Cfg)
    sig = {
        "or_m_sqrt": (C.c_double, [C.c_double]), "or_m_exp": (C.c_double, [C.c_double]),
        "or_m_log": (C.c_double, [C.c_double]), "or_m_pow": (C.c_double, [C.c_double, C.c_double]),
        "or_m_sin": (C.c_double, [C.c_double]), "or_m_cos": (C.c_double, [C.c_double]),
        "or_m_sqrtf": (C.c_float, [C.c_float]), "or_m_expf": (C.c_float, [C.c_float]),
        "or_m_logf": (C.c_float, [C.c_float]), "or_m_powf": (C.c_float, [C.c_float, C.c_float]),
        "or_m_sinf": (C.c_float, [C.c_float]), "or_m_cosf": (C.c_float, [C.c_float]),
        "or_pcg_seed": (None, [C.POINTER(Pcg), C.c_uint64, C.c_uint64]),
        "or_pcg_next_u32": (C.c_uint32, [C.POINTER(Pcg)]),
        "or_pcg_range_i64": (C.c_int64, [C.POINTER(Pcg), C.c_int64, C.c_int64]),
        "or_pcg_gaussian": (C.c_double, [C.POINTER(Pcg), C.c_double, C.c_double]),
        "or_num_params": (C.c_uint32, [cfgp]),
        "or_param_layout": (C.c_uint64, [cfgp, u64p, u64p]),
        "or_lm_init": (None, [cfgp, C.c_uint64, C.c_uint64, f32p]),
        "or_rope_tables": (None, [C.c_uint32, C.c_uint32, f32p, f32p]),
        "or_sample_batch": (None, [u32p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint64, u32p, u32p]),
        "or_matmul": (None, [C.c_uint32, C.c_uint32, C.c_uint32, f32p, C.c_int64, C.c_int64,
                             f32p, C.c_int64, C.c_int64, f32p]),
        "or_forward_logits": (None, [cfgp, f32p, u32p, C.c_uint32, C.c_uint32, f32p, C.c_int]),
        "or_forward_backward": (C.c_float, [cfgp, f32p, u32p, u32p, C.c_uint32, C.c_uint32,
                                            C.c_void_p, C.c_void_p, C.c_int]),
        "or_adam_step": (None, [f32p, f32p, f32p, f32p, C.c_uint64, C.c_uint64, C.c_float,
                                C.c_float, C.c_float, C.c_float, C.c_float, C.c_float]),
        "or_argmax": (C.c_uint32, [f32p, C.c_uint32]),
        "or_sample_next": (C.c_uint32, [f32p, C.c_uint32, C.c_float, C.POINTER(Pcg), f32p]),
        "or_lr_warmup_cosine": (C.c_float, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _threads():
    return max(1, min(16, os.cpu_count() or 1))


class Model:
    """A model configuration plus the oracle's flat parameter layout."""

    def __init__(self, V, D, H, L, F, eps=1e-5):
        self.cfg = Cfg(V, D, H, L, F, eps)
        self.V, self.D, self.H, self.L, self.F, self.eps = V, D, H, L, F, eps
        n = lib().or_num_params(C.byref(self.cfg))
        self.offsets = np.zeros(n, np.uint64)
        self.numels = np.zeros(n, np.uint64)
        self.total = int(lib().or_param_layout(C.byref(self.cfg), self.offsets, self.numels))
        self.num_params = n

    def shapes(self):
        """Per-tensor shapes in lm_collect_params order (lm_model.c:134-148)."""
        D, F = self.D, self.F
        out = [(self.V, D)]
        for _ in range(self.L):
            out += [(D,), (D, 3 * D), (3 * D,), (D, D), (D,), (D,), (D, 2 * F), (2 * F,), (F, D), (D,)]
        out.append((D,))
        return out

    def names(self):
        """Per-tensor names in lm_collect_params order (embed, l<i>.<kind>, final_norm)."""
        kinds = ["attn_norm", "w_qkv", "b_qkv", "wo", "bo", "ffn_norm", "w_gate_up", "b_gate_up", "w_down", "b_down"]
        return ["embed"] + ["l%d.%s" % (l, k) for l in range(self.L) for k in kinds] + ["final_norm"]

    def split(self, flat):
        return [flat[int(o):int(o) + int(n)].reshape(s)
                for o, n, s in zip(self.offsets, self.numels, self.shapes())]

    def init(self, seed_a=1337, seed_b=1):
        p = np.zeros(self.total, np.float32)
        lib().or_lm_init(C.byref(self.cfg), seed_a, seed_b, p)
        return p

    def forward_logits(self, params, ids, B, T, nthreads=None):
        out = np.zeros((B * T, self.V), np.float32)
        lib().or_forward_logits(C.byref(self.cfg), params, np.ascontiguousarray(ids, np.uint32),
                                B, T, out, nthreads or _threads())
        return out

    def forward_backward(self, params, ids, tgt, B, T, want_grads=True, nthreads=None):
        grads = np.zeros(self.total, np.float32) if want_grads else None
        rows = np.zeros(B * T, np.float32)
        loss = lib().or_forward_backward(
            C.byref(self.cfg), params, np.ascontiguousarray(ids, np.uint32),
            np.ascontiguousarray(tgt, np.uint32), B, T,
            grads.ctypes.data if grads is not None else None, rows.ctypes.data, nthreads or _threads())
        return np.float32(loss), grads, rows


def matmul(A, B):
    """Reference-order fp32 C = A @ B (tensor.c:351-373)."""
    A = np.ascontiguousarray(A, np.float32)
    B = np.ascontiguousarray(B, np.float32)
    M, K = A.shape
    N = B.shape[1]
    out = np.zeros((M, N), np.float32)
    lib().or_matmul(M, N, K, A, K, 1, B, N, 1, out)
    return out


def rope_tables(T, hd):
    c = np.zeros((T, hd // 2), np.float32)
    s = np.zeros((T, hd // 2), np.float32)
    lib().or_rope_tables(T, hd, c, s)
    return c, s


def sample_batch(tokens, T, B, seed_base):
    tokens = np.ascontiguousarray(tokens, np.uint32)
    ids = np.zeros(B * T, np.uint32)
    tgt = np.zeros(B * T, np.uint32)
    lib().or_sample_batch(tokens, len(tokens), T, B, seed_base, ids, tgt)
    return ids, tgt


def pcg_stream(seed_a, seed_b):
    r = Pcg()
    lib().or_pcg_seed(C.byref(r), seed_a, seed_b)
    return r


# ---- checkpoint TRLM v1 (training/checkpoint.h:6-12, checkpoint.c:22-137) ----
# [4 B "TRLM"][u32 version=1][u32 num_params][u32 has_opt]
# per parameter: [u32 ndim][ndim x u64 shape][numel x f32]
# if has_opt: per parameter [numel x f32 m][numel x f32 v], then [u64 t]
# Little-endian, as written by the x86-64 reference.

def trlm_bytes(shapes, params, m=None, v=None, t=0):
    """The bytes checkpoint_save writes for these flat buffers."""
    import struct
    has_opt = m is not None
    out = [b"TRLM", struct.pack("<III", 1, len(shapes), 1 if has_opt else 0)]
    off = 0
    p = np.ascontiguousarray(params, np.float32)
    for sh in shapes:
        n = int(np.prod(sh))
        out.append(struct.pack("<I", len(sh)) + struct.pack("<%dQ" % len(sh), *sh))
        out.append(p[off:off + n].tobytes())
        off += n
    if has_opt:
        mm, vv = np.ascontiguousarray(m, np.float32), np.ascontiguousarray(v, np.float32)
        off = 0
        for sh in shapes:
            n = int(np.prod(sh))
            out.append(mm[off:off + n].tobytes())
            out.append(vv[off:off + n].tobytes())
            off += n
        out.append(struct.pack("<Q", t))
    return b"".join(out)


def trlm_parse(data, shapes, want_opt):
    """checkpoint_load's validation and copy: (params, m, v, t) or None when
    the reference would return FALSE (bad magic/version/count, a shape that
    differs, a size that is not exactly the expected one, optimizer state
    asked for but absent)."""
    import struct
    if len(data) < 16 or data[:4] != b"TRLM":
        return None
    version, num, has_opt = struct.unpack_from("<III", data, 4)
    if version != 1 or num != len(shapes) or (want_opt and not has_opt):
        return None
    pos = 16
    offs = []
    total = 0
    for sh in shapes:
        if pos + 4 > len(data):
            return None
        nd = struct.unpack_from("<I", data, pos)[0]
        pos += 4
        if nd != len(sh):
            return None
        for d in sh:
            if pos + 8 > len(data) or struct.unpack_from("<Q", data, pos)[0] != d:
                return None
            pos += 8
        n = int(np.prod(sh))
        if pos + 4 * n > len(data):
            return None
        offs.append((pos, n))
        pos += 4 * n
        total += n
    opt_at = pos
    if has_opt:
        pos += 8 * total + 8
    if pos != len(data):
        return None
    params = np.concatenate([np.frombuffer(data, np.float32, n, o) for o, n in offs])
    if not want_opt:
        return params, None, None, None
    m, v = [], []
    pos = opt_at
    for _, n in offs:
        m.append(np.frombuffer(data, np.float32, n, pos)); pos += 4 * n
        v.append(np.frombuffer(data, np.float32, n, pos)); pos += 4 * n
    t = struct.unpack_from("<Q", data, pos)[0]
    return params, np.concatenate(m), np.concatenate(v), t


def lr_warmup_cosine(step, warmup, total, peak, min_lr):
    """The reference's learning-rate schedule (training/lr_schedule.c) as f32."""
    return np.float32(lib().or_lr_warmup_cosine(step, warmup, total, peak, min_lr))


def sample_next(row, temperature, pcg):
    """sample_next on one row of logits; pcg (a Pcg) advances by one draw."""
    row = np.ascontiguousarray(row, np.float32)
    scratch = np.zeros(row.size, np.float32)
    return int(lib().or_sample_next(row, row.size, temperature, C.byref(pcg), scratch))


def random_tokens(n, V, seed_a=4242, seed_b=7, hi_exclusive=None):
    """n token ids from pcg_range_i64(0, hi) (test_gpu_train.c:74-75 uses hi = V-1)."""
    r = pcg_stream(seed_a, seed_b)
    hi = V - 1 if hi_exclusive is None else hi_exclusive
    f = lib().or_pcg_range_i64
    return np.array([f(C.byref(r), 0, hi) for _ in range(n)], np.uint32)


def gaussian_array(n, seed_a, seed_b, std=1.0):
    r = pcg_stream(seed_a, seed_b)
    f = lib().or_pcg_gaussian
    return np.array([f(C.byref(r), 0.0, std) for _ in range(n)], np.float32)


def adam_step(p, g, m, v, t, lr, b1, b2, eps, wd=0.0, grad_scale=1.0):
    """In-place Adam/AdamW step; t is the step count after increment."""
    lib().or_adam_step(p, g, m, v, p.size, t, lr, b1, b2, eps, wd, grad_scale)


class RefCfg(Cfg):
    pass


class Reference:
    """The reference's own CPU path (oracle/_ref), when it was built here."""

    def __init__(self):
        if not (os.path.exists(REF_LIB) and os.path.exists(REF_HARNESS)):
            raise FileNotFoundError("oracle/_ref not built")
        self.h = C.CDLL(REF_HARNESS)
        h = self.h
        h.refh_open.restype = C.c_int
        h.refh_open.argtypes = [C.c_char_p]
        rc = h.refh_open(REF_LIB.encode())
        if rc != 0:
            raise RuntimeError("refh_open failed: %d" % rc)
        cfgp = C.POINTER(Cfg)
        h.refh_m.restype = C.c_double
        h.refh_m.argtypes = [C.c_int, C.c_double, C.c_double]
        h.refh_pcg_u32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32, u32p]
        h.refh_pcg_range.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_int64, C.c_uint32, i64p]
        h.refh_pcg_gauss.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32, f64p]
        h.refh_rope_tables.argtypes = [C.c_uint32, C.c_uint32, f32p, f32p]
        h.refh_lm_init.argtypes = [cfgp, C.c_uint64, C.c_uint64, f32p]
        h.refh_forward_logits.argtypes = [cfgp, f32p, u32p, C.c_uint32, C.c_uint32, f32p, C.c_int]
        h.refh_forward_backward.restype = C.c_float
        h.refh_forward_backward.argtypes = [cfgp, f32p, u32p, u32p, C.c_uint32, C.c_uint32,
                                            C.c_uint64, C.c_void_p, C.c_void_p, C.c_int]
        h.refh_adam_step.argtypes = [cfgp, f32p, f32p, f32p, f32p, C.c_uint64, C.c_float,
                                     C.c_float, C.c_float, C.c_float]
        h.refh_matmul.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p, f32p]
        h.refh_sample_batch.argtypes = [u32p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint64, u32p, u32p]
        h.refh_lr_schedule.argtypes = [C.c_uint64, C.c_uint32, C.c_uint64, C.c_uint64, C.c_float, C.c_float, f32p]
        h.refh_time_train_step.restype = C.c_double
        h.refh_time_train_step.argtypes = [cfgp, f32p, u32p, u32p, C.c_uint32, C.c_uint32,
                                           C.c_uint64, f32p, f32p, C.c_int]
        h.refh_time_forward.restype = C.c_double
        h.refh_time_forward.argtypes = [cfgp, f32p, u32p, C.c_uint32, C.c_uint32, f32p, C.c_int]
        h.refh_time_matmul.restype = C.c_double
        h.refh_checkpoint_save.restype = C.c_int
        h.refh_checkpoint_save.argtypes = [C.POINTER(RefCfg), f32p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_int,
                                           C.c_char_p]
        h.refh_checkpoint_save_init.restype = C.c_int
        h.refh_checkpoint_save_init.argtypes = [C.POINTER(RefCfg), C.c_uint64, C.c_uint64, C.c_char_p]
        h.refh_checkpoint_load.restype = C.c_int
        h.refh_checkpoint_load.argtypes = [C.POINTER(RefCfg), C.c_char_p, f32p, C.c_void_p, C.c_void_p,
                                           C.POINTER(C.c_uint64), C.c_int]
        h.refh_time_matmul.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p, f32p]
        h.refh_time_matmul_threads.restype = C.c_double
        h.refh_time_matmul_threads.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, f32p, f32p, f32p, C.c_int]
        h.refh_time_pieces.restype = C.c_int
        h.refh_time_pieces.argtypes = [cfgp, f32p, u32p, u32p, C.c_uint32, C.c_uint32, C.c_int, f64p]
        h.refh_time_adam.restype = C.c_double
        h.refh_time_adam.argtypes = [cfgp, f32p, f32p, C.c_int]

    def lm_init(self, model, seed_a=1337, seed_b=1):
        p = np.zeros(model.total, np.float32)
        self.h.refh_lm_init(C.byref(model.cfg), seed_a, seed_b, p)
        return p

    def forward_logits(self, model, params, ids, B, T, nthreads=None):
        out = np.zeros((B * T, model.V), np.float32)
        self.h.refh_forward_logits(C.byref(model.cfg), params, np.ascontiguousarray(ids, np.uint32),
                                   B, T, out, nthreads or _threads())
        return out

    def forward_backward(self, model, params, ids, tgt, B, T, nthreads=None):
        grads = np.zeros(model.total, np.float32)
        scratch = np.zeros(model.total * B, np.float32)
        loss = self.h.refh_forward_backward(C.byref(model.cfg), params, np.ascontiguousarray(ids, np.uint32),
                                            np.ascontiguousarray(tgt, np.uint32), B, T, model.total,
                                            grads.ctypes.data, scratch.ctypes.data, nthreads or _threads())
        return np.float32(loss), grads

    def adam_step(self, model, p, g, m, v, t_before, lr, b1, b2, eps):
        self.h.refh_adam_step(C.byref(model.cfg), p, g, m, v, t_before, lr, b1, b2, eps)

    def checkpoint_save(self, model, path, params, m=None, v=None, t=0):
        c = RefCfg(model.V, model.D, model.H, model.L, model.F, model.eps)
        has = m is not None
        mm = np.ascontiguousarray(m, np.float32) if has else None
        vv = np.ascontiguousarray(v, np.float32) if has else None
        return bool(self.h.refh_checkpoint_save(C.byref(c), np.ascontiguousarray(params, np.float32),
                                                mm.ctypes.data if has else None, vv.ctypes.data if has else None,
                                                t, int(has), path.encode()))

    def checkpoint_save_init(self, model, path, seed_a=1337, seed_b=1):
        c = RefCfg(model.V, model.D, model.H, model.L, model.F, model.eps)
        return bool(self.h.refh_checkpoint_save_init(C.byref(c), seed_a, seed_b, path.encode()))

    def checkpoint_load(self, model, path, total, want_opt):
        c = RefCfg(model.V, model.D, model.H, model.L, model.F, model.eps)
        p = np.zeros(total, np.float32)
        m = np.zeros(total, np.float32) if want_opt else None
        v = np.zeros(total, np.float32) if want_opt else None
        t = C.c_uint64(0)
        ok = self.h.refh_checkpoint_load(C.byref(c), path.encode(), p, m.ctypes.data if want_opt else None,
                                         v.ctypes.data if want_opt else None, C.byref(t), int(want_opt))
        return (p, m, v, t.value) if ok else None

    def sample_batch(self, tokens, T, B, seed_base):
        """gpu_trainer_sample_batch of the reference (model/gpu_train.c:296-307)."""
        tokens = np.ascontiguousarray(tokens, np.uint32)
        ids = np.zeros(B * T, np.uint32)
        tgt = np.zeros(B * T, np.uint32)
        self.h.refh_sample_batch(tokens, len(tokens), T, B, seed_base, ids, tgt)
        return ids, tgt

    def lr_schedule(self, first, n, warmup, total, peak, min_lr):
        out = np.zeros(n, np.float32)
        self.h.refh_lr_schedule(first, n, warmup, total, peak, min_lr, out)
        return out

    def matmul(self, A, B):
        A = np.ascontiguousarray(A, np.float32)
        B = np.ascontiguousarray(B, np.float32)
        out = np.zeros((A.shape[0], B.shape[1]), np.float32)
        self.h.refh_matmul(A.shape[0], B.shape[1], A.shape[1], A, B, out)
        return out


def reference_available():
    return os.path.exists(REF_LIB) and os.path.exists(REF_HARNESS)
