"""Python front end of the MI355X GPU path: a ctypes binding of the C ABI.

The product is the C library (libtrlm_hip.so, declared in include/*.h) and
its gfx950 code object; this module only binds it, mirrors the host
structures its signatures take (layout-checked against the C side by
trlm_host_layout), and offers numpy conveniences for building an LMModel and
reading gradients back.  It never falls back to a CPU computation: if the
built libraries are missing it raises.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_HIP = os.path.join(HERE, "libtrlm_hip.so")
LIB_HOST = os.path.join(HERE, "libtrlm_host.so")
KERNELS = os.path.join(HERE, "trlm_kernels.hsaco")

f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")

LM_MAX_LAYERS = 32


class Tensor(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_float)), ("shape", C.c_uint64 * 6), ("strides", C.c_int64 * 6),
                ("ndim", C.c_uint32), ("numel", C.c_uint64), ("owns_data", C.c_uint32)]


class Node(C.Structure):
    pass


Node._fields_ = [("value", Tensor), ("grad", Tensor), ("requires_grad", C.c_uint32),
                 ("parents", C.POINTER(Node) * 3), ("num_parents", C.c_uint32), ("backward_fn", C.c_void_p),
                 ("visited", C.c_uint32), ("aux_dim0", C.c_uint32), ("aux_dim1", C.c_uint32),
                 ("aux_scalar", C.c_float), ("aux_ptr", C.c_void_p)]

NodeP = C.POINTER(Node)


class AttentionWeights(C.Structure):
    _fields_ = [("w_qkv", NodeP), ("b_qkv", NodeP), ("wo", NodeP), ("bo", NodeP)]


class FeedForwardWeights(C.Structure):
    _fields_ = [("w_gate_up", NodeP), ("b_gate_up", NodeP), ("w_down", NodeP), ("b_down", NodeP)]


class BlockWeights(C.Structure):
    _fields_ = [("attn_norm_w", NodeP), ("attn", AttentionWeights), ("ffn_norm_w", NodeP),
                ("ffn", FeedForwardWeights)]


class LMModel(C.Structure):
    _fields_ = [("embed_table", NodeP), ("blocks", BlockWeights * LM_MAX_LAYERS), ("final_norm_w", NodeP),
                ("num_layers", C.c_uint32), ("num_heads", C.c_uint32), ("d_model", C.c_uint32),
                ("vocab_size", C.c_uint32), ("eps", C.c_float)]


class AdamOptimizer(C.Structure):
    _fields_ = [("params", C.POINTER(NodeP)), ("m", C.POINTER(Tensor)), ("v", C.POINTER(Tensor)),
                ("num_params", C.c_uint32), ("t", C.c_uint64), ("lr", C.c_float), ("beta1", C.c_float),
                ("beta2", C.c_float), ("eps", C.c_float)]


class Arena(C.Structure):
    _fields_ = [("base", C.c_void_p), ("reserved", C.c_uint64), ("committed", C.c_uint64), ("used", C.c_uint64)]


class Allocator(C.Structure):
    _fields_ = [("backing", Arena), ("free_list", C.c_void_p), ("last_phys", C.c_void_p)]


class PCGState(C.Structure):
    _fields_ = [("state", C.c_uint64), ("inc", C.c_uint64), ("has_cached_gaussian", C.c_uint32),
                ("cached_gaussian", C.c_double)]


class HipCtx(C.Structure):
    _fields_ = [("device", C.c_int32), ("module", C.c_void_p), ("stream", C.c_void_p), ("allocs", C.c_void_p),
                ("side", C.c_void_p)]


class TrlmTimer(C.Structure):
    _fields_ = [("start", C.c_void_p), ("stop", C.c_void_p)]


class TrlmSchedule(C.Structure):
    """Mirror of TrlmSchedule (trlm_ext.h): the driver loop's lr schedule,
    clip, weight decay and batch seed base."""
    _fields_ = [("warmup_steps", C.c_uint64), ("total_steps", C.c_uint64), ("peak_lr", C.c_float),
                ("min_lr", C.c_float), ("grad_clip", C.c_double), ("weight_decay", C.c_float),
                ("seed_base", C.c_uint64)]


_libs = None


def built():
    return all(os.path.exists(p) for p in (LIB_HIP, LIB_HOST, KERNELS))


def libs():
    """(host, hip) ctypes libraries; raises if the build outputs are missing."""
    global _libs
    if _libs is not None:
        return _libs
    if not built():
        raise FileNotFoundError("MI355X path not built: run __graft_entry__.build() (missing %s)" %
                                ", ".join(p for p in (LIB_HIP, LIB_HOST, KERNELS) if not os.path.exists(p)))
    host = C.CDLL(LIB_HOST, mode=C.RTLD_GLOBAL)
    hip = C.CDLL(LIB_HIP, mode=C.RTLD_GLOBAL)
    _bind(host, hip)
    _libs = (host, hip)
    return _libs


def _sig(lib, name, res, args):
    fn = getattr(lib, name)
    fn.restype = res
    fn.argtypes = args


def _bind(host, hip):
    AP = C.POINTER(Allocator)
    _sig(host, "allocator_create", Allocator, [C.c_uint64])
    _sig(host, "allocator_alloc", C.c_void_p, [AP, C.c_uint64])
    _sig(host, "allocator_destroy", None, [AP])
    _sig(host, "tensor_create", Tensor, [AP, C.POINTER(C.c_uint64), C.c_uint32])
    _sig(host, "tensor_transpose", Tensor, [C.POINTER(Tensor), C.c_uint32, C.c_uint32])
    _sig(host, "node_leaf", NodeP, [AP, Tensor, C.c_uint32])
    _sig(host, "backward", None, [AP, NodeP])
    _sig(host, "pcg_seed", PCGState, [C.c_uint64, C.c_uint64])
    _sig(host, "pcg_next_u32", C.c_uint32, [C.POINTER(PCGState)])
    _sig(host, "pcg_range_i64", C.c_int64, [C.POINTER(PCGState), C.c_int64, C.c_int64])
    _sig(host, "pcg_gaussian", C.c_double, [C.POINTER(PCGState), C.c_double, C.c_double])
    for n in ("m_sqrt", "m_exp", "m_log", "m_sin", "m_cos"):
        _sig(host, n, C.c_double, [C.c_double])
    _sig(host, "m_pow", C.c_double, [C.c_double, C.c_double])
    _sig(host, "m_powf", C.c_float, [C.c_float, C.c_float])
    _sig(host, "m_sqrtf", C.c_float, [C.c_float])
    _sig(host, "m_sinf", C.c_float, [C.c_float])
    _sig(host, "m_cosf", C.c_float, [C.c_float])
    _sig(host, "rope_build_tables", None, [C.POINTER(Tensor), C.POINTER(Tensor), C.c_uint64, C.c_uint64,
                                          C.c_float])
    _sig(host, "trlm_host_layout", None, [C.POINTER(C.c_uint64)])

    _sig(hip, "trlm_version", C.c_char_p, [])
    _sig(hip, "trlm_sizeof_gpu_trainer", C.c_uint64, [])
    _sig(hip, "trlm_sizeof_hip_ctx", C.c_uint64, [])
    global GpuTrainer
    n = hip.trlm_sizeof_gpu_trainer()
    GpuTrainer = type("GpuTrainer", (C.Structure,), {"_fields_": [("raw", C.c_uint64 * (n // 8))]})
    GP = C.POINTER(GpuTrainer)
    _sig(hip, "gpu_trainer_create", GpuTrainer, [AP, C.c_char_p, C.POINTER(LMModel), C.POINTER(NodeP),
                                                 C.c_uint32, C.c_uint32, C.c_uint32])
    _sig(hip, "gpu_trainer_destroy", None, [GP])
    _sig(hip, "gpu_trainer_upload", None, [GP, C.POINTER(NodeP), C.POINTER(AdamOptimizer)])
    _sig(hip, "gpu_trainer_download", None, [GP, C.POINTER(NodeP), C.POINTER(AdamOptimizer)])
    _sig(hip, "gpu_trainer_download_grads", None, [GP, C.POINTER(NodeP)])
    _sig(hip, "gpu_trainer_upload_grads", None, [GP, C.POINTER(NodeP)])
    _sig(hip, "gpu_trainer_sample_batch", None, [u32p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint64, u32p,
                                                 u32p])
    _sig(hip, "gpu_trainer_forward_backward", C.c_float, [GP, u32p, u32p])
    _sig(hip, "gpu_trainer_eval_loss", C.c_float, [GP, u32p, u32p])
    _sig(hip, "gpu_trainer_grad_norm", C.c_double, [GP])
    _sig(hip, "gpu_trainer_adam_step", None, [GP, C.POINTER(AdamOptimizer)])
    _sig(hip, "gpu_trainer_adam_step_scaled", None, [GP, C.POINTER(AdamOptimizer), C.c_float])
    _sig(hip, "gpu_trainer_adamw_step_scaled", None, [GP, C.POINTER(AdamOptimizer), C.c_float, C.c_float])
    _sig(hip, "gpu_trainer_forward_logits", None, [GP, u32p, C.c_void_p])
    _sig(hip, "gpu_trainer_forward_loss_logits", C.c_float, [GP, u32p, u32p, C.c_void_p])
    _sig(hip, "gpu_trainer_greedy_argmax", None, [GP, u32p])
    _sig(hip, "gpu_trainer_gemm_engine", C.c_void_p, [GP])
    ckpt_args = [GP, C.c_char_p, C.POINTER(NodeP), C.POINTER(AdamOptimizer)]
    _sig(hip, "gpu_trainer_checkpoint_save", C.c_uint32, ckpt_args)
    _sig(hip, "gpu_trainer_checkpoint_load", C.c_uint32, ckpt_args)
    _sig(hip, "gpu_trainer_train_steps", None, [GP, C.POINTER(AdamOptimizer), u32p, C.c_uint64,
                                                C.POINTER(TrlmSchedule), C.c_uint64, C.c_uint32, C.c_void_p,
                                                C.c_void_p, C.c_void_p])
    _sig(hip, "gpu_trainer_eval_windows", C.c_float, [GP, u32p, C.c_uint64, C.c_uint64, C.c_uint32])
    _sig(hip, "trlm_lr_warmup_cosine", C.c_float, [C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_float])
    DP = C.c_void_p
    f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
    _sig(hip, "gpu_decoder_create", DP, [GP, C.c_uint32, C.c_uint32])
    _sig(hip, "gpu_decoder_destroy", None, [DP])
    _sig(hip, "gpu_decoder_prefill", None, [DP, u32p, C.c_uint32])
    _sig(hip, "gpu_decoder_step", None, [DP, u32p])
    _sig(hip, "gpu_decoder_length", C.c_uint32, [DP])
    _sig(hip, "gpu_decoder_logits", None, [DP, f32p])
    _sig(hip, "gpu_decoder_greedy", None, [DP, u32p])
    _sig(hip, "gpu_decoder_sample", None, [DP, C.POINTER(PCGState), C.c_float, u32p])
    _sig(hip, "gpu_decoder_generate_greedy", None, [DP, u32p, C.c_uint32, C.c_uint32, u32p])
    _sig(hip, "gpu_decoder_generate_sampled", None, [DP, u32p, C.c_uint32, C.c_uint32, C.POINTER(PCGState),
                                                     C.c_float, u32p])

    HP = C.POINTER(HipCtx)
    _sig(hip, "hip_init", HipCtx, [AP, C.c_char_p])
    _sig(hip, "hip_device_count", C.c_int32, [])
    _sig(hip, "hip_shutdown", None, [HP])
    _sig(hip, "hip_side_serial", None, [C.c_int32])
    _sig(hip, "hip_set_current", None, [HP])
    _sig(hip, "hip_get_kernel", C.c_void_p, [HP, C.c_char_p])
    _sig(hip, "hip_alloc", C.c_void_p, [C.c_uint64])
    _sig(hip, "hip_free", None, [C.c_void_p])
    _sig(hip, "hip_h2d", None, [C.c_void_p, C.c_void_p, C.c_uint64])
    _sig(hip, "hip_d2h", None, [C.c_void_p, C.c_void_p, C.c_uint64])
    _sig(hip, "hip_launch", None, [C.c_void_p] + [C.c_uint32] * 7 + [C.POINTER(C.c_void_p)])
    _sig(hip, "hip_memset_zero", None, [C.c_void_p, C.c_uint64])
    _sig(hip, "hip_sync", None, [])
    _sig(hip, "trlm_gemm_create", C.c_void_p, [HP])
    _sig(hip, "trlm_gemm_destroy", None, [C.c_void_p])
    _sig(hip, "trlm_gemm", None, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p, C.c_void_p,
                                  C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                  C.c_uint32, C.c_int64, C.c_int64, C.c_int64, C.c_float, C.c_float,
                                  C.c_void_p, C.c_void_p, C.c_int32])
    _sig(hip, "trlm_gemm_noalloc", C.c_int32, [C.c_void_p, C.c_int32, C.c_int32, C.c_void_p, C.c_void_p,
                                              C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32,
                                              C.c_int32, C.c_uint32, C.c_int64, C.c_int64, C.c_int64, C.c_float,
                                              C.c_float, C.c_void_p, C.c_void_p, C.c_int32])
    _sig(hip, "trlm_gemm_last_variant", C.c_char_p, [C.c_void_p, C.POINTER(C.c_int32)])
    _sig(hip, "trlm_gemm_plan", C.c_char_p, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_uint32,
                                             C.POINTER(C.c_int32)])
    _sig(hip, "trlm_gemm_force", C.c_int32, [C.c_void_p, C.c_char_p, C.c_int32])
    _sig(hip, "trlm_attn_job_table", C.c_int32, [C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                                 C.POINTER(C.c_int32)])
    TP = C.POINTER(TrlmTimer)
    _sig(hip, "trlm_timer_create", None, [TP])
    _sig(hip, "trlm_timer_destroy", None, [TP])
    _sig(hip, "trlm_timer_start", None, [TP])
    _sig(hip, "trlm_timer_stop_ms", C.c_float, [TP])
    _sig(hip, "gpu_ops_init", None, [AP, C.c_char_p])
    _sig(hip, "gpu_ops_init_workers", None, [AP, C.c_char_p, C.c_uint32])
    _sig(hip, "gpu_ops_shutdown", None, [])
    _sig(hip, "gpu_ops_set_worker_id", None, [C.c_int32])
    _sig(hip, "node_matmul2d_gpu", NodeP, [AP, NodeP, NodeP])
    _sig(hip, "gpu_ops_debug_stats", None, [C.POINTER(C.c_double), C.POINTER(C.c_uint32)])
    _sig(hip, "gpu_ops_debug_reset", None, [])
    _sig(hip, "gpu_ops_pin", None, [C.c_void_p, C.c_uint64])
    _sig(hip, "gpu_ops_unpin_all", None, [])


GpuTrainer = None


def check_layout():
    """Compare this module's structure mirrors with the C compiler's layout."""
    host, _ = libs()
    out = (C.c_uint64 * 12)()
    host.trlm_host_layout(out)
    want = [C.sizeof(Tensor), C.sizeof(Node), Node.backward_fn.offset, Node.aux_ptr.offset, C.sizeof(LMModel),
            LMModel.final_norm_w.offset, LMModel.eps.offset, C.sizeof(AdamOptimizer), AdamOptimizer.t.offset,
            C.sizeof(Allocator), C.sizeof(PCGState), Tensor.numel.offset]
    return list(out) == want, list(out), want


# ---------------------------------------------------------------- helpers

def tensor_np(t, n=None):
    """numpy view of a contiguous Tensor's data."""
    n = int(t.numel) if n is None else n
    return np.ctypeslib.as_array(t.data, shape=(n,))


class HostModel:
    """An LMModel whose parameter Nodes live in a host Allocator and hold
    copies of a flat fp32 parameter buffer (lm_collect_params order)."""

    def __init__(self, V, D, H, L, F, flat_params, eps=1e-5, arena_bytes=None):
        host, _ = libs()
        self.V, self.D, self.H, self.L, self.F = V, D, H, L, F
        shapes = [(V, D)]
        for _ in range(L):
            shapes += [(D,), (D, 3 * D), (3 * D,), (D, D), (D,), (D,), (D, 2 * F), (2 * F,), (F, D), (D,)]
        shapes.append((D,))
        self.shapes = shapes
        total = sum(int(np.prod(s)) for s in shapes)
        assert flat_params.size == total, (flat_params.size, total)
        need = arena_bytes or (total * 4 * 48 + (V + 1) * 4 * 4 + (1 << 28))
        self.alloc = host.allocator_create(need)
        self.nodes = (NodeP * len(shapes))()
        off = 0
        for i, s in enumerate(shapes):
            shp = (C.c_uint64 * 2)(*s) if len(s) == 2 else (C.c_uint64 * 1)(*s)
            t = host.tensor_create(C.byref(self.alloc), shp, len(s))
            n = int(np.prod(s))
            tensor_np(t)[:] = flat_params[off:off + n]
            self.nodes[i] = host.node_leaf(C.byref(self.alloc), t, 1)
            off += n
        m = LMModel()
        m.embed_table = self.nodes[0]
        for l in range(L):
            b = m.blocks[l]
            k = 1 + 10 * l
            b.attn_norm_w = self.nodes[k]
            b.attn.w_qkv, b.attn.b_qkv, b.attn.wo, b.attn.bo = [self.nodes[k + j] for j in (1, 2, 3, 4)]
            b.ffn_norm_w = self.nodes[k + 5]
            b.ffn.w_gate_up, b.ffn.b_gate_up, b.ffn.w_down, b.ffn.b_down = [self.nodes[k + j] for j in (6, 7, 8, 9)]
        m.final_norm_w = self.nodes[1 + 10 * L]
        m.num_layers, m.num_heads, m.d_model, m.vocab_size, m.eps = L, H, D, V, eps
        self.model = m
        self.num_params = len(shapes)
        self.total = total

    def values(self):
        return np.concatenate([tensor_np(self.nodes[i].contents.value).copy() for i in range(self.num_params)])

    def grads(self):
        return np.concatenate([tensor_np(self.nodes[i].contents.grad).copy() for i in range(self.num_params)])

    def set_values(self, flat):
        off = 0
        for i in range(self.num_params):
            a = tensor_np(self.nodes[i].contents.value)
            a[:] = flat[off:off + a.size]
            off += a.size

    def set_grads(self, flat):
        off = 0
        for i in range(self.num_params):
            a = tensor_np(self.nodes[i].contents.grad)
            a[:] = flat[off:off + a.size]
            off += a.size

    def close(self):
        host, _ = libs()
        host.allocator_destroy(C.byref(self.alloc))


class Adam:
    """An AdamOptimizer over a HostModel's parameters with numpy-backed m/v."""

    def __init__(self, hm, lr=3e-4, b1=0.9, b2=0.999, eps=1e-8):
        host, _ = libs()
        self.hm = hm
        n = hm.num_params
        self.m_arr = (Tensor * n)()
        self.v_arr = (Tensor * n)()
        for i in range(n):
            s = hm.shapes[i]
            shp = (C.c_uint64 * len(s))(*s)
            self.m_arr[i] = host.tensor_create(C.byref(hm.alloc), shp, len(s))
            self.v_arr[i] = host.tensor_create(C.byref(hm.alloc), shp, len(s))
            tensor_np(self.m_arr[i])[:] = 0
            tensor_np(self.v_arr[i])[:] = 0
        self.opt = AdamOptimizer(hm.nodes, self.m_arr, self.v_arr, n, 0, lr, b1, b2, eps)

    def flat(self, which):
        arr = self.m_arr if which == "m" else self.v_arr
        return np.concatenate([tensor_np(arr[i]).copy() for i in range(self.hm.num_params)])

    def set_flat(self, which, flat):
        arr = self.m_arr if which == "m" else self.v_arr
        off = 0
        for i in range(self.hm.num_params):
            a = tensor_np(arr[i])
            a[:] = flat[off:off + a.size]
            off += a.size


class Trainer:
    """gpu_trainer_* through the C ABI for one HostModel."""

    def __init__(self, hm, B, T, image=KERNELS):
        _, hip = libs()
        self.hip = hip
        self.hm = hm
        self.B, self.T = B, T
        self.g = hip.gpu_trainer_create(C.byref(hm.alloc), image.encode(), C.byref(hm.model), hm.nodes,
                                        hm.num_params, B, T)

    def forward_backward(self, ids, tgt):
        return self.hip.gpu_trainer_forward_backward(C.byref(self.g), _u32(ids), _u32(tgt))

    def eval_loss(self, ids, tgt):
        return self.hip.gpu_trainer_eval_loss(C.byref(self.g), _u32(ids), _u32(tgt))

    def grads(self):
        self.hip.gpu_trainer_download_grads(C.byref(self.g), self.hm.nodes)
        return self.hm.grads()

    def upload_grads(self, flat):
        self.hm.set_grads(flat)
        self.hip.gpu_trainer_upload_grads(C.byref(self.g), self.hm.nodes)

    def upload(self, adam=None):
        self.hip.gpu_trainer_upload(C.byref(self.g), self.hm.nodes, C.byref(adam.opt) if adam else None)

    def download(self, adam=None):
        self.hip.gpu_trainer_download(C.byref(self.g), self.hm.nodes, C.byref(adam.opt) if adam else None)
        return self.hm.values()

    def grad_norm(self):
        return self.hip.gpu_trainer_grad_norm(C.byref(self.g))

    def adam_step(self, adam, scale=None):
        if scale is None:
            self.hip.gpu_trainer_adam_step(C.byref(self.g), C.byref(adam.opt))
        else:
            self.hip.gpu_trainer_adam_step_scaled(C.byref(self.g), C.byref(adam.opt), scale)

    def adamw_step(self, adam, wd, scale=1.0):
        self.hip.gpu_trainer_adamw_step_scaled(C.byref(self.g), C.byref(adam.opt), wd, scale)

    def checkpoint_save(self, path, adam=None):
        return bool(self.hip.gpu_trainer_checkpoint_save(C.byref(self.g), path.encode(), self.hm.nodes,
                                                         C.byref(adam.opt) if adam else None))

    def checkpoint_load(self, path, adam=None):
        return bool(self.hip.gpu_trainer_checkpoint_load(C.byref(self.g), path.encode(), self.hm.nodes,
                                                         C.byref(adam.opt) if adam else None))

    def train_steps(self, adam, tokens, schedule, first_step, n_steps):
        """Steps first_step .. first_step+n_steps-1 of the driver loop;
        returns (losses f32[n], grad_norms f64[n], lrs f32[n])."""
        losses = np.zeros(n_steps, np.float32)
        norms = np.zeros(n_steps, np.float64)
        lrs = np.zeros(n_steps, np.float32)
        tok = _u32(tokens)
        self.hip.gpu_trainer_train_steps(C.byref(self.g), C.byref(adam.opt), tok, tok.size, C.byref(schedule),
                                         first_step, n_steps, losses.ctypes.data, norms.ctypes.data,
                                         lrs.ctypes.data)
        return losses, norms, lrs

    def eval_windows(self, tokens, train_tokens, val_tokens, val_batches):
        return np.float32(self.hip.gpu_trainer_eval_windows(C.byref(self.g), _u32(tokens), train_tokens,
                                                            val_tokens, val_batches))

    def forward_logits(self, ids):
        out = np.zeros((self.B * self.T, self.hm.V), np.float32)
        self.hip.gpu_trainer_forward_logits(C.byref(self.g), _u32(ids), out.ctypes.data)
        return out

    def forward_loss_logits(self, ids, tgt, want_logits=True):
        out = np.zeros((self.B * self.T, self.hm.V), np.float32) if want_logits else None
        loss = self.hip.gpu_trainer_forward_loss_logits(C.byref(self.g), _u32(ids), _u32(tgt),
                                                        out.ctypes.data if want_logits else None)
        return loss, out

    def greedy_argmax(self):
        out = np.zeros(self.B * self.T, np.uint32)
        self.hip.gpu_trainer_greedy_argmax(C.byref(self.g), out)
        return out

    def force_gemm(self, tile=None, splits=0):
        """trlm_gemm_force on the trainer's main-stream GEMM engine: later
        forward, LM-head and dX products use that tile variant (None restores
        automatic selection)."""
        eng = self.hip.gpu_trainer_gemm_engine(C.byref(self.g))
        if self.hip.trlm_gemm_force(eng, tile.encode() if tile else None, splits) != 0:
            raise ValueError("unknown GEMM tile variant %r" % tile)

    def gemm_last_variant(self):
        """(kernel, splits) of the main engine's last GEMM."""
        eng = self.hip.gpu_trainer_gemm_engine(C.byref(self.g))
        sp = C.c_int32(0)
        return self.hip.trlm_gemm_last_variant(eng, C.byref(sp)).decode(), sp.value

    def destroy(self):
        if self.g is not None:
            self.hip.gpu_trainer_destroy(C.byref(self.g))
            self.g = None


class Decoder:
    """gpu_decoder_* (KV-cache decode) over a Trainer's resident parameters."""

    def __init__(self, trainer, batch, max_ctx):
        self.hip = trainer.hip
        self.tr = trainer
        self.B, self.V = batch, trainer.hm.V
        self.d = self.hip.gpu_decoder_create(C.byref(trainer.g), batch, max_ctx)

    def prefill(self, ids):
        ids = _u32(ids)
        self.hip.gpu_decoder_prefill(self.d, ids.ravel(), ids.shape[-1] if ids.ndim > 1 else ids.size // self.B)

    def step(self, ids):
        self.hip.gpu_decoder_step(self.d, _u32(ids).ravel())

    def length(self):
        return self.hip.gpu_decoder_length(self.d)

    def logits(self):
        out = np.zeros((self.B, self.V), np.float32)
        self.hip.gpu_decoder_logits(self.d, out)
        return out

    def greedy(self):
        out = np.zeros(self.B, np.uint32)
        self.hip.gpu_decoder_greedy(self.d, out)
        return out

    def sample(self, rngs, temperature):
        """rngs: ctypes array of PCGState (one per sequence), advanced in place."""
        out = np.zeros(self.B, np.uint32)
        self.hip.gpu_decoder_sample(self.d, rngs, temperature, out)
        return out

    def generate_greedy(self, prompt, steps):
        prompt = _u32(prompt)
        out = np.zeros((self.B, steps), np.uint32)
        self.hip.gpu_decoder_generate_greedy(self.d, prompt.ravel(), prompt.shape[-1], steps, out)
        return out

    def generate_sampled(self, prompt, steps, rngs, temperature):
        """rngs: ctypes array of PCGState (one per sequence), advanced in place."""
        prompt = _u32(prompt)
        out = np.zeros((self.B, steps), np.uint32)
        self.hip.gpu_decoder_generate_sampled(self.d, prompt.ravel(), prompt.shape[-1], steps, rngs, temperature, out)
        return out

    def destroy(self):
        if self.d is not None:
            self.hip.gpu_decoder_destroy(self.d)
            self.d = None


def _u32(a):
    return np.ascontiguousarray(a, np.uint32)


class Device:
    """A bare HIP context (kernel image loaded) with device-buffer helpers,
    for exercising the GEMM and timing through the C ABI."""

    def __init__(self, image=KERNELS):
        _, hip = libs()
        self.hip = hip
        self.ctx = hip.hip_init(None, image.encode())
        hip.hip_set_current(C.byref(self.ctx))
        self.gemm = hip.trlm_gemm_create(C.byref(self.ctx))

    def current(self):
        self.hip.hip_set_current(C.byref(self.ctx))

    def upload(self, arr):
        arr = np.ascontiguousarray(arr)
        p = self.hip.hip_alloc(max(arr.nbytes, 4))
        self.hip.hip_h2d(p, arr.ctypes.data, arr.nbytes)
        return p

    def empty(self, nbytes):
        p = self.hip.hip_alloc(max(nbytes, 4))
        self.hip.hip_memset_zero(p, max(nbytes, 4))
        return p

    def download(self, p, shape, dtype=np.float32):
        out = np.zeros(shape, dtype)
        self.hip.hip_d2h(out.ctypes.data, p, out.nbytes)
        return out

    def free(self, p):
        self.hip.hip_free(p)

    def matmul(self, ta, tb, A, B, C_, M, N, K, lda, ldb, ldc, batch=1, sA=0, sB=0, sC=0, alpha=1.0, beta=0.0,
               bias=None, resid=None, ldr=0):
        self.hip.trlm_gemm(self.gemm, ta, tb, A, B, C_, M, N, K, lda, ldb, ldc, batch, sA, sB, sC, alpha, beta,
                           bias, resid, ldr or ldc)

    def matmul_noalloc(self, ta, tb, A, B, C_, M, N, K, lda, ldb, ldc, batch=1, sA=0, sB=0, sC=0, alpha=1.0,
                       beta=0.0, bias=None, resid=None, ldr=0):
        """trlm_gemm_noalloc: returns 0 (a plan whose split-K partials
        exceed the 32 MiB scratch runs with the most splits that fit), or -1
        when the engine's device is not the current one (nothing launched)."""
        return self.hip.trlm_gemm_noalloc(self.gemm, ta, tb, A, B, C_, M, N, K, lda, ldb, ldc, batch, sA, sB, sC,
                                          alpha, beta, bias, resid, ldr or ldc)

    def last_variant(self):
        sp = C.c_int32(0)
        name = self.hip.trlm_gemm_last_variant(self.gemm, C.byref(sp))
        return name.decode(), sp.value

    def force(self, tile=None, splits=0):
        """Pin later GEMMs on this device to one tile variant / split-K factor
        (None restores automatic selection)."""
        if self.hip.trlm_gemm_force(self.gemm, tile.encode() if tile else None, splits) != 0:
            raise ValueError("unknown GEMM tile variant %r" % tile)

    def sync(self):
        self.hip.hip_sync()

    def close(self):
        self.current()   # the engine's workspace is freed in its own context
        self.hip.trlm_gemm_destroy(self.gemm)
        self.hip.hip_shutdown(C.byref(self.ctx))
