"""The drop-in C ABI, checked without a GPU.

  - every function declared in include/*.h is exported by the built
    libraries (gpu_train.h / gpu_ops.h / hip_backend.h / trlm_ext.h by
    libtrlm_hip.so, trlm_host.h by libtrlm_host.so);
  - libtrlm_hip.so leaves undefined only the reference-runtime symbols the
    reference's own gpu_train.c / gpu_ops.c use (so the reference's objects
    can provide them) plus libc / HIP runtime;
  - the gfx950 code object holds every kernel the host code looks up;
  - the Python structure mirror matches the C compiler's layout, and
    trlm_host.h's host types match the reference's own headers (sizeof and
    every field offset, compiled from /root/reference when present);
  - the drop-in binding is real: oracle/dropin.sh compiles every program of
    the reference (all but tests/test_cuda.c) from its own sources against
    include/ installed as model/gpu_train.h, model/gpu_ops.h, ... and links
    it with libtrlm_hip.so instead of the CUDA objects (when
    /root/reference is present);
  - the host-side logic of the path is bit-identical to the oracle: PCG,
    scalar maths feeding RoPE and Adam, RoPE tables, batch sampling.
No GPU call is made here (HIP calls without a device would end the process).
"""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INC = os.path.join(ROOT, "include")

PROTO = re.compile(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s+\**\s*([a-z_][a-z0-9_]*)\s*\(", re.M)


def declared(header):
    with open(os.path.join(INC, header)) as fh:
        text = fh.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set(PROTO.findall(text))
    return {n for n in names if n not in ("if", "while", "for", "return", "sizeof")}


def test_headers_declare_the_reference_api():
    train = declared("gpu_train.h")
    assert {"gpu_trainer_create", "gpu_trainer_destroy", "gpu_trainer_upload", "gpu_trainer_download",
            "gpu_trainer_download_grads", "gpu_trainer_upload_grads", "gpu_trainer_sample_batch",
            "gpu_trainer_forward_backward", "gpu_trainer_eval_loss", "gpu_trainer_grad_norm",
            "gpu_trainer_adam_step", "gpu_trainer_adam_step_scaled"} <= train
    ops = declared("gpu_ops.h")
    assert {"gpu_ops_init", "gpu_ops_shutdown", "gpu_ops_init_workers", "gpu_ops_set_worker_id",
            "node_matmul2d_gpu", "gpu_ops_debug_stats", "gpu_ops_debug_reset"} <= ops


def test_every_declared_symbol_is_exported(trlm):
    host, hip = trlm.libs()
    for header, lib in [("gpu_train.h", hip), ("gpu_ops.h", hip), ("hip_backend.h", hip), ("trlm_ext.h", hip),
                        ("trlm_host.h", host)]:
        for name in declared(header):
            assert hasattr(lib, name), (header, name)


def test_reference_prototypes_unchanged():
    """The prototypes of the reference's model/gpu_train.h:86-125 and
    model/gpu_ops.h:23-60, as text, appear unchanged in include/."""
    want = [
        "GpuTrainer gpu_trainer_create(Allocator* alloc, const char* ptx_path, const LMModel* model,\n"
        "                              Node** params, u32 num_params, u32 batch_size, u32 seq_len);",
        "void gpu_trainer_destroy(GpuTrainer* g);",
        "void gpu_trainer_upload(GpuTrainer* g, Node** params, const AdamOptimizer* opt);",
        "void gpu_trainer_download(GpuTrainer* g, Node** params, AdamOptimizer* opt);",
        "void gpu_trainer_download_grads(GpuTrainer* g, Node** params);",
        "void gpu_trainer_upload_grads(GpuTrainer* g, Node** params);",
        "void gpu_trainer_sample_batch(const u32* tokens, u64 num_tokens, u32 seq_len, u32 batch_size,\n"
        "                              u64 seed_base, u32* ids_out, u32* targets_out);",
        "f32 gpu_trainer_forward_backward(GpuTrainer* g, const u32* ids, const u32* targets);",
        "f32 gpu_trainer_eval_loss(GpuTrainer* g, const u32* ids, const u32* targets);",
        "f64 gpu_trainer_grad_norm(GpuTrainer* g);",
        "void gpu_trainer_adam_step(GpuTrainer* g, AdamOptimizer* opt);",
        "void gpu_trainer_adam_step_scaled(GpuTrainer* g, AdamOptimizer* opt, f32 grad_scale);",
        "#define GPU_TRAIN_MAX_PARAMS (LM_MAX_LAYERS * 10u + 2u)",
        "#define GPU_TRAIN_NORM_BLOCKS 1024u",
    ]
    text = open(os.path.join(INC, "gpu_train.h")).read()
    for w in want:
        assert w in text, w
    ops = open(os.path.join(INC, "gpu_ops.h")).read()
    for w in ["void gpu_ops_init(Allocator* scratch, const char* ptx_path);", "void gpu_ops_shutdown(void);",
              "void gpu_ops_init_workers(Allocator* scratch, const char* ptx_path, u32 num_workers);",
              "void gpu_ops_set_worker_id(i32 worker_id);", "Node* node_matmul2d_gpu(Allocator* alloc, Node* a, Node* b);",
              "void gpu_ops_debug_stats(f64* out_total_seconds, u32* out_call_count);",
              "void gpu_ops_debug_reset(void);"]:
        assert w in ops, w


def test_undefined_symbols_are_runtime_only(trlm):
    out = subprocess.run(["nm", "-D", "--undefined-only", trlm.LIB_HIP], capture_output=True, text=True,
                         check=True).stdout
    names = {ln.split()[-1].split("@")[0] for ln in out.splitlines() if ln.strip()}
    runtime = {"allocator_alloc", "tensor_create", "tensor_transpose", "tensor_contiguous", "tensor_add_inplace",
               "node_make_custom", "rope_build_tables", "pcg_seed", "pcg_range_i64", "pcg_next_u32", "m_powf",
               "m_sqrt", "m_sqrtf", "m_cos"}
    other = {n for n in names if not (n.startswith("hip") or n.startswith("_") or n in runtime)}
    libc = {"fprintf", "fflush", "_exit", "fopen", "fseek", "ftell", "fread", "fclose", "malloc", "calloc",
            "realloc", "free", "memset", "memcpy", "memcmp", "strcmp", "strlen", "snprintf", "fwrite", "rename",
            "remove", "stderr", "stdout", "clock_gettime", "getenv", "pthread_create", "pthread_join",
            "pthread_mutex_lock", "pthread_mutex_unlock", "pthread_mutex_init", "pthread_mutex_destroy"}
    assert other <= libc, other - libc
    assert runtime & names == runtime, runtime - names


def test_code_object_has_every_kernel(trlm):
    with open(trlm.KERNELS, "rb") as fh:
        blob = fh.read()
    src = ""
    for f in ("gpu_train.c", "gpu_decode.c", "trlm_gemm.c"):
        src += open(os.path.join(ROOT, "turkce-llm_amd", "csrc", f)).read()
    names = set(re.findall(r'"(k_[a-z0-9_]+)"', src))
    names |= {"k_attn_fwd_hd%d" % d for d in (16, 32, 64)} | {"k_attn_bwd_dq_hd%d" % d for d in (16, 32, 64)}
    names |= {"k_attn_dvec_hd%d" % d for d in (16, 32, 64)}
    names |= {"k_attn_bwd_dkv_hd%d" % d for d in (16, 32, 64)}
    names |= {"k_dec_qkv_attn_hd%d" % d for d in (16, 32, 64)} | {"k_dec_head_k%d" % n for n in (8, 24, 32)}
    names |= {"k_gemm_%s_%s" % (l, t) for l in ("nn", "nt", "tn") for t in (
        "256x128", "128x256", "128x128", "128x128_k32", "64x128", "64x128_k32", "64x64", "64x64_k32")}
    names |= {"k_gemm_%s_64x64_u" % l for l in ("nn", "nt", "tn", "tt")} | {"k_gemm_nn_64x64_k32_glu"}
    for n in sorted(names):
        assert n.encode() + b"\0" in blob, n


LLVM = "/opt/rocm/llvm/bin"


@pytest.mark.skipif(not os.path.exists(os.path.join(LLVM, "llvm-readobj")), reason="ROCm LLVM tools not present")
def test_kernel_argument_blocks_match_host_structs(trlm, tmp_path):
    """Every kernel that takes an argument block by value declares, in the
    code object's own metadata, exactly one explicit argument whose size is
    sizeof() of the host struct the library fills (kernel_params.h, compiled
    by the host compiler): the bytes HIP copies from the host pointer are
    exactly the host struct, no more and no less."""
    import yaml
    csrc = os.path.join(ROOT, "turkce-llm_amd", "csrc")
    src = tmp_path / "kp.c"
    src.write_text('#include <stdio.h>\n#include "kernel_params.h"\n'
                   'int main(void) { printf("%zu %zu %zu\\n", sizeof(GemmParams), sizeof(AttnParams), '
                   'sizeof(DecGemmParams)); return 0; }\n')
    exe = tmp_path / "kp"
    subprocess.run(["gcc", "-std=c11", "-I" + csrc, str(src), "-o", str(exe)], check=True)
    gemm, attn, dec = map(int, subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split())
    co = tmp_path / "k.co"
    subprocess.run([os.path.join(LLVM, "clang-offload-bundler"), "--unbundle", "--type=o", "--input=" + trlm.KERNELS,
                    "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", "--output=" + str(co)], check=True)
    notes = subprocess.run([os.path.join(LLVM, "llvm-readobj"), "--notes", str(co)], check=True, capture_output=True,
                           text=True).stdout
    a = notes.index("---")
    kernels = yaml.safe_load(notes[a:notes.index("\n...", a)])["amdhsa.kernels"]
    want = {}
    for k in kernels:
        n = k[".name"]
        if n.startswith("k_gemm_") and not n.startswith("k_gemm_splitk"):
            want[n] = gemm
        elif re.match(r"k_attn_(fwd|bwd_dkv|bwd_dq|dvec)_hd\d+$", n):
            want[n] = attn
        elif n in ("k_dec_out", "k_dec_gu", "k_dec_down") or re.match(r"k_dec_(qkv_attn_hd|head_k)\d+$", n):
            want[n] = dec
    assert len([n for n in want if n.startswith("k_gemm_")]) == 29   # 8 tiles x 3 layouts, 4 unaligned, SwiGLU
    assert len([n for n in want if n.startswith("k_attn_")]) == 12
    assert len([n for n in want if n.startswith("k_dec_")]) == 9   # out, gu, down, head x 3, QKV + attention x 3
    for k in kernels:
        n = k[".name"]
        if n not in want:
            continue
        explicit = [x for x in k[".args"] if not x[".value_kind"].startswith("hidden_")]
        assert len(explicit) == 1 and explicit[0][".value_kind"] == "by_value", (n, explicit)
        assert explicit[0][".size"] == want[n], (n, explicit[0][".size"], want[n])


def test_structure_layout(trlm):
    ok, got, want = trlm.check_layout()
    assert ok, (got, want)
    _, hip = trlm.libs()
    assert hip.trlm_sizeof_hip_ctx() == C.sizeof(trlm.HipCtx)


def test_host_runtime_matches_oracle(trlm, orc):
    host, hip = trlm.libs()
    L = orc.lib()
    r1 = host.pcg_seed(4242, 7)
    r2 = orc.pcg_stream(4242, 7)
    for _ in range(50):
        assert host.pcg_range_i64(C.byref(r1), 0, 31769) == L.or_pcg_range_i64(C.byref(r2), 0, 31769)
    for _ in range(20):
        assert float(host.pcg_gaussian(C.byref(r1), 0.0, 0.02)).hex() == \
            float(L.or_pcg_gaussian(C.byref(r2), 0.0, 0.02)).hex()
    rng = np.random.default_rng(1)
    for x in rng.uniform(1e-8, 1e8, 200):
        assert float(host.m_sqrt(x)).hex() == float(L.or_m_sqrt(x)).hex()
    for b in (0.9, 0.95, 0.999):
        for t in range(1, 200, 7):
            assert np.float32(host.m_powf(b, float(t))) == np.float32(L.or_m_powf(b, float(t)))
    for x in rng.uniform(-1100, 1100, 200):
        assert np.float32(host.m_sinf(x)) == np.float32(L.or_m_sinf(x))
        assert np.float32(host.m_cosf(x)) == np.float32(L.or_m_cosf(x))


@pytest.mark.parametrize("T,hd", [(128, 64), (1024, 64), (12, 16), (100, 32)])
def test_rope_tables_bit_exact(trlm, orc, T, hd):
    host, _ = trlm.libs()
    alloc = host.allocator_create(1 << 26)
    try:
        sh = (C.c_uint64 * 2)(T, hd // 2)
        ct = host.tensor_create(C.byref(alloc), sh, 2)
        st = host.tensor_create(C.byref(alloc), sh, 2)
        host.rope_build_tables(C.byref(ct), C.byref(st), T, hd, 10000.0)
        c, s = orc.rope_tables(T, hd)
        assert np.array_equal(trlm.tensor_np(ct).view(np.uint32), c.ravel().view(np.uint32))
        assert np.array_equal(trlm.tensor_np(st).view(np.uint32), s.ravel().view(np.uint32))
    finally:
        host.allocator_destroy(C.byref(alloc))


@pytest.mark.parametrize("T,B,seed", [(12, 5, 2026), (128, 4, 7), (1024, 8, 2026 + 99)])
def test_sample_batch_bit_exact(trlm, orc, T, B, seed):
    _, hip = trlm.libs()
    toks = orc.random_tokens(50000, 31769)
    ids = np.zeros(B * T, np.uint32)
    tgt = np.zeros(B * T, np.uint32)
    hip.gpu_trainer_sample_batch(toks, len(toks), T, B, seed, ids, tgt)
    wi, wt = orc.sample_batch(toks, T, B, seed)
    assert np.array_equal(ids, wi) and np.array_equal(tgt, wt)


def test_gemm_plan_is_a_pure_function_of_the_shape(trlm):
    """The GEMM plan (variant, split-K) depends on (layout, M, N, K, batch)
    only -- reruns of a shape take the same kernels, so results repeat bit for
    bit -- and respects the split-K limits: single GEMMs only, every split at
    least 256 deep, at most 32 splits."""
    _, hip = trlm.libs()
    sp = C.c_int32()
    shapes = [(8192, 1152, 384), (8192, 384, 2048), (384, 1152, 8192), (8192, 31769, 384), (8192, 384, 31769),
              (31769, 384, 8192), (1, 1, 1), (4, 5, 3), (512, 384, 1024), (100, 68, 4000), (64, 64, 0)]
    for ta, tb in [(0, 0), (0, 1), (1, 0)]:
        for M, N, K in shapes:
            for batch in (1, 6):
                first = hip.trlm_gemm_plan(ta, tb, M, N, K, batch, C.byref(sp)).decode(), sp.value
                again = hip.trlm_gemm_plan(ta, tb, M, N, K, batch, C.byref(sp)).decode(), sp.value
                assert first == again
                name, splits = first
                assert name.startswith("k_gemm_%s_" % ["nn", "nt", "tn"][ta * 2 + tb]), name
                assert 1 <= splits <= 32
                if splits > 1:
                    assert batch == 1 and K // splits >= 224, (M, N, K, splits)
    assert hip.trlm_gemm_plan(1, 1, 64, 64, 64, 1, C.byref(sp)) == b"k_gemm_tt_64x64_u" and sp.value == 1
    # the LM-head forward (15,936 tiles of 128x128, 62 per CU) keeps the
    # large tile and needs no split
    name = hip.trlm_gemm_plan(0, 1, 8192, 31769, 384, 1, C.byref(sp)).decode()
    assert name == "k_gemm_nt_128x128" and sp.value == 1


def test_attention_job_table(trlm):
    """trlm_attn_job_table: every (query block, head) job exactly once; the
    three workgroups L, L + cus, L + 2 cus that share a compute unit hold
    floor or ceil of 3(n + 1)/2 key-block stages (query block q is q + 1
    stages); and every head's workgroups have one L mod xcds (the XCD whose L2
    holds that head's K and V) -- checked by counting, for every n up to 64
    and some larger, with 1, 2 and 16 triples of heads per XCD over 1 to 8
    XCDs; B8 T1024 (48 heads, 16 blocks, 256 units, 8 XCDs) gives 25 or 26
    per unit.  Any grid that is not exactly three workgroups per unit, or
    whose head triples do not divide among the XCDs, gets 0 and an untouched
    table."""
    import numpy as np
    _, hip = trlm.libs()
    for n in list(range(1, 65)) + [100, 127, 128, 256]:
        for trip, xcds in ((1, 1), (2, 2), (16, 8), (8, 8), (3, 1)):
            heads, cus = 3 * trip, trip * n
            jobs = (C.c_int32 * (heads * n))()
            assert hip.trlm_attn_job_table(heads, n, cus, xcds, jobs) == 1
            a = np.frombuffer(jobs, dtype=np.int32)
            qb, hd = a >> 16, a & 0xFFFF
            assert sorted(zip(qb.tolist(), hd.tolist())) == [(q, h) for q in range(n) for h in range(heads)]
            stages = (qb + 1).reshape(3, cus).sum(axis=0)
            assert stages.min() >= 3 * (n + 1) // 2 and stages.max() <= -(-3 * (n + 1) // 2), (n, trip)
            xcd = np.arange(heads * n) % xcds
            for h in range(heads):
                assert len(set(xcd[hd == h].tolist())) == 1, (n, trip, xcds, h)
    jobs = (C.c_int32 * 768)()
    assert hip.trlm_attn_job_table(48, 16, 256, 8, jobs) == 1
    stages = ((np.frombuffer(jobs, dtype=np.int32) >> 16) + 1).reshape(3, 256).sum(axis=0)
    assert set(stages.tolist()) == {25, 26}
    for heads, n, cus, xcds in [(48, 8, 256, 8), (50, 16, 256, 8), (48, 16, 255, 8), (3, 16, 0, 1), (48, 0, 256, 8),
                                (6, 4, 7, 1), (24, 16, 128, 16), (48, 16, 256, 0), (6, 4, 8, 4)]:
        size = max(1, heads * n)
        jobs = (C.c_int32 * size)(*([-7] * size))
        assert hip.trlm_attn_job_table(heads, n, cus, xcds, jobs) == 0
        assert all(v == -7 for v in jobs)


REF = "/root/reference"
LAYOUT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
%s
#define S(T) printf(#T " %%zu\n", sizeof(T))
#define O(T, m) printf(#T "." #m " %%zu\n", offsetof(T, m))
int main(void) {
    S(Arena); S(Allocator); S(Tensor); S(Node); S(PCGState); S(AttentionWeights); S(FeedForwardWeights);
    S(BlockWeights); S(LMModel); S(AdamOptimizer);
    O(Arena, reserved); O(Arena, committed); O(Arena, used);
    O(Allocator, free_list); O(Allocator, last_phys);
    O(Tensor, shape); O(Tensor, strides); O(Tensor, ndim); O(Tensor, numel); O(Tensor, owns_data);
    O(Node, grad); O(Node, requires_grad); O(Node, parents); O(Node, num_parents); O(Node, backward_fn);
    O(Node, visited); O(Node, aux_dim0); O(Node, aux_dim1); O(Node, aux_scalar); O(Node, aux_ptr);
    O(PCGState, inc); O(PCGState, has_cached_gaussian); O(PCGState, cached_gaussian);
    O(AttentionWeights, b_qkv); O(AttentionWeights, wo); O(AttentionWeights, bo);
    O(FeedForwardWeights, b_gate_up); O(FeedForwardWeights, w_down); O(FeedForwardWeights, b_down);
    O(BlockWeights, attn); O(BlockWeights, ffn_norm_w); O(BlockWeights, ffn);
    O(LMModel, blocks); O(LMModel, final_norm_w); O(LMModel, num_layers); O(LMModel, num_heads);
    O(LMModel, d_model); O(LMModel, vocab_size); O(LMModel, eps);
    O(AdamOptimizer, m); O(AdamOptimizer, v); O(AdamOptimizer, num_params); O(AdamOptimizer, t);
    O(AdamOptimizer, lr); O(AdamOptimizer, beta1); O(AdamOptimizer, beta2); O(AdamOptimizer, eps);
    printf("LM_MAX_LAYERS %%d\n", (int)LM_MAX_LAYERS);
    return 0;
}
"""


def _probe(tmp_path, name, includes, flags):
    src = tmp_path / (name + ".c")
    src.write_text(LAYOUT_PROBE % includes)
    exe = tmp_path / name
    subprocess.run(["gcc", "-std=c11", "-D_DEFAULT_SOURCE"] + flags + [str(src), "-o", str(exe)], check=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not present")
def test_host_types_match_reference_headers(tmp_path):
    """sizeof and every field offset of the host types in trlm_host.h equal
    the reference's own definitions (runtime/types.h, runtime/memory.h,
    runtime/prng.h, tensor/tensor.h, autograd/node.h, model/*.h,
    training/adam.h), compiled by the same compiler."""
    ref_inc = "\n".join('#include "%s"' % h for h in (
        "runtime/types.h", "runtime/memory.h", "runtime/prng.h", "tensor/tensor.h", "autograd/node.h",
        "model/lm_model.h", "training/adam.h"))
    want = _probe(tmp_path, "ref_layout", ref_inc, ["-I" + REF])
    got = _probe(tmp_path, "our_layout", '#include "trlm_host.h"', ["-I" + INC])
    assert got == want
    assert len(got.splitlines()) >= 50


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference tree not present")
def test_reference_programs_link_against_the_library(trlm):
    """oracle/dropin.sh: the reference's own programs, compiled against
    include/ as model/gpu_train.h, model/gpu_ops.h (+ hip_backend.h,
    trlm_host.h, trlm_ext.h), link with libtrlm_hip.so and need no CUDA
    library.  Among them the callers of the GPU path: train_lm_gpu, generate,
    chat, train_lm, train_faz4/5, data_parallel's tests, test_gpu_train and
    test_gpu_ops."""
    trlm.libs()
    r = subprocess.run([os.path.join(ROOT, "oracle", "dropin.sh"), REF], capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    out = os.path.join(ROOT, "oracle", "_ref", "dropin")
    # no warning comes from this build's headers
    assert not re.search(r"model/(gpu_train|gpu_ops|hip_backend|trlm_host|trlm_ext)\.h", r.stderr), r.stderr[-3000:]
    progs = ["training_train_lm_gpu", "training_generate", "training_chat", "training_train_lm",
             "training_train_faz4", "training_train_faz5", "training_probe_batched_step", "tests_test_gpu_train",
             "tests_test_gpu_ops", "tests_test_lm_model_gpu", "tests_test_batched_lm", "tests_test_data_parallel",
             "tests_test_resume"]
    for p in progs:
        exe = os.path.join(out, p)
        assert os.path.exists(exe), p
        needed = subprocess.run(["readelf", "-d", exe], capture_output=True, text=True, check=True).stdout
        assert "libtrlm_hip.so" in needed and "libcuda" not in needed, (p, needed)
