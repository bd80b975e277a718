/* train_loop.c -- the reference GPU training driver's inner loop
 * (training/train_lm_gpu.c:212-223) and its validation windows (:241-258),
 * queued on the device.
 *
 * The reference waits for the device several times per step (the loss
 * readback in forward_backward, the grad-norm partials, the synchronous
 * Adam step, and blocking uploads of every batch).  Here a step is one run
 * of launches with no wait: the host samples batch s+1 and groups its rows
 * for the embedding backward while the device runs step s; batches go up
 * through a ring of pinned buffers with asynchronous copies (stream order
 * puts each upload after the previous step's kernels); the loss mean, the
 * grad norm and the clip scale are computed on the device (k_loss_mean,
 * k_norm_clip, with the host functions' operation order) and the Adam kernel
 * reads the scale from device memory (k_adam_ds).  The per-step values come
 * back once, at the end of the call.  Same results as the reference's loop,
 * bit for bit.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#include "gpu_internal.h"

#define LR_PI 3.14159265358979323846
#define SLOTS 3          /* pinned batch buffers in flight */

static void loop_fatal(const char* what) {
    fprintf(stderr, "[HIP ERROR] train_loop: %s\n", what);
    fflush(stderr);
    _exit(1);
}

static void check_hip(hipError_t r, const char* what) {
    if (r != hipSuccess) {
        fprintf(stderr, "[HIP ERROR] train_loop: %s -> %s: %s\n", what, hipGetErrorName(r), hipGetErrorString(r));
        fflush(stderr);
        _exit(1);
    }
}

f32 trlm_lr_warmup_cosine(u64 step, u64 warmup_steps, u64 total_steps, f32 peak_lr, f32 min_lr) {
    if (warmup_steps > 0 && step < warmup_steps) return peak_lr * (f32)(step + 1) / (f32)warmup_steps;
    if (total_steps <= warmup_steps) return min_lr;
    f64 p = (f64)(step - warmup_steps) / (f64)(total_steps - warmup_steps);
    if (p > 1.0) p = 1.0;
    f64 c = 0.5 * (1.0 + m_cos(LR_PI * p));
    return (f32)((f64)min_lr + ((f64)peak_lr - (f64)min_lr) * c);
}

/* One pinned batch: ids, targets, row order, segments. */
typedef struct Slot {
    u32 *ids, *tgt, *order, *seg;
    hipEvent_t uploaded;
    int busy;
} Slot;

typedef struct Ring {
    u32* host;
    Slot slot[SLOTS];
} Ring;

static void ring_open(Ring* r, u32 N) {
    u64 per = (u64)N * 5 + 1;    /* ids N, tgt N, order N, seg 2N+1 */
    check_hip(hipHostMalloc((void**)&r->host, per * SLOTS * sizeof(u32), hipHostMallocDefault), "hipHostMalloc");
    for (int i = 0; i < SLOTS; i++) {
        Slot* s = &r->slot[i];
        s->ids = r->host + per * (u64)i;
        s->tgt = s->ids + N;
        s->order = s->tgt + N;
        s->seg = s->order + N;
        s->busy = 0;
        check_hip(hipEventCreateWithFlags(&s->uploaded, hipEventDisableTiming), "hipEventCreate");
    }
}

static void ring_close(Ring* r) {
    for (int i = 0; i < SLOTS; i++) check_hip(hipEventDestroy(r->slot[i].uploaded), "hipEventDestroy");
    check_hip(hipHostFree(r->host), "hipHostFree");
}

/* Wait until the slot's previous upload has left its buffers. */
static Slot* ring_take(Ring* r, u64 i) {
    Slot* s = &r->slot[i % SLOTS];
    if (s->busy) check_hip(hipEventSynchronize(s->uploaded), "hipEventSynchronize");
    s->busy = 0;
    return s;
}

static void upload_async(GpuTrainer* g, hipDeviceptr_t dst, const void* src, u64 bytes) {
    check_hip(hipMemcpyHtoDAsync(dst, (void*)src, bytes, g->hip.stream), "hipMemcpyHtoDAsync");
}

static void ring_sent(GpuTrainer* g, Slot* s) {
    check_hip(hipEventRecord(s->uploaded, g->hip.stream), "hipEventRecord");
    s->busy = 1;
}

void gpu_trainer_train_steps(GpuTrainer* g, AdamOptimizer* opt, const u32* tokens, u64 num_tokens,
                             const TrlmSchedule* sch, u64 first_step, u32 n_steps, f32* losses, f64* grad_norms,
                             f32* lrs) {
    trlm_bind(g);
    if (n_steps == 0) return;
    if (num_tokens < (u64)g->T + 2) loop_fatal("token stream shorter than seq_len + 2");
    u32 N = g->N;
    Ring ring;
    ring_open(&ring, N);
    hipDeviceptr_t d_loss = hip_alloc((u64)n_steps * sizeof(f32));
    hipDeviceptr_t d_norm = hip_alloc((u64)n_steps * sizeof(f64));
    hipDeviceptr_t d_scale = hip_alloc(sizeof(f32));
    for (u32 i = 0; i < n_steps; i++) {
        u64 step = first_step + i;
        f32 lr = trlm_lr_warmup_cosine(step, sch->warmup_steps, sch->total_steps, sch->peak_lr, sch->min_lr);
        opt->lr = lr;
        if (lrs) lrs[i] = lr;
        Slot* s = ring_take(&ring, i);
        gpu_trainer_sample_batch(tokens, num_tokens, g->T, g->B, sch->seed_base + step, s->ids, s->tgt);
        trlm_check_ids(g, s->ids, "ids");
        trlm_check_ids(g, s->tgt, "targets");
        u32 nseg = trlm_embed_groups(g, s->ids, s->order, s->seg);
        upload_async(g, g->ids, s->ids, (u64)N * sizeof(u32));
        upload_async(g, g->targets, s->tgt, (u64)N * sizeof(u32));
        upload_async(g, g->emb_order, s->order, (u64)N * sizeof(u32));
        upload_async(g, g->emb_seg, s->seg, (2ull * nseg + 1) * sizeof(u32));
        ring_sent(g, s);
        g->emb_nseg = nseg;
        trlm_train_step_queued(g, opt, sch->weight_decay, sch->grad_clip,
                               (hipDeviceptr_t)((char*)d_loss + (u64)i * sizeof(f32)),
                               (hipDeviceptr_t)((char*)d_norm + (u64)i * sizeof(f64)), d_scale);
    }
    if (losses) hip_d2h(losses, d_loss, (u64)n_steps * sizeof(f32));
    if (grad_norms) hip_d2h(grad_norms, d_norm, (u64)n_steps * sizeof(f64));
    hip_sync();
    hip_free(d_scale);
    hip_free(d_norm);
    hip_free(d_loss);
    ring_close(&ring);
}

f32 gpu_trainer_eval_windows(GpuTrainer* g, const u32* tokens, u64 train_tokens, u64 val_tokens, u32 val_batches) {
    trlm_bind(g);
    if (val_batches == 0) loop_fatal("val_batches is 0");
    u64 windows = (u64)val_batches * g->B;
    if (val_tokens < (u64)g->T + 1) loop_fatal("validation block shorter than seq_len + 1");
    u64 stride = (val_tokens - g->T - 1) / windows;
    u32 N = g->N, T = g->T;
    Ring ring;
    ring_open(&ring, N);
    hipDeviceptr_t d_sum = hip_alloc(sizeof(f32));
    for (u32 vb = 0; vb < val_batches; vb++) {
        Slot* s = ring_take(&ring, vb);
        for (u32 w = 0; w < g->B; w++) {
            u64 start = train_tokens + ((u64)vb * g->B + w) * stride;
            for (u32 t = 0; t < T; t++) {
                s->ids[(u64)w * T + t] = tokens[start + t];
                s->tgt[(u64)w * T + t] = tokens[start + t + 1];
            }
        }
        trlm_check_ids(g, s->ids, "ids");
        trlm_check_ids(g, s->tgt, "targets");
        upload_async(g, g->ids, s->ids, (u64)N * sizeof(u32));
        upload_async(g, g->targets, s->tgt, (u64)N * sizeof(u32));
        ring_sent(g, s);
        trlm_eval_queued(g, d_sum, vb > 0);
    }
    f32 sum;
    hip_d2h(&sum, d_sum, sizeof(f32));
    hip_free(d_sum);
    ring_close(&ring);
    return sum / (f32)val_batches;
}
