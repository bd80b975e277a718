/* checkpoint.c -- TRLM v1 checkpoints straight from / to a GpuTrainer.
 *
 * Same file format and acceptance rules as the reference's
 * training/checkpoint.c (format: checkpoint.h:6-12; save :22-66; load
 * :68-137), so files move freely between the two:
 *   ["TRLM"][u32 version = 1][u32 num_params][u32 has_opt]
 *   per parameter: [u32 ndim][ndim x u64 shape][numel x f32 value]
 *   if has_opt:    per parameter [numel x f32 m][numel x f32 v], then [u64 t]
 * The reference drivers save after gpu_trainer_download and load before
 * gpu_trainer_upload; here the values come from / go to the device buffers
 * directly (the host mirror is refreshed on load), with the reference's
 * guarantees: a save goes to path.tmp and is renamed over path only when
 * every byte was written; a load validates the whole file first and
 * changes nothing when it returns FALSE.  Shapes come from the caller's
 * parameter nodes, as in the reference.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "trlm_ext.h"

#define CKPT_MAX_PATH 512
#define F4 ((u64)sizeof(f32))

static hipDeviceptr_t dev_at(hipDeviceptr_t base, u64 floats) { return (hipDeviceptr_t)((char*)base + floats * F4); }

static int shapes_match(const GpuTrainer* g, Node** params, u32 num_params) {
    if (num_params != g->num_params) return 0;
    for (u32 i = 0; i < num_params; i++)
        if (params[i]->value.numel != g->numels[i]) return 0;
    return 1;
}

bool32 gpu_trainer_checkpoint_save(GpuTrainer* g, const char* path, Node** params, const AdamOptimizer* opt) {
    hip_set_current(&g->hip);
    if (!shapes_match(g, params, g->num_params)) return FALSE;
    u64 n = strlen(path);
    char tmp[CKPT_MAX_PATH];
    if (n + 5 > CKPT_MAX_PATH) return FALSE;
    memcpy(tmp, path, n);
    memcpy(tmp + n, ".tmp", 5);
    u64 maxn = 0;
    for (u32 i = 0; i < g->num_params; i++)
        if (g->numels[i] > maxn) maxn = g->numels[i];
    f32* buf = (f32*)malloc(maxn * F4);
    if (!buf) return FALSE;
    FILE* f = fopen(tmp, "wb");
    if (!f) { free(buf); return FALSE; }

    int ok = 1;
    u32 hdr[3] = { 1u, g->num_params, opt != NULL_PTR ? 1u : 0u };
    ok = ok && fwrite("TRLM", 1, 4, f) == 4;
    ok = ok && fwrite(hdr, sizeof(u32), 3, f) == 3;
    for (u32 i = 0; ok && i < g->num_params; i++) {
        const Tensor* t = &params[i]->value;
        ok = ok && fwrite(&t->ndim, sizeof(u32), 1, f) == 1;
        ok = ok && fwrite(t->shape, sizeof(u64), t->ndim, f) == t->ndim;
        hip_d2h(buf, dev_at(g->params, g->offsets[i]), g->numels[i] * F4);
        ok = ok && fwrite(buf, F4, g->numels[i], f) == g->numels[i];
    }
    if (opt != NULL_PTR) {
        for (u32 i = 0; ok && i < g->num_params; i++) {
            hip_d2h(buf, dev_at(g->adam_m, g->offsets[i]), g->numels[i] * F4);
            ok = ok && fwrite(buf, F4, g->numels[i], f) == g->numels[i];
            hip_d2h(buf, dev_at(g->adam_v, g->offsets[i]), g->numels[i] * F4);
            ok = ok && fwrite(buf, F4, g->numels[i], f) == g->numels[i];
        }
        ok = ok && fwrite(&opt->t, sizeof(u64), 1, f) == 1;
    }
    if (fclose(f) != 0) ok = 0;
    free(buf);
    if (ok) ok = rename(tmp, path) == 0;
    if (!ok) remove(tmp);
    return ok ? TRUE : FALSE;
}

bool32 gpu_trainer_checkpoint_load(GpuTrainer* g, const char* path, Node** params, AdamOptimizer* opt) {
    hip_set_current(&g->hip);
    if (!shapes_match(g, params, g->num_params)) return FALSE;
    FILE* f = fopen(path, "rb");
    if (!f) return FALSE;
    long sz = -1;
    if (fseek(f, 0, SEEK_END) == 0) sz = ftell(f);
    if (sz < 0 || fseek(f, 0, SEEK_SET) != 0) { fclose(f); return FALSE; }
    u64 size = (u64)sz;
    u8* b = (u8*)malloc(size ? size : 1);
    if (!b) { fclose(f); return FALSE; }
    int ok = fread(b, 1, size, f) == size;
    fclose(f);

    /* pass 1: validate everything, copy nothing */
    u32 version = 0, num = 0, has_opt = 0;
    u64 pos = 16, total = 0;
    u64* offs = (u64*)malloc((u64)g->num_params * sizeof(u64));
    if (!offs) ok = 0;
    if (ok) ok = size >= 16 && memcmp(b, "TRLM", 4) == 0;
    if (ok) {
        memcpy(&version, b + 4, 4);
        memcpy(&num, b + 8, 4);
        memcpy(&has_opt, b + 12, 4);
        ok = version == 1 && num == g->num_params && (opt == NULL_PTR || has_opt);
    }
    for (u32 i = 0; ok && i < g->num_params; i++) {
        const Tensor* t = &params[i]->value;
        u32 nd;
        if (pos + 4 > size) { ok = 0; break; }
        memcpy(&nd, b + pos, 4);
        pos += 4;
        if (nd != t->ndim) { ok = 0; break; }
        for (u32 d = 0; d < nd; d++) {
            u64 dim;
            if (pos + 8 > size) { ok = 0; break; }
            memcpy(&dim, b + pos, 8);
            pos += 8;
            if (dim != t->shape[d]) { ok = 0; break; }
        }
        if (!ok) break;
        u64 bytes = g->numels[i] * F4;
        if (pos + bytes > size) { ok = 0; break; }
        offs[i] = pos;
        pos += bytes;
        total += g->numels[i];
    }
    u64 opt_at = pos;
    if (ok && has_opt) pos += 2 * total * F4 + sizeof(u64);
    if (ok) ok = pos == size;

    /* pass 2: the file is consistent -- device buffers and host mirror */
    if (ok) {
        for (u32 i = 0; i < g->num_params; i++) {
            hip_h2d(dev_at(g->params, g->offsets[i]), b + offs[i], g->numels[i] * F4);
            memcpy(params[i]->value.data, b + offs[i], g->numels[i] * F4);
        }
        if (opt != NULL_PTR) {
            u64 p = opt_at;
            for (u32 i = 0; i < g->num_params; i++) {
                u64 bytes = g->numels[i] * F4;
                hip_h2d(dev_at(g->adam_m, g->offsets[i]), b + p, bytes);
                memcpy(opt->m[i].data, b + p, bytes);
                p += bytes;
                hip_h2d(dev_at(g->adam_v, g->offsets[i]), b + p, bytes);
                memcpy(opt->v[i].data, b + p, bytes);
                p += bytes;
            }
            memcpy(&opt->t, b + p, sizeof(u64));
        }
    }
    free(offs);
    free(b);
    return ok ? TRUE : FALSE;
}
