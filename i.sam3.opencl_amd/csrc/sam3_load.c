/* SPDX-License-Identifier: Unlicense
 *
 * sam3_load.c - checkpoint weights into device memory.
 *
 * pth_upload moves one tensor of an open checkpoint into a new device
 * buffer: the storage span the tensor covers goes from the file mapping
 * through two pinned staging buffers (the host copy into one overlaps
 * the DMA out of the other) into device memory, and k_pth_convert turns
 * it into the C-order tensor of the requested element type (float32,
 * half or bfloat16; strided views gathered). A contiguous tensor whose
 * storage type is already the requested one lands in its buffer
 * directly. The reference instead converts every tensor to float32 on
 * the host (pth_read_f32, pth_loader.c:962-1012), rounds weight matrices
 * to half there too and uploads (load_dev / load_dev_w,
 * sam3_model.c:52-76).
 *
 * On top: the reference's load helpers (sam3_ops.h:26-38) and sam_load /
 * sam_free for the image encoder trunk and the point-prompt decoder
 * (sam3_model.c:473-583, 657-758, 918-962, 1532).
 */
#include "hipb_internal.h"
#include "pth_loader.h"
#include "sam3_launch.h"

#include <hip/hip_runtime_api.h>

#include <math.h>
#include <pthread.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

#define STAGE_BYTES ((size_t)32 << 20)
/* Host threads of one staging copy, and the least bytes per thread. */
#define COPY_THREADS 8
#define COPY_MIN ((size_t)2 << 20)

#define TRUNK "detector.backbone.vision_backbone.trunk"
#define DEC "tracker.sam_mask_decoder"
#define PROMPT "tracker.sam_prompt_encoder"

static size_t elem_bytes(enum pth_dtype d)
{
    return d == PTH_C64 ? 8 : d == PTH_F32 ? 4 : 2;
}

static int stage_ready(struct hipb_backend *b)
{
    int i;

    for (i = 0; i < 2; i++) {
        if (!b->stage[i])
            hipb_check(hipHostMalloc(&b->stage[i], STAGE_BYTES,
                                     hipHostMallocDefault),
                       "hipHostMalloc (checkpoint staging)");
        if (!b->stage_ev[i])
            hipb_check(hipEventCreateWithFlags((hipEvent_t *)&b->stage_ev[i],
                                               hipEventDisableTiming),
                       "hipEventCreate (checkpoint staging)");
        if (hipb_failed())
            return 0;
    }
    return 1;
}

struct part {
    void *dst;
    const void *src;
    size_t n;
};

static void *copy_part(void *arg)
{
    const struct part *p = arg;

    memcpy(p->dst, p->src, p->n);
    return NULL;
}

/* memcpy split over up to COPY_THREADS threads: one core's copy from the
 * page cache into pinned memory runs far below the DMA rate. */
static void copy_wide(void *dst, const void *src, size_t n)
{
    struct part parts[COPY_THREADS];
    pthread_t th[COPY_THREADS];
    int started[COPY_THREADS] = {0};
    size_t per, off = 0;
    int k, nt = (int)(n / COPY_MIN);

    nt = nt < 1 ? 1 : nt > COPY_THREADS ? COPY_THREADS : nt;
    per = (n / (size_t)nt + 4095) & ~(size_t)4095;
    for (k = 0; k < nt; k++) {
        const size_t len = off >= n ? 0 : n - off < per ? n - off : per;

        parts[k].dst = (char *)dst + off;
        parts[k].src = (const char *)src + off;
        parts[k].n = len;
        off += len;
        if (k > 0 && len)
            started[k] = !pthread_create(&th[k], NULL, copy_part, &parts[k]);
    }
    copy_part(&parts[0]);
    for (k = 1; k < nt; k++) {
        if (started[k])
            pthread_join(th[k], NULL);
        else if (parts[k].n)
            copy_part(&parts[k]);
    }
}

/* n bytes of host memory to device address dst on the backend stream,
 * through the staging buffers in turn. */
static void h2d(struct hipb_backend *b, char *dst, const unsigned char *src,
                size_t n)
{
    const uintptr_t pg = (uintptr_t)sysconf(_SC_PAGESIZE);
    const uintptr_t a0 = (uintptr_t)src & ~(pg - 1);
    size_t off;

    /* Start the file read-ahead for the whole span. */
    madvise((void *)a0, (uintptr_t)src + n - a0, MADV_WILLNEED);
    for (off = 0; off < n && !hipb_failed(); off += STAGE_BYTES) {
        const size_t len = n - off < STAGE_BYTES ? n - off : STAGE_BYTES;
        const int k = b->stage_next;

        b->stage_next ^= 1;
        hipb_check(hipEventSynchronize((hipEvent_t)b->stage_ev[k]),
                   "hipEventSynchronize (checkpoint staging)");
        copy_wide(b->stage[k], src + off, len);
        hipb_check(hipMemcpyAsync(dst + off, b->stage[k], len,
                                  hipMemcpyHostToDevice,
                                  (hipStream_t)b->stream),
                   "hipMemcpyAsync (checkpoint upload)");
        hipb_check(hipEventRecord((hipEvent_t)b->stage_ev[k],
                                  (hipStream_t)b->stream),
                   "hipEventRecord (checkpoint staging)");
    }
}

hipb_mem pth_upload(struct hipb_backend *b, const struct pth_file *pf,
                    const struct pth_tensor *t, int dtype, const char *what)
{
    const size_t es = elem_bytes(t->dtype);
    const long n = pth_numel(t);
    long span = 1, expect = 1;
    int contiguous = 1, direct, d, err;
    hipb_mem out;
    void *raw;

    if (dtype < HIPB_F32 || dtype > HIPB_BF16) {
        hipb_fatal("pth_upload: invalid element type %d", dtype);
        return NULL;
    }
    if (t->dtype == PTH_C64 && dtype != HIPB_F32) {
        hipb_fatal("Tensor <%s> is complex, a real tensor is expected",
                   t->name);
        return NULL;
    }
    /* pth_open accepted the view only if storage_offset + span elements
     * lie inside the storage and the element count stays below 2^56, so
     * none of this overflows. */
    for (d = t->ndim - 1; d >= 0; d--) {
        if (t->shape[d] != 1 && t->stride[d] != expect)
            contiguous = 0;
        expect *= t->shape[d];
        span += (t->shape[d] - 1) * t->stride[d];
    }
    if (!stage_ready(b))
        return NULL;
    out = hipb_alloc_typed(b, (size_t)n * (t->dtype == PTH_C64 ? 2 : 1),
                           dtype, what);
    if (!out)
        return NULL;
    /* enum pth_dtype and HIPB_* agree on f32 / f16 / bf16; complex
     * elements are float pairs. */
    direct = contiguous && (t->dtype == PTH_C64 || (int)t->dtype == dtype);
    raw = direct ? out->ptr : hipb_scratch(b, (size_t)span * es);
    if (!raw) {
        hipb_release(&out);
        return NULL;
    }
    h2d(b, raw,
        pf->map + t->data_offset + (size_t)t->storage_offset * es,
        (size_t)span * es);
    if (!direct && !hipb_failed()) {
        hipb_run_begin(b);
        err = launch_pth_convert(raw, (int)t->dtype, out->ptr, dtype, n,
                                 t->ndim, t->shape, t->stride, contiguous,
                                 b->stream);
        hipb_run_end(b, err, "pth_convert", 0.0);
    }
    if (hipb_failed())
        hipb_release(&out);
    return out;
}

/* ------------------------------------------------- sam3_ops.h helpers */

static int weight_dtype(const struct hipb_backend *b)
{
    return b->fp16w ? HIPB_F16 : b->bf16 ? HIPB_BF16 : HIPB_F32;
}

static hipb_mem load_as(struct sam_model *m, const struct pth_file *pf,
                        const char *name, int ndim, const long *shape,
                        int dtype)
{
    const struct pth_tensor *t = pth_require(pf, name, ndim, shape);

    if (!t)
        return NULL;
    if (t->dtype == PTH_C64) {
        hipb_fatal("Tensor <%s> is complex, a real tensor is expected", name);
        return NULL;
    }
    return pth_upload(m->hip, pf, t, dtype, name);
}

hipb_mem load_dev(struct sam_model *m, const struct pth_file *pf,
                  const char *name, int ndim, const long *shape)
{
    return load_as(m, pf, name, ndim, shape, HIPB_F32);
}

hipb_mem load_dev_w(struct sam_model *m, const struct pth_file *pf,
                    const char *name, int ndim, const long *shape)
{
    return load_as(m, pf, name, ndim, shape, weight_dtype(m->hip));
}

hipb_mem load_dev_fmt(struct sam_model *m, const struct pth_file *pf,
                      int ndim, const long *shape, const char *fmt, ...)
{
    char name[256];
    va_list ap;

    va_start(ap, fmt);
    vsnprintf(name, sizeof(name), fmt, ap);
    va_end(ap);
    return load_dev(m, pf, name, ndim, shape);
}

hipb_mem load_dev_w_fmt(struct sam_model *m, const struct pth_file *pf,
                        int ndim, const long *shape, const char *fmt, ...)
{
    char name[256];
    va_list ap;

    va_start(ap, fmt);
    vsnprintf(name, sizeof(name), fmt, ap);
    va_end(ap);
    return load_dev_w(m, pf, name, ndim, shape);
}

float *load_host(const struct pth_file *pf, const char *name, int ndim,
                 const long *shape)
{
    const struct pth_tensor *t = pth_require(pf, name, ndim, shape);

    return t ? pth_read_f32(pf, t) : NULL;
}

void load_host_into(const struct pth_file *pf, const char *name, int ndim,
                    const long *shape, float *dst)
{
    float *h = load_host(pf, name, ndim, shape);

    if (h)
        memcpy(dst, h, (size_t)pth_numel(pth_find(pf, name)) * sizeof(float));
    free(h);
}

/* ------------------------------------------------- the trunk */

/* Sizes the trunk takes from the checkpoint (sam3_model.c:473-520). */
struct trunk_dims {
    long E, pt_side, patch, hd, heads, mlp, grid, win;
    int depth;
};

static long square_side(long n)
{
    long s = (long)llround(sqrt((double)n));

    return s * s == n ? s : -1;
}

static long rope_npos(const struct pth_file *pf, int i, long hd)
{
    char name[160];
    const struct pth_tensor *t;

    snprintf(name, sizeof(name), TRUNK ".blocks.%d.attn.freqs_cis", i);
    t = pth_require(pf, name, 2, (long[]){-1, hd / 2});
    return t ? t->shape[0] : -1;
}

/* The trunk's sizes, or 0 after a fatal error. The token grid is the
 * extent of the global-attention blocks' rope tables (72 x 72 in SAM 3,
 * SAM_GRID of the reference); the other blocks attend in windows of
 * the side of theirs. */
static int trunk_dims(const struct pth_file *pf, struct trunk_dims *k)
{
    const struct pth_tensor *t;
    char name[160];
    int i;

    memset(k, 0, sizeof(*k));
    t = pth_require(pf, TRUNK ".pos_embed", 3, (long[]){1, -1, -1});
    if (!t)
        return 0;
    k->E = t->shape[2];
    /* The pretraining grid plus the class token that SAM 3 drops. */
    k->pt_side = square_side(t->shape[1] - 1);
    for (k->depth = 0;; k->depth++) {
        snprintf(name, sizeof(name), TRUNK ".blocks.%d.norm1.weight",
                 k->depth);
        if (!pth_find(pf, name))
            break;
    }
    t = pth_require(pf, TRUNK ".blocks.0.attn.freqs_cis", 2, NULL);
    if (!t)
        return 0;
    k->hd = 2 * t->shape[1];
    if (k->hd != 64 || k->E % k->hd) {
        hipb_fatal("Unsupported attention head width %ld", k->hd);
        return 0;
    }
    k->heads = k->E / k->hd;
    t = pth_require(pf, TRUNK ".blocks.0.mlp.fc1.weight", 2,
                    (long[]){-1, k->E});
    if (!t)
        return 0;
    k->mlp = t->shape[0];
    t = pth_require(pf, TRUNK ".patch_embed.proj.weight", 4,
                    (long[]){k->E, 3, -1, -1});
    if (!t)
        return 0;
    k->patch = t->shape[2];
    if (t->shape[3] != k->patch) {
        hipb_fatal("Unsupported patch embedding in <%s>", pf->path);
        return 0;
    }
    for (i = 0; i < k->depth; i++) {
        const long side = square_side(rope_npos(pf, i, k->hd));

        if (hipb_failed())
            return 0;
        if (side < 1) {
            hipb_fatal("Unsupported attention extent in <%s>", pf->path);
            return 0;
        }
        if (side > k->grid)
            k->grid = side;
    }
    for (i = 0; i < k->depth; i++) {
        const long side = square_side(rope_npos(pf, i, k->hd));

        if (side == k->grid)
            continue;
        if (k->win && side != k->win) {
            hipb_fatal("Blocks with different window sizes in <%s>", pf->path);
            return 0;
        }
        k->win = side;
    }
    if (!k->win || !k->grid) {
        hipb_fatal("<%s> lacks windowed or global attention blocks", pf->path);
        return 0;
    }
    if (k->pt_side < 1 || k->grid % k->pt_side) {
        hipb_fatal("Unsupported position embedding in <%s>", pf->path);
        return 0;
    }
    return 1;
}

static void load_block(struct sam_model *m, const struct pth_file *pf, int i,
                       const struct trunk_dims *k, struct vit_block *b)
{
    const char *p = TRUNK ".blocks";
    const long E = k->E, M = k->mlp;

    b->n1w = load_dev_fmt(m, pf, 1, (long[]){E}, "%s.%d.norm1.weight", p, i);
    b->n1b = load_dev_fmt(m, pf, 1, (long[]){E}, "%s.%d.norm1.bias", p, i);
    b->n2w = load_dev_fmt(m, pf, 1, (long[]){E}, "%s.%d.norm2.weight", p, i);
    b->n2b = load_dev_fmt(m, pf, 1, (long[]){E}, "%s.%d.norm2.bias", p, i);
    b->qkvw = load_dev_w_fmt(m, pf, 2, (long[]){3 * E, E},
                             "%s.%d.attn.qkv.weight", p, i);
    b->qkvb = load_dev_fmt(m, pf, 1, (long[]){3 * E}, "%s.%d.attn.qkv.bias",
                           p, i);
    b->projw = load_dev_w_fmt(m, pf, 2, (long[]){E, E},
                              "%s.%d.attn.proj.weight", p, i);
    b->projb = load_dev_fmt(m, pf, 1, (long[]){E}, "%s.%d.attn.proj.bias", p,
                            i);
    b->l1w = load_dev_w_fmt(m, pf, 2, (long[]){M, E}, "%s.%d.mlp.fc1.weight",
                            p, i);
    b->l1b = load_dev_fmt(m, pf, 1, (long[]){M}, "%s.%d.mlp.fc1.bias", p, i);
    b->l2w = load_dev_w_fmt(m, pf, 2, (long[]){E, M}, "%s.%d.mlp.fc2.weight",
                            p, i);
    b->l2b = load_dev_fmt(m, pf, 1, (long[]){E}, "%s.%d.mlp.fc2.bias", p, i);
}

static hipb_mem load_rope(struct sam_model *m, const struct pth_file *pf,
                          int i)
{
    char name[160];
    const struct pth_tensor *t;

    snprintf(name, sizeof(name), TRUNK ".blocks.%d.attn.freqs_cis", i);
    t = pth_require(pf, name, 2, (long[]){-1, m->hd / 2});
    if (!t)
        return NULL;
    if (t->dtype != PTH_C64) {
        hipb_fatal("Tensor <%s> is not complex", name);
        return NULL;
    }
    /* Complex64 (re, im) = (cos, sin): the rope table's float pairs. */
    return pth_upload(m->hip, pf, t, HIPB_F32, name);
}

/* tile_abs_pos: the pretraining grid's embedding repeated over the
 * token grid, class token dropped (sam3_model.c:482-502). */
static hipb_mem load_pos(struct sam_model *m, const struct pth_file *pf,
                         long pt)
{
    const long G = m->grid, E = m->embed;
    float *pe = load_host(pf, TRUNK ".pos_embed", 3, (long[]){1, -1, E});
    float *pos;
    hipb_mem r = NULL;
    long i;

    if (!pe)
        return NULL;
    pos = malloc((size_t)G * G * E * sizeof(float));
    for (i = 0; i < G * G; i++) {
        const long y = i / G % pt, x = i % G % pt;

        memcpy(pos + (size_t)i * E, pe + (size_t)(1 + y * pt + x) * E,
               (size_t)E * sizeof(float));
    }
    r = hipb_upload(m->hip, pos, (size_t)G * G * E * sizeof(float),
                    "position embedding");
    free(pos);
    free(pe);
    return r;
}

/* ------------------------------------------------- the decoder */

static void load_attn(struct sam_model *m, const struct pth_file *pf,
                      const char *prefix, int dint, struct sam_attn_w *a)
{
    const long win[2] = {dint, SAM_DIM}, wout[2] = {SAM_DIM, dint};
    const long bin[1] = {dint}, bout[1] = {SAM_DIM};

    a->dint = dint;
    a->qw = load_dev_w_fmt(m, pf, 2, win, "%s.q_proj.weight", prefix);
    a->qb = load_dev_fmt(m, pf, 1, bin, "%s.q_proj.bias", prefix);
    a->kw = load_dev_w_fmt(m, pf, 2, win, "%s.k_proj.weight", prefix);
    a->kb = load_dev_fmt(m, pf, 1, bin, "%s.k_proj.bias", prefix);
    a->vw = load_dev_w_fmt(m, pf, 2, win, "%s.v_proj.weight", prefix);
    a->vb = load_dev_fmt(m, pf, 1, bin, "%s.v_proj.bias", prefix);
    a->ow = load_dev_w_fmt(m, pf, 2, wout, "%s.out_proj.weight", prefix);
    a->ob = load_dev_fmt(m, pf, 1, bout, "%s.out_proj.bias", prefix);
}

/* The decoder's weights (sam3_model.c:657-758). The upscaling and MLP
 * head matrices are device GEMM operands here, in the weight type. */
static void load_decoder(struct sam_model *m, const struct pth_file *pf,
                         struct sam_decoder *d)
{
    const long v256[1] = {SAM_DIM}, e1[2] = {1, SAM_DIM};
    const char *tl = DEC ".transformer.layers";
    char name[200];
    int i, j;

    load_host_into(pf, PROMPT ".pe_layer.positional_encoding_gaussian_matrix",
                   2, (long[]){2, SAM_DIM / 2}, d->gauss);
    for (i = 0; i < 4; i++) {
        snprintf(name, sizeof(name), PROMPT ".point_embeddings.%d.weight", i);
        load_host_into(pf, name, 2, e1, d->point_emb[i]);
    }
    load_host_into(pf, PROMPT ".not_a_point_embed.weight", 2, e1,
                   d->not_a_point);
    load_host_into(pf, PROMPT ".no_mask_embed.weight", 2, e1, d->no_mask);
    load_host_into(pf, DEC ".obj_score_token.weight", 2, e1, d->obj_token);
    load_host_into(pf, DEC ".iou_token.weight", 2, e1, d->iou_token);
    load_host_into(pf, DEC ".mask_tokens.weight", 2, (long[]){4, SAM_DIM},
                   d->mask_tokens);
    for (i = 0; i < 2 && !hipb_failed(); i++) {
        struct sam_dec_layer *L = &d->layers[i];

        snprintf(name, sizeof(name), "%s.%d.self_attn", tl, i);
        load_attn(m, pf, name, SAM_DIM, &L->self);
        snprintf(name, sizeof(name), "%s.%d.cross_attn_token_to_image", tl, i);
        load_attn(m, pf, name, SAM_DIM / 2, &L->t2i);
        snprintf(name, sizeof(name), "%s.%d.cross_attn_image_to_token", tl, i);
        load_attn(m, pf, name, SAM_DIM / 2, &L->i2t);
        L->n1w = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm1.weight", tl, i);
        L->n1b = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm1.bias", tl, i);
        L->n2w = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm2.weight", tl, i);
        L->n2b = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm2.bias", tl, i);
        L->n3w = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm3.weight", tl, i);
        L->n3b = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm3.bias", tl, i);
        L->n4w = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm4.weight", tl, i);
        L->n4b = load_dev_fmt(m, pf, 1, v256, "%s.%d.norm4.bias", tl, i);
        L->m1w = load_dev_w_fmt(m, pf, 2, (long[]){2048, SAM_DIM},
                                "%s.%d.mlp.lin1.weight", tl, i);
        L->m1b = load_dev_fmt(m, pf, 1, (long[]){2048}, "%s.%d.mlp.lin1.bias",
                              tl, i);
        L->m2w = load_dev_w_fmt(m, pf, 2, (long[]){SAM_DIM, 2048},
                                "%s.%d.mlp.lin2.weight", tl, i);
        L->m2b = load_dev_fmt(m, pf, 1, v256, "%s.%d.mlp.lin2.bias", tl, i);
    }
    load_attn(m, pf, DEC ".transformer.final_attn_token_to_image",
              SAM_DIM / 2, &d->final_t2i);
    d->nfw = load_dev(m, pf, DEC ".transformer.norm_final_attn.weight", 1,
                      v256);
    d->nfb = load_dev(m, pf, DEC ".transformer.norm_final_attn.bias", 1,
                      v256);
    d->up0w = load_dev_w(m, pf, DEC ".output_upscaling.0.weight", 4,
                         (long[]){SAM_DIM, 64, 2, 2});
    d->up0b = load_dev(m, pf, DEC ".output_upscaling.0.bias", 1,
                       (long[]){64});
    d->up1w = load_dev(m, pf, DEC ".output_upscaling.1.weight", 1,
                       (long[]){64});
    d->up1b = load_dev(m, pf, DEC ".output_upscaling.1.bias", 1,
                       (long[]){64});
    d->up3w = load_dev_w(m, pf, DEC ".output_upscaling.3.weight", 4,
                         (long[]){64, 32, 2, 2});
    d->up3b = load_dev(m, pf, DEC ".output_upscaling.3.bias", 1,
                       (long[]){32});
    for (i = 0; i < 4; i++)
        for (j = 0; j < 3; j++) {
            const long rows = j == 2 ? 32 : SAM_DIM;

            d->hyper_w[i][j] = load_dev_w_fmt(
                m, pf, 2, (long[]){rows, SAM_DIM},
                "%s.output_hypernetworks_mlps.%d.layers.%d.weight", DEC, i, j);
            d->hyper_b[i][j] = load_dev_fmt(
                m, pf, 1, (long[]){rows},
                "%s.output_hypernetworks_mlps.%d.layers.%d.bias", DEC, i, j);
        }
    for (j = 0; j < 3; j++) {
        const long rows = j == 2 ? 4 : SAM_DIM;

        d->iou_w[j] = load_dev_w_fmt(m, pf, 2, (long[]){rows, SAM_DIM},
                                     "%s.iou_prediction_head.layers.%d.weight",
                                     DEC, j);
        d->iou_b[j] = load_dev_fmt(m, pf, 1, (long[]){rows},
                                   "%s.iou_prediction_head.layers.%d.bias",
                                   DEC, j);
    }
}

static void release_attn(struct sam_attn_w *a)
{
    hipb_release(&a->qw);
    hipb_release(&a->qb);
    hipb_release(&a->kw);
    hipb_release(&a->kb);
    hipb_release(&a->vw);
    hipb_release(&a->vb);
    hipb_release(&a->ow);
    hipb_release(&a->ob);
}

static void release_decoder(struct sam_decoder *d)
{
    hipb_mem *v[] = {&d->nfw, &d->nfb, &d->up0w, &d->up0b, &d->up1w,
                     &d->up1b, &d->up3w, &d->up3b, &d->emb, &d->feat_s0,
                     &d->feat_s1};
    size_t k;
    int i, j;

    for (i = 0; i < 2; i++) {
        struct sam_dec_layer *L = &d->layers[i];
        hipb_mem *lv[] = {&L->n1w, &L->n1b, &L->n2w, &L->n2b, &L->n3w,
                          &L->n3b, &L->n4w, &L->n4b, &L->m1w, &L->m1b,
                          &L->m2w, &L->m2b};

        release_attn(&L->self);
        release_attn(&L->t2i);
        release_attn(&L->i2t);
        for (k = 0; k < sizeof(lv) / sizeof(lv[0]); k++)
            hipb_release(lv[k]);
    }
    release_attn(&d->final_t2i);
    for (k = 0; k < sizeof(v) / sizeof(v[0]); k++)
        hipb_release(v[k]);
    for (i = 0; i < 4; i++)
        for (j = 0; j < 3; j++) {
            hipb_release(&d->hyper_w[i][j]);
            hipb_release(&d->hyper_b[i][j]);
        }
    for (j = 0; j < 3; j++) {
        hipb_release(&d->iou_w[j]);
        hipb_release(&d->iou_b[j]);
    }
}

/* ------------------------------------------------- sam_load / sam_free */

int sam_is_sam3(const struct pth_file *pf)
{
    return pth_find(pf, TRUNK ".pos_embed") &&
           pth_find(pf, DEC ".iou_token.weight") &&
           pth_find(pf, "detector.backbone.vision_backbone.sam2_convs.0.conv_1x1.weight");
}

void sam_load(struct sam_model *m, struct hipb_backend *b,
              const struct pth_file *pf, int batch, int point_head)
{
    struct trunk_dims k;
    struct vit_block *blocks;
    struct sam_decoder *d;
    int i, rope_win = -1, rope_glob = -1;

    memset(m, 0, sizeof(*m));
    if (!trunk_dims(pf, &k))
        return;
    blocks = calloc((size_t)k.depth, sizeof(*blocks));
    for (i = 0; i < k.depth; i++)
        blocks[i].window =
            square_side(rope_npos(pf, i, k.hd)) == k.grid ? 0 : (int)k.win;
    /* Work buffers sized for these blocks (alloc_buffers). */
    sam_path_init(m, b, (int)k.grid, (int)k.E, (int)k.heads, (int)k.hd,
                  (int)k.mlp, blocks, k.depth);
    m->blocks = blocks;
    m->depth = k.depth;
    m->owns_weights = 1;
    if (hipb_failed())
        return;
    m->patch = (int)k.patch;
    m->pe_w = load_dev_w(m, pf, TRUNK ".patch_embed.proj.weight", 4,
                         (long[]){k.E, 3, k.patch, k.patch});
    m->lnpw = load_dev(m, pf, TRUNK ".ln_pre.weight", 1, (long[]){k.E});
    m->lnpb = load_dev(m, pf, TRUNK ".ln_pre.bias", 1, (long[]){k.E});
    m->pos = load_pos(m, pf, k.pt_side);
    for (i = 0; i < k.depth && !hipb_failed(); i++) {
        load_block(m, pf, i, &k, &blocks[i]);
        if (blocks[i].window && rope_win < 0)
            m->rope_win = load_rope(m, pf, rope_win = i);
        else if (!blocks[i].window && rope_glob < 0)
            m->rope_glob = load_rope(m, pf, rope_glob = i);
    }
    if (hipb_failed() || !point_head)
        return;
    d = calloc(1, sizeof(*d));
    m->dec = d;
    d->img = m->grid * m->patch;
    load_decoder(m, pf, d);
    if (hipb_failed())
        return;
    sam_dec_init(m, d, batch);
}

void sam_free(struct sam_model *m)
{
    struct sam_decoder *d = m->dec;
    struct vit_block *blocks = m->blocks;
    int i, owned = m->owns_weights, depth = m->depth;

    if (m->hip)
        hipb_finish(m->hip);
    if (owned) {
        hipb_mem *v[] = {&m->pe_w, &m->pos, &m->lnpw, &m->lnpb, &m->rope_win,
                         &m->rope_glob};
        size_t k;

        for (k = 0; k < sizeof(v) / sizeof(v[0]); k++)
            hipb_release(v[k]);
        for (i = 0; i < depth; i++) {
            struct vit_block *b = &blocks[i];
            hipb_mem *bv[] = {&b->n1w, &b->n1b, &b->qkvw, &b->qkvb,
                              &b->projw, &b->projb, &b->n2w, &b->n2b,
                              &b->l1w, &b->l1b, &b->l2w, &b->l2b};

            for (k = 0; k < sizeof(bv) / sizeof(bv[0]); k++)
                hipb_release(bv[k]);
        }
    }
    /* sam_path_free runs sam_dec_free (the decoder's work buffers). */
    sam_path_free(m);
    if (owned) {
        if (d) {
            release_decoder(d);
            free(d);
        }
        free(blocks);
    }
    memset(m, 0, sizeof(*m));
}
