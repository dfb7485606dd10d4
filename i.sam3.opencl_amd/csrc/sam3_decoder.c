/* SPDX-License-Identifier: Unlicense
 *
 * sam3_decoder.c - the point-prompt mask decoder on HIP: prompt tokens,
 * the two-way transformer (self attention, token -> image and image ->
 * token attention, token MLP), the output upscaling, the hypernetwork
 * and IoU heads, the low-resolution logits and the postprocessing
 * (sam3_model.c:1212-1530), over the operators of sam3_ops.c.
 *
 * The host-side parts (prompt encoding, the small MLP heads, hole
 * filling) are plain C as in the reference; the tensor work is queued on
 * the backend's stream.
 */
#include "hipb_internal.h"
#include "sam3_launch.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define NTOK 8         /* prompt tokens per prompt (sam3_model.c:35) */
#define DEC_EPS 1e-5f  /* decoder LayerNorm eps (sam3_model.c:31) */
#define LN2D_EPS 1e-6f /* LayerNorm2d of the upscaling (sam3_model.c:32) */

/* PositionEmbeddingRandom of normalized (x, y) in [0, 1]
 * (sam3_model.c:760-773). */
static void pe_encode(const struct sam_decoder *d, float x, float y,
                      float *out)
{
    int i;

    x = 2.0f * x - 1.0f;
    y = 2.0f * y - 1.0f;
    for (i = 0; i < SAM_DIM / 2; i++) {
        float v = x * d->gauss[i] + y * d->gauss[SAM_DIM / 2 + i];

        v *= 2.0f * (float)M_PI;
        out[i] = sinf(v);
        out[SAM_DIM / 2 + i] = cosf(v);
    }
}

static hipb_mem dalloc(struct sam_model *m, size_t floats, const char *what)
{
    return hipb_alloc(m->hip, floats * sizeof(float), what);
}

void sam_dec_init(struct sam_model *m, struct sam_decoder *d, int batch)
{
    const long G = m->grid, T = G * G, P = batch;
    float *pe;
    long x, y;

    if (G < 1 || batch < 1 || d->img < 1) {
        hipb_fatal("sam_dec_init: invalid grid %ld, batch %d or image side %d",
                   G, batch, d->img);
        return;
    }
    m->dec = d;
    d->batch = batch;
    d->src = dalloc(m, T * SAM_DIM, "decoder src");
    d->srcpe = dalloc(m, T * SAM_DIM, "decoder src+pe");
    d->kp0 = dalloc(m, T * 128, "decoder k0");
    d->vp0 = dalloc(m, T * 128, "decoder v0");
    d->qp0 = dalloc(m, T * 128, "decoder q0");
    pe = malloc(T * SAM_DIM * sizeof(float));
    for (y = 0; y < G; y++)
        for (x = 0; x < G; x++)
            pe_encode(d, (x + 0.5f) / G, (y + 0.5f) / G,
                      pe + (y * G + x) * SAM_DIM);
    d->pe_img = hipb_upload(m->hip, pe, T * SAM_DIM * sizeof(float),
                            "decoder pe");
    free(pe);
    d->qpe = dalloc(m, P * NTOK * SAM_DIM, "query pe");
    d->qry = dalloc(m, P * NTOK * SAM_DIM, "queries");
    d->qin = dalloc(m, P * NTOK * SAM_DIM, "queries+pe");
    d->sq = dalloc(m, P * NTOK * SAM_DIM, "token q");
    d->sk = dalloc(m, P * NTOK * SAM_DIM, "token k");
    d->sv = dalloc(m, P * NTOK * SAM_DIM, "token v");
    d->so = dalloc(m, P * NTOK * SAM_DIM, "token attention");
    d->sh = dalloc(m, P * NTOK * 2048, "token mlp");
    d->keys = dalloc(m, P * T * SAM_DIM, "keys");
    d->kin = dalloc(m, P * T * SAM_DIM, "keys+pe");
    d->bq = dalloc(m, P * T * 128, "image q");
    d->bk = dalloc(m, P * T * 128, "image k");
    d->bv = dalloc(m, P * T * 128, "image v");
    d->bo = dalloc(m, P * T * 128, "image attention");
    if (!m->hip->bf16) {
        /* The fp32 path's upscaled maps (the bf16 path fuses them away). */
        d->u1 = dalloc(m, P * 4 * T * 64, "upscaling 1");
        d->g2 = dalloc(m, P * 4 * T * 128, "upscaling 2 gemm");
        d->u2 = dalloc(m, P * 16 * T * 32, "upscaling 2");
    }
    d->hyper = dalloc(m, P * 3 * 32, "hypernetwork");
    d->lowres = dalloc(m, P * 3 * 16 * T, "low-res masks");
    d->h_queries = malloc(P * NTOK * SAM_DIM * sizeof(float));
    d->h_lowres = malloc(P * 3 * 16 * T * sizeof(float));
    d->sel = hipb_alloc(m->hip, P * 3 * sizeof(int), "mask selection");
    d->stats = hipb_alloc(m->hip, P * 3 * 6 * sizeof(int), "mask statistics");
    d->mask = NULL;
    d->mask_cap = 0;
    if (m->hip->bf16) {
        d->fold_w = hipb_alloc_typed(m->hip, P * 64 * SAM_DIM, HIPB_BF16,
                                     "folded image queries");
        d->fold_b = dalloc(m, P * 64, "folded score bias");
        d->fold_y = hipb_alloc_typed(m->hip, P * SAM_DIM * 64, HIPB_BF16,
                                     "folded output projection");
        d->up_w1t = hipb_alloc_typed(m->hip, 256 * 256, HIPB_BF16,
                                     "upscaling weights 1");
        d->up_w2t = hipb_alloc_typed(m->hip, 128 * 64, HIPB_BF16,
                                     "upscaling weights 2");
        d->t2i_part = dalloc(m, (2L * m->hip->cu_count + P) * 64 * 258,
                             "token -> image partials");
        d->t2i_z = dalloc(m, P * 64 * SAM_DIM, "token -> image key sums");
        d->fold_c = hipb_alloc_typed(m->hip, P * 64 * 16, HIPB_BF16,
                                     "folded token rows");
        d->pe_q1 = hipb_alloc_typed(m->hip, T * 128, HIPB_BF16,
                                    "PE image-query projection");
        d->pe_k1 = hipb_alloc_typed(m->hip, T * 128, HIPB_BF16,
                                    "PE key projection");
        d->pe_kf = hipb_alloc_typed(m->hip, T * 128, HIPB_BF16,
                                    "PE final key projection");
    }
}

static void dec_graph_drop(struct sam_decoder *d)
{
    if (d->graph_exec)
        hipGraphExecDestroy((hipGraphExec_t)d->graph_exec);
    if (d->graph)
        hipGraphDestroy((hipGraph_t)d->graph);
    d->graph_exec = d->graph = NULL;
    d->graph_P = 0;
}

void sam_dec_free(struct sam_model *m)
{
    struct sam_decoder *d = m->dec;
    size_t i;

    if (!d)
        return;
    hipb_mem *bufs[] = {&d->src, &d->pe_img, &d->srcpe, &d->kp0, &d->vp0,
                        &d->qp0, &d->qpe, &d->qry, &d->qin, &d->sq, &d->sk,
                        &d->sv, &d->so, &d->sh, &d->keys, &d->kin, &d->bq,
                        &d->bk, &d->bv, &d->bo, &d->u1, &d->g2, &d->u2,
                        &d->hyper, &d->lowres, &d->mask, &d->sel, &d->stats,
                        &d->fold_w, &d->fold_b, &d->fold_y, &d->up_w1t,
                        &d->up_w2t, &d->t2i_part, &d->t2i_z, &d->fold_c,
                        &d->pe_q1, &d->pe_k1, &d->pe_kf};

    if (m->hip)
        hipb_finish(m->hip);
    dec_graph_drop(d);
    for (i = 0; i < sizeof(bufs) / sizeof(bufs[0]); i++)
        hipb_release(bufs[i]);
    free(d->h_queries);
    free(d->h_lowres);
    d->h_queries = d->h_lowres = NULL;
    d->mask_cap = 0;
    m->dec = NULL;
}

static struct sam_decoder *dec_of(struct sam_model *m, const char *op)
{
    if (!m->dec)
        hipb_fatal("%s: no decoder (sam_dec_init)", op);
    return m->dec;
}

void sam_dec_prepare(struct sam_model *m)
{
    struct sam_decoder *d = dec_of(m, "sam_dec_prepare");
    const long T = (long)m->grid * m->grid;
    const struct sam_dec_layer *L0;
    hipb_mem nm;

    if (!d)
        return;
    L0 = &d->layers[0];
    nm = hipb_upload(m->hip, d->no_mask, SAM_DIM * sizeof(float),
                     "no-mask embedding");
    if (!nm)
        return;
    add_bcast(m, d->src, d->emb, nm, T * SAM_DIM, SAM_DIM);
    add_bcast(m, d->srcpe, d->src, d->pe_img, T * SAM_DIM, T * SAM_DIM);
    linear(m, (int)T, SAM_DIM, 128, d->srcpe, 0, L0->t2i.kw, L0->t2i.kb,
           d->kp0, 0, ACT_NONE, 0);
    linear(m, (int)T, SAM_DIM, 128, d->src, 0, L0->t2i.vw, L0->t2i.vb, d->vp0,
           0, ACT_NONE, 0);
    linear(m, (int)T, SAM_DIM, 128, d->srcpe, 0, L0->i2t.qw, L0->i2t.qb,
           d->qp0, 0, ACT_NONE, 0);
    if (d->fold_w) {
        /* The position term of the fused layer-1 and final blocks: PE
         * through the projections that meet it there, without their
         * biases (the fused blocks add those through the folds). */
        const struct sam_dec_layer *L1 = &d->layers[1];

        linear(m, (int)T, SAM_DIM, 128, d->pe_img, 0, L1->i2t.qw, NULL,
               d->pe_q1, 0, ACT_NONE, 0);
        linear(m, (int)T, SAM_DIM, 128, d->pe_img, 0, L1->t2i.kw, NULL,
               d->pe_k1, 0, ACT_NONE, 0);
        linear(m, (int)T, SAM_DIM, 128, d->pe_img, 0, d->final_t2i.kw, NULL,
               d->pe_kf, 0, ACT_NONE, 0);
    }
    hipb_finish(m->hip);
    hipb_release(&nm);
}

void t2i_attention(struct sam_model *m, int P, const struct sam_attn_w *a)
{
    struct sam_decoder *d = dec_of(m, "t2i_attention");
    const long T = (long)m->grid * m->grid, n = (long)P * NTOK * SAM_DIM;

    if (!d)
        return;
    if (P < 1 || P > d->batch) {
        hipb_fatal("t2i_attention: %d prompts for a batch of %d", P,
                   d->batch);
        return;
    }
    add_bcast(m, d->qin, d->qry, d->qpe, n, n);
    if (d->fold_w) {
        /* bf16: the queries folded through the key projection, then one
         * pass over the prompt's keys (keys + PE formed on the fly, the
         * key and value projections never applied to the 256-wide image
         * tokens), then Wv per head, then the output projection. kin is
         * not written: the fused image -> token block forms it itself. */
        struct hipb_backend *be = m->hip;
        const int nblk = (int)((T + 63) / 64);
        int nsplit = (2 * be->cu_count + P - 1) / P, err;
        /* The position term needs PE through this block's key projection,
         * cached per image for the two blocks that attend to per-prompt
         * keys. */
        const hipb_mem pk = a == &d->layers[1].t2i ? d->pe_k1
                            : a == &d->final_t2i   ? d->pe_kf
                                                   : NULL;

        if (!pk) {
            hipb_fatal("t2i_attention: precision=bf16 runs the layer-1 and "
                       "final token -> image blocks only");
            return;
        }
        if (nsplit > nblk)
            nsplit = nblk;

        linear(m, P * NTOK, SAM_DIM, 128, d->qin, 0, a->qw, a->qb, d->sq, 0,
               ACT_NONE, 0);
        if (hipb_failed())
            return;
        hipb_run_begin(be);
        err = launch_i2t_fold(d->sq->ptr, NULL, 1, a->kw->ptr, a->kw->dtype,
                              NULL, NULL, 0,
                              1.4426950408889634f / sqrtf(16.0f), P,
                              d->fold_w->ptr, NULL, NULL, d->fold_c->ptr,
                              be->stream);
        hipb_run_end(be, err, "t2i_fold", 0.0);
        hipb_run_begin(be);
        err = launch_t2i_fused(d->keys->ptr, pk->ptr, d->fold_w->ptr,
                               d->fold_c->ptr, d->t2i_part->ptr,
                               d->t2i_z->ptr, a->vw->ptr, a->vw->dtype,
                               a->vb->ptr, d->so->ptr, (int)T, P, nsplit,
                               be->stream);
        hipb_run_end(be, err, "t2i_fused", 4.0 * P * 64.0 * T * SAM_DIM);
        linear(m, P * NTOK, 128, SAM_DIM, d->so, 0, a->ow, a->ob, d->qry, 0,
               ACT_NONE, 1);
        return;
    }
    add_bcast(m, d->kin, d->keys, d->pe_img, P * T * SAM_DIM, T * SAM_DIM);
    linear(m, P * NTOK, SAM_DIM, 128, d->qin, 0, a->qw, a->qb, d->sq, 0,
           ACT_NONE, 0);
    linear(m, (int)(P * T), SAM_DIM, 128, d->kin, 0, a->kw, a->kb, d->bk, 0,
           ACT_NONE, 0);
    linear(m, (int)(P * T), SAM_DIM, 128, d->keys, 0, a->vw, a->vb, d->bv, 0,
           ACT_NONE, 0);
    mha(m, P, NTOK, (int)T, 128, d->sq, NTOK * 128, d->bk, T * 128, d->bv,
        T * 128, d->so);
    linear(m, P * NTOK, 128, SAM_DIM, d->so, 0, a->ow, a->ob, d->qry, 0,
           ACT_NONE, 1);
}

void i2t_attention(struct sam_model *m, int layer, int P)
{
    struct sam_decoder *d = dec_of(m, "i2t_attention");
    const long T = (long)m->grid * m->grid, n = (long)P * NTOK * SAM_DIM;
    const struct sam_dec_layer *L;

    if (!d)
        return;
    if (P < 1 || P > d->batch || layer < 0 || layer > 1) {
        hipb_fatal("i2t_attention: layer %d, %d prompts for a batch of %d",
                   layer, P, d->batch);
        return;
    }
    L = &d->layers[layer];
    add_bcast(m, d->qin, d->qry, d->qpe, n, n);
    if (d->fold_w) {
        /* bf16: the token keys / values as in the reference, then the
         * folded block, one pass over the image tokens (keys + PE formed
         * on the fly in layer 1, so kin is not read). */
        struct hipb_backend *be = m->hip;
        const float s = 1.4426950408889634f / sqrtf(16.0f);
        int err;

        linear(m, P * NTOK, SAM_DIM, 128, d->qin, 0, L->i2t.kw, L->i2t.kb,
               d->sk, 0, ACT_NONE, 0);
        linear(m, P * NTOK, SAM_DIM, 128, d->qry, 0, L->i2t.vw, L->i2t.vb,
               d->sv, 0, ACT_NONE, 0);
        if (hipb_failed())
            return;
        hipb_run_begin(be);
        err = launch_i2t_fold(d->sk->ptr, d->sv->ptr, layer,
                              layer ? L->i2t.qw->ptr : NULL,
                              L->i2t.qw->dtype, layer ? L->i2t.qb->ptr : NULL,
                              L->i2t.ow->ptr, L->i2t.ow->dtype, s, P,
                              d->fold_w->ptr, d->fold_b->ptr, d->fold_y->ptr,
                              layer ? d->fold_c->ptr : NULL, be->stream);
        hipb_run_end(be, err, "i2t_fold", 0.0);
        hipb_run_begin(be);
        err = launch_i2t_fused(layer ? d->keys->ptr : d->qp0->ptr,
                               layer ? T * SAM_DIM : 0, layer ? 256 : 128,
                               layer ? d->pe_q1->ptr : NULL,
                               layer ? d->fold_c->ptr : NULL, d->fold_w->ptr,
                               d->fold_b->ptr, d->fold_y->ptr, L->i2t.ob->ptr,
                               layer ? d->keys->ptr : d->src->ptr,
                               layer ? T * SAM_DIM : 0, L->n4w->ptr,
                               L->n4b->ptr, d->keys->ptr, (int)T, P, DEC_EPS,
                               be->stream);
        hipb_run_end(be, err, "i2t_fused",
                     4.0 * P * T * 64.0 * ((layer ? 256 : 128) + SAM_DIM));
        return;
    }
    if (layer == 0) {
        linear(m, P * NTOK, SAM_DIM, 128, d->qin, 0, L->i2t.kw, L->i2t.kb,
               d->sk, 0, ACT_NONE, 0);
        linear(m, P * NTOK, SAM_DIM, 128, d->qry, 0, L->i2t.vw, L->i2t.vb,
               d->sv, 0, ACT_NONE, 0);
        mha(m, P, (int)T, NTOK, 128, d->qp0, 0, d->sk, NTOK * 128, d->sv,
            NTOK * 128, d->bo);
        linear(m, (int)(P * T), 128, SAM_DIM, d->bo, 0, L->i2t.ow, L->i2t.ob,
               d->keys, 0, ACT_NONE, 0);
        add_bcast(m, d->keys, d->keys, d->src, P * T * SAM_DIM, T * SAM_DIM);
    }
    else {
        linear(m, (int)(P * T), SAM_DIM, 128, d->kin, 0, L->i2t.qw,
               L->i2t.qb, d->bq, 0, ACT_NONE, 0);
        linear(m, P * NTOK, SAM_DIM, 128, d->qin, 0, L->i2t.kw, L->i2t.kb,
               d->sk, 0, ACT_NONE, 0);
        linear(m, P * NTOK, SAM_DIM, 128, d->qry, 0, L->i2t.vw, L->i2t.vb,
               d->sv, 0, ACT_NONE, 0);
        mha(m, P, (int)T, NTOK, 128, d->bq, T * 128, d->sk, NTOK * 128,
            d->sv, NTOK * 128, d->bo);
        linear(m, (int)(P * T), 128, SAM_DIM, d->bo, 0, L->i2t.ow, L->i2t.ob,
               d->keys, 0, ACT_NONE, 1);
    }
    layernorm(m, P * T, SAM_DIM, d->keys, d->keys, L->n4w, L->n4b, DEC_EPS,
              ACT_NONE);
}

/* Prompt-token self attention (sam3_model.c:1274-1286 for layer 0, no
 * positional encoding and no residual; 1316-1327 for layer 1), norm1. */
static void self_attention(struct sam_model *m, int layer, int P)
{
    struct sam_decoder *d = m->dec;
    const struct sam_dec_layer *L = &d->layers[layer];
    const long n = (long)P * NTOK * SAM_DIM;
    hipb_mem qk = d->qry;

    if (layer) {
        add_bcast(m, d->qin, d->qry, d->qpe, n, n);
        qk = d->qin;
    }
    linear(m, P * NTOK, SAM_DIM, SAM_DIM, qk, 0, L->self.qw, L->self.qb,
           d->sq, 0, ACT_NONE, 0);
    linear(m, P * NTOK, SAM_DIM, SAM_DIM, qk, 0, L->self.kw, L->self.kb,
           d->sk, 0, ACT_NONE, 0);
    linear(m, P * NTOK, SAM_DIM, SAM_DIM, d->qry, 0, L->self.vw, L->self.vb,
           d->sv, 0, ACT_NONE, 0);
    mha(m, P, NTOK, NTOK, SAM_DIM, d->sq, NTOK * SAM_DIM, d->sk,
        NTOK * SAM_DIM, d->sv, NTOK * SAM_DIM, d->so);
    linear(m, P * NTOK, SAM_DIM, SAM_DIM, d->so, 0, L->self.ow, L->self.ob,
           d->qry, 0, ACT_NONE, layer);
    layernorm(m, P * NTOK, SAM_DIM, d->qry, d->qry, L->n1w, L->n1b, DEC_EPS,
              ACT_NONE);
}

static void token_mlp(struct sam_model *m, int P,
                      const struct sam_dec_layer *L)
{
    struct sam_decoder *d = m->dec;

    linear(m, P * NTOK, SAM_DIM, 2048, d->qry, 0, L->m1w, L->m1b, d->sh, 0,
           ACT_RELU, 0);
    linear(m, P * NTOK, 2048, SAM_DIM, d->sh, 0, L->m2w, L->m2b, d->qry, 0,
           ACT_NONE, 1);
}

void convt_scatter(struct sam_model *m, hipb_mem G, hipb_mem out,
                   hipb_mem bias, hipb_mem add, int P, int H, int W, int Co,
                   int act)
{
    struct hipb_backend *be = m->hip;
    const size_t total = (size_t)P * 4 * H * W * Co;
    int err;

    if (P < 1 || H < 1 || W < 1 || Co < 1 || act < ACT_NONE ||
        act > ACT_RELU) {
        hipb_fatal("convt_scatter: invalid shape P=%d H=%d W=%d Co=%d", P, H,
                   W, Co);
        return;
    }
    if (!G || !out || !bias || G->dtype != HIPB_F32 ||
        out->dtype != HIPB_F32 || hipb_count(G) < total ||
        hipb_count(out) < total || hipb_count(bias) < (size_t)Co ||
        (add && hipb_count(add) < (size_t)4 * H * W * Co)) {
        hipb_fatal("convt_scatter: operand missing or too small");
        return;
    }
    hipb_run_begin(be);
    err = launch_convt_scatter(G->ptr, out->ptr, bias->ptr,
                               add ? add->ptr : NULL, P, H, W, Co, act,
                               be->stream);
    hipb_run_end(be, err, "convt_scatter", 0.0);
}

/* The device part of sam_decode for P prompts whose tokens are in qpe /
 * qry: the two-way transformer, the hypernetwork and IoU heads (raw IoU
 * outputs in sv), the upscaling and the logits. Host-synchronisation
 * free, so that sam_dec_graph can capture it. */
static void dec_kernels(struct sam_model *m, int P)
{
    struct sam_decoder *d = m->dec;
    const int G = m->grid;
    const long T = (long)G * G, n = (long)P * NTOK * SAM_DIM;
    const struct sam_dec_layer *L0 = &d->layers[0], *L1 = &d->layers[1];
    int i, err;

    /* Layer 0: self attention, token -> image attention on the shared
     * image keys (stride 0), token MLP, image -> token attention. */
    self_attention(m, 0, P);
    add_bcast(m, d->qin, d->qry, d->qpe, n, n);
    linear(m, P * NTOK, SAM_DIM, 128, d->qin, 0, L0->t2i.qw, L0->t2i.qb,
           d->sq, 0, ACT_NONE, 0);
    mha(m, P, NTOK, (int)T, 128, d->sq, NTOK * 128, d->kp0, 0, d->vp0, 0,
        d->so);
    linear(m, P * NTOK, 128, SAM_DIM, d->so, 0, L0->t2i.ow, L0->t2i.ob,
           d->qry, 0, ACT_NONE, 1);
    layernorm(m, P * NTOK, SAM_DIM, d->qry, d->qry, L0->n2w, L0->n2b,
              DEC_EPS, ACT_NONE);
    token_mlp(m, P, L0);
    layernorm(m, P * NTOK, SAM_DIM, d->qry, d->qry, L0->n3w, L0->n3b,
              DEC_EPS, ACT_NONE);
    i2t_attention(m, 0, P);

    /* Layer 1. */
    self_attention(m, 1, P);
    t2i_attention(m, P, &L1->t2i);
    layernorm(m, P * NTOK, SAM_DIM, d->qry, d->qry, L1->n2w, L1->n2b,
              DEC_EPS, ACT_NONE);
    token_mlp(m, P, L1);
    layernorm(m, P * NTOK, SAM_DIM, d->qry, d->qry, L1->n3w, L1->n3b,
              DEC_EPS, ACT_NONE);
    i2t_attention(m, 1, P);

    /* Final token -> image attention. */
    t2i_attention(m, P, &d->final_t2i);
    layernorm(m, P * NTOK, SAM_DIM, d->qry, d->qry, d->nfw, d->nfb, DEC_EPS,
              ACT_NONE);

    /* Hypernetwork MLPs of mask tokens 1..3 (into d->hyper [P][3][32])
     * and the IoU head (4 raw outputs into d->sv): on the bf16 path one
     * kernel for all four; else GEMMs over the P prompts' token rows (row
     * stride NTOK x 256) with the hidden layers in d->sq / d->sk. */
    if (d->fold_w && d->iou_w[0]->dtype == d->hyper_w[1][0]->dtype) {
        const void *w0[4], *w1[4], *w2[4];
        const float *b0[4], *b1[4], *b2[4];

        for (i = 0; i <= 3; i++) {
            hipb_mem const *W = i ? d->hyper_w[i] : d->iou_w;
            hipb_mem const *B = i ? d->hyper_b[i] : d->iou_b;

            w0[i] = W[0]->ptr;
            w1[i] = W[1]->ptr;
            w2[i] = W[2]->ptr;
            b0[i] = B[0]->ptr;
            b1[i] = B[1]->ptr;
            b2[i] = B[2]->ptr;
        }
        hipb_run_begin(m->hip);
        err = launch_dec_heads(d->qry->ptr, w0, w1, w2, b0, b1, b2,
                               d->iou_w[0]->dtype, d->hyper->ptr, d->sv->ptr,
                               P, m->hip->stream);
        hipb_run_end(m->hip, err, "dec_heads", 0.0);
    }
    else {
        for (i = 0; i <= 3; i++) {
            hipb_mem const *W = i ? d->hyper_w[i] : d->iou_w;
            hipb_mem const *B = i ? d->hyper_b[i] : d->iou_b;
            const int tok_row = i ? 2 + i : 1, nout = i ? 32 : 4;

            gemm(m, P, SAM_DIM, SAM_DIM, mat(d->qry, (long)tok_row * SAM_DIM,
                                             NTOK * SAM_DIM),
                 mat(W[0], 0, SAM_DIM), 1, mat(d->sq, 0, SAM_DIM), 1, 1, B[0],
                 NULL, 0, 1.0f, ACT_RELU);
            gemm(m, P, SAM_DIM, SAM_DIM, mat(d->sq, 0, SAM_DIM),
                 mat(W[1], 0, SAM_DIM), 1, mat(d->sk, 0, SAM_DIM), 1, 1, B[1],
                 NULL, 0, 1.0f, ACT_RELU);
            gemm(m, P, nout, SAM_DIM, mat(d->sk, 0, SAM_DIM),
                 mat(W[2], 0, SAM_DIM), 1,
                 i ? mat(d->hyper, (long)(i - 1) * 32, 96) : mat(d->sv, 0, 4), 1,
                 1, B[2], NULL, 0, 1.0f, ACT_NONE);
        }
    }
    if (hipb_failed())
        return;

    if (d->up_w1t) {
        /* bf16: the whole upscaling and the logits in one pass over the
         * keys, per token 16 output pixels of the 3 masks. */
        hipb_run_begin(m->hip);
        err = launch_upscale_prep(d->up0w->ptr, d->up0w->dtype, d->up3w->ptr,
                                  d->up3w->dtype, d->up_w1t->ptr,
                                  d->up_w2t->ptr, m->hip->stream);
        hipb_run_end(m->hip, err, "upscale_prep", 0.0);
        hipb_run_begin(m->hip);
        err = launch_upscale_fused(d->keys->ptr, d->up_w1t->ptr,
                                   d->up_w2t->ptr, d->up0b->ptr, d->up1w->ptr,
                                   d->up1b->ptr, d->up3b->ptr,
                                   d->feat_s1->ptr, d->feat_s0->ptr,
                                   d->hyper->ptr, d->lowres->ptr, G, P,
                                   LN2D_EPS, m->hip->cu_count,
                                   m->hip->stream);
        hipb_run_end(m->hip, err, "upscale_fused",
                     2.0 * P * T * (256.0 * 256 + 4 * 64 * 128 + 16 * 96));
    }
    else {
        /* Output upscaling: ConvT 256 -> 64 + feat_s1, LayerNorm2d, GELU,
         * ConvT 64 -> 32 + feat_s0, GELU (the kin buffer holds the first
         * GEMM), then the logits. */
        gemm(m, (int)(P * T), 256, SAM_DIM, mat(d->keys, 0, SAM_DIM),
             mat(d->up0w, 0, 256), 0, mat(d->kin, 0, 256), 1, 1, NULL, NULL,
             0, 1.0f, ACT_NONE);
        convt_scatter(m, d->kin, d->u1, d->up0b, d->feat_s1, P, G, G, 64,
                      ACT_NONE);
        layernorm(m, P * 4 * T, 64, d->u1, d->u1, d->up1w, d->up1b, LN2D_EPS,
                  ACT_GELU);
        gemm(m, (int)(P * 4 * T), 128, 64, mat(d->u1, 0, 64),
             mat(d->up3w, 0, 128), 0, mat(d->g2, 0, 128), 1, 1, NULL, NULL, 0,
             1.0f, ACT_NONE);
        convt_scatter(m, d->g2, d->u2, d->up3b, d->feat_s0, P, 2 * G, 2 * G,
                      32, ACT_GELU);
        mask_logits(m, d->u2, d->hyper, d->lowres, P, (int)(16 * T));
    }
}

void sam_dec_graph(struct sam_model *m, int P, int enable)
{
    struct sam_decoder *d = dec_of(m, "sam_dec_graph");
    struct hipb_backend *b = m->hip;
    hipGraph_t g = NULL;
    hipGraphExec_t x = NULL;
    void *scratch;
    int err;

    if (!d)
        return;
    hipb_finish(b);
    dec_graph_drop(d);
    if (!enable)
        return;
    if (b->profile) {
        hipb_fatal("sam_dec_graph: profiling runs the kernels one by one");
        return;
    }
    if (P < 1 || P > d->batch) {
        hipb_fatal("sam_dec_graph: %d prompts for a batch of %d", P, d->batch);
        return;
    }
    dec_kernels(m, P); /* allocates whatever scratch is still missing */
    hipb_finish(b);
    if (hipb_failed())
        return;
    scratch = b->scratch;
    err = hipStreamBeginCapture((hipStream_t)b->stream,
                                hipStreamCaptureModeRelaxed);
    if (err != hipSuccess) {
        hipb_fatal("sam_dec_graph: hipStreamBeginCapture: %s (%d)",
                   hipb_errstr(err), err);
        return;
    }
    dec_kernels(m, P);
    err = hipStreamEndCapture((hipStream_t)b->stream, &g);
    if (hipb_failed() || err != hipSuccess || !g || b->scratch != scratch) {
        if (g)
            hipGraphDestroy(g);
        if (!hipb_failed())
            hipb_fatal("sam_dec_graph: capture failed: %s (%d)",
                       hipb_errstr(err), err);
        return;
    }
    err = hipGraphInstantiate(&x, g, NULL, NULL, 0);
    if (err != hipSuccess) {
        hipGraphDestroy(g);
        hipb_fatal("sam_dec_graph: hipGraphInstantiate: %s (%d)",
                   hipb_errstr(err), err);
        return;
    }
    d->graph = g;
    d->graph_exec = x;
    d->graph_P = P;
    d->graph_scratch = scratch;
}

void mask_logits(struct sam_model *m, hipb_mem U, hipb_mem hyper,
                 hipb_mem out, int P, int npix)
{
    struct hipb_backend *be = m->hip;
    int err;

    if (P < 1 || npix < 1 || !U || !hyper || !out ||
        hipb_count(U) < (size_t)P * npix * 32 ||
        hipb_count(hyper) < (size_t)P * 96 ||
        hipb_count(out) < (size_t)P * 3 * npix || U->dtype != HIPB_F32 ||
        hyper->dtype != HIPB_F32 || out->dtype != HIPB_F32) {
        hipb_fatal("mask_logits: invalid shape P=%d npix=%d or operand", P,
                   npix);
        return;
    }
    hipb_run_begin(be);
    err = launch_mask_logits(U->ptr, hyper->ptr, out->ptr, P, npix,
                             be->stream);
    hipb_run_end(be, err, "mask_logits", 0.0);
}

void sam_decode(struct sam_model *m, int P, const float *points, float *iou)
{
    struct sam_decoder *d = dec_of(m, "sam_decode");
    const long n = (long)P * NTOK * SAM_DIM;
    float *tok;
    int p, i, err;

    if (!d)
        return;
    if (P < 1 || P > d->batch) {
        hipb_fatal("sam_decode: batch overflow");
        return;
    }
    tok = d->h_queries;

    /* Prompt tokens: object score token, IoU token, 4 mask tokens, the
     * positive point and the padding point (no box prompt). */
    for (p = 0; p < P; p++) {
        float *t = tok + (long)p * NTOK * SAM_DIM;

        memcpy(t, d->obj_token, SAM_DIM * sizeof(float));
        memcpy(t + SAM_DIM, d->iou_token, SAM_DIM * sizeof(float));
        memcpy(t + 2 * SAM_DIM, d->mask_tokens, 4 * SAM_DIM * sizeof(float));
        pe_encode(d, (points[2 * p] + 0.5f) / d->img,
                  (points[2 * p + 1] + 0.5f) / d->img, t + 6 * SAM_DIM);
        for (i = 0; i < SAM_DIM; i++) {
            t[6 * SAM_DIM + i] += d->point_emb[1][i];
            t[7 * SAM_DIM + i] = d->not_a_point[i];
        }
    }
    hipb_write(m->hip, d->qpe, 0, tok, n * sizeof(float));
    hipb_copy(m->hip, d->qpe, d->qry, 0, 0, n * sizeof(float));

    /* The captured device sequence when it was captured for this P and
     * the backend scratch it uses has not moved since. */
    if (d->graph_exec && !m->hip->profile) {
        if (d->graph_P == P && d->graph_scratch == m->hip->scratch) {
            err = hipGraphLaunch((hipGraphExec_t)d->graph_exec,
                                 (hipStream_t)m->hip->stream);
            hipb_run_end(m->hip, err, "decoder_graph", 0.0);
        }
        else
            dec_kernels(m, P);
    }
    else
        dec_kernels(m, P);
    if (hipb_failed())
        return;
    /* IoU predictions 1..3 through the sigmoid (iou_prediction_use_sigmoid). */
    {
        float *raw = d->h_queries;

        hipb_read(m->hip, d->sv, 0, raw, (size_t)P * 4 * sizeof(float));
        for (p = 0; p < P; p++)
            for (i = 0; i < 3; i++)
                iou[p * 3 + i] = 1.0f / (1.0f + expf(-raw[p * 4 + 1 + i]));
    }
}

/* Root of pixel i's set, halving the path on the way up. */
static int hole_root(int *par, int i)
{
    while (par[i] != i) {
        par[i] = par[par[i]];
        i = par[i];
    }
    return i;
}

/* Background components (v <= 0, 8-connected) of at most max_area pixels
 * of an L x L map become 10 (the hole filling of sam3_model.c:1406-1443).
 * Union-find over one raster pass: each background pixel starts its own
 * set and joins the sets of its background neighbours already passed
 * (left, upper left, up, upper right), every set rooted at its smallest
 * pixel index; a second pass counts each root's pixels and a third fills
 * the pixels of the small sets. par and cnt hold L^2 ints each (par -1:
 * foreground). A NaN logit counts as foreground here. Returns 1 if the
 * map changed. */
static int fill_holes(float *v, int L, int max_area, int *par, int *cnt)
{
    const int n = L * L;
    int i, changed = 0;

    for (i = 0; i < n; i++) {
        const int x = i % L;
        int nb[4], k;

        par[i] = -1;
        if (!(v[i] <= 0.0f))
            continue;
        par[i] = i;
        nb[0] = x > 0 ? i - 1 : -1;
        nb[1] = x > 0 && i >= L ? i - L - 1 : -1;
        nb[2] = i >= L ? i - L : -1;
        nb[3] = x + 1 < L && i >= L ? i - L + 1 : -1;
        for (k = 0; k < 4; k++) {
            int ra, rb;

            if (nb[k] < 0 || par[nb[k]] < 0)
                continue;
            ra = hole_root(par, i);
            rb = hole_root(par, nb[k]);
            if (ra < rb)
                par[rb] = ra;
            else if (rb < ra)
                par[ra] = rb;
        }
    }
    memset(cnt, 0, (size_t)n * sizeof(int));
    for (i = 0; i < n; i++)
        if (par[i] >= 0)
            cnt[hole_root(par, i)]++;
    for (i = 0; i < n; i++)
        if (par[i] >= 0 && cnt[hole_root(par, i)] <= max_area) {
            v[i] = 10.0f;
            changed = 1;
        }
    return changed;
}

void sam_postprocess(struct sam_model *m, int n, const int *sel, int out_h,
                     int out_w, float offset, int fill, int *stats)
{
    struct sam_decoder *d = dec_of(m, "sam_postprocess");
    const int L = 4 * m->grid;
    const size_t plane = (size_t)L * L * sizeof(float);
    const size_t need = (size_t)n * out_h * out_w;
    int i, err;

    if (!d || n <= 0)
        return;
    if (n > 3 * d->batch || out_h < 1 || out_w < 1) {
        hipb_fatal("sam_postprocess: %d masks of %d x %d", n, out_h, out_w);
        return;
    }
    for (i = 0; i < n; i++)
        if (sel[i] < 0 || (size_t)sel[i] >= hipb_count(d->lowres) / (L * L)) {
            hipb_fatal("sam_postprocess: plane %d out of range", sel[i]);
            return;
        }
    if (fill) {
        int *par = malloc((size_t)L * L * sizeof(int));
        int *cnt = malloc((size_t)L * L * sizeof(int));

        for (i = 0; i < n; i++) {
            float *v = d->h_lowres + (size_t)i * L * L;

            hipb_read(m->hip, d->lowres, sel[i] * plane, v, plane);
            if (fill_holes(v, L, SAM_HOLE, par, cnt))
                hipb_write(m->hip, d->lowres, sel[i] * plane, v, plane);
        }
        free(par);
        free(cnt);
    }
    if (need > d->mask_cap) {
        hipb_release(&d->mask);
        d->mask = hipb_alloc(m->hip, need, "postprocessed masks");
        if (!d->mask)
            return;
        d->mask_cap = need;
    }
    for (i = 0; i < n; i++) {
        stats[6 * i + 0] = 0;
        stats[6 * i + 1] = 0;
        stats[6 * i + 2] = 0x7fffffff;
        stats[6 * i + 3] = 0x7fffffff;
        stats[6 * i + 4] = -1;
        stats[6 * i + 5] = -1;
    }
    hipb_write(m->hip, d->sel, 0, sel, n * sizeof(int));
    hipb_write(m->hip, d->stats, 0, stats, 6 * n * sizeof(int));
    hipb_run_begin(m->hip);
    err = launch_mask_post(d->lowres->ptr, d->sel->ptr, n, L, out_h, out_w,
                           offset, d->mask->ptr, d->stats->ptr,
                           m->hip->stream);
    hipb_run_end(m->hip, err, "mask_post", 0.0);
    hipb_read(m->hip, d->stats, 0, stats, 6 * n * sizeof(int));
}

void sam_read_mask(struct sam_model *m, int k, int out_h, int out_w, int x0,
                   int y0, int x1, int y1, unsigned char *dst)
{
    struct sam_decoder *d = dec_of(m, "sam_read_mask");
    const int w = x1 - x0 + 1;
    hipError_t err;

    if (!d)
        return;
    if (!d->mask || k < 0 || x0 < 0 || y0 < 0 || x1 < x0 || y1 < y0 ||
        x1 >= out_w || y1 >= out_h ||
        (size_t)(k + 1) * out_h * out_w > d->mask_cap) {
        hipb_fatal("sam_read_mask: region outside the postprocessed masks");
        return;
    }
    err = hipMemcpy2DAsync(dst, (size_t)w,
                           (const char *)d->mask->ptr +
                               ((size_t)k * out_h + y0) * out_w + x0,
                           (size_t)out_w, (size_t)w, (size_t)(y1 - y0 + 1),
                           hipMemcpyDeviceToHost, (hipStream_t)m->hip->stream);
    if (err == hipSuccess)
        err = hipStreamSynchronize((hipStream_t)m->hip->stream);
    hipb_check(err, "hipMemcpy2DAsync");
}
