/* CPU oracle, mask decoder part (TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline, never by
 * the product library).
 *
 * Restates the SAM 3 point-prompt mask decoder of the reference: the
 * prompt encoder and token set-up (sam3_model.c:760-773, 1239-1268), the
 * two-way transformer (sam3_model.c:1212-1351), the output upscaling
 * with convt_scatter (sam3_kernels.cl:762-786, sam3_model.c:1352-1366),
 * the host hypernetwork / IoU MLPs (sam3_model.c:1185-1209, 1367-1385),
 * mask_logits (sam3_kernels.cl:789-805), and the postprocessing
 * (fill_holes sam3_model.c:1406-1443, mask_post sam3_kernels.cl:807-883,
 * sam_postprocess sam3_model.c:1445-1517). Every GEMM goes through the
 * reference's GPU dispatch (or_gemm_dispatch with cpu = 0).
 */
#include "sam3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define DIM 256      /* SAM_DIM, sam3_model.h:12 */
#define NTOK 8       /* prompt tokens, sam3_model.c:35 */
#define DEC_EPS 1e-5f
#define LN2D_EPS 1e-6f

/* linear() (sam3_model.c:305-310) through the GPU dispatcher. */
static void lin(int rows, int in, int out, const float *X, const float *W,
                const float *b, float *Y, int act, int residual)
{
    or_gemm_dispatch(0, rows, out, in, X, 0, in, 0, 0, W, 0, in, 0, 0, 1, Y,
                     0, out, 0, 0, 1, 1, b, residual ? Y : NULL, 0, 1.0f, act);
}

/* PositionEmbeddingRandom of normalized (x, y) (sam3_model.c:760-773). */
void or_pe_encode(const float *gauss, float x, float y, float *out)
{
    int i;

    x = 2.0f * x - 1.0f;
    y = 2.0f * y - 1.0f;
    for (i = 0; i < DIM / 2; i++) {
        float v = x * gauss[i] + y * gauss[DIM / 2 + i];

        v *= 2.0f * (float)M_PI;
        out[i] = sinf(v);
        out[DIM / 2 + i] = cosf(v);
    }
}

/* host_linear (sam3_model.c:1185-1198): double accumulation from the
 * bias, products in index order, optional ReLU, rounded once. */
void or_host_linear(const float *W, const float *b, const float *x, int nin,
                    int nout, int relu, float *y)
{
    int o, i;

    for (o = 0; o < nout; o++) {
        const float *w = W + (long)o * nin;
        double acc = b[o];

        for (i = 0; i < nin; i++)
            acc += (double)w[i] * x[i];
        y[o] = relu && acc < 0.0 ? 0.0f : (float)acc;
    }
}

static void host_mlp3(const float *const W[3], const float *const B[3],
                      const float *x, int nout, float *y)
{
    float h1[DIM], h2[DIM];

    or_host_linear(W[0], B[0], x, DIM, DIM, 1, h1);
    or_host_linear(W[1], B[1], h1, DIM, DIM, 1, h2);
    or_host_linear(W[2], B[2], h2, DIM, nout, 0, y);
}

/* convt_scatter (sam3_kernels.cl:762-786): G is (P H W) x (Co 4) with
 * column co 4 + dy 2 + dx; out is P x 2H x 2W x Co; add (2H x 2W x Co,
 * shared by the prompts) is summed in before the activation. */
void or_convt_scatter(const float *G, float *out, const float *bias,
                      const float *add, int P, int H, int W, int Co, int act)
{
    const long total = (long)P * 4 * H * W * Co;
    long gid;

#pragma omp parallel for schedule(static)
    for (gid = 0; gid < total; gid++) {
        const int co = (int)(gid % Co);
        const long pix = gid / Co;
        const int ox = (int)(pix % (2 * W));
        const long rest = pix / (2 * W);
        const int oy = (int)(rest % (2 * H));
        const long p = rest / (2 * H);
        const int y = oy >> 1, x = ox >> 1, dy = oy & 1, dx = ox & 1;
        float v = G[((p * H + y) * W + x) * (Co * 4) + co * 4 + dy * 2 + dx] +
                  bias[co];

        if (add)
            v += add[gid % (4L * H * W * Co)];
        out[gid] = or_act(v, act);
    }
}

/* mask_logits (sam3_kernels.cl:789-805): out[p, k, pix] = hyper[p, k, :]
 * . U[p, pix, :] over 32 channels as two dot16 (sam3_kernels.cl:516-520)
 * summed, for the 3 multimask outputs. */
void or_mask_logits(const float *U, const float *hyper, float *out, int P,
                    int npix)
{
    const long total = (long)P * npix;
    long gid;

#pragma omp parallel for schedule(static)
    for (gid = 0; gid < total; gid++) {
        const long p = gid / npix, pix = gid % npix;
        const float *h = hyper + p * 96, *u = U + gid * 32;
        int k;

        for (k = 0; k < 3; k++)
            out[(p * 3 + k) * npix + pix] =
                or_dot16(u, h + 32 * k) + or_dot16(u + 16, h + 32 * k + 16);
    }
}

/* PyTorch bilinear source coordinate (align_corners = False),
 * sam3_kernels.cl:808-813. */
static float src_coord(float scale, int dst)
{
    const float s = scale * ((float)dst + 0.5f) - 0.5f;

    return s < 0.0f ? 0.0f : s;
}

/* mask_post (sam3_kernels.cl:815-883) for the n planes sel[] of lowres
 * (L x L each): the bilinear value at each output pixel, written as
 * (1 - ly) ((1 - lx) a + lx b) + ly ((1 - lx) c + lx d) with every
 * a * b + c contracted to fmaf (the reference compiles with
 * -cl-mad-enable; where clang contracts is parity unpinned at the last
 * bit), mask = v > 0, and per mask the stats inter = #(v > offset),
 * union = #(v > -offset), bounding box of the mask. stats must hold the
 * initial values sam_postprocess writes (0, 0, INT_MAX, INT_MAX, -1,
 * -1). */
void or_mask_post(const float *lowres, const int *sel, int n, int L,
                  int out_h, int out_w, float offset, unsigned char *mask,
                  int *stats)
{
    int k;

#pragma omp parallel for schedule(dynamic)
    for (k = 0; k < n; k++) {
        const float *lr = lowres + (long)sel[k] * L * L;
        int *st = stats + 6 * k;
        int oy, ox;

        for (oy = 0; oy < out_h; oy++)
            for (ox = 0; ox < out_w; ox++) {
                const float sy = src_coord((float)L / out_h, oy);
                const float sx = src_coord((float)L / out_w, ox);
                const int y0 = (int)sy, x0 = (int)sx;
                const int y1 = y0 + (y0 < L - 1), x1 = x0 + (x0 < L - 1);
                const float ly = sy - y0, lx = sx - x0;
                const float top = fmaf(lx, lr[y0 * L + x1],
                                       (1.0f - lx) * lr[y0 * L + x0]);
                const float bot = fmaf(lx, lr[y1 * L + x1],
                                       (1.0f - lx) * lr[y1 * L + x0]);
                const float v = fmaf(ly, bot, (1.0f - ly) * top);

                mask[((long)k * out_h + oy) * out_w + ox] = v > 0.0f;
                if (v > offset)
                    st[0]++;
                if (v > -offset)
                    st[1]++;
                if (v > 0.0f) {
                    if (ox < st[2])
                        st[2] = ox;
                    if (oy < st[3])
                        st[3] = oy;
                    if (ox > st[4])
                        st[4] = ox;
                    if (oy > st[5])
                        st[5] = oy;
                }
            }
    }
}

/* fill_holes (sam3_model.c:1406-1443): background components (v <= 0,
 * 8-connected) of at most max_area pixels become 10. Returns 1 if the
 * map changed. */
int or_fill_holes(float *v, int L, int max_area)
{
    const int n = L * L;
    int *lab = calloc(n, sizeof(int)), *queue = malloc(n * sizeof(int));
    int i, changed = 0;

    for (i = 0; i < n; i++) {
        int sp = 0, j;

        if (lab[i] || v[i] > 0.0f)
            continue;
        lab[i] = 1;
        queue[sp++] = i;
        for (j = 0; j < sp; j++) {
            const int c = queue[j], cx = c % L, cy = c / L;
            int dy, dx;

            for (dy = -1; dy <= 1; dy++)
                for (dx = -1; dx <= 1; dx++) {
                    const int nx = cx + dx, ny = cy + dy;

                    if (nx < 0 || ny < 0 || nx >= L || ny >= L)
                        continue;
                    if (!lab[ny * L + nx] && v[ny * L + nx] <= 0.0f) {
                        lab[ny * L + nx] = 1;
                        queue[sp++] = ny * L + nx;
                    }
                }
        }
        if (sp <= max_area) {
            for (j = 0; j < sp; j++)
                v[queue[j]] = 10.0f;
            changed = 1;
        }
    }
    free(lab);
    free(queue);
    return changed;
}

/* sam_postprocess (sam3_model.c:1445-1517) on host copies: lowres
 * [planes][L][L] is modified in place by the hole filling (fill != 0,
 * holes of at most max_area pixels) of the selected planes; then
 * or_mask_post with freshly initialised stats. */
void or_postprocess(float *lowres, int L, int n, const int *sel, int out_h,
                    int out_w, float offset, int fill, int max_area,
                    unsigned char *mask, int *stats)
{
    int i;

    if (fill)
        for (i = 0; i < n; i++)
            or_fill_holes(lowres + (long)sel[i] * L * L, L, max_area);
    for (i = 0; i < n; i++) {
        stats[6 * i + 0] = 0;
        stats[6 * i + 1] = 0;
        stats[6 * i + 2] = 0x7fffffff;
        stats[6 * i + 3] = 0x7fffffff;
        stats[6 * i + 4] = -1;
        stats[6 * i + 5] = -1;
    }
    or_mask_post(lowres, sel, n, L, out_h, out_w, offset, mask, stats);
}

/* Prompt-independent decoder inputs (sam3_model.c:1150-1171, dense
 * positional encoding sam3_model.c:886-892): pe_img, src = emb +
 * no_mask, srcpe = src + pe_img, and the layer-0 projections kp0 =
 * t2i.k(srcpe), vp0 = t2i.v(src), qp0 = i2t.q(srcpe). */
void or_dec_prepare(const struct or_decoder *d, const float *emb, float *pe,
                    float *src, float *srcpe, float *kp0, float *vp0,
                    float *qp0)
{
    const int G = d->grid, T = G * G;
    const struct or_dec_layer *L0 = &d->layers[0];
    int x, y;

    for (y = 0; y < G; y++)
        for (x = 0; x < G; x++)
            or_pe_encode(d->gauss, (x + 0.5f) / G, (y + 0.5f) / G,
                         pe + ((long)y * G + x) * DIM);
    or_add_bcast(src, emb, d->no_mask, (long)T * DIM, DIM);
    or_add_bcast(srcpe, src, pe, (long)T * DIM, (long)T * DIM);
    lin(T, DIM, 128, srcpe, L0->t2i.kw, L0->t2i.kb, kp0, OR_ACT_NONE, 0);
    lin(T, DIM, 128, src, L0->t2i.vw, L0->t2i.vb, vp0, OR_ACT_NONE, 0);
    lin(T, DIM, 128, srcpe, L0->i2t.qw, L0->i2t.qb, qp0, OR_ACT_NONE, 0);
}

/* Token -> image attention on per-prompt keys with the residual into
 * the queries (t2i_attention, sam3_model.c:1212-1229): kin = keys + pe
 * is left in kin (the next image -> token attention reads it). */
void or_t2i_attention(int P, int T, float *qry, const float *qpe,
                      const float *keys, const float *pe,
                      const struct or_attn_w *a, float *kin)
{
    const long n = (long)P * NTOK * DIM;
    float *qin = malloc(n * sizeof(float));
    float *sq = malloc((size_t)P * NTOK * 128 * sizeof(float));
    float *so = malloc((size_t)P * NTOK * 128 * sizeof(float));
    float *bk = malloc((size_t)P * T * 128 * sizeof(float));
    float *bv = malloc((size_t)P * T * 128 * sizeof(float));

    or_add_bcast(qin, qry, qpe, n, n);
    or_add_bcast(kin, keys, pe, (long)P * T * DIM, (long)T * DIM);
    lin(P * NTOK, DIM, 128, qin, a->qw, a->qb, sq, OR_ACT_NONE, 0);
    lin(P * T, DIM, 128, kin, a->kw, a->kb, bk, OR_ACT_NONE, 0);
    lin(P * T, DIM, 128, keys, a->vw, a->vb, bv, OR_ACT_NONE, 0);
    or_mha(P, NTOK, T, 128, sq, NTOK * 128, bk, (long)T * 128, bv,
           (long)T * 128, so);
    lin(P * NTOK, 128, DIM, so, a->ow, a->ob, qry, OR_ACT_NONE, 1);
    free(qin);
    free(sq);
    free(so);
    free(bk);
    free(bv);
}

/* Image -> token attention of layer `layer` (sam3_model.c:1298-1312 for
 * layer 0, 1330-1345 for layer 1), keys updated in place: layer 0 takes
 * the shared queries qp0 and replaces keys by src + out-projection;
 * layer 1 projects kin per prompt and adds the out-projection to keys.
 * Both end with norm4. */
void or_i2t_attention(int layer, int P, int T, const float *qry,
                      const float *qpe, float *keys, const float *kin,
                      const float *qp0, const float *src,
                      const struct or_dec_layer *L)
{
    const long n = (long)P * NTOK * DIM;
    float *qin = malloc(n * sizeof(float));
    float *sk = malloc((size_t)P * NTOK * 128 * sizeof(float));
    float *sv = malloc((size_t)P * NTOK * 128 * sizeof(float));
    float *bo = malloc((size_t)P * T * 128 * sizeof(float));

    or_add_bcast(qin, qry, qpe, n, n);
    if (layer == 0) {
        lin(P * NTOK, DIM, 128, qin, L->i2t.kw, L->i2t.kb, sk, OR_ACT_NONE,
            0);
        lin(P * NTOK, DIM, 128, qry, L->i2t.vw, L->i2t.vb, sv, OR_ACT_NONE,
            0);
        or_mha(P, T, NTOK, 128, qp0, 0, sk, NTOK * 128, sv, NTOK * 128, bo);
        lin(P * T, 128, DIM, bo, L->i2t.ow, L->i2t.ob, keys, OR_ACT_NONE, 0);
        or_add_bcast(keys, keys, src, (long)P * T * DIM, (long)T * DIM);
    }
    else {
        float *bq = malloc((size_t)P * T * 128 * sizeof(float));

        lin(P * T, DIM, 128, kin, L->i2t.qw, L->i2t.qb, bq, OR_ACT_NONE, 0);
        lin(P * NTOK, DIM, 128, qin, L->i2t.kw, L->i2t.kb, sk, OR_ACT_NONE,
            0);
        lin(P * NTOK, DIM, 128, qry, L->i2t.vw, L->i2t.vb, sv, OR_ACT_NONE,
            0);
        or_mha(P, T, NTOK, 128, bq, (long)T * 128, sk, NTOK * 128, sv,
               NTOK * 128, bo);
        lin(P * T, 128, DIM, bo, L->i2t.ow, L->i2t.ob, keys, OR_ACT_NONE, 1);
        free(bq);
    }
    or_layernorm(keys, keys, (long)P * T, DIM, L->n4w, L->n4b, DEC_EPS,
                 OR_ACT_NONE);
    free(qin);
    free(sk);
    free(sv);
    free(bo);
}

/* Self attention of the prompt tokens (sam3_model.c:1274-1286 for layer
 * 0: no positional encoding, no residual; 1316-1327 for layer 1), then
 * norm1. */
static void self_attention(int layer, int P, float *qry, const float *qpe,
                           const struct or_dec_layer *L)
{
    const long n = (long)P * NTOK * DIM;
    float *qin = malloc(n * sizeof(float));
    float *sq = malloc(n * sizeof(float)), *sk = malloc(n * sizeof(float));
    float *sv = malloc(n * sizeof(float)), *so = malloc(n * sizeof(float));
    const float *qk = qry;

    if (layer) {
        or_add_bcast(qin, qry, qpe, n, n);
        qk = qin;
    }
    lin(P * NTOK, DIM, DIM, qk, L->self.qw, L->self.qb, sq, OR_ACT_NONE, 0);
    lin(P * NTOK, DIM, DIM, qk, L->self.kw, L->self.kb, sk, OR_ACT_NONE, 0);
    lin(P * NTOK, DIM, DIM, qry, L->self.vw, L->self.vb, sv, OR_ACT_NONE, 0);
    or_mha(P, NTOK, NTOK, DIM, sq, NTOK * DIM, sk, NTOK * DIM, sv, NTOK * DIM,
           so);
    lin(P * NTOK, DIM, DIM, so, L->self.ow, L->self.ob, qry, OR_ACT_NONE,
        layer);
    or_layernorm(qry, qry, P * NTOK, DIM, L->n1w, L->n1b, DEC_EPS,
                 OR_ACT_NONE);
    free(qin);
    free(sq);
    free(sk);
    free(sv);
    free(so);
}

static void token_mlp(int P, float *qry, const struct or_dec_layer *L)
{
    float *sh = malloc((size_t)P * NTOK * 2048 * sizeof(float));

    lin(P * NTOK, DIM, 2048, qry, L->m1w, L->m1b, sh, OR_ACT_RELU, 0);
    lin(P * NTOK, 2048, DIM, sh, L->m2w, L->m2b, qry, OR_ACT_NONE, 1);
    free(sh);
}

/* Prompt tokens of P single-point prompts (sam3_model.c:1249-1265):
 * object score token, IoU token, 4 mask tokens, the point (PE + point
 * embedding 1) and the padding point. */
void or_prompt_tokens(const struct or_decoder *d, int P, const float *points,
                      float *tok)
{
    const float img = (float)d->img;
    int p, i;

    for (p = 0; p < P; p++) {
        float *t = tok + (long)p * NTOK * DIM;

        memcpy(t, d->obj_token, DIM * sizeof(float));
        memcpy(t + DIM, d->iou_token, DIM * sizeof(float));
        memcpy(t + 2 * DIM, d->mask_tokens, 4 * DIM * sizeof(float));
        or_pe_encode(d->gauss, (points[2 * p] + 0.5f) / img,
                     (points[2 * p + 1] + 0.5f) / img, t + 6 * DIM);
        for (i = 0; i < DIM; i++) {
            t[6 * DIM + i] += d->point_emb[DIM + i];
            t[7 * DIM + i] = d->not_a_point[i];
        }
    }
}

/* sam_decode (sam3_model.c:1239-1400) after or_dec_prepare: iou [P][3],
 * lowres [P][3][4G][4G]; tokens (if not NULL) receives the final tokens
 * [P][8][256] and hyper (if not NULL) the hypernetwork outputs
 * [P][3][32]. */
void or_sam_decode(const struct or_decoder *d, int P, const float *points,
                   const float *pe, const float *src, const float *kp0,
                   const float *vp0, const float *qp0, const float *feat_s0,
                   const float *feat_s1, float *iou, float *lowres,
                   float *tokens, float *hyper_out)
{
    const int G = d->grid, T = G * G;
    const long n = (long)P * NTOK * DIM;
    const struct or_dec_layer *L0 = &d->layers[0], *L1 = &d->layers[1];
    float *qpe = malloc(n * sizeof(float)), *qry = malloc(n * sizeof(float));
    float *qin = malloc(n * sizeof(float));
    float *sq = malloc((size_t)P * NTOK * 128 * sizeof(float));
    float *so = malloc((size_t)P * NTOK * 128 * sizeof(float));
    float *keys = malloc((size_t)P * T * DIM * sizeof(float));
    float *kin = malloc((size_t)P * T * DIM * sizeof(float));
    float *u1 = malloc((size_t)P * 4 * T * 64 * sizeof(float));
    float *g2 = malloc((size_t)P * 4 * T * 128 * sizeof(float));
    float *u2 = malloc((size_t)P * 16 * T * 32 * sizeof(float));
    float *hyper = malloc((size_t)P * 96 * sizeof(float));
    int p, i;

    or_prompt_tokens(d, P, points, qpe);
    memcpy(qry, qpe, n * sizeof(float));

    /* Layer 0. */
    self_attention(0, P, qry, qpe, L0);
    or_add_bcast(qin, qry, qpe, n, n);
    lin(P * NTOK, DIM, 128, qin, L0->t2i.qw, L0->t2i.qb, sq, OR_ACT_NONE, 0);
    or_mha(P, NTOK, T, 128, sq, NTOK * 128, kp0, 0, vp0, 0, so);
    lin(P * NTOK, 128, DIM, so, L0->t2i.ow, L0->t2i.ob, qry, OR_ACT_NONE, 1);
    or_layernorm(qry, qry, P * NTOK, DIM, L0->n2w, L0->n2b, DEC_EPS,
                 OR_ACT_NONE);
    token_mlp(P, qry, L0);
    or_layernorm(qry, qry, P * NTOK, DIM, L0->n3w, L0->n3b, DEC_EPS,
                 OR_ACT_NONE);
    or_i2t_attention(0, P, T, qry, qpe, keys, NULL, qp0, src, L0);

    /* Layer 1. */
    self_attention(1, P, qry, qpe, L1);
    or_t2i_attention(P, T, qry, qpe, keys, pe, &L1->t2i, kin);
    or_layernorm(qry, qry, P * NTOK, DIM, L1->n2w, L1->n2b, DEC_EPS,
                 OR_ACT_NONE);
    token_mlp(P, qry, L1);
    or_layernorm(qry, qry, P * NTOK, DIM, L1->n3w, L1->n3b, DEC_EPS,
                 OR_ACT_NONE);
    or_i2t_attention(1, P, T, qry, qpe, keys, kin, NULL, NULL, L1);

    /* Final token -> image attention. */
    or_t2i_attention(P, T, qry, qpe, keys, pe, &d->final_t2i, kin);
    or_layernorm(qry, qry, P * NTOK, DIM, d->nfw, d->nfb, DEC_EPS,
                 OR_ACT_NONE);

    /* Output upscaling (sam3_model.c:1352-1366). */
    or_gemm_dispatch(0, P * T, 256, DIM, keys, 0, DIM, 0, 0, d->up0w, 0, 256,
                     0, 0, 0, kin, 0, 256, 0, 0, 1, 1, NULL, NULL, 0, 1.0f,
                     OR_ACT_NONE);
    or_convt_scatter(kin, u1, d->up0b, feat_s1, P, G, G, 64, OR_ACT_NONE);
    or_layernorm(u1, u1, (long)P * 4 * T, 64, d->up1w, d->up1b, LN2D_EPS,
                 OR_ACT_GELU);
    or_gemm_dispatch(0, P * 4 * T, 128, 64, u1, 0, 64, 0, 0, d->up3w, 0, 128,
                     0, 0, 0, g2, 0, 128, 0, 0, 1, 1, NULL, NULL, 0, 1.0f,
                     OR_ACT_NONE);
    or_convt_scatter(g2, u2, d->up3b, feat_s0, P, 2 * G, 2 * G, 32,
                     OR_ACT_GELU);

    /* Hypernetwork MLPs and IoU head (sam3_model.c:1367-1385). */
    for (p = 0; p < P; p++) {
        const float *t = qry + (long)p * NTOK * DIM;
        float out[4];

        for (i = 1; i <= 3; i++)
            host_mlp3(d->hyper_w[i], d->hyper_b[i], t + (2 + i) * DIM, 32,
                      hyper + (long)p * 96 + (i - 1) * 32);
        host_mlp3(d->iou_w, d->iou_b, t + DIM, 4, out);
        for (i = 0; i < 3; i++)
            iou[p * 3 + i] = 1.0f / (1.0f + expf(-out[1 + i]));
    }
    or_mask_logits(u2, hyper, lowres, P, 16 * T);
    if (tokens)
        memcpy(tokens, qry, n * sizeof(float));
    if (hyper_out)
        memcpy(hyper_out, hyper, (size_t)P * 96 * sizeof(float));
    free(qpe);
    free(qry);
    free(qin);
    free(sq);
    free(so);
    free(keys);
    free(kin);
    free(u1);
    free(g2);
    free(u2);
    free(hyper);
}
