/* SPDX-License-Identifier: Unlicense
 *
 * sam3_ops.c - the operator layer of the attention path on HIP: the
 * functions of sam3_ops.h (gemm, linear, layernorm, add_bcast, mat,
 * bmat), the attention helpers of sam3_model.c (softmax_rows,
 * rope_apply, window_partition, window_unpartition_add, mha), and the
 * fused attention entry points attn_fused / vit_attention.
 *
 * Each operator validates its shapes and that every element it will
 * touch lies inside its buffers before anything is queued (a bad
 * operand is a fatal error naming the call, never a device fault), then
 * queues its kernel(s) on the backend's stream inside the profiling
 * bracket of the reference's run() (sam3_model.c:167-207).
 */
#include "hipb_internal.h"
#include "sam3_launch.h"

#include <hip/hip_runtime_api.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define ENC_EPS 1e-5f   /* ViT LayerNorm eps (sam3_model.c:30) */
#define SAM_PATCH 14    /* ViT patch side (sam3_model.h:10) */
#define DEC_HEADS 8     /* decoder heads (sam3_model.c:36) */
#define LOG2E_HOST 1.4426950408889634f /* the bf16 kernel scores in log2 units */

struct opnd mat(hipb_mem buf, long off, int ld)
{
    struct opnd o = {buf, off, ld, 0, 0};

    return o;
}

struct opnd bmat(hipb_mem buf, long off, int ld, long s0, long s1)
{
    struct opnd o = {buf, off, ld, s0, s1};

    return o;
}

/* True if rows x cols elements at (off, ld) for every batch b < nb,
 * b = (b / nb1) * s0 + (b % nb1) * s1, lie inside o.buf; fatal
 * otherwise. */
static int opnd_ok(const char *op, const char *name, struct opnd o, long rows,
                   long cols, int nb, int nb1)
{
    long last, b0max, b1max;

    if (!o.buf) {
        hipb_fatal("%s: operand %s has no buffer", op, name);
        return 0;
    }
    if (rows <= 0 || cols <= 0)
        return 1;
    if (o.off < 0 || o.s0 < 0 || o.s1 < 0 || o.ld < 0 ||
        (rows > 1 && o.ld < cols)) {
        hipb_fatal("%s: operand %s has a negative offset or stride, or "
                   "ld %d < %ld columns",
                   op, name, o.ld, cols);
        return 0;
    }
    b0max = (nb - 1) / nb1;
    b1max = (nb < nb1 ? nb : nb1) - 1;
    last = o.off + b0max * o.s0 + b1max * o.s1 + (rows - 1) * (long)o.ld +
           cols - 1;
    if ((size_t)last >= hipb_count(o.buf)) {
        hipb_fatal("%s: operand %s reaches element %ld of buffer <%s> "
                   "(%lu elements)",
                   op, name, last, o.buf->what,
                   (unsigned long)hipb_count(o.buf));
        return 0;
    }
    return 1;
}

static int buf_ok(const char *op, const char *name, hipb_mem m, size_t count,
                  int dtype)
{
    if (!m) {
        hipb_fatal("%s: %s has no buffer", op, name);
        return 0;
    }
    if (dtype >= 0 && m->dtype != dtype) {
        hipb_fatal("%s: %s <%s> has element type %d, expected %d", op, name,
                   m->what, m->dtype, dtype);
        return 0;
    }
    if (hipb_count(m) < count) {
        hipb_fatal("%s: %s <%s> holds %lu elements, %lu needed", op, name,
                   m->what, (unsigned long)hipb_count(m),
                   (unsigned long)count);
        return 0;
    }
    return 1;
}

/* ------------------------------------------------------------ GEMM */

void gemm(struct sam_model *m, int M, int N, int K, struct opnd A,
          struct opnd B, int transb, struct opnd C, int nb, int nb1,
          hipb_mem bias, hipb_mem R, long roff, float alpha, int act)
{
    struct hipb_backend *b = m->hip;
    struct gemm_desc d;
    struct opnd Ro;
    const char *what;
    int err;

    if (M < 0 || N < 0 || K < 0 || nb < 1 || nb1 < 1 || act < ACT_NONE ||
        act > ACT_RELU) {
        hipb_fatal("gemm: invalid shape M=%d N=%d K=%d nb=%d nb1=%d act=%d",
                   M, N, K, nb, nb1, act);
        return;
    }
    if (M == 0 || N == 0)
        return;
    if (!opnd_ok("gemm", "A", A, M, K, nb, nb1) ||
        !opnd_ok("gemm", "B", B, transb ? N : K, transb ? K : N, nb, nb1) ||
        !opnd_ok("gemm", "C", C, M, N, nb, nb1))
        return;
    if (A.buf->dtype == HIPB_F16 || C.buf->dtype == HIPB_F16) {
        hipb_fatal("gemm: half storage is for operand B only");
        return;
    }
    if (bias && !buf_ok("gemm", "bias", bias, (size_t)N, HIPB_F32))
        return;
    if (R) {
        Ro = C;
        Ro.buf = R;
        Ro.off = roff;
        if (!opnd_ok("gemm", "R", Ro, M, N, nb, nb1))
            return;
        if (R->dtype != C.buf->dtype) {
            hipb_fatal("gemm: residual R must have C's element type");
            return;
        }
    }
    memset(&d, 0, sizeof(d));
    d.M = M;
    d.N = N;
    d.K = K;
    d.A = A.buf->ptr;
    d.aoff = A.off;
    d.lda = A.ld;
    d.sa0 = A.s0;
    d.sa1 = A.s1;
    d.adt = A.buf->dtype;
    d.B = B.buf->ptr;
    d.boff = B.off;
    d.ldb = B.ld;
    d.sb0 = B.s0;
    d.sb1 = B.s1;
    d.bdt = B.buf->dtype;
    d.transb = transb != 0;
    d.C = C.buf->ptr;
    d.coff = C.off;
    d.ldc = C.ld;
    d.sc0 = C.s0;
    d.sc1 = C.s1;
    d.cdt = C.buf->dtype;
    d.nb = nb;
    d.nb1 = nb1;
    d.bias = bias ? (const float *)bias->ptr : NULL;
    d.R = R ? R->ptr : NULL;
    d.roff = roff;
    d.alpha = alpha;
    d.act = act;
    d.mode = (b->bf16 || d.adt == HIPB_BF16 || d.bdt == HIPB_BF16)
                 ? MODE_BF16
                 : MODE_F32;
    what = gemm_nt_ok(&d)           ? "gemm_nt_bf16"
           : d.mode == MODE_BF16 ? "gemm_bf16"
                                 : "gemm_f32";
    hipb_run_begin(b);
    err = launch_gemm(&d, b->stream);
    hipb_run_end(b, err, what, 2.0 * M * N * K * (double)nb);
}

/* Y[rows, out] = act(X[rows, in] W^T + b) (+ Y when residual)
 * (sam3_model.c:305-310). */
void linear(struct sam_model *m, int rows, int in, int out, hipb_mem X,
            long xoff, hipb_mem W, hipb_mem b, hipb_mem Y, long yoff, int act,
            int residual)
{
    gemm(m, rows, out, in, mat(X, xoff, in), mat(W, 0, in), 1,
         mat(Y, yoff, out), 1, 1, b, residual ? Y : NULL, yoff, 1.0f, act);
}

/* ------------------------------------------------------------ row ops */

void layernorm(struct sam_model *m, long rows, int C, hipb_mem X, hipb_mem Y,
               hipb_mem g, hipb_mem b, float eps, int act)
{
    struct hipb_backend *be = m->hip;
    int err;

    if (rows < 0 || C < 1 || act < ACT_NONE || act > ACT_RELU) {
        hipb_fatal("layernorm: invalid shape rows=%ld C=%d", rows, C);
        return;
    }
    if (!buf_ok("layernorm", "X", X, (size_t)rows * C, HIPB_F32) ||
        !buf_ok("layernorm", "Y", Y, (size_t)rows * C, -1) ||
        !buf_ok("layernorm", "g", g, (size_t)C, HIPB_F32) ||
        !buf_ok("layernorm", "b", b, (size_t)C, HIPB_F32))
        return;
    if (Y->dtype == HIPB_F16 || (Y->dtype == HIPB_BF16 && X == Y)) {
        hipb_fatal("layernorm: Y must be float, or bf16 distinct from X");
        return;
    }
    if (rows == 0)
        return;
    hipb_run_begin(be);
    err = launch_layernorm(X->ptr, Y->ptr, Y->dtype, g->ptr, b->ptr, rows, C,
                           eps, act, 0, 0, 0, be->stream);
    hipb_run_end(be, err, "layernorm", 0.0);
}

void add_bcast(struct sam_model *m, hipb_mem out, hipb_mem a, hipb_mem b,
               long n, long bmod)
{
    struct hipb_backend *be = m->hip;
    int err;

    if (n < 0 || bmod < 1) {
        hipb_fatal("add_bcast: invalid n=%ld bmod=%ld", n, bmod);
        return;
    }
    if (!buf_ok("add_bcast", "out", out, (size_t)n, HIPB_F32) ||
        !buf_ok("add_bcast", "a", a, (size_t)n, HIPB_F32) ||
        !buf_ok("add_bcast", "b", b, (size_t)(bmod < n ? bmod : n),
                HIPB_F32))
        return;
    if (n == 0)
        return;
    hipb_run_begin(be);
    err = launch_add_bcast(out->ptr, a->ptr, b->ptr, n, bmod, be->stream);
    hipb_run_end(be, err, "add_bcast", 0.0);
}

void softmax_rows(struct sam_model *m, hipb_mem S, long rows, int L)
{
    struct hipb_backend *be = m->hip;
    int err;

    if (rows < 0 || L < 1) {
        hipb_fatal("softmax_rows: invalid shape rows=%ld L=%d", rows, L);
        return;
    }
    if (!buf_ok("softmax_rows", "S", S, (size_t)rows * L, HIPB_F32))
        return;
    if (rows == 0)
        return;
    hipb_run_begin(be);
    err = launch_softmax_rows(S->ptr, rows, L, be->stream);
    hipb_run_end(be, err, "softmax_rows", 0.0);
}

void softmax_ext(struct sam_model *m, hipb_mem S, long rows, int L, int Nq,
                 int h0, int causal, hipb_mem dy, hipb_mem dx, int W, int nh)
{
    struct hipb_backend *be = m->hip;
    int err;

    if (rows < 0 || L < 1 || Nq < 1 || h0 < 0 || (dy && !dx) || (dx && !dy) ||
        (dy && (W < 1 || L % W || nh < 1 || h0 + (rows + Nq - 1) / Nq > nh))) {
        hipb_fatal("softmax_ext: invalid shape rows=%ld L=%d Nq=%d h0=%d W=%d "
                   "nh=%d",
                   rows, L, Nq, h0, W, nh);
        return;
    }
    if (!buf_ok("softmax_ext", "S", S, (size_t)rows * L, HIPB_F32) ||
        (dy && (!buf_ok("softmax_ext", "dy", dy, (size_t)Nq * (L / W) * nh,
                        HIPB_F32) ||
                !buf_ok("softmax_ext", "dx", dx, (size_t)Nq * W * nh,
                        HIPB_F32))))
        return;
    if (rows == 0)
        return;
    hipb_run_begin(be);
    err = launch_softmax_ext(S->ptr, rows, L, Nq, h0, causal != 0,
                             dy ? dy->ptr : NULL, dx ? dx->ptr : NULL, W, nh,
                             be->stream);
    hipb_run_end(be, err, "softmax_ext", 0.0);
}

void rope_apply(struct sam_model *m, hipb_mem table, long rows, int npos)
{
    struct hipb_backend *be = m->hip;
    const int E = m->embed, hd = m->hd;
    int err;

    if (rows < 0 || npos < 1 || hd < 2 || hd % 2 || E % hd) {
        hipb_fatal("rope_apply: invalid shape rows=%ld npos=%d", rows, npos);
        return;
    }
    if (!buf_ok("rope_apply", "qkv", m->qkv, (size_t)rows * 3 * E, HIPB_F32) ||
        !buf_ok("rope_apply", "table", table, (size_t)npos * hd, HIPB_F32))
        return;
    if (rows == 0)
        return;
    hipb_run_begin(be);
    err = launch_rope_apply(m->qkv->ptr, rows, E, hd, npos, table->ptr,
                            be->stream);
    hipb_run_end(be, err, "rope_apply", 0.0);
}

void window_partition(struct sam_model *m, hipb_mem X, hipb_mem out, int H,
                      int C, int ws, int nwx)
{
    struct hipb_backend *be = m->hip;
    int err;

    if (H < 1 || C < 1 || ws < 1 || nwx < 1 || (long)nwx * ws < H) {
        hipb_fatal("window_partition: invalid geometry H=%d ws=%d nwx=%d", H,
                   ws, nwx);
        return;
    }
    if (!buf_ok("window_partition", "X", X, (size_t)H * H * C, HIPB_F32) ||
        !buf_ok("window_partition", "out", out,
                (size_t)nwx * nwx * ws * ws * C, HIPB_F32))
        return;
    hipb_run_begin(be);
    err = launch_window_partition(X->ptr, out->ptr, H, H, C, ws, nwx,
                                  be->stream);
    hipb_run_end(be, err, "window_partition", 0.0);
}

void window_unpartition_add(struct sam_model *m, hipb_mem X, hipb_mem Wd,
                            int H, int C, int ws, int nwx)
{
    struct hipb_backend *be = m->hip;
    int err;

    if (H < 1 || C < 1 || ws < 1 || nwx < 1 || (long)nwx * ws < H) {
        hipb_fatal("window_unpartition_add: invalid geometry H=%d ws=%d "
                   "nwx=%d",
                   H, ws, nwx);
        return;
    }
    if (!buf_ok("window_unpartition_add", "X", X, (size_t)H * H * C,
                HIPB_F32) ||
        !buf_ok("window_unpartition_add", "Wd", Wd,
                (size_t)nwx * nwx * ws * ws * C, HIPB_F32))
        return;
    hipb_run_begin(be);
    err = launch_window_unpartition_add(X->ptr, Wd->ptr, H, H, C, ws, nwx,
                                        be->stream);
    hipb_run_end(be, err, "window_unpartition_add", 0.0);
}

/* ------------------------------------------------------------ decoder */

/* Extent in elements of P prompts of `rows` rows of dint channels with
 * per-prompt stride s (0 = shared). */
static size_t dec_extent(int P, long s, int rows, int dint)
{
    return (size_t)((long)(P - 1) * s + (long)rows * dint);
}

/* mha and mha_noalloc: the many-keys split partials in the backend's
 * scratch (grown on demand) or, with noalloc, in the library's static
 * device scratch (no allocation, no profiling events). */
static void mha_run(struct sam_model *m, const char *who, int noalloc, int P,
                    int Nq, int Nk, int dint, hipb_mem qp, long sq, hipb_mem kp,
                    long sk, hipb_mem vp, long sv, hipb_mem o)
{
    struct hipb_backend *be = m->hip;
    const int c = dint / DEC_HEADS;
    const float scale = 1.0f / sqrtf((float)c);
    const int many = Nk > 64;
    const char *what;
    double flops;
    int err;

    if (P < 1 || Nq < 1 || Nk < 1 || dint < DEC_HEADS || sq < 0 || sk < 0 ||
        sv < 0) {
        hipb_fatal("%s: invalid shape P=%d Nq=%d Nk=%d dint=%d", who, P, Nq, Nk,
                   dint);
        return;
    }
    /* The reference takes c == 16 for many keys and its float16 vector
     * kernels need c of 16 or 32 (sam3_kernels.cl:527-569). */
    if ((many && c != 16) || dint % DEC_HEADS || (c != 16 && c != 32)) {
        hipb_fatal("%s: unsupported shape", who);
        return;
    }
    /* The many-keys kernel reads rows as 16-byte vectors. */
    if (many && (sq % 4 || sk % 4 || sv % 4)) {
        hipb_fatal("%s: per-prompt strides must be multiples of 4 floats "
                   "with many keys (sq=%ld sk=%ld sv=%ld)", who, sq, sk, sv);
        return;
    }
    if (!buf_ok(who, "q", qp, dec_extent(P, sq, Nq, dint), HIPB_F32) ||
        !buf_ok(who, "k", kp, dec_extent(P, sk, Nk, dint), HIPB_F32) ||
        !buf_ok(who, "v", vp, dec_extent(P, sv, Nk, dint), HIPB_F32) ||
        !buf_ok(who, "o", o, (size_t)P * Nq * dint, HIPB_F32))
        return;
    flops = 4.0 * P * DEC_HEADS * (double)Nq * Nk * c;
    if (!noalloc)
        hipb_run_begin(be);
    if (many) {
        const size_t need = mha_manykeys_scratch(P, Nq, Nk);
        void *scr = NULL;

        if (need && noalloc) {
            if (need > MHA_NOALLOC_BYTES) {
                hipb_fatal("%s: %zu bytes of split partials exceed the static "
                           "scratch of %zu bytes", who, need, MHA_NOALLOC_BYTES);
                return;
            }
            scr = dec_scratch(be->device);
            if (!scr) {
                hipb_fatal("%s: no device scratch on device %d (hipb_init "
                           "resolves it)", who, be->device);
                return;
            }
        }
        else if (need) {
            scr = hipb_scratch(be, need);
            if (!scr)
                return;
        }
        err = launch_mha_manykeys(qp->ptr, sq, kp->ptr, sk, vp->ptr, sv,
                                  o->ptr, P, Nq, Nk, dint, scale, scr,
                                  be->stream);
        what = "attn_manykeys";
    }
    else if (be->bf16 && c == 32 && Nk <= 8 && (sq | sk | sv) % 4 == 0) {
        /* precision=bf16: the decoder's token self-attention, four lanes
         * per (query, head) instead of the reference's one. */
        err = launch_mha_few32x4(qp->ptr, sq, kp->ptr, sk, vp->ptr, sv,
                                 o->ptr, P, Nq, Nk, dint, scale, be->stream);
        what = "attn_fewkeys";
    }
    else {
        err = launch_mha_fewkeys(qp->ptr, sq, kp->ptr, sk, vp->ptr, sv,
                                 o->ptr, P, Nq, Nk, dint, scale, be->stream);
        what = "attn_fewkeys";
    }
    if (!noalloc)
        hipb_run_end(be, err, what, flops);
    else if (err != hipSuccess)
        hipb_fatal("HIP: %s failed: %s (%d)", what, hipb_errstr(err), err);
}

void mha(struct sam_model *m, int P, int Nq, int Nk, int dint, hipb_mem qp,
         long sq, hipb_mem kp, long sk, hipb_mem vp, long sv, hipb_mem o)
{
    mha_run(m, "mha", 0, P, Nq, Nk, dint, qp, sq, kp, sk, vp, sv, o);
}

void mha_noalloc(struct sam_model *m, int P, int Nq, int Nk, int dint,
                 hipb_mem qp, long sq, hipb_mem kp, long sk, hipb_mem vp,
                 long sv, hipb_mem o)
{
    mha_run(m, "mha_noalloc", 1, P, Nq, Nk, dint, qp, sq, kp, sk, vp, sv, o);
}

/* ------------------------------------------------------------ attention */

/* Grow a model-owned staging buffer of element type dt to count
 * elements. */
/* Bumped by every work-buffer (re)allocation: a captured trunk graph
 * holds buffer addresses and is valid only while this has not moved. */
static unsigned long work_gen;

static int ensure_typed(struct hipb_backend *b, hipb_mem *buf, size_t count,
                        int dt, const char *what)
{
    if (*buf && hipb_count(*buf) >= count)
        return 1;
    if (*buf) {
        hipb_finish(b);
        hipb_release(buf);
    }
    *buf = hipb_alloc_typed(b, count, dt, what);
    work_gen++;
    return *buf != NULL;
}

static int ensure_bf16(struct hipb_backend *b, hipb_mem *buf, size_t count,
                       const char *what)
{
    return ensure_typed(b, buf, count, HIPB_BF16, what);
}

/* Key splits of the bf16 attention: enough (unit, query tile, split)
 * workgroups to fill one round of three per CU when the units and query
 * tiles alone leave CUs idle, each split keeping at least two 64-key
 * blocks, at most 64 splits. The ViT shapes (656 and 720 workgroups)
 * stay at one. */
static int attn_splits(const struct hipb_backend *b, int N, int Nk, int nb)
{
    const long items = (long)nb * ((N + 127) / 128);
    const int nblk = (Nk + 63) / 64, cus = b->cu_count > 0 ? b->cu_count : 256;
    long ns = 3L * cus / (items > 0 ? items : 1);

    if (ns > nblk / 2)
        ns = nblk / 2;
    if (ns > 64) /* the launchers' limit */
        ns = 64;
    return ns > 1 ? (int)ns : 1;
}

/* Key groups inside the workgroup (launch_attn_bf16_grp) for plain
 * attention that the query tiles alone leave launch-starved (attn_splits
 * would split the keys): 4 groups of 64-query tiles when those tiles fit
 * on the CUs at once with two key blocks per group, else 2 groups of
 * 128-query tiles with two blocks each, else 0 (the split launch, its
 * splits merged by their last workgroup). One 576-token window of 16 heads: 144 workgroups of four
 * groups of 2-3 key blocks. */
static int attn_groups(const struct hipb_backend *b, const struct attn_desc *d, int N,
                       int Nk, int nb)
{
    const int nblk = (Nk + 63) / 64, cus = b->cu_count > 0 ? b->cu_count : 256;
    const long t64 = (long)nb * ((N + 63) / 64), t128 = (long)nb * ((N + 127) / 128);

    if (d->hd != 64 || d->bias || d->causal || attn_splits(b, N, Nk, nb) <= 1)
        return 0;
    if (t64 <= cus && nblk >= 8)
        return 4;
    if (t128 <= cus && nblk >= 4)
        return 2;
    return 0;
}

/* Records of nsplit key splits merged inside their launch (both paths):
 * nb, 128-query tiles, SPLIT_RECS(nsplit) records of 9216 floats. */
static float *attn_part(struct sam_model *m, int N, int nb, int nsplit)
{
    const size_t tiles = ((size_t)N + 127) / 128;
    const size_t count = (size_t)nb * tiles * SPLIT_RECS((size_t)nsplit) * 9216;

    if (nsplit <= 1)
        return NULL;
    if (!ensure_typed(m->hip, &m->apart, count, HIPB_F32, "attention split partials"))
        return NULL;
    return (float *)m->apart->ptr;
}

/* n arrival counts (one per 128-query tile for the balanced bf16 launch,
 * SPLIT_CNT per tile for key splits), zero between launches: zero-filled
 * when (re)allocated, and every launch that counts in resets each count it
 * used. */
static unsigned *attn_cnt(struct sam_model *m, long tiles)
{
    struct hipb_backend *b = m->hip;
    const int fresh = !m->askcnt || hipb_count(m->askcnt) < (size_t)tiles;
    int err;

    if (!ensure_typed(b, &m->askcnt, (size_t)tiles, HIPB_F32, "attention arrival counts"))
        return NULL;
    if (fresh) {
        hipb_run_begin(b);
        err = launch_attn_sk_zero((unsigned *)m->askcnt->ptr, tiles, b->stream);
        hipb_run_end(b, err, "attn_sk_zero", 0.0);
        if (hipb_failed())
            return NULL;
    }
    return (unsigned *)m->askcnt->ptr;
}

/* Balanced launch of the bf16 attention (launch_attn_bf16's skG, skdp):
 * when an XCD's share of the 128-query tiles lies strictly between two
 * and three per CU (the global ViT block: 82 tiles per XCD on 32 CUs),
 * two whole tiles per CU run as before and one more workgroup per CU
 * takes an even share of the remaining tiles' key blocks (stream-K), so
 * that no CU runs three whole tiles while others run two. Only for head
 * width 64 without bias or causal mask, with tiles of at least 16 key
 * blocks. Returns skG (0: the plain grid) and sets *dp. */
static int attn_sk(const struct hipb_backend *b, const struct attn_desc *d, int N,
                   int Nk, int nb, int nsplit, int *dp)
{
    const long tiles = (long)nb * ((N + 127) / 128), per = (tiles + 7) / 8;
    const int nblk = (Nk + 63) / 64, cus = b->cu_count > 0 ? b->cu_count : 256;
    const int c = cus / 8; /* CUs per XCD */

    *dp = 0;
    if (nsplit != 1 || d->hd != 64 || d->bias || d->causal || nblk < 16 || c < 1 ||
        per <= 2L * c || per >= 3L * c || (per - 2L * c) * nblk < c ||
        (per - 2L * c) * nblk * c > 0x7fffffffL)
        return 0;
    *dp = 2 * c;
    return c;
}

/* Records and per-tile arrival counters of the balanced attention (G
 * stream-K workgroups per XCD); the counters are cleared by a fill kernel
 * when (re)allocated, which happens outside graph capture (the eager pass
 * before a capture allocates every work buffer), and every launch leaves
 * them zero. */
static int attn_skbuf(struct sam_model *m, int G, long tiles, float **rec,
                      unsigned **cnt)
{
    if (!ensure_typed(m->hip, &m->askrec, (size_t)8 * G * ATTN_SK_REC_FLOATS, HIPB_F32,
                      "balanced attention records") ||
        !(*cnt = attn_cnt(m, tiles)))
        return 0;
    *rec = (float *)m->askrec->ptr;
    return 1;
}

/* The fused attention of attn_fused at head width hd: 64 on both paths,
 * 32 on the bf16 path (operands packed with zero channels 32..63). */
static void attn_fused_hd(struct sam_model *m, const char *who, int hd, int N,
                          int Nk, int nb, int nb1, struct opnd Q, struct opnd K,
                          struct opnd V, struct opnd O, hipb_mem rope,
                          int npos, float scale, int causal, hipb_mem bias, int bW)
{
    struct hipb_backend *b = m->hip;
    struct attn_desc d;
    int err;

    if (N < 0 || Nk < 0 || nb < 1 || nb1 < 1 || (rope && npos < 1)) {
        hipb_fatal("%s: invalid shape N=%d Nk=%d nb=%d nb1=%d npos=%d", who, N,
                   Nk, nb, nb1, npos);
        return;
    }
    if (!(hd == 64 || (hd == 32 && !rope))) {
        hipb_fatal("%s: unsupported head width %d", who, hd);
        return;
    }
    if (N == 0 || Nk == 0)
        return;
    if (!opnd_ok(who, "Q", Q, N, hd, nb, nb1) ||
        !opnd_ok(who, "K", K, Nk, hd, nb, nb1) ||
        !opnd_ok(who, "V", V, Nk, hd, nb, nb1) ||
        !opnd_ok(who, "O", O, N, hd, nb, nb1))
        return;
    if (Q.buf->dtype != HIPB_F32 || K.buf->dtype != HIPB_F32 ||
        V.buf->dtype != HIPB_F32 || O.buf->dtype == HIPB_F16) {
        hipb_fatal("%s: Q, K, V must be float; O float or bf16", who);
        return;
    }
    if (rope && !buf_ok(who, "rope", rope, (size_t)npos * hd, HIPB_F32))
        return;
    d.N = N;
    d.nb = nb;
    d.nb1 = nb1;
    d.Q = Q.buf->ptr;
    d.qoff = Q.off;
    d.ldq = Q.ld;
    d.sq0 = Q.s0;
    d.sq1 = Q.s1;
    d.K = K.buf->ptr;
    d.koff = K.off;
    d.ldk = K.ld;
    d.sk0 = K.s0;
    d.sk1 = K.s1;
    d.V = V.buf->ptr;
    d.voff = V.off;
    d.ldv = V.ld;
    d.sv0 = V.s0;
    d.sv1 = V.s1;
    d.O = O.buf->ptr;
    d.ooff = O.off;
    d.ldo = O.ld;
    d.so0 = O.s0;
    d.so1 = O.s1;
    d.odt = O.buf->dtype;
    d.rope = rope ? (const float *)rope->ptr : NULL;
    d.npos = rope ? npos : 1;
    d.scale = scale;
    d.hd = hd;
    d.Nk = Nk;
    d.causal = causal != 0;
    d.bias = bias ? (const float *)bias->ptr : NULL;
    d.bW = bias ? bW : 0;
    if (bias && bW > 0 &&
        (bW < 64 || bW % 8 || Nk % bW || (Nk / bW) % 4 || (b->bf16 && hd != 32) ||
         !buf_ok(who, "bias rows", bias, (size_t)nb * N * ((size_t)Nk / bW + bW),
                 HIPB_F32))) {
        if (!hipb_failed())
            hipb_fatal("%s: bias rows need W >= 64, a multiple of 8 dividing Nk "
                       "into a multiple of 4 rows (bf16: head width 32)", who);
        return;
    }
    if (bias && bW == 0 &&
        !buf_ok(who, "bias table", bias,
                (size_t)nb * N * (((size_t)Nk + 63) / 64 * 64), HIPB_F32))
        return;
    if (b->bf16) {
        const size_t np = ((size_t)N + 63) / 64 * 64;
        const size_t npk = ((size_t)Nk + 63) / 64 * 64;

        if (!ensure_bf16(b, &m->q16, (size_t)nb * np * 64, "packed q") ||
            !ensure_bf16(b, &m->k16, (size_t)nb * npk * 64, "packed k") ||
            !ensure_bf16(b, &m->vt16, (size_t)nb * npk * 64, "packed v^T") ||
            !ensure_typed(b, &m->knorm, (size_t)nb * (npk / 64), HIPB_F32,
                          "key block norms"))
            return;
        hipb_run_begin(b);
        err = launch_qkv_pack(&d, m->q16->ptr, m->k16->ptr, m->vt16->ptr,
                              (float *)m->knorm->ptr, b->stream);
        hipb_run_end(b, err, "qkv_pack", 0.0);
        if (hipb_failed())
            return;
        {
            const int ng = attn_groups(b, &d, N, Nk, nb);
            const int ns = ng ? 1 : attn_splits(b, N, Nk, nb);
            int dp;
            const int G = attn_sk(b, &d, N, Nk, nb, ns, &dp);
            float *part = attn_part(m, N, nb, ns), *skrec = NULL;
            unsigned *skcnt =
                ns > 1 ? attn_cnt(m, (long)nb * ((N + 127) / 128) * SPLIT_CNT) : NULL;

            if ((ns > 1 && (!part || !skcnt)) ||
                (G && !attn_skbuf(m, G, (long)nb * ((N + 127) / 128), &skrec, &skcnt)))
                return;
            hipb_run_begin(b);
            err = ng ? launch_attn_bf16_grp(&d, m->q16->ptr, m->k16->ptr, m->vt16->ptr,
                                            (const float *)m->knorm->ptr, ng, b->stream)
                     : launch_attn_bf16(&d, m->q16->ptr, m->k16->ptr, m->vt16->ptr,
                                        (const float *)m->knorm->ptr, part, ns, skrec,
                                        skcnt, G, dp, b->stream);
            hipb_run_end(b, err, "attn_bf16", 4.0 * N * (double)Nk * hd * nb);
        }
        return;
    }
    {
        /* The exact kernel's key blocks are 32 keys: split by those, at
         * least three blocks per split, into one full round of three
         * workgroups per CU when the blocks allow it, else one round of
         * one per CU (at least two splits); the splits merge inside the
         * launch. A round that leaves most CUs with two workgroups and
         * some with one ran slower than either. One 576-token window of
         * 16 heads (80 tiles, 18 blocks): 3 splits, 240 workgroups, 26.0
         * us (6 splits 27.4 us, 9 splits 33 us); the decoder's box-biased
         * cross-attention (16 tiles, 162 blocks): 48 splits, 768
         * workgroups, 42.1 us (27 splits 44.1 us, 16 splits 50.2 us). */
        int ns = attn_splits(b, N, Nk, nb);

        if (ns > 1) {
            const int cus = b->cu_count > 0 ? b->cu_count : 256;
            const long items = (long)nb * ((N + 127) / 128), cap = (Nk + 31) / 32 / 3;
            long n32 = 3L * cus / items;

            if (n32 > cap)
                n32 = cus / items;
            if (n32 < 2)
                n32 = 2;
            if (n32 > cap)
                n32 = cap;
            if (n32 > 64)
                n32 = 64;
            ns = n32 > 1 ? (int)n32 : 1;
        }
        float *part = attn_part(m, N, nb, ns);
        unsigned *cnt = ns > 1 ? attn_cnt(m, (long)nb * ((N + 127) / 128) * SPLIT_CNT) : NULL;

        if (ns > 1 && (!part || !cnt))
            return;
        hipb_run_begin(b);
        err = launch_attn_f32(&d, part, cnt, ns, b->stream);
        hipb_run_end(b, err, "attn_f32", 4.0 * N * (double)Nk * hd * nb);
    }
}

void attn_fused(struct sam_model *m, int N, int nb, int nb1, struct opnd Q,
                struct opnd K, struct opnd V, struct opnd O, hipb_mem rope,
                int npos, float scale)
{
    if (m->hd != 0 && m->hd != 64) {
        hipb_fatal("attn_fused: unsupported head width %d", m->hd);
        return;
    }
    attn_fused_hd(m, "attn_fused", 64, N, N, nb, nb1, Q, K, V, O, rope, npos,
                  scale, 0, NULL, 0);
}

void attn_packed(struct sam_model *m, int N, int nb, int nb1, struct opnd O)
{
    struct hipb_backend *b = m->hip;
    const size_t np = ((size_t)N + 63) / 64 * 64;
    struct attn_desc d;
    float *part, *skrec = NULL;
    unsigned *skcnt = NULL;
    int err, ns, G, dp, ng;

    if (N < 1 || nb < 1 || nb1 < 1) {
        hipb_fatal("attn_packed: invalid shape N=%d nb=%d nb1=%d", N, nb, nb1);
        return;
    }
    if (!buf_ok("attn_packed", "q16", m->q16, (size_t)nb * np * 64, HIPB_BF16) ||
        !buf_ok("attn_packed", "k16", m->k16, (size_t)nb * np * 64, HIPB_BF16) ||
        !buf_ok("attn_packed", "vt16", m->vt16, (size_t)nb * np * 64,
                HIPB_BF16) ||
        !buf_ok("attn_packed", "knorm", m->knorm, (size_t)nb * (np / 64),
                HIPB_F32) ||
        !opnd_ok("attn_packed", "O", O, N, 64, nb, nb1))
        return;
    if (O.buf->dtype == HIPB_F16) {
        hipb_fatal("attn_packed: O must be float or bf16");
        return;
    }
    memset(&d, 0, sizeof(d));
    d.N = N;
    d.nb = nb;
    d.nb1 = nb1;
    d.hd = 64;
    d.Nk = N;
    d.O = O.buf->ptr;
    d.ooff = O.off;
    d.ldo = O.ld;
    d.so0 = O.s0;
    d.so1 = O.s1;
    d.odt = O.buf->dtype;
    ng = attn_groups(b, &d, N, N, nb);
    ns = ng ? 1 : attn_splits(b, N, N, nb);
    G = attn_sk(b, &d, N, N, nb, ns, &dp);
    part = attn_part(m, N, nb, ns);
    if (ns > 1 && !(skcnt = attn_cnt(m, (long)nb * ((N + 127) / 128) * SPLIT_CNT)))
        return;
    if ((ns > 1 && !part) ||
        (G && !attn_skbuf(m, G, (long)nb * ((N + 127) / 128), &skrec, &skcnt)))
        return;
    hipb_run_begin(b);
    err = ng ? launch_attn_bf16_grp(&d, m->q16->ptr, m->k16->ptr, m->vt16->ptr,
                                    (const float *)m->knorm->ptr, ng, b->stream)
             : launch_attn_bf16(&d, m->q16->ptr, m->k16->ptr, m->vt16->ptr,
                                (const float *)m->knorm->ptr, part, ns, skrec, skcnt,
                                G, dp, b->stream);
    hipb_run_end(b, err, "attn_bf16", 4.0 * N * (double)N * 64 * nb);
}

void attend(struct sam_model *m, int Nq, int Nk, int heads, int hd, hipb_mem Q,
            int ldq, hipb_mem K, int ldk, hipb_mem V, int ldv, hipb_mem O,
            int ldo, int causal, hipb_mem dy, hipb_mem dx, int W)
{
    struct hipb_backend *b = m->hip;
    const long plane = (long)Nq * Nk;
    const float scale = 1.0f / sqrtf((float)hd);
    long hcl;
    int hc, h0;

    if (Nq < 0 || Nk < 0 || heads < 1 || hd < 1) {
        hipb_fatal("attend: invalid shape Nq=%d Nk=%d heads=%d hd=%d", Nq, Nk,
                   heads, hd);
        return;
    }
    if (Nq == 0 || Nk == 0)
        return;
    if (dy && (!dx || W < 1 || Nk % W ||
               !buf_ok("attend", "dy", dy, (size_t)Nq * (Nk / W) * heads,
                       HIPB_F32) ||
               !buf_ok("attend", "dx", dx, (size_t)Nq * W * heads, HIPB_F32))) {
        if (!hipb_failed())
            hipb_fatal("attend: box bias needs dy, dx and W dividing Nk");
        return;
    }
    /* Fused for head width 64 or 32 with any mask or bias, on both paths.
     * The box bias goes to the kernels as rows of each (head, query)'s dy
     * and dx values, H + W floats, which they add as dy[j / W] + dx[j % W]
     * per key, when W >= 64 is a multiple of 8 and H of 4 (the decoder's
     * 72 x 72 grid) on the exact path or at head width 32 on bf16; else as
     * a table [head][Nq][Nk padded to 64] of the sums. On the bf16 path
     * both are scaled to its exp2 domain. Heads are the units, head h at
     * column h hd of every operand. */
    if (hd == 64 || hd == 32) {
        const int rows = dy && W >= 64 && W % 8 == 0 && (Nk / W) % 4 == 0 &&
                         (!b->bf16 || hd == 32);

        if (dy) {
            const float us = b->bf16 ? LOG2E_HOST : 1.0f;
            const size_t n = rows ? (size_t)heads * Nq * ((size_t)Nk / W + W)
                                  : (size_t)heads * Nq * (((size_t)Nk + 63) / 64 * 64);
            int err;

            if (!ensure_typed(b, &m->abias, n, HIPB_F32, "attention bias"))
                return;
            hipb_run_begin(b);
            err = rows ? launch_box_rows((float *)m->abias->ptr, (const float *)dy->ptr,
                                         (const float *)dx->ptr, heads, Nq, Nk, W, heads, us,
                                         b->stream)
                       : launch_box_bias((float *)m->abias->ptr, (const float *)dy->ptr,
                                         (const float *)dx->ptr, heads, Nq, Nk, W, heads, us,
                                         b->stream);
            hipb_run_end(b, err, rows ? "box_rows" : "box_bias", 0.0);
            if (hipb_failed())
                return;
        }
        attn_fused_hd(m, "attend", hd, Nq, Nk, heads, heads,
                      bmat(Q, 0, ldq, 0, hd), bmat(K, 0, ldk, 0, hd),
                      bmat(V, 0, ldv, 0, hd), bmat(O, 0, ldo, 0, hd), NULL, 1,
                      scale, causal, dy ? m->abias : NULL, rows ? W : 0);
        return;
    }
    /* The reference's sequence (sam3_text.c:305-343): per chunk of heads
     * whose scores fit the score buffer, Q K^T / sqrt(hd), softmax_ext,
     * P V. */
    hcl = m->score_cap / plane;
    hc = hcl > heads ? heads : (int)hcl;
    if (hc < 1) {
        hipb_fatal("attend: device cannot hold %d x %d attention scores", Nq,
                   Nk);
        return;
    }
    if (!ensure_typed(b, &m->scores, (size_t)hc * plane, HIPB_F32,
                      "attention scores"))
        return;
    for (h0 = 0; h0 < heads && !hipb_failed(); h0 += hc) {
        const int hcc = heads - h0 < hc ? heads - h0 : hc;

        gemm(m, Nq, Nk, hd, bmat(Q, (long)h0 * hd, ldq, 0, hd),
             bmat(K, (long)h0 * hd, ldk, 0, hd), 1,
             bmat(m->scores, 0, Nk, 0, plane), hcc, hcc, NULL, NULL, 0, scale,
             ACT_NONE);
        softmax_ext(m, m->scores, (long)hcc * Nq, Nk, Nq, h0, causal, dy, dx, W,
                    heads);
        gemm(m, Nq, hd, Nk, bmat(m->scores, 0, Nk, 0, plane),
             bmat(V, (long)h0 * hd, ldv, 0, hd), 0,
             bmat(O, (long)h0 * hd, ldo, 0, hd), hcc, hcc, NULL, NULL, 0, 1.0f,
             ACT_NONE);
    }
}

/* Attention geometry of a block (block_geom, sam3_model.c:777-791). */
struct geom {
    int s, nwx, nwin, N;
};

static struct geom block_geom(const struct sam_model *m,
                              const struct vit_block *blk)
{
    struct geom g;

    g.s = blk->window ? blk->window : m->grid;
    g.nwx = (m->grid + g.s - 1) / g.s;
    g.nwin = g.nwx * g.nwx;
    g.N = g.s * g.s;
    return g;
}

/* Heads whose score planes fit the score buffer (head_chunk,
 * sam3_model.c:793-798). */
static int head_chunk(const struct sam_model *m, const struct geom *g)
{
    long hc = m->score_cap / ((long)g->nwin * g->N * g->N);

    return hc > m->heads ? m->heads : (int)hc;
}

/* The attention region of vit_attention with its output operand O
 * (rows of the block's window order, head h at column h * hd). */
/* QKV projection of a block written straight as the packed attention
 * operands (the NT GEMM's packed store: RoPE, scale, bf16, V^T and the
 * key block norms in the GEMM epilogue, no fp32 qkv round trip). Returns
 * 0 without queueing anything when the shape does not allow it (head
 * width 64, E % 128 == 0 and N % 64 == 0 are needed), 1 when queued. */
static int qkv_projection_packed(struct sam_model *m, const struct vit_block *blk,
                                 long rows, int N, hipb_mem table, float scale)
{
    struct hipb_backend *b = m->hip;
    const int E = m->embed;
    const long nb = rows / (N > 0 ? N : 1) * m->heads;
    struct gemm_desc d;
    int err;

    if (m->hd != 64 || E % 128 || N < 64 || N % 64 || rows % N ||
        !blk->qkvw || blk->qkvw->dtype != HIPB_BF16 || !m->xn16 ||
        (blk->qkvb && blk->qkvb->dtype != HIPB_F32))
        return 0;
    memset(&d, 0, sizeof(d));
    d.M = (int)rows;
    d.N = 3 * E;
    d.K = E;
    d.A = m->xn16->ptr;
    d.lda = E;
    d.adt = HIPB_BF16;
    d.B = blk->qkvw->ptr;
    d.ldb = E;
    d.bdt = HIPB_BF16;
    d.transb = 1;
    d.cdt = HIPB_F32;
    d.nb = d.nb1 = 1;
    d.bias = blk->qkvb ? (const float *)blk->qkvb->ptr : NULL;
    d.alpha = 1.0f;
    d.act = ACT_NONE;
    d.mode = MODE_BF16;
    d.pack_N = N;
    d.pack_E = E;
    d.pack_npos = N;
    d.pack_scale = scale;
    d.pack_rope = (const float *)table->ptr;
    if (!gemm_nt_ok(&d))
        return 0;
    if (!buf_ok("vit_attention", "normalized tokens", m->xn16, (size_t)rows * E,
                HIPB_BF16) ||
        !buf_ok("vit_attention", "qkv weight", blk->qkvw, (size_t)3 * E * E,
                HIPB_BF16) ||
        (blk->qkvb && !buf_ok("vit_attention", "qkv bias", blk->qkvb,
                              (size_t)3 * E, HIPB_F32)) ||
        !buf_ok("vit_attention", "rope", table, (size_t)N * 64, HIPB_F32) ||
        !ensure_bf16(b, &m->q16, (size_t)nb * N * 64, "packed q") ||
        !ensure_bf16(b, &m->k16, (size_t)nb * N * 64, "packed k") ||
        !ensure_bf16(b, &m->vt16, (size_t)nb * N * 64, "packed v^T") ||
        !ensure_typed(b, &m->knorm, (size_t)nb * (N / 64), HIPB_F32,
                      "key block norms"))
        return 0;
    d.pack_q16 = m->q16->ptr;
    d.pack_k16 = m->k16->ptr;
    d.pack_vt16 = m->vt16->ptr;
    d.pack_knorm = (float *)m->knorm->ptr;
    hipb_run_begin(b);
    err = launch_gemm_nt(&d, b->stream);
    hipb_run_end(b, err, "gemm_nt_qkv_pack", 2.0 * rows * 3.0 * E * E);
    return !hipb_failed();
}

static void attention_region(struct sam_model *m, const struct vit_block *blk,
                             int unfused, hipb_mem obuf)
{
    struct hipb_backend *b = m->hip;
    const struct geom g = block_geom(m, blk);
    const int T = m->grid * m->grid, E = m->embed, hd = m->hd;
    const long rows = (long)g.nwin * g.N;
    const float scale = 1.0f / sqrtf((float)hd);
    hipb_mem table = blk->window ? m->rope_win : m->rope_glob;
    hipb_mem A = m->xn;
    int h0;

    if (!table) {
        hipb_fatal("vit_attention: no RoPE table for this block");
        return;
    }
    if (rows > (long)(hipb_count(m->qkv) / (3 * (size_t)E))) {
        hipb_fatal("vit_attention: block needs %ld rows, work buffers hold "
                   "fewer",
                   rows);
        return;
    }
    if (b->bf16 && !unfused) {
        /* LayerNorm straight into bf16 in window-partitioned row order,
         * QKV projection on bf16 MFMA, then the packed fast path. */
        if (!ensure_bf16(b, &m->xn16, (size_t)rows * E, "normalized tokens "
                                                        "(bf16)") ||
            !buf_ok("vit_attention", "x", m->x, (size_t)T * E, HIPB_F32))
            return;
        hipb_run_begin(b);
        {
            int err = launch_layernorm(
                m->x->ptr, m->xn16->ptr, HIPB_BF16, blk->n1w->ptr,
                blk->n1b->ptr, T, E, ENC_EPS, ACT_NONE,
                blk->window ? m->grid : 0, blk->window ? g.s : 0, g.nwx,
                b->stream);
            hipb_run_end(b, err, "layernorm", 0.0);
        }
        if (hipb_failed())
            return;
        if (qkv_projection_packed(m, blk, rows, g.N, table, scale)) {
            attn_packed(m, g.N, g.nwin * m->heads, m->heads,
                        bmat(obuf, 0, E, (long)g.N * E, hd));
            return;
        }
        if (hipb_failed())
            return;
        linear(m, (int)rows, E, 3 * E, m->xn16, 0, blk->qkvw, blk->qkvb,
               m->qkv, 0, ACT_NONE, 0);
        if (hipb_failed())
            return;
        attn_fused(m, g.N, g.nwin * m->heads, m->heads,
                   bmat(m->qkv, 0, 3 * E, (long)g.N * 3 * E, hd),
                   bmat(m->qkv, E, 3 * E, (long)g.N * 3 * E, hd),
                   bmat(m->qkv, 2L * E, 3 * E, (long)g.N * 3 * E, hd),
                   bmat(obuf, 0, E, (long)g.N * E, hd), table, g.N, scale);
        return;
    }

    layernorm(m, T, E, m->x, m->xn, blk->n1w, blk->n1b, ENC_EPS, ACT_NONE);
    if (blk->window) {
        window_partition(m, m->xn, m->xw, m->grid, E, g.s, g.nwx);
        A = m->xw;
    }
    linear(m, (int)rows, E, 3 * E, A, 0, blk->qkvw, blk->qkvb, m->qkv, 0,
           ACT_NONE, 0);
    if (hipb_failed())
        return;
    if (!unfused) {
        /* RoPE and the scale are applied on the Q/K loads. */
        attn_fused(m, g.N, g.nwin * m->heads, m->heads,
                   bmat(m->qkv, 0, 3 * E, (long)g.N * 3 * E, hd),
                   bmat(m->qkv, E, 3 * E, (long)g.N * 3 * E, hd),
                   bmat(m->qkv, 2L * E, 3 * E, (long)g.N * 3 * E, hd),
                   bmat(obuf, 0, E, (long)g.N * E, hd), table, g.N, scale);
        return;
    }

    /* The reference's sequence (sam3_model.c:998-1013). */
    rope_apply(m, table, rows, g.N);
    if (!m->scores) {
        size_t need = 0;
        int i;

        for (i = 0; i < m->depth; i++) {
            const struct geom gi = block_geom(m, &m->blocks[i]);
            size_t n = (size_t)head_chunk(m, &gi) * gi.nwin * gi.N * gi.N;

            if (n > need)
                need = n;
        }
        if (need == 0)
            need = (size_t)head_chunk(m, &g) * g.nwin * g.N * g.N;
        m->scores = hipb_alloc(b, need * sizeof(float), "attention scores");
        if (!m->scores)
            return;
    }
    {
        const int hc = head_chunk(m, &g);

        for (h0 = 0; h0 < m->heads && !hipb_failed(); h0 += hc) {
            int hcc = m->heads - h0 < hc ? m->heads - h0 : hc;
            long plane = (long)g.N * g.N, tstride = (long)g.N * 3 * E;

            gemm(m, g.N, g.N, hd,
                 bmat(m->qkv, (long)h0 * hd, 3 * E, tstride, hd),
                 bmat(m->qkv, E + (long)h0 * hd, 3 * E, tstride, hd), 1,
                 bmat(m->scores, 0, g.N, hcc * plane, plane), g.nwin * hcc,
                 hcc, NULL, NULL, 0, scale, ACT_NONE);
            softmax_rows(m, m->scores, (long)g.nwin * hcc * g.N, g.N);
            gemm(m, g.N, hd, g.N, bmat(m->scores, 0, g.N, hcc * plane, plane),
                 bmat(m->qkv, 2L * E + (long)h0 * hd, 3 * E, tstride, hd), 0,
                 bmat(obuf, (long)h0 * hd, E, (long)g.N * E, hd),
                 g.nwin * hcc, hcc, NULL, NULL, 0, 1.0f, ACT_NONE);
        }
    }
}

void vit_attention(struct sam_model *m, const struct vit_block *blk,
                   int unfused)
{
    attention_region(m, blk, unfused, m->attn);
}

/* ------------------------------------------------------------ trunk */

/* x[token(r)] += A[r] W^T + b for the window-partitioned rows r of a
 * windowed block: the projection and window_unpartition_add
 * (sam3_model.c:1015-1019) in one bf16 NT GEMM whose epilogue maps each
 * row to its grid token. Returns 0 (nothing queued) when the operands do
 * not take the NT kernel. */
static int proj_unpartition(struct sam_model *m, long rows, hipb_mem A,
                            const struct vit_block *blk, int ws, int nwx)
{
    struct hipb_backend *b = m->hip;
    const int E = m->embed, T = m->grid * m->grid;
    struct gemm_desc d;
    int err;

    if (!opnd_ok("vit_block", "A", mat(A, 0, E), rows, E, 1, 1) ||
        !opnd_ok("vit_block", "projw", mat(blk->projw, 0, E), E, E, 1, 1) ||
        !buf_ok("vit_block", "x", m->x, (size_t)T * E, HIPB_F32) ||
        !buf_ok("vit_block", "projb", blk->projb, (size_t)E, HIPB_F32))
        return 1;
    memset(&d, 0, sizeof(d));
    d.M = (int)rows;
    d.N = E;
    d.K = E;
    d.A = A->ptr;
    d.lda = E;
    d.adt = A->dtype;
    d.B = blk->projw->ptr;
    d.ldb = E;
    d.bdt = blk->projw->dtype;
    d.transb = 1;
    d.C = m->x->ptr;
    d.ldc = E;
    d.cdt = HIPB_F32;
    d.nb = d.nb1 = 1;
    d.bias = (const float *)blk->projb->ptr;
    d.R = m->x->ptr;
    d.alpha = 1.0f;
    d.act = ACT_NONE;
    d.mode = b->bf16 ? MODE_BF16 : MODE_F32;
    d.unpart_H = m->grid;
    d.unpart_ws = ws;
    d.unpart_nwx = nwx;
    if (!gemm_nt_ok(&d))
        return 0;
    hipb_run_begin(b);
    err = launch_gemm_nt(&d, b->stream);
    hipb_run_end(b, err, "gemm_nt_bf16", 2.0 * rows * E * (double)E);
    return 1;
}

void vit_block(struct sam_model *m, const struct vit_block *blk, int unfused)
{
    struct hipb_backend *b = m->hip;
    const struct geom g = block_geom(m, blk);
    const int T = m->grid * m->grid, E = m->embed, mlp = m->mlp;
    const long rows = (long)g.nwin * g.N;
    hipb_mem A = m->attn;

    if (mlp < 1 || !m->tmp || !m->mlpbuf) {
        hipb_fatal("vit_block: no MLP work buffers (sam_path_init with "
                   "mlp > 0)");
        return;
    }
    /* With precision=bf16 the attention output goes to the MLP hidden
     * buffer as bf16 (free until norm2): the A operand of the bf16
     * projection. */
    if (b->bf16 && !unfused) {
        if (!ensure_bf16(b, &m->mlp16, (size_t)(rows > T ? rows : T) *
                                           (mlp > E ? mlp : E),
                         "mlp (bf16)"))
            return;
        A = m->mlp16;
    }
    attention_region(m, blk, unfused, A);
    if (hipb_failed())
        return;
    /* Projection with residual (sam3_model.c:1015-1022). */
    if (blk->window && proj_unpartition(m, rows, A, blk, g.s, g.nwx)) {
        /* fused into the NT GEMM (or an operand check failed: reported) */
    }
    else if (blk->window) {
        linear(m, (int)rows, E, E, A, 0, blk->projw, blk->projb, m->tmp, 0,
               ACT_NONE, 0);
        window_unpartition_add(m, m->x, m->tmp, m->grid, E, g.s, g.nwx);
    }
    else
        linear(m, T, E, E, A, 0, blk->projw, blk->projb, m->x, 0, ACT_NONE,
               1);
    if (hipb_failed())
        return;
    /* norm2 and the MLP (sam3_model.c:1024-1027); with precision=bf16 the
     * normalised tokens and the hidden layer are stored as bf16. */
    if (b->bf16 && !unfused) {
        if (!ensure_bf16(b, &m->xn16, (size_t)T * E, "normalized tokens "
                                                     "(bf16)") ||
            !ensure_bf16(b, &m->mlp16, (size_t)T * mlp, "mlp (bf16)"))
            return;
        layernorm(m, T, E, m->x, m->xn16, blk->n2w, blk->n2b, ENC_EPS,
                  ACT_NONE);
        linear(m, T, E, mlp, m->xn16, 0, blk->l1w, blk->l1b, m->mlp16, 0,
               ACT_GELU, 0);
        linear(m, T, mlp, E, m->mlp16, 0, blk->l2w, blk->l2b, m->x, 0,
               ACT_NONE, 1);
    }
    else {
        layernorm(m, T, E, m->x, m->xn, blk->n2w, blk->n2b, ENC_EPS,
                  ACT_NONE);
        linear(m, T, E, mlp, m->xn, 0, blk->l1w, blk->l1b, m->mlpbuf, 0,
               ACT_GELU, 0);
        linear(m, T, mlp, E, m->mlpbuf, 0, blk->l2w, blk->l2b, m->x, 0,
               ACT_NONE, 1);
    }
}

/* Trunk preconditions and the image buffer; 1 when the trunk can run. */
static int trunk_ready(struct sam_model *m, const char *who)
{
    const int G = m->grid, ps = m->patch, E = m->embed, K = 3 * ps * ps;
    const long T = (long)G * G, side = (long)G * ps;

    if (ps < 1 || !m->pe_w || !m->pos || !m->lnpw || !m->lnpb) {
        hipb_fatal("%s: no patch size or trunk weights", who);
        return 0;
    }
    if (!m->mlpbuf || hipb_count(m->mlpbuf) < (size_t)T * K) {
        hipb_fatal("%s: work buffers hold fewer than %ld patch columns", who,
                   T * K);
        return 0;
    }
    return buf_ok(who, "pe_w", m->pe_w, (size_t)E * K, -1) &&
           buf_ok(who, "pos", m->pos, (size_t)T * E, HIPB_F32) &&
           ensure_typed(m->hip, &m->img, (size_t)3 * side * side, HIPB_F32,
                        "image");
}

/* Everything of the trunk after the image upload. */
static void trunk_kernels(struct sam_model *m)
{
    struct hipb_backend *b = m->hip;
    const int G = m->grid, ps = m->patch, E = m->embed, K = 3 * ps * ps;
    const long T = (long)G * G, side = (long)G * ps;
    int i, err;

    /* Patch embedding (no bias), tiled position embedding, ln_pre
     * (sam3_model.c:1119-1130); the position embedding (pos: [T][E], the
     * tokens' layout) is the product's residual operand, added in its
     * store as add_bcast would add it. With precision=bf16 the patch columns
     * (K = 588 at patch 14) and the weight rows are padded with zeros to
     * a multiple of 64 in the bf16 MLP buffer (free until the first
     * block's projection), so the product takes the NT GEMM's 64-wide K
     * steps instead of the general kernel; the zero columns add nothing. */
    if (b->bf16 && K % 64 != 0 && m->mlp > 0 &&
        (m->pe_w->dtype == HIPB_BF16 || m->pe_w->dtype == HIPB_F32)) {
        const int KP = (K + 63) / 64 * 64;
        const size_t need = (size_t)(T + E) * KP, blk = (size_t)T * (m->mlp > E ? m->mlp : E);

        if (!ensure_bf16(b, &m->mlp16, need > blk ? need : blk, "mlp (bf16)"))
            return;
        hipb_run_begin(b);
        err = launch_patch_im2col(m->img->ptr, m->mlp16->ptr, HIPB_BF16, (int)side, G, ps, KP,
                                  b->stream);
        hipb_run_end(b, err, "patch_im2col", 0.0);
        hipb_run_begin(b);
        err = launch_pad_rows_bf16(m->pe_w->ptr, m->pe_w->dtype,
                                   (uint16_t *)m->mlp16->ptr + (size_t)T * KP, E, K, KP,
                                   b->stream);
        hipb_run_end(b, err, "pad_rows", 0.0);
        if (hipb_failed())
            return;
        gemm(m, (int)T, E, KP, mat(m->mlp16, 0, KP), mat(m->mlp16, T * KP, KP), 1,
             mat(m->x, 0, E), 1, 1, NULL, m->pos, 0, 1.0f, ACT_NONE);
    }
    else {
        hipb_run_begin(b);
        err = launch_patch_im2col(m->img->ptr, m->mlpbuf->ptr, HIPB_F32, (int)side, G, ps, K,
                                  b->stream);
        hipb_run_end(b, err, "patch_im2col", 0.0);
        if (hipb_failed())
            return;
        gemm(m, (int)T, E, K, mat(m->mlpbuf, 0, K), mat(m->pe_w, 0, K), 1, mat(m->x, 0, E), 1,
             1, NULL, m->pos, 0, 1.0f, ACT_NONE);
    }
    layernorm(m, T, E, m->x, m->x, m->lnpw, m->lnpb, ENC_EPS, ACT_NONE);
    for (i = 0; i < m->depth && !hipb_failed(); i++)
        vit_block(m, &m->blocks[i], 0);
}

static void trunk_graph_drop(struct sam_model *m)
{
    if (m->trunk_exec)
        hipGraphExecDestroy((hipGraphExec_t)m->trunk_exec);
    if (m->trunk_graph)
        hipGraphDestroy((hipGraph_t)m->trunk_graph);
    m->trunk_exec = NULL;
    m->trunk_graph = NULL;
}

void sam_encode_trunk(struct sam_model *m, const float *img)
{
    struct hipb_backend *b = m->hip;
    const long side = (long)m->grid * m->patch;
    int err;

    if (!img) {
        hipb_fatal("sam_encode_trunk: no image");
        return;
    }
    if (!trunk_ready(m, "sam_encode_trunk"))
        return;
    hipb_write(b, m->img, 0, img, (size_t)3 * side * side * sizeof(float));
    if (hipb_failed())
        return;
    if (m->trunk_exec && !b->profile) {
        if (m->trunk_gen == work_gen) {
            err = hipGraphLaunch((hipGraphExec_t)m->trunk_exec,
                                 (hipStream_t)b->stream);
            hipb_run_end(b, err, "trunk_graph", 0.0);
            return;
        }
        trunk_graph_drop(m); /* a work buffer moved since the capture */
    }
    trunk_kernels(m);
}

void sam_trunk_graph(struct sam_model *m, int enable)
{
    struct hipb_backend *b = m->hip;
    hipGraph_t g = NULL;
    hipGraphExec_t x = NULL;
    unsigned long gen;
    int err, err2;

    if (b)
        hipb_finish(b);
    trunk_graph_drop(m);
    if (!enable)
        return;
    if (b->profile) {
        hipb_fatal("sam_trunk_graph: profiling runs the kernels one by one");
        return;
    }
    if (!trunk_ready(m, "sam_trunk_graph"))
        return;
    trunk_kernels(m); /* allocates whatever is still missing */
    hipb_finish(b);
    if (hipb_failed())
        return;
    gen = work_gen;
    err = hipStreamBeginCapture((hipStream_t)b->stream,
                                hipStreamCaptureModeRelaxed);
    if (err != hipSuccess) {
        hipb_fatal("sam_trunk_graph: hipStreamBeginCapture: %s (%d)",
                   hipb_errstr(err), err);
        return;
    }
    trunk_kernels(m);
    err = hipStreamEndCapture((hipStream_t)b->stream, &g);
    if (hipb_failed() || err != hipSuccess || !g || work_gen != gen) {
        if (g)
            hipGraphDestroy(g);
        if (!hipb_failed())
            hipb_fatal("sam_trunk_graph: capture failed: %s (%d)",
                       hipb_errstr(err), err);
        return;
    }
    err2 = hipGraphInstantiate(&x, g, NULL, NULL, 0);
    if (err2 != hipSuccess) {
        hipGraphDestroy(g);
        hipb_fatal("sam_trunk_graph: hipGraphInstantiate: %s (%d)",
                   hipb_errstr(err2), err2);
        return;
    }
    m->trunk_graph = g;
    m->trunk_exec = x;
    m->trunk_gen = gen;
}

/* ------------------------------------------------------------ setup */

void sam_path_init(struct sam_model *m, struct hipb_backend *b, int grid,
                   int embed, int heads, int hd, int mlp,
                   struct vit_block *blocks, int depth)
{
    const size_t f = sizeof(float);
    const long T = (long)grid * grid;
    size_t cap;
    long rows = T;
    int i;

    memset(m, 0, sizeof(*m));
    m->hip = b;
    m->grid = grid;
    m->embed = embed;
    m->heads = heads;
    m->hd = hd;
    m->blocks = blocks;
    m->depth = depth;
    m->mlp = mlp;
    m->patch = SAM_PATCH;
    if (grid < 1 || hd != 64 || embed != heads * hd || mlp < 0) {
        hipb_fatal("Unsupported attention head width %d", hd);
        return;
    }
    cap = b->max_alloc < ((size_t)512 << 20) ? b->max_alloc
                                             : ((size_t)512 << 20);
    m->score_cap = (long)(cap / f);
    for (i = 0; i < depth; i++) {
        const struct geom g = block_geom(m, &blocks[i]);
        const int hc = head_chunk(m, &g);

        if (hc < 1) {
            hipb_fatal("HIP device cannot hold the attention scores of one "
                       "head (%lu MiB)",
                       (unsigned long)((size_t)g.nwin * g.N * g.N * f >> 20));
            return;
        }
        if ((long)g.nwin * g.N > rows)
            rows = (long)g.nwin * g.N;
    }
    m->x = hipb_alloc(b, T * embed * f, "tokens");
    m->xn = hipb_alloc(b, T * embed * f, "normalized tokens");
    m->xw = hipb_alloc(b, rows * embed * f, "window partition");
    m->qkv = hipb_alloc(b, rows * 3 * embed * f, "qkv");
    m->attn = hipb_alloc(b, rows * embed * f, "attention output");
    if (mlp > 0) {
        /* MLP hidden, also the patch columns (sam3_model.c:841-843). */
        const long cols = mlp > 3 * SAM_PATCH * SAM_PATCH
                              ? mlp
                              : 3 * SAM_PATCH * SAM_PATCH;

        m->tmp = hipb_alloc(b, rows * embed * f, "projection");
        m->mlpbuf = hipb_alloc(b, T * cols * f, "mlp");
    }
}

void sam_path_free(struct sam_model *m)
{
    if (m->dec)
        sam_dec_free(m);
    if (m->hip)
        hipb_finish(m->hip);
    trunk_graph_drop(m);
    hipb_release(&m->x);
    hipb_release(&m->xn);
    hipb_release(&m->xw);
    hipb_release(&m->qkv);
    hipb_release(&m->scores);
    hipb_release(&m->attn);
    hipb_release(&m->xn16);
    hipb_release(&m->q16);
    hipb_release(&m->k16);
    hipb_release(&m->vt16);
    hipb_release(&m->knorm);
    hipb_release(&m->img);
    hipb_release(&m->tmp);
    hipb_release(&m->mlpbuf);
    hipb_release(&m->mlp16);
    hipb_release(&m->abias);
    hipb_release(&m->apart);
    hipb_release(&m->askrec);
    hipb_release(&m->askcnt);
}
