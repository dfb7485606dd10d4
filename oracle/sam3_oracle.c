/* CPU oracle for the SAM 3 attention path of i.sam3.opencl.
 *
 * TEST INFRASTRUCTURE ONLY: the checker of the HIP library and the CPU
 * baseline of bench.py. Nothing in the product links or loads it.
 *
 * Each function restates the arithmetic (operation order, reduction
 * trees, fused multiply-adds) of one reference kernel or host helper and
 * cites it. The reference's work-item decomposition only matters where
 * it fixes an order of floating-point operations; elsewhere the loops
 * are written for the host and parallelised with OpenMP, which does not
 * change any result.
 *
 * Pinning, by function (tests/test_oracle.py holds the checks):
 *   or_gemm (both kinds)        exact small-integer products, fp64 matmul,
 *                                batch/stride/alias/epilogue cases
 *   or_softmax_rows             fp64 softmax, shift invariance, row sums
 *   or_softmax_ext / or_attend  softmax_rows without terms (bit for bit),
 *                                fp64 masked / biased softmax and SDPA with
 *                                the bias built by broadcasting, causal
 *                                row 0 = V[0], per-row bias shifts, head
 *                                chunking
 *   or_layernorm                fp64 textbook LayerNorm
 *   or_rope_apply               identity table, pair norms, relative
 *                                position property of the rotation
 *   or_window_partition/_add    index algebra: round trip, padding
 *   or_attn_fewkeys/_manykeys   fp64 SDPA, Nk = 1, Q = 0, key permutation
 *   or_vit_attention            fp64 pipeline, window = grid == global
 *   or_patch_im2col             index algebra (numpy reshape of patches)
 *   or_vit_block / _encode_trunk fp64 textbook block and trunk
 * and, for every function, the golden vectors of the reference's own
 * kernels (tests/golden, sam3_kernels.cl run unchanged through the ROCm
 * OpenCL runtime): bit-exact for RoPE and window data movement, rel-L2
 * <= 1e-6 elsewhere (tests/test_golden.py). The last-bit choices (mad as
 * fma, the runtime's exp/erf/rsqrt, dot()'s internal order) stay parity
 * unpinned: those vectors bound them, none fixes them.
 */
#include "sam3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

int or_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Exact-erf GELU and activation epilogue (sam3_kernels.cl:43-55). */
static float act_f(float v, int act)
{
    if (act == OR_ACT_GELU)
        return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    if (act == OR_ACT_RELU)
        return fmaxf(v, 0.0f);
    return v;
}

float or_act(float v, int act)
{
    return act_f(v, act);
}

/* Epilogue shared by every reference GEMM: alpha, bias, activation, then
 * residual (store_one sam3_kernels.cl:306-319; the same sequence in
 * gemm sam3_kernels.cl:141-155 and store_row8 sam3_kernels.cl:158-181). */
static void store_out(float *C, const float *R, const float *bias, long m,
                      int n, int ldc, float alpha, int act, float acc)
{
    float v = alpha * acc;

    if (bias)
        v += bias[n];
    v = act_f(v, act);
    if (R)
        v += R[m * ldc + n];
    C[m * ldc + n] = v;
}

/* gemm / gemm_big / gemm_cpu_n: each output is one accumulator updated by
 * mad(a, b, acc) for k = 0, 1, ..., K - 1 (sam3_kernels.cl:114-125,
 * the k0 loop of gemm_big sam3_kernels.cl:221-297, and
 * sam3_kernels.cl:424-447 for gemm_cpu_n). */
static void gemm_seq_one(int M, int N, int K, const float *A, int lda,
                         const float *B, int ldb, int transb, float *C,
                         int ldc, const float *bias, const float *R,
                         float alpha, int act)
{
    long m;

#pragma omp parallel for schedule(static)
    for (m = 0; m < M; m++) {
        const float *a = A + m * lda;
        float *acc = malloc(sizeof(float) * (size_t)N);
        int n, k;

        for (n = 0; n < N; n++)
            acc[n] = 0.0f;
        if (transb) {
            for (n = 0; n < N; n++) {
                const float *bn = B + (long)n * ldb;
                float s = 0.0f;

                for (k = 0; k < K; k++)
                    s = fmaf(a[k], bn[k], s);
                acc[n] = s;
            }
        }
        else {
            /* Same per-output order, k outermost so the rows of B stream. */
            for (k = 0; k < K; k++) {
                const float *bk = B + (long)k * ldb;
                const float av = a[k];

                for (n = 0; n < N; n++)
                    acc[n] = fmaf(av, bk[n], acc[n]);
            }
        }
        for (n = 0; n < N; n++)
            store_out(C, R, bias, m, n, ldc, alpha, act, acc[n]);
        free(acc);
    }
}

/* gemm_cpu_t (sam3_kernels.cl:334-391). A work-item owns outputs
 * m0 .. m0 + 1, n0 .. n0 + 3 with m0 = 2 * gy, n0 = 4 * gx. When that
 * whole 2 x 4 block is inside C, k advances in steps of 8 with eight
 * independent lanes (lane q sums k = q, q + 8, ...); hsum8 then adds
 * lane q and q + 4 pairwise and sums the four results left to right;
 * the remaining k < K are chained with mad from there. A partial block
 * skips the lanes and chains every k from zero. */
static void gemm_cpu_t_one(int M, int N, int K, const float *A, int lda,
                           const float *B, int ldb, float *C, int ldc,
                           const float *bias, const float *R, float alpha,
                           int act)
{
    const int gy = (M + 1) / 2, gx = (N + 3) / 4;
    long blk;

#pragma omp parallel for schedule(static)
    for (blk = 0; blk < (long)gy * gx; blk++) {
        const int m0 = (int)(blk / gx) * 2, n0 = (int)(blk % gx) * 4;
        float lane[2][4][8];
        int i, j, q, k = 0;

        memset(lane, 0, sizeof(lane));
        if (m0 + 1 < M && n0 + 3 < N) {
            for (k = 0; k + 8 <= K; k += 8)
                for (i = 0; i < 2; i++)
                    for (j = 0; j < 4; j++) {
                        const float *a = A + (long)(m0 + i) * lda + k;
                        const float *b = B + (long)(n0 + j) * ldb + k;

                        for (q = 0; q < 8; q++)
                            lane[i][j][q] = fmaf(a[q], b[q], lane[i][j][q]);
                    }
        }
        for (i = 0; i < 2; i++)
            for (j = 0; j < 4; j++) {
                const int m = m0 + i, n = n0 + j;
                float h[4], v;
                int kk;

                if (m >= M || n >= N)
                    continue;
                for (q = 0; q < 4; q++)
                    h[q] = lane[i][j][q] + lane[i][j][q + 4];
                v = ((h[0] + h[1]) + h[2]) + h[3];
                for (kk = k; kk < K; kk++)
                    v = fmaf(A[(long)m * lda + kk], B[(long)n * ldb + kk], v);
                store_out(C, R, bias, m, n, ldc, alpha, act, v);
            }
    }
}

/* Batch loop of every reference GEMM: b = get_group_id(2) (or
 * get_global_id(2)) split as (b / nb1, b % nb1), each part with its own
 * element stride per operand (sam3_kernels.cl:84-91). */
void or_gemm(int kind, int M, int N, int K, const float *A, long aoff, int lda,
             long sa0, long sa1, const float *B, long boff, int ldb, long sb0,
             long sb1, int transb, float *C, long coff, int ldc, long sc0,
             long sc1, int nb, int nb1, const float *bias, const float *R,
             long roff, float alpha, int act)
{
    int b;

    for (b = 0; b < nb; b++) {
        const long b0 = b / nb1, b1 = b % nb1;
        const float *a = A + aoff + b0 * sa0 + b1 * sa1;
        const float *bb = B + boff + b0 * sb0 + b1 * sb1;
        float *c = C + coff + b0 * sc0 + b1 * sc1;
        const float *r = R ? R + roff + b0 * sc0 + b1 * sc1 : NULL;

        if (kind == OR_GEMM_CPU_T && transb)
            gemm_cpu_t_one(M, N, K, a, lda, bb, ldb, c, ldc, bias, r, alpha,
                           act);
        else
            gemm_seq_one(M, N, K, a, lda, bb, ldb, transb, c, ldc, bias, r,
                         alpha, act);
    }
}

/* Kernel choice of gemm() (sam3_model.c:230-302). Its GPU kernels gemm
 * and gemm_big, and gemm_cpu_n, all chain k sequentially; only gemm_cpu_t
 * (profile=cpu, transb != 0) has a different summation order. */
void or_gemm_dispatch(int cpu, int M, int N, int K, const float *A, long aoff,
                      int lda, long sa0, long sa1, const float *B, long boff,
                      int ldb, long sb0, long sb1, int transb, float *C,
                      long coff, int ldc, long sc0, long sc1, int nb, int nb1,
                      const float *bias, const float *R, long roff,
                      float alpha, int act)
{
    or_gemm(cpu && transb ? OR_GEMM_CPU_T : OR_GEMM_SEQ, M, N, K, A, aoff, lda,
            sa0, sa1, B, boff, ldb, sb0, sb1, transb, C, coff, ldc, sc0, sc1,
            nb, nb1, bias, R, roff, alpha, act);
}

/* Work-group tree reductions wg_sum / wg_max (sam3_kernels.cl:454-484):
 * n partial values (n a power of two) are folded as v[i] op= v[i + s]
 * for s = n / 2, n / 4, ..., 1; the result is v[0]. */
static float tree_sum(float *v, int n)
{
    int s, i;

    for (s = n / 2; s > 0; s >>= 1)
        for (i = 0; i < s; i++)
            v[i] += v[i + s];
    return v[0];
}

static float tree_max(float *v, int n)
{
    int s, i;

    for (s = n / 2; s > 0; s >>= 1)
        for (i = 0; i < s; i++)
            v[i] = fmaxf(v[i], v[i + s]);
    return v[0];
}

/* softmax_rows (sam3_kernels.cl:637-656) with the host's work-group size
 * ls = 256 for L >= 256, else 64 (sam3_model.c:336). Item t owns the
 * entries j = t, t + ls, ...: a strided max, tree max, then
 * v = exp(s - m) stored and summed per item in order, tree sum, and a
 * final multiply by 1 / sum. */
void or_softmax_rows(float *S, long rows, int L)
{
    const int ls = L >= 256 ? 256 : 64;
    long r;

#pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        float *s = S + r * L;
        float part[256], m, inv;
        int t, j;

        for (t = 0; t < ls; t++) {
            float v = -INFINITY;

            for (j = t; j < L; j += ls)
                v = fmaxf(v, s[j]);
            part[t] = v;
        }
        m = tree_max(part, ls);
        for (t = 0; t < ls; t++) {
            float sum = 0.0f;

            for (j = t; j < L; j += ls) {
                const float v = expf(s[j] - m);

                s[j] = v;
                sum += v;
            }
            part[t] = sum;
        }
        inv = 1.0f / tree_sum(part, ls);
        for (j = 0; j < L; j++)
            s[j] *= inv;
    }
}

/* softmax_ext (sam3_kernels.cl:885-921): softmax_rows' reduction
 * order with the causal mask or box bias added in the first pass, which
 * stores the biased scores back (so the exp pass reads them). */
void or_softmax_ext(float *S, long rows, int L, int Nq, int h0, int causal,
                    const float *dy, const float *dx, int W, int nh)
{
    const int ls = L >= 256 ? 256 : 64, H = W > 0 ? L / W : 0;
    long r;

#pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        const int i = (int)(r % Nq), h = h0 + (int)(r / Nq);
        float *s = S + r * L;
        float part[256], m, inv;
        int t, j;

        for (t = 0; t < ls; t++) {
            float mx = -INFINITY;

            for (j = t; j < L; j += ls) {
                float v = s[j];

                if (causal && j > i)
                    v = -INFINITY;
                else if (dy)
                    v += dy[((long)i * H + j / W) * nh + h] +
                         dx[((long)i * W + j % W) * nh + h];
                s[j] = v;
                mx = fmaxf(mx, v);
            }
            part[t] = mx;
        }
        m = tree_max(part, ls);
        for (t = 0; t < ls; t++) {
            float sum = 0.0f;

            for (j = t; j < L; j += ls) {
                const float v = expf(s[j] - m);

                s[j] = v;
                sum += v;
            }
            part[t] = sum;
        }
        inv = 1.0f / tree_sum(part, ls);
        for (j = 0; j < L; j++)
            s[j] *= inv;
    }
}

/* attend() (sam3_text.c:305-343): the head chunking, the two GEMMs of
 * each chunk (alpha 1 / sqrtf(hd), heads as the batch with stride hd) and
 * softmax_ext between them. */
int or_attend(int cpu, int Nq, int Nk, int heads, int hd, const float *Q,
              int ldq, const float *K, int ldk, const float *V, int ldv,
              float *O, int ldo, int causal, const float *dy, const float *dx,
              int W, long score_cap)
{
    const long plane = (long)Nq * Nk;
    const long hcl = score_cap / plane;
    const int hc = hcl > heads ? heads : (int)hcl;
    float *scores;
    int h0;

    if (hc < 1)
        return -1;
    scores = malloc((size_t)hc * plane * sizeof(float));
    if (!scores)
        return -1;
    for (h0 = 0; h0 < heads; h0 += hc) {
        const int hcc = heads - h0 < hc ? heads - h0 : hc;

        or_gemm_dispatch(cpu, Nq, Nk, hd, Q, (long)h0 * hd, ldq, 0, hd, K,
                         (long)h0 * hd, ldk, 0, hd, 1, scores, 0, Nk, 0, plane,
                         hcc, hcc, NULL, NULL, 0, 1.0f / sqrtf((float)hd),
                         OR_ACT_NONE);
        or_softmax_ext(scores, (long)hcc * Nq, Nk, Nq, h0, causal, dy, dx, W,
                       heads);
        or_gemm_dispatch(cpu, Nq, hd, Nk, scores, 0, Nk, 0, plane, V,
                         (long)h0 * hd, ldv, 0, hd, 0, O, (long)h0 * hd, ldo, 0,
                         hd, hcc, hcc, NULL, NULL, 0, 1.0f, OR_ACT_NONE);
    }
    free(scores);
    return hc;
}

/* layernorm (sam3_kernels.cl:489-514), ls = 256 for C >= 1024 else 64
 * (sam3_model.c:320). Per-item strided sums, tree sum, mean = sum / C;
 * the same for the squared deviations (s += d * d contracted to a fused
 * multiply-add); rs = rsqrt(var + eps);
 * y = act(((x - mean) * rs) * g + b) with the last multiply-add fused. */
void or_layernorm(const float *X, float *Y, long rows, int C, const float *g,
                  const float *b, float eps, int act)
{
    const int ls = C >= 1024 ? 256 : 64;
    long r;

#pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        const float *x = X + r * C;
        float *y = Y + r * C;
        float part[256], mean, var, rs;
        int t, c;

        for (t = 0; t < ls; t++) {
            float s = 0.0f;

            for (c = t; c < C; c += ls)
                s += x[c];
            part[t] = s;
        }
        mean = tree_sum(part, ls) / C;
        for (t = 0; t < ls; t++) {
            float s = 0.0f;

            for (c = t; c < C; c += ls) {
                const float d = x[c] - mean;

                s = fmaf(d, d, s);
            }
            part[t] = s;
        }
        var = tree_sum(part, ls) / C;
        rs = 1.0f / sqrtf(var + eps);
        for (c = 0; c < C; c++)
            y[c] = act_f(fmaf((x[c] - mean) * rs, g[c], b[c]), act);
    }
}

/* rope_apply (sam3_kernels.cl:679-698): for row r, the q (qk = 0) and
 * k (qk = 1) thirds, head h and pair j < hd / 2, (a, b) = x[2j, 2j + 1]
 * becomes (a cos - b sin, a sin + b cos) with (cos, sin) =
 * cs[(r % npos) * hd / 2 + j]; each expression contracted on its first
 * product. */
void or_rope_apply(float *qkv, long rows, int E, int hd, int npos,
                   const float *cs)
{
    const int nf = hd / 2;
    long r;

#pragma omp parallel for schedule(static)
    for (r = 0; r < rows; r++) {
        const float *rot = cs + (r % npos) * 2L * nf;
        int qk, p;

        for (qk = 0; qk < 2; qk++)
            for (p = 0; p < E / 2; p++) {
                const int h = p / nf, j = p % nf;
                float *x = qkv + r * 3L * E + (long)qk * E + (long)h * hd + 2 * j;
                const float a = x[0], bb = x[1];
                const float c = rot[2 * j], s = rot[2 * j + 1];

                x[0] = fmaf(a, c, -(bb * s));
                x[1] = fmaf(a, s, bb * c);
            }
    }
}

/* window_partition (sam3_kernels.cl:712-724): output row w * ws^2 + i,
 * window w = (wy, wx) row-major with nwx windows per side, in-window
 * position i = (iy, ix); zero outside the H x W grid. */
void or_window_partition(const float *X, float *out, int H, int W, int C,
                         int ws, int nwx)
{
    const long nrows = (long)nwx * nwx * ws * ws;
    long r;

#pragma omp parallel for schedule(static)
    for (r = 0; r < nrows; r++) {
        const int w = (int)(r / (ws * ws)), i = (int)(r % (ws * ws));
        const int y = (w / nwx) * ws + i / ws, x = (w % nwx) * ws + i % ws;

        if (y < H && x < W)
            memcpy(out + r * C, X + ((long)y * W + x) * C, sizeof(float) * C);
        else
            memset(out + r * C, 0, sizeof(float) * C);
    }
}

/* window_unpartition_add (sam3_kernels.cl:728-741): X[t] += Wd[row of t]. */
void or_window_unpartition_add(float *X, const float *Wd, int H, int W, int C,
                               int ws, int nwx)
{
    long t;

#pragma omp parallel for schedule(static)
    for (t = 0; t < (long)H * W; t++) {
        const int y = (int)(t / W), x = (int)(t % W);
        const long w = (long)(y / ws) * nwx + x / ws;
        const long i = (long)(y % ws) * ws + x % ws;
        const float *src = Wd + (w * ws * ws + i) * C;
        float *dst = X + t * C;
        int c;

        for (c = 0; c < C; c++)
            dst[c] += src[c];
    }
}

void or_add_bcast(float *out, const float *a, const float *b, long n,
                  long bmod)
{
    long i;

#pragma omp parallel for schedule(static)
    for (i = 0; i < n; i++)
        out[i] = a[i] + b[i % bmod];
}

/* OpenCL dot() of two float4, taken as the chain of fused multiply-adds
 * fma(a3, b3, fma(a2, b2, fma(a1, b1, a0 * b0))) (parity unpinned), and
 * dot16 = ((d0 + d1) + d2) + d3 over the four float4 quarters
 * (sam3_kernels.cl:516-520). */
static float dot4(const float *a, const float *b)
{
    return fmaf(a[3], b[3], fmaf(a[2], b[2], fmaf(a[1], b[1], a[0] * b[0])));
}

static float dot16(const float *a, const float *b)
{
    return ((dot4(a, b) + dot4(a + 4, b + 4)) + dot4(a + 8, b + 8)) +
           dot4(a + 12, b + 12);
}

float or_dot16(const float *a, const float *b)
{
    return dot16(a, b);
}

#define DEC_HEADS 8

/* attn_fewkeys (sam3_kernels.cl:527-569): one work-item per (prompt p,
 * head h, query i); online softmax over the Nk keys in order:
 * s = scale * q . k (c = 32 adds the second dot16 before scaling),
 * mn = max(m, s), corr = exp(m - mn), e = exp(s - mn),
 * sum = fma(sum, corr, e), o = fma(o, corr, e * v); O = o / sum. */
void or_attn_fewkeys(const float *Q, long sq, const float *K, long sk,
                     const float *V, long sv, float *O, int P, int Nq, int Nk,
                     int dint, int c, float scale)
{
    const long total = (long)P * DEC_HEADS * Nq;
    long gid;

#pragma omp parallel for schedule(static)
    for (gid = 0; gid < total; gid++) {
        const int i = (int)(gid % Nq);
        const long ph = gid / Nq;
        const int h = (int)(ph % DEC_HEADS);
        const long p = ph / DEC_HEADS;
        const float *q = Q + p * sq + (long)i * dint + (long)h * c;
        const float *kb = K + p * sk + (long)h * c;
        const float *vb = V + p * sv + (long)h * c;
        float o[32] = {0}, m = -INFINITY, sum = 0.0f;
        float *out = O + (p * Nq + i) * dint + (long)h * c;
        int j, d;

        for (j = 0; j < Nk; j++) {
            const float *kr = kb + (long)j * dint, *vr = vb + (long)j * dint;
            float s = dot16(q, kr), mn, corr, e;

            if (c > 16)
                s += dot16(q + 16, kr + 16);
            s *= scale;
            mn = fmaxf(m, s);
            corr = expf(m - mn);
            e = expf(s - mn);
            sum = fmaf(sum, corr, e);
            for (d = 0; d < c; d++)
                o[d] = fmaf(o[d], corr, e * vr[d]);
            m = mn;
        }
        for (d = 0; d < c; d++)
            out[d] = o[d] / sum;
    }
}

/* attn_manykeys (sam3_kernels.cl:577-633): one 256-item work-group per
 * (p, h, i) row, c = 16. Item t runs the online softmax of attn_fewkeys
 * over keys j = t, t + 256, ...; then mall = tree max of the items' m,
 * f = exp(m - mall) (0 for an item without keys), o *= f,
 * inv = 1 / tree sum of sum * f, each output channel tree-summed over
 * the items and multiplied by inv. */
void or_attn_manykeys(const float *Q, long sq, const float *K, long sk,
                      const float *V, long sv, float *O, int P, int Nq,
                      int Nk, int dint, int c, float scale)
{
    const long total = (long)P * DEC_HEADS * Nq;
    long row;

    (void)c;
#pragma omp parallel for schedule(static)
    for (row = 0; row < total; row++) {
        const int i = (int)(row % Nq);
        const long ph = row / Nq;
        const int h = (int)(ph % DEC_HEADS);
        const long p = ph / DEC_HEADS;
        const float *kb = K + p * sk + (long)h * 16;
        const float *vb = V + p * sv + (long)h * 16;
        const float *q = Q + p * sq + (long)i * dint + (long)h * 16;
        float *out = O + (p * Nq + i) * dint + (long)h * 16;
        float *part = malloc(sizeof(float) * 17 * 256);
        float mt[256], st[256], mall, inv;
        int t, j, d;

        for (t = 0; t < 256; t++) {
            float o[16] = {0}, m = -INFINITY, sum = 0.0f;

            for (j = t; j < Nk; j += 256) {
                const float *kr = kb + (long)j * dint,
                            *vr = vb + (long)j * dint;
                const float s = dot16(q, kr) * scale;
                const float mn = fmaxf(m, s), corr = expf(m - mn),
                            e = expf(s - mn);

                sum = fmaf(sum, corr, e);
                for (d = 0; d < 16; d++)
                    o[d] = fmaf(o[d], corr, e * vr[d]);
                m = mn;
            }
            mt[t] = m;
            st[t] = sum;
            for (d = 0; d < 16; d++)
                part[d * 256 + t] = o[d];
        }
        memcpy(part + 16 * 256, mt, sizeof(mt));
        mall = tree_max(part + 16 * 256, 256);
        for (t = 0; t < 256; t++) {
            const float f = mt[t] == -INFINITY ? 0.0f : expf(mt[t] - mall);

            for (d = 0; d < 16; d++)
                part[d * 256 + t] *= f;
            st[t] = st[t] * f;
        }
        inv = 1.0f / tree_sum(st, 256);
        for (d = 0; d < 16; d++)
            out[d] = tree_sum(part + d * 256, 256) * inv;
        free(part);
    }
}

/* mha() (sam3_model.c:413-451): c = dint / 8, scale = 1 / sqrtf(c);
 * Nk > 64 takes attn_manykeys, which needs c == 16 (else fatal), the
 * rest attn_fewkeys. */
int or_mha(int P, int Nq, int Nk, int dint, const float *qp, long sq,
           const float *kp, long sk, const float *vp, long sv, float *o)
{
    const int c = dint / DEC_HEADS;
    const float scale = 1.0f / sqrtf((float)c);

    if (Nk > 64) {
        if (c != 16)
            return -1;
        or_attn_manykeys(qp, sq, kp, sk, vp, sv, o, P, Nq, Nk, dint, c, scale);
    }
    else
        or_attn_fewkeys(qp, sq, kp, sk, vp, sv, o, P, Nq, Nk, dint, c, scale);
    return 0;
}

/* Attention region of vit_block (sam3_model.c:981-1013) with its
 * geometry block_geom / head_chunk (sam3_model.c:777-798). */
int or_vit_attention(int cpu, const float *x, int grid, int E, int heads,
                     int hd, int ws, const float *n1w, const float *n1b,
                     const float *qkvw, const float *qkvb, const float *rope,
                     long score_cap, float *attn, float *qkv_out)
{
    const int s = ws ? ws : grid;
    const int nwx = (grid + s - 1) / s, nwin = nwx * nwx, N = s * s;
    const long T = (long)grid * grid, rows = (long)nwin * N;
    const float scale = 1.0f / sqrtf((float)hd);
    const long plane = (long)N * N, tstride = (long)N * 3 * E;
    long hc = score_cap / ((long)nwin * N * N);
    float *xn, *xw, *qkv, *scores;
    int h0;

    if (hc < 1)
        return -1;
    if (hc > heads)
        hc = heads;
    xn = malloc(sizeof(float) * T * E);
    qkv = qkv_out ? qkv_out : malloc(sizeof(float) * rows * 3 * E);
    scores = malloc(sizeof(float) * hc * nwin * plane);
    or_layernorm(x, xn, T, E, n1w, n1b, 1e-5f, OR_ACT_NONE);
    xw = xn;
    if (ws) {
        xw = malloc(sizeof(float) * rows * E);
        or_window_partition(xn, xw, grid, grid, E, s, nwx);
    }
    /* linear(): X W^T + b as a transb GEMM (sam3_model.c:305-310). */
    or_gemm_dispatch(cpu, (int)rows, 3 * E, E, xw, 0, E, 0, 0, qkvw, 0, E, 0,
                     0, 1, qkv, 0, 3 * E, 0, 0, 1, 1, qkvb, NULL, 0, 1.0f,
                     OR_ACT_NONE);
    or_rope_apply(qkv, rows, E, hd, N, rope);
    for (h0 = 0; h0 < heads; h0 += (int)hc) {
        const int hcc = heads - h0 < hc ? heads - h0 : (int)hc;

        or_gemm_dispatch(cpu, N, N, hd, qkv, (long)h0 * hd, 3 * E, tstride,
                         hd, qkv, E + (long)h0 * hd, 3 * E, tstride, hd, 1,
                         scores, 0, N, hcc * plane, plane, nwin * hcc, hcc,
                         NULL, NULL, 0, scale, OR_ACT_NONE);
        or_softmax_rows(scores, (long)nwin * hcc * N, N);
        or_gemm_dispatch(cpu, N, hd, N, scores, 0, N, hcc * plane, plane, qkv,
                         2L * E + (long)h0 * hd, 3 * E, tstride, hd, 0, attn,
                         (long)h0 * hd, E, (long)N * E, hd, nwin * hcc, hcc,
                         NULL, NULL, 0, 1.0f, OR_ACT_NONE);
    }
    if (xw != xn)
        free(xw);
    free(xn);
    free(scores);
    if (!qkv_out)
        free(qkv);
    return (int)hc;
}

void or_patch_im2col(const float *img, float *out, int side, int grid, int ps)
{
    const int K = 3 * ps * ps;
    const long T = (long)grid * grid;
    long t;

#pragma omp parallel for schedule(static)
    for (t = 0; t < T; t++) {
        const int ty = (int)(t / grid), tx = (int)(t % grid);
        int col;

        for (col = 0; col < K; col++) {
            const int c = col / (ps * ps), ky = (col % (ps * ps)) / ps,
                      kx = col % ps;

            out[t * K + col] =
                img[((long)c * side + ty * ps + ky) * side + tx * ps + kx];
        }
    }
}

int or_vit_block(int cpu, float *x, int grid, int E, int heads, int hd,
                 int mlp, const struct or_block_w *b, const float *rope,
                 long score_cap)
{
    const int s = b->window ? b->window : grid;
    const int nwx = (grid + s - 1) / s, N = s * s;
    const long T = (long)grid * grid, rows = (long)nwx * nwx * N;
    float *attn = malloc(sizeof(float) * rows * E);
    float *xn = malloc(sizeof(float) * T * E);
    float *h = malloc(sizeof(float) * T * mlp);
    int hc = or_vit_attention(cpu, x, grid, E, heads, hd, b->window, b->n1w,
                              b->n1b, b->qkvw, b->qkvb, rope, score_cap, attn,
                              NULL);

    if (hc > 0) {
        /* Projection (sam3_model.c:1015-1022). */
        if (b->window) {
            float *tmp = malloc(sizeof(float) * rows * E);

            or_gemm_dispatch(cpu, (int)rows, E, E, attn, 0, E, 0, 0, b->projw,
                             0, E, 0, 0, 1, tmp, 0, E, 0, 0, 1, 1, b->projb,
                             NULL, 0, 1.0f, OR_ACT_NONE);
            or_window_unpartition_add(x, tmp, grid, grid, E, s, nwx);
            free(tmp);
        }
        else
            or_gemm_dispatch(cpu, (int)T, E, E, attn, 0, E, 0, 0, b->projw, 0,
                             E, 0, 0, 1, x, 0, E, 0, 0, 1, 1, b->projb, x, 0,
                             1.0f, OR_ACT_NONE);
        /* norm2 and the MLP (sam3_model.c:1024-1027). */
        or_layernorm(x, xn, T, E, b->n2w, b->n2b, 1e-5f, OR_ACT_NONE);
        or_gemm_dispatch(cpu, (int)T, mlp, E, xn, 0, E, 0, 0, b->l1w, 0, E, 0,
                         0, 1, h, 0, mlp, 0, 0, 1, 1, b->l1b, NULL, 0, 1.0f,
                         OR_ACT_GELU);
        or_gemm_dispatch(cpu, (int)T, E, mlp, h, 0, mlp, 0, 0, b->l2w, 0, mlp,
                         0, 0, 1, x, 0, E, 0, 0, 1, 1, b->l2b, x, 0, 1.0f,
                         OR_ACT_NONE);
    }
    free(attn);
    free(xn);
    free(h);
    return hc;
}

int or_encode_trunk(int cpu, const float *img, int grid, int ps, int E,
                    int heads, int hd, int mlp, const float *pe_w,
                    const float *pos, const float *lnpw, const float *lnpb,
                    const struct or_block_w *blocks, int depth,
                    const float *rope_win, const float *rope_glob,
                    long score_cap, float *x)
{
    const long T = (long)grid * grid;
    const int K = 3 * ps * ps;
    float *col = malloc(sizeof(float) * T * K);
    int i, ok = 0;

    or_patch_im2col(img, col, grid * ps, grid, ps);
    or_gemm_dispatch(cpu, (int)T, E, K, col, 0, K, 0, 0, pe_w, 0, K, 0, 0, 1,
                     x, 0, E, 0, 0, 1, 1, NULL, NULL, 0, 1.0f, OR_ACT_NONE);
    or_add_bcast(x, x, pos, T * E, T * E);
    or_layernorm(x, x, T, E, lnpw, lnpb, 1e-5f, OR_ACT_NONE);
    free(col);
    for (i = 0; i < depth && ok == 0; i++)
        if (or_vit_block(cpu, x, grid, E, heads, hd, mlp, &blocks[i],
                         blocks[i].window ? rope_win : rope_glob,
                         score_cap) < 0)
            ok = -1;
    return ok;
}

/* Textbook softmax attention in double precision. */
void or_sdpa_f64(int Nq, int Nk, int d, const double *Q, int ldq,
                 const double *K, int ldk, const double *V, int ldv, double *O,
                 int ldo, double scale)
{
    int i;

#pragma omp parallel for schedule(static)
    for (i = 0; i < Nq; i++) {
        double *s = malloc(sizeof(double) * (size_t)Nk), m = -INFINITY,
               sum = 0.0;
        int j, k;

        for (j = 0; j < Nk; j++) {
            double acc = 0.0;

            for (k = 0; k < d; k++)
                acc += Q[(long)i * ldq + k] * K[(long)j * ldk + k];
            s[j] = scale * acc;
            if (s[j] > m)
                m = s[j];
        }
        for (j = 0; j < Nk; j++) {
            s[j] = exp(s[j] - m);
            sum += s[j];
        }
        for (k = 0; k < d; k++) {
            double acc = 0.0;

            for (j = 0; j < Nk; j++)
                acc += s[j] * V[(long)j * ldv + k];
            O[(long)i * ldo + k] = acc / sum;
        }
        free(s);
    }
}
