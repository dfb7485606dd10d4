/* SPDX-License-Identifier: Unlicense
 *
 * Mask-decoder attention on gfx950 (8 heads, fp32), the kernels behind
 * mha() (sam3_model.c:413-451). Both directions are HBM-bound (a few
 * FLOP per byte), so they are organised around reading each byte once
 * with full-row coalescing rather than around arithmetic.
 *
 * Few keys (attn_fewkeys, sam3_kernels.cl:527-569: image->token and the
 * token self-attention): one thread per (prompt, query, head); the 8
 * heads of a query are 8 adjacent threads, so a query row (dint floats)
 * is read and written as one contiguous segment. Online softmax over the
 * keys in order, as the reference.
 *
 * Many keys (attn_manykeys, sam3_kernels.cl:577-633: token->image over
 * the 5184 image tokens): the reference runs one 256-item workgroup per
 * (prompt, head, query) and so reads a prompt's image keys once per
 * query and head. Here a workgroup owns one key range of one prompt for
 * all heads and up to 8 queries (split-K): a wave covers 8 heads x 8
 * queries, each image key row (8 heads x 16 channels) is read once per
 * workgroup, and the partial softmax states (m, sum, o) are merged across
 * the workgroup in LDS, written per split, and merged across splits by a
 * second kernel.
 */
#include "k_common.h"

#define DEC_HEADS 8
#define QCH 8  /* queries per many-keys workgroup */
#define KLN 4  /* key lanes per (head, query) in a many-keys workgroup */

__global__ __launch_bounds__(256) void k_mha_fewkeys(
    const float *__restrict__ Q, long sq, const float *__restrict__ K,
    long sk, const float *__restrict__ V, long sv, float *__restrict__ O,
    int Nq, int Nk, int dint, int c, float scale)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;
    const long p = blockIdx.y;
    const int h = (int)(gid & 7);
    const long i = gid >> 3;
    float q[32], o[32], m = -INFINITY, sum = 0.0f;

    if (i >= Nq)
        return;
    const float *qr = Q + p * sq + i * dint + h * c;
    const float *kb = K + p * sk + h * c;
    const float *vb = V + p * sv + h * c;

    for (int e = 0; e < 32; e++) {
        q[e] = e < c ? qr[e] : 0.0f;
        o[e] = 0.0f;
    }
    for (int j = 0; j < Nk; j++) {
        const float *kr = kb + (long)j * dint, *vr = vb + (long)j * dint;
        float s = 0.0f, mn, corr, e;

        for (int x = 0; x < 32; x++)
            if (x < c)
                s = fmaf(q[x], kr[x], s);
        s *= scale;
        mn = fmaxf(m, s);
        corr = expf(m - mn);
        e = expf(s - mn);
        sum = fmaf(sum, corr, e);
        for (int x = 0; x < 32; x++)
            if (x < c)
                o[x] = fmaf(o[x], corr, e * vr[x]);
        m = mn;
    }
    {
        float *out = O + (p * Nq + i) * dint + h * c;
        const float inv = 1.0f / sum;

        for (int x = 0; x < 32; x++)
            if (x < c)
                out[x] = o[x] * inv;
    }
}

extern "C" int launch_mha_fewkeys(const float *Q, long sq, const float *K,
                                  long sk, const float *V, long sv, float *O,
                                  int P, int Nq, int Nk, int dint, float scale,
                                  void *stream)
{
    const long threads = (long)Nq * DEC_HEADS;

    if (P > 65535)
        return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_mha_fewkeys, dim3((threads + 255) / 256, P),
                       dim3(256), 0, (hipStream_t)stream, Q, sq, K, sk, V, sv,
                       O, Nq, Nk, dint, dint / DEC_HEADS, scale);
    return hipGetLastError();
}

/* Splits of the key range: enough workgroups to fill the device (about
 * 1024), at least 64 keys each. */
static int many_splits(int P, int Nk)
{
    int by_keys = (Nk + 63) / 64;
    int by_fill = (1024 + P - 1) / P;
    int n = by_keys < by_fill ? by_keys : by_fill;

    return n < 1 ? 1 : n;
}

/* Partial state of one (prompt, split, query, head): m, sum, o[16]. */
#define PART 18

__global__ __launch_bounds__(256) void k_mha_many_part(
    const float *__restrict__ Q, long sq, const float *__restrict__ K,
    long sk, const float *__restrict__ V, long sv, float *__restrict__ part,
    int Nq, int Nk, int dint, float scale, int nsplit)
{
    __shared__ float red[KLN][QCH][DEC_HEADS][PART];
    const int t = threadIdx.x, h = t & 7, qq = (t >> 3) & 7, kl = t >> 6;
    const int split = blockIdx.x;
    const long p = blockIdx.y;
    const int qi = blockIdx.z * QCH + qq;
    const int chunk = (Nk + nsplit - 1) / nsplit;
    const int k0 = split * chunk, k1 = min(Nk, k0 + chunk);
    float q[16], o[16], m = -INFINITY, sum = 0.0f;

    for (int e = 0; e < 16; e++) {
        q[e] = 0.0f;
        o[e] = 0.0f;
    }
    if (qi < Nq) {
        const float *qr = Q + p * sq + (long)qi * dint + h * 16;

        for (int e = 0; e < 16; e++)
            q[e] = qr[e];
    }
    {
        const float *kb = K + p * sk + h * 16;
        const float *vb = V + p * sv + h * 16;

        for (int j = k0 + kl; j < k1; j += KLN) {
            const f32x4 *kr = (const f32x4 *)(kb + (long)j * dint);
            const f32x4 *vr = (const f32x4 *)(vb + (long)j * dint);
            f32x4 kv[4], vv[4];
            float s = 0.0f, e;

            for (int x = 0; x < 4; x++)
                kv[x] = kr[x];
            for (int x = 0; x < 4; x++)
                vv[x] = vr[x];
            for (int x = 0; x < 16; x++)
                s = fmaf(q[x], kv[x >> 2][x & 3], s);
            s *= scale;
            if (s > m) {
                const float corr = expf(m - s);

                sum *= corr;
                for (int x = 0; x < 16; x++)
                    o[x] *= corr;
                m = s;
            }
            e = expf(s - m);
            sum += e;
            for (int x = 0; x < 16; x++)
                o[x] = fmaf(e, vv[x >> 2][x & 3], o[x]);
        }
    }
    red[kl][qq][h][0] = m;
    red[kl][qq][h][1] = sum;
    for (int x = 0; x < 16; x++)
        red[kl][qq][h][2 + x] = o[x];
    __syncthreads();
    if (t < QCH * DEC_HEADS * 2) {
        /* Two threads per (query, head): channels 0..8 and 9..17. */
        const int hh = (t >> 1) & 7, q2 = t >> 4, half = t & 1;
        const int qo = blockIdx.z * QCH + q2;
        float M = -INFINITY, f[KLN];

        if (qo < Nq) {
            for (int k = 0; k < KLN; k++)
                M = fmaxf(M, red[k][q2][hh][0]);
            for (int k = 0; k < KLN; k++)
                f[k] = red[k][q2][hh][0] == -INFINITY
                           ? 0.0f
                           : expf(red[k][q2][hh][0] - M);
            float *dst = part + (((p * nsplit + split) * Nq + qo) * DEC_HEADS + hh) * PART;

            for (int x = half * 9; x < half * 9 + 9; x++) {
                float v = 0.0f;

                if (x == 0)
                    v = M;
                else
                    for (int k = 0; k < KLN; k++)
                        v = fmaf(red[k][q2][hh][x], f[k], v);
                dst[x] = v;
            }
        }
    }
}

__global__ __launch_bounds__(256) void k_mha_many_merge(
    const float *__restrict__ part, float *__restrict__ O, long rows, int Nq,
    int dint, int nsplit)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= rows)
        return;
    const int h = (int)(gid & 7);
    const long pq = gid >> 3, p = pq / Nq, qi = pq % Nq;
    float M = -INFINITY, sum = 0.0f, o[16];

    for (int x = 0; x < 16; x++)
        o[x] = 0.0f;
    for (int s = 0; s < nsplit; s++)
        M = fmaxf(M, part[(((p * nsplit + s) * Nq + qi) * DEC_HEADS + h) * PART]);
    for (int s = 0; s < nsplit; s++) {
        const float *src = part + (((p * nsplit + s) * Nq + qi) * DEC_HEADS + h) * PART;
        const float f = src[0] == -INFINITY ? 0.0f : expf(src[0] - M);

        sum = fmaf(src[1], f, sum);
        for (int x = 0; x < 16; x++)
            o[x] = fmaf(src[2 + x], f, o[x]);
    }
    {
        float *out = O + (p * Nq + qi) * dint + h * 16;
        const float inv = 1.0f / sum;

        for (int x = 0; x < 16; x++)
            out[x] = o[x] * inv;
    }
}

extern "C" size_t mha_manykeys_scratch(int P, int Nq, int Nk)
{
    return (size_t)P * many_splits(P, Nk) * Nq * DEC_HEADS * PART *
           sizeof(float);
}

extern "C" int launch_mha_manykeys(const float *Q, long sq, const float *K,
                                   long sk, const float *V, long sv, float *O,
                                   int P, int Nq, int Nk, int dint,
                                   float scale, void *scratch, void *stream)
{
    const int nsplit = many_splits(P, Nk);
    const long rows = (long)P * Nq * DEC_HEADS;
    hipStream_t s = (hipStream_t)stream;
    int err;

    if (P > 65535 || (Nq + QCH - 1) / QCH > 65535)
        return hipErrorInvalidConfiguration;
    /* 16-byte row loads of K and V need their rows and offsets aligned. */
    if (dint % 4 || sk % 4 || sv % 4)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mha_many_part, dim3(nsplit, P, (Nq + QCH - 1) / QCH),
                       dim3(256), 0, s, Q, sq, K, sk, V, sv, (float *)scratch,
                       Nq, Nk, dint, scale, nsplit);
    err = hipGetLastError();
    if (err != hipSuccess)
        return err;
    hipLaunchKernelGGL(k_mha_many_merge, dim3((rows + 255) / 256), dim3(256),
                       0, s, (const float *)scratch, O, rows, Nq, dint,
                       nsplit);
    return hipGetLastError();
}
