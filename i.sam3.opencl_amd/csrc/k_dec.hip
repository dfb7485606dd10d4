/* SPDX-License-Identifier: Unlicense
 *
 * Mask-decoder attention on gfx950 (8 heads, fp32), the kernels behind
 * mha() (sam3_model.c:413-451). Both directions are HBM-bound (a few
 * FLOP per byte), so they are organised around reading each byte once
 * with whole-wave coalescing rather than around arithmetic.
 *
 * Head width 16 (dint = 128, every call of the two-way transformer's
 * cross-attention, sam3_model.c:1212-1229 and 1290-1306): a lane owns
 * four channels of one (row, head). A wave then covers two 128-float
 * rows with one 1 KiB load per row pair (lane l reads floats 4l..4l+3),
 * and the 16-channel dot product of a (row, head) closes over its four
 * lanes with two DPP quad-permute adds, which leave the same sum in all
 * four lanes, so the softmax state stays identical across the quad.
 *
 * Few keys (attn_fewkeys, sam3_kernels.cl:527-569: image->token): the
 * prompt's <= 8 key and value rows live in registers for the whole
 * workgroup; each query row is read once, its scores, exact softmax and
 * weighted sum are formed in registers and the output row is written
 * once.
 *
 * Many keys (attn_manykeys, sam3_kernels.cl:577-633: token->image over
 * the image tokens): the reference runs one workgroup per (prompt, head,
 * query) and so reads a prompt's image keys once per query and head.
 * Here a workgroup owns one key range of one prompt for all heads and up
 * to 8 queries (split-K): each image key / value row is read once per
 * workgroup, each lane runs an online softmax over its keys for all the
 * queries, and the partial states (m, l, o) are merged across the wave,
 * across the workgroup in LDS and, when the key range is split, across
 * splits by a second kernel.
 *
 * Scores are formed in the exp2 domain: the key rows (few keys) or the
 * query rows (many keys) are multiplied by scale * log2(e) once, so the
 * softmax uses v_exp_f32 directly.
 *
 * Other shapes (head width 32, the token self-attention, or strides not
 * a multiple of 4 floats) take the generic one-thread-per-(query, head)
 * few-keys kernel.
 */
#include "k_common.h"

#define DEC_HEADS 8
#define DEC_W 128      /* dint of the head-width-16 kernels */
#define UNR 4          /* row pairs per wave per step (few keys) */
#define STEP_ROWS (4 * 2 * UNR) /* rows per workgroup step: 32 */
#define M_INIT -1.0e30f /* running max before any key: finite, so that
                           exp2(m - m_new) never sees inf - inf */

/* DPP quad permutes: [1,0,3,2] and [2,3,0,1]. */
#define DPP_QXOR1 0xB1
#define DPP_QXOR2 0x4E

template <int CTRL> __device__ __forceinline__ float dppf(float x)
{
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                           0xF, 0xF, false));
}

/* Sum over the four lanes of a quad, the same bits in all four: each step
 * adds a lane's value to its partner's in both lanes (a + b == b + a). */
__device__ __forceinline__ float quad_sum(float x)
{
    x += dppf<DPP_QXOR1>(x);
    return x + dppf<DPP_QXOR2>(x);
}

__device__ __forceinline__ float dot4(f32x4 a, f32x4 b)
{
    return fmaf(a.w, b.w, fmaf(a.z, b.z, fmaf(a.y, b.y, a.x * b.x)));
}

__device__ __forceinline__ f32x4 ld4(const float *p)
{
    return *(const f32x4 *)p;
}

/* ------------------------------------------------------------------ */
/* Few keys, head width 16                                             */
/* ------------------------------------------------------------------ */

template <int NK>
__global__ __launch_bounds__(256) void k_mha_few16(
    const float *__restrict__ Q, long sq, const float *__restrict__ K,
    long sk, const float *__restrict__ V, long sv, float *__restrict__ O,
    int Nq, float kscale, int steps)
{
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = (lane & 31) * 4, r = lane >> 5;
    const long p = blockIdx.y;
    const float *qb = Q + p * sq + col;
    float *ob = O + p * (long)Nq * DEC_W + col;
    f32x4 kf[NK], vf[NK];

    for (int j = 0; j < NK; j++) {
        kf[j] = ld4(K + p * sk + j * DEC_W + col) * kscale;
        vf[j] = ld4(V + p * sv + j * DEC_W + col);
    }
    for (int st = 0; st < steps; st++) {
        const long i0 = ((long)blockIdx.x * steps + st) * STEP_ROWS +
                        w * 2 * UNR + r;
        f32x4 q[UNR];

        for (int u = 0; u < UNR; u++) {
            const long i = i0 + 2 * u;

            q[u] = i < Nq ? ld4(qb + i * DEC_W) : (f32x4){0, 0, 0, 0};
        }
        for (int u = 0; u < UNR; u++) {
            const long i = i0 + 2 * u;
            float s[NK], mx = -INFINITY, l = 0.0f;
            f32x4 o = {0, 0, 0, 0};

            for (int j = 0; j < NK; j++) {
                s[j] = quad_sum(dot4(q[u], kf[j]));
                mx = __builtin_fmaxf(mx, s[j]);
            }
            for (int j = 0; j < NK; j++) {
                const float e = __builtin_amdgcn_exp2f(s[j] - mx);

                l += e;
                o += e * vf[j];
            }
            if (i < Nq)
                *(f32x4 *)(ob + i * DEC_W) = o * (1.0f / l);
        }
    }
}

/* ------------------------------------------------------------------ */
/* Few keys, any head width up to 32 (generic)                         */
/* ------------------------------------------------------------------ */

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

/* Few keys (<= 8), head width 32, for precision=bf16: four lanes per
 * (prompt, query, head), each holding 8 of the 32 channels; the partial
 * dot products close over the four lanes, the softmax runs on the exp2
 * domain, and each lane writes its 8 output channels. Rows are read as
 * float4 (16-byte aligned strides, checked by the launcher). */
__global__ __launch_bounds__(256) void k_mha_few32x4(
    const float *__restrict__ Q, long sq, const float *__restrict__ K,
    long sk, const float *__restrict__ V, long sv, float *__restrict__ O,
    int Nq, int Nk, int dint, float scale2, long total)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= total)
        return;
    const int qt = (int)(gid & 3), h = (int)((gid >> 2) & 7);
    const long row = gid >> 5, p = row / Nq, i = row % Nq;
    const int c0 = 32 * h + 8 * qt;
    const float *qr = Q + p * sq + i * dint + c0;
    const f32x4 q0 = *(const f32x4 *)qr, q1 = *(const f32x4 *)(qr + 4);
    float sc[8], mx = -INFINITY;

    for (int j = 0; j < 8; j++) {
        float s = 0.0f;

        if (j < Nk) {
            const float *kr = K + p * sk + (long)j * dint + c0;
            const f32x4 k0 = *(const f32x4 *)kr, k1 = *(const f32x4 *)(kr + 4);

            for (int e = 0; e < 4; e++) {
                s = fmaf(q0[e], k0[e], s);
                s = fmaf(q1[e], k1[e], s);
            }
        }
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        sc[j] = j < Nk ? s * scale2 : -INFINITY;
        mx = fmaxf(mx, sc[j]);
    }
    float sum = 0.0f;
    f32x4 o0 = {}, o1 = {};

    for (int j = 0; j < 8; j++) {
        if (j >= Nk)
            break;
        const float e = __builtin_amdgcn_exp2f(sc[j] - mx);
        const float *vr = V + p * sv + (long)j * dint + c0;
        const f32x4 v0 = *(const f32x4 *)vr, v1 = *(const f32x4 *)(vr + 4);

        sum += e;
        for (int x = 0; x < 4; x++) {
            o0[x] = fmaf(e, v0[x], o0[x]);
            o1[x] = fmaf(e, v1[x], o1[x]);
        }
    }
    const float inv = 1.0f / sum;
    float *out = O + (p * Nq + i) * dint + c0;

    *(f32x4 *)out = o0 * inv;
    *(f32x4 *)(out + 4) = o1 * inv;
}

extern "C" int launch_mha_few32x4(const float *Q, long sq, const float *K,
                                  long sk, const float *V, long sv, float *O,
                                  int P, int Nq, int Nk, int dint, float scale,
                                  void *stream)
{
    const long total = (long)P * Nq * 32;

    if (dint != 256 || Nk < 1 || Nk > 8 || ((sq | sk | sv) & 3) ||
        (((uintptr_t)Q | (uintptr_t)K | (uintptr_t)V | (uintptr_t)O) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mha_few32x4, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, (hipStream_t)stream, Q, sq, K, sk, V, sv,
                       O, Nq, Nk, dint, scale * LOG2E_F, total);
    return hipGetLastError();
}

static bool aligned16(long sq, long sk, long sv)
{
    return sq % 4 == 0 && sk % 4 == 0 && sv % 4 == 0;
}

extern "C" int launch_mha_fewkeys(const float *Q, long sq, const float *K,
                                  long sk, const float *V, long sv, float *O,
                                  int P, int Nq, int Nk, int dint, float scale,
                                  void *stream)
{
    hipStream_t s = (hipStream_t)stream;

    if (P > 65535)
        return hipErrorInvalidConfiguration;
    if (dint == DEC_W && Nk <= 8 && aligned16(sq, sk, sv)) {
        /* Enough workgroups to fill the device several times over, then
         * more rows per workgroup. */
        const long per_prompt = (Nq + STEP_ROWS - 1) / STEP_ROWS;
        long steps = per_prompt * P / 4096;
        dim3 grid;

        steps = steps < 1 ? 1 : steps > 8 ? 8 : steps;
        grid = dim3((unsigned)((per_prompt + steps - 1) / steps), P);
        if (grid.x > 2147483647u)
            return hipErrorInvalidConfiguration;
#define FEW(n)                                                                \
    case n:                                                                   \
        hipLaunchKernelGGL(k_mha_few16<n>, grid, dim3(256), 0, s, Q, sq, K,  \
                           sk, V, sv, O, Nq, scale * LOG2E_F, (int)steps);    \
        break;
        switch (Nk) {
            FEW(1) FEW(2) FEW(3) FEW(4) FEW(5) FEW(6) FEW(7) FEW(8)
        }
#undef FEW
        return hipGetLastError();
    }
    {
        const long threads = (long)Nq * DEC_HEADS;

        hipLaunchKernelGGL(k_mha_fewkeys, dim3((threads + 255) / 256, P),
                           dim3(256), 0, s, Q, sq, K, sk, V, sv, O, Nq, Nk,
                           dint, dint / DEC_HEADS, scale);
    }
    return hipGetLastError();
}

/* ------------------------------------------------------------------ */
/* Many keys, head width 16 (split-K)                                  */
/* ------------------------------------------------------------------ */

/* Partial record of one (prompt, split, query): m[8 heads], l[8 heads],
 * o[128] (unnormalised), in the exp2 domain. */
#define PREC (2 * DEC_HEADS + DEC_W)

/* Merge two online-softmax states into the first. */
__device__ __forceinline__ void merge_state(float &m, float &l, f32x4 &o,
                                            float m2, float l2, f32x4 o2)
{
    const float M = __builtin_fmaxf(m, m2);
    const float f = __builtin_amdgcn_exp2f(m - M);
    const float f2 = __builtin_amdgcn_exp2f(m2 - M);

    l = fmaf(l, f, l2 * f2);
    o = o * f + o2 * f2;
    m = M;
}

/* Reduce-scatter over a quad: p[u] are this lane's partial dot products
 * with the quad's four keys; lane cq (b0 = cq & 1, b1 = cq >> 1) returns
 * key cq's full score. Step 1 keeps keys b0 and b0 + 2 and hands the
 * other two to lane ^ 1; step 2 keeps key cq and hands the other to
 * lane ^ 2. */
__device__ __forceinline__ float quad_rs4(const float p[4], bool b0, bool b1)
{
    const float k0 = b0 ? p[1] : p[0], g0 = b0 ? p[0] : p[1];
    const float k1 = b0 ? p[3] : p[2], g1 = b0 ? p[2] : p[3];
    const float a0 = k0 + dppf<DPP_QXOR1>(g0);
    const float a1 = k1 + dppf<DPP_QXOR1>(g1);

    return (b1 ? a1 : a0) + dppf<DPP_QXOR2>(b1 ? a0 : a1);
}

__device__ __forceinline__ float quad_max(float x)
{
    x = __builtin_fmaxf(x, dppf<DPP_QXOR1>(x));
    return __builtin_fmaxf(x, dppf<DPP_QXOR2>(x));
}

/* Key groups of four per lane per step of the many-keys kernel, and the
 * keys a workgroup covers per step (4 waves x 2 row halves x 4 keys x
 * groups). */
#define MANY_G 1
#define MANY_STEP (4 * 2 * 4 * MANY_G)

/* Lazy rescale: the running max only moves when a score exceeds it by
 * more than this (log2 units), so exp2(s - m) <= 2^8 in between. */
#define LAZY_TH 8.0f

/* Many keys: a quad (lanes 4g..4g+3 of one row half) holds, per group
 * of a step, four keys j0 + r + 8g + 2u (u = 0..3) x 16 channels of one
 * head, four channels per lane. Per query: partial dots, a reduce-scatter that
 * leaves key cq's score in lane cq, one exp per lane, and the PV update
 * o += e_u * v_u with e_u broadcast from lane u (DPP quad_perm u,u,u,u).
 * The running max m is the same in the quad's four lanes; the row sum l
 * is per lane (its own keys) and summed over the quad at the end. */
template <int NQ>
__global__ __launch_bounds__(256) void k_mha_many16(
    const float *__restrict__ Q, long sq, const float *__restrict__ K,
    long sk, const float *__restrict__ V, long sv, float *__restrict__ part,
    float *__restrict__ O, int Nq, int Nk, float qscale, int chunk,
    int nsplit)
{
    __shared__ float red[4][NQ][6][32];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = (lane & 31) * 4, r = lane >> 5, cq = lane & 3;
    const bool b0 = cq & 1, b1 = cq >> 1;
    const int split = blockIdx.x, qz = blockIdx.z * 8;
    const long p = blockIdx.y;
    const int nq = min(NQ, Nq - qz);
    const int k0 = split * chunk, k1 = min(Nk, k0 + chunk);
    const float *kb = K + p * sk + col, *vb = V + p * sv + col;
    f32x4 q[NQ], o[NQ];
    float m[NQ], l[NQ];

    for (int t = 0; t < NQ; t++) {
        q[t] = t < nq ? ld4(Q + p * sq + (long)(qz + t) * DEC_W + col) * qscale
                      : (f32x4){0, 0, 0, 0};
        o[t] = (f32x4){0, 0, 0, 0};
        m[t] = M_INIT;
        l[t] = 0.0f;
    }
    for (int kbase = k0; kbase < k1; kbase += MANY_STEP) {
        const int j0 = kbase + w * 8 * MANY_G + r;
        f32x4 kf[4 * MANY_G], vf[4 * MANY_G];
        float s[MANY_G][NQ], madd[MANY_G];
        bool need = false;

        for (int u = 0; u < 4 * MANY_G; u++) {
            const long j = j0 + 2 * u;

            kf[u] = j < k1 ? ld4(kb + j * DEC_W) : (f32x4){0, 0, 0, 0};
            vf[u] = j < k1 ? ld4(vb + j * DEC_W) : (f32x4){0, 0, 0, 0};
        }
        for (int g = 0; g < MANY_G; g++)
            madd[g] = j0 + 8 * g + 2 * cq < k1 ? 0.0f : -INFINITY;
        for (int g = 0; g < MANY_G; g++)
            for (int t = 0; t < NQ; t++) {
                float pd[4];

                for (int u = 0; u < 4; u++)
                    pd[u] = dot4(q[t], kf[4 * g + u]);
                s[g][t] = quad_rs4(pd, b0, b1) + madd[g];
                need |= s[g][t] > m[t] + LAZY_TH;
            }
        if (__builtin_amdgcn_ballot_w64(need)) {
            for (int t = 0; t < NQ; t++) {
                float mx = s[0][t];

                for (int g = 1; g < MANY_G; g++)
                    mx = __builtin_fmaxf(mx, s[g][t]);
                {
                    const float mn = __builtin_fmaxf(m[t], quad_max(mx));
                    const float corr = __builtin_amdgcn_exp2f(m[t] - mn);

                    l[t] *= corr;
                    o[t] *= corr;
                    m[t] = mn;
                }
            }
        }
        for (int g = 0; g < MANY_G; g++)
            for (int t = 0; t < NQ; t++) {
                const float e = __builtin_amdgcn_exp2f(s[g][t] - m[t]);

                l[t] += e;
                o[t] += dppf<0x00>(e) * vf[4 * g];
                o[t] += dppf<0x55>(e) * vf[4 * g + 1];
                o[t] += dppf<0xAA>(e) * vf[4 * g + 2];
                o[t] += dppf<0xFF>(e) * vf[4 * g + 3];
            }
    }
    for (int t = 0; t < NQ; t++)
        l[t] = quad_sum(l[t]);
    /* Lanes l and l ^ 32 hold the same (head, channels) over different
     * keys. */
    for (int t = 0; t < NQ; t++) {
        f32x4 o2;

        o2.x = __shfl_xor(o[t].x, 32);
        o2.y = __shfl_xor(o[t].y, 32);
        o2.z = __shfl_xor(o[t].z, 32);
        o2.w = __shfl_xor(o[t].w, 32);
        merge_state(m[t], l[t], o[t], __shfl_xor(m[t], 32),
                    __shfl_xor(l[t], 32), o2);
    }
    if (lane < 32)
        for (int t = 0; t < NQ; t++) {
            red[w][t][0][lane] = m[t];
            red[w][t][1][lane] = l[t];
            red[w][t][2][lane] = o[t].x;
            red[w][t][3][lane] = o[t].y;
            red[w][t][4][lane] = o[t].z;
            red[w][t][5][lane] = o[t].w;
        }
    __syncthreads();
    if (w != 0 || lane >= 32)
        return;
    for (int t = 0; t < NQ; t++) {
        for (int v = 1; v < 4; v++) {
            const f32x4 o2 = {red[v][t][2][lane], red[v][t][3][lane],
                              red[v][t][4][lane], red[v][t][5][lane]};

            merge_state(m[t], l[t], o[t], red[v][t][0][lane],
                        red[v][t][1][lane], o2);
        }
        if (t >= nq)
            continue;
        if (nsplit == 1) {
            *(f32x4 *)(O + (p * Nq + qz + t) * DEC_W + col) = o[t] * (1.0f / l[t]);
        }
        else {
            float *rec = part + ((p * nsplit + split) * Nq + qz + t) * PREC;

            if (cq == 0) {
                rec[lane >> 2] = m[t];
                rec[DEC_HEADS + (lane >> 2)] = l[t];
            }
            *(f32x4 *)(rec + 2 * DEC_HEADS + col) = o[t];
        }
    }
}

/* Merge of the split partial records: one workgroup per (prompt, query);
 * lane (t & 31) owns four channels, the 8 lane groups (t >> 5) take every
 * 8th split, four records in flight at a time, and the 8 group states are
 * merged through LDS. */
#define MERGE_GROUPS 8

__global__ __launch_bounds__(256) void k_mha_many_merge(
    const float *__restrict__ part, float *__restrict__ O, int Nq, int nsplit)
{
    __shared__ float red[MERGE_GROUPS][6][32];
    const int t = threadIdx.x, c = t & 31, sg = t >> 5;
    const int col = c * 4, h = col >> 4;
    const long pq = blockIdx.x, p = pq / Nq, qi = pq % Nq;
    const float *rec = part + (p * nsplit * Nq + qi) * PREC;
    const long stride = (long)Nq * PREC;
    float m = M_INIT, l = 0.0f;
    f32x4 o = {0, 0, 0, 0};

    for (int s0 = sg; s0 < nsplit; s0 += 4 * MERGE_GROUPS) {
        float mm[4], ll[4];
        f32x4 oo[4];

        for (int u = 0; u < 4; u++) {
            const int s = s0 + u * MERGE_GROUPS;
            const float *r2 = rec + (s < nsplit ? s : 0) * stride;

            mm[u] = r2[h];
            ll[u] = r2[DEC_HEADS + h];
            oo[u] = ld4(r2 + 2 * DEC_HEADS + col);
        }
        for (int u = 0; u < 4; u++)
            if (s0 + u * MERGE_GROUPS < nsplit)
                merge_state(m, l, o, mm[u], ll[u], oo[u]);
    }
    red[sg][0][c] = m;
    red[sg][1][c] = l;
    red[sg][2][c] = o.x;
    red[sg][3][c] = o.y;
    red[sg][4][c] = o.z;
    red[sg][5][c] = o.w;
    __syncthreads();
    if (sg != 0)
        return;
    for (int g = 1; g < MERGE_GROUPS; g++) {
        const f32x4 o2 = {red[g][2][c], red[g][3][c], red[g][4][c],
                          red[g][5][c]};

        merge_state(m, l, o, red[g][0][c], red[g][1][c], o2);
    }
    *(f32x4 *)(O + pq * DEC_W + col) = o * (1.0f / l);
}

/* Key range per workgroup: a multiple of the workgroup step, chosen so
 * that the grid holds about 512 workgroups (half a resident round at four
 * workgroups per CU; longer workgroups amortise the merge). */
static int many_chunk(int P, int Nq, int Nk)
{
    const long groups = (long)P * ((Nq + 7) / 8);
    long splits = (512 + groups - 1) / groups;
    long chunk;

    if (splits < 1)
        splits = 1;
    chunk = (Nk + splits - 1) / splits;
    chunk = (chunk + MANY_STEP - 1) / MANY_STEP * MANY_STEP;
    return (int)(chunk < MANY_STEP ? MANY_STEP : chunk);
}

/* Static device scratch of mha_noalloc: the split-K partial records of
 * the many-keys kernel, for callers that cannot allocate (HIP graph
 * capture, serving loops). Every GPU the library runs on holds its own
 * copy, at its own address, until the process ends. The host refers to
 * it only through the address hipGetSymbolAddress returns on each
 * device (the array's name is a host-side stand-in). */
static __device__ __align__(256) float scratch[MHA_NOALLOC_BYTES / sizeof(float)];

#define SCRATCH_DEVICES 64
static void *scratch_at[SCRATCH_DEVICES];

extern "C" int dec_scratch_init(int device)
{
    void *p = NULL;
    int err;

    if (device < 0 || device >= SCRATCH_DEVICES)
        return hipErrorInvalidDevice;
    err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (err != hipSuccess)
        return err;
    __atomic_store_n(&scratch_at[device], p, __ATOMIC_RELEASE);
    return hipSuccess;
}

extern "C" void *dec_scratch(int device)
{
    if (device < 0 || device >= SCRATCH_DEVICES)
        return NULL;
    return __atomic_load_n(&scratch_at[device], __ATOMIC_ACQUIRE);
}

extern "C" size_t mha_manykeys_scratch(int P, int Nq, int Nk)
{
    const int chunk = many_chunk(P, Nq, Nk);
    const int nsplit = (Nk + chunk - 1) / chunk;

    return nsplit > 1 ? (size_t)P * nsplit * Nq * PREC * sizeof(float) : 0;
}

extern "C" int launch_mha_manykeys(const float *Q, long sq, const float *K,
                                   long sk, const float *V, long sv, float *O,
                                   int P, int Nq, int Nk, int dint,
                                   float scale, void *scratch, void *stream)
{
    const int chunk = many_chunk(P, Nq, Nk);
    const int nsplit = (Nk + chunk - 1) / chunk;
    const dim3 grid(nsplit, P, (Nq + 7) / 8);
    const float qscale = scale * LOG2E_F;
    hipStream_t s = (hipStream_t)stream;
    int err;

    if (dint != DEC_W)
        return hipErrorInvalidValue;
    if (P > 65535 || grid.z > 65535)
        return hipErrorInvalidConfiguration;
    /* 16-byte row loads need 4-float aligned per-prompt strides. */
    if (!aligned16(sq, sk, sv))
        return hipErrorInvalidValue;
    if (nsplit > 1 && !scratch)
        return hipErrorInvalidValue;
#define MANY(n)                                                               \
    case n:                                                                   \
        hipLaunchKernelGGL(k_mha_many16<n>, grid, dim3(256), 0, s, Q, sq, K, \
                           sk, V, sv, (float *)scratch, O, Nq, Nk, qscale,   \
                           chunk, nsplit);                                    \
        break;
    switch (Nq < 8 ? Nq : 8) {
        MANY(1) MANY(2) MANY(3) MANY(4) MANY(5) MANY(6) MANY(7) MANY(8)
    }
#undef MANY
    err = hipGetLastError();
    if (err != hipSuccess || nsplit == 1)
        return err;
    if ((long)P * Nq > 2147483647L)
        return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_mha_many_merge, dim3(P * Nq), dim3(256), 0, s,
                       (const float *)scratch, O, Nq, nsplit);
    return hipGetLastError();
}
