/* SPDX-License-Identifier: Unlicense
 *
 * Row and element kernels of the attention path on gfx950: LayerNorm
 * (optionally fused with the window partition and a bf16 store),
 * softmax_rows, rope_apply, window partition / unpartition, add_bcast
 * and storage conversions. All are HBM-bound; they use one workgroup
 * per row or one thread per element with 64-bit index arithmetic.
 */
#include "k_common.h"

/* ------------------------------------------------------------ LayerNorm */

/* Block-wide sum of 256 threads: wave64 butterflies, then 4 partials. */
__device__ __forceinline__ float block_sum256(float v, float *red)
{
    const int w = threadIdx.x >> 6, l = threadIdx.x & 63;

    v = wave_sum(v);
    __syncthreads();
    if (l == 0)
        red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

/* One 256-thread workgroup per output row. The row is held in registers
 * (up to 8 values per thread, C <= 2048) between the mean, variance and
 * normalisation passes; wider rows are re-read. With ws > 0 output row r
 * is window-partition position r of an H x H grid (sam3_kernels.cl:
 * 712-724) and takes its token from there, or zeros in the padding. */
template <typename TY>
__global__ __launch_bounds__(256) void k_layernorm(
    const float *__restrict__ X, TY *__restrict__ Y, const float *__restrict__ g,
    const float *__restrict__ bt, int C, float eps, int act, int H, int ws,
    int nwx)
{
    __shared__ float red[4];
    const long r = blockIdx.x;
    long src = r;
    float v[8];
    float s = 0.0f, mean, var, rs;
    const int t = threadIdx.x;
    int i, c;

    if (ws > 0) {
        const int w = (int)(r / ((long)ws * ws)), p = (int)(r % ((long)ws * ws));
        const int y = (w / nwx) * ws + p / ws, x = (w % nwx) * ws + p % ws;

        if (y >= H || x >= H) {
            for (c = t; c < C; c += 256)
                Y[r * C + c] = (TY)0.0f;
            return;
        }
        src = (long)y * H + x;
    }
    const float *xr = X + src * C;
    for (i = 0; i < 8; i++) {
        c = t + 256 * i;
        v[i] = c < C ? xr[c] : 0.0f;
        s += v[i];
    }
    for (c = t + 2048; c < C; c += 256)
        s += xr[c];
    mean = block_sum256(s, red) / (float)C;
    s = 0.0f;
    for (i = 0; i < 8; i++) {
        c = t + 256 * i;
        if (c < C) {
            const float d = v[i] - mean;

            s = fmaf(d, d, s);
        }
    }
    for (c = t + 2048; c < C; c += 256) {
        const float d = xr[c] - mean;

        s = fmaf(d, d, s);
    }
    var = block_sum256(s, red) / (float)C;
    rs = 1.0f / sqrtf(var + eps);
    for (i = 0; i < 8; i++) {
        c = t + 256 * i;
        if (c < C)
            Y[r * C + c] = (TY)act_k(fmaf((v[i] - mean) * rs, g[c], bt[c]), act);
    }
    for (c = t + 2048; c < C; c += 256)
        Y[r * C + c] = (TY)act_k(fmaf((xr[c] - mean) * rs, g[c], bt[c]), act);
}

/* Sum over a wave64, the same bits in every lane: DPP adds inside each
 * row of 16 lanes (swap within pairs, then within quads, then the half-row
 * and row mirrors: every lane of a row ends with the row's sum), then the
 * four row sums read into scalars and added in a fixed order. Six dependent
 * VALU steps instead of six LDS-crossbar round trips of the shuffle form. */
__device__ __forceinline__ float wave_sum_rows(float v)
{
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                       0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                       0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                       0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                       0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0)),
                r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16)),
                r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32)),
                r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));

    return (r0 + r1) + (r2 + r3);
}

/* Rows of C = 256 V floats (V <= 16): one wave per output row, four
 * rows per workgroup. Lane l holds floats 4 l + 256 i .. +3 (i < V) in
 * registers from one 16-byte load each, its gamma and beta loaded beside
 * them for C <= 2048 (not after the sums, where they would add an L2 trip
 * to every wave's path); the mean and variance close with wave_sum_rows
 * (no LDS, no barrier); outputs leave as 16-byte (float) or 8-byte (bf16)
 * stores. Window partition as in k_layernorm, in 32-bit arithmetic (the
 * launcher keeps the rows below 2^32). At 5184 x 1024 (bf16 out) after a
 * kernel that wrote X: 7.9 -> 6.6 us against the shuffle sums with late
 * gamma / beta loads and 64-bit partition divisions. Every loop over the
 * row is unrolled (left rolled at C >= 3072, the row went to scratch). */
template <typename TY, int V>
__global__ __launch_bounds__(256) void k_layernorm_w(
    const float *__restrict__ X, TY *__restrict__ Y, const float *__restrict__ g,
    const float *__restrict__ bt, long rows, float eps, int act, int H,
    int ws, int nwx)
{
    constexpr int C = 256 * V;
    /* Gamma and beta held from the start up to 8 float4 each (96 VGPRs
     * with the row); wider rows load them at the end. */
    constexpr bool EARLY = V <= 8;
    const int l = threadIdx.x & 63;
    const unsigned r = blockIdx.x * 4u + (threadIdx.x >> 6);
    unsigned src = r;
    f32x4 v[V], gv[V], bv[V];
    float s = 0.0f, mean, var, rs;

    if (r >= rows)
        return;
    TY *yr = Y + (long)r * C + 4 * l;
    if (ws > 0) {
        const unsigned a = (unsigned)ws * (unsigned)ws, w = r / a, p = r - w * a;
        const unsigned wy = w / (unsigned)nwx, py = p / (unsigned)ws;
        const unsigned y = wy * ws + py, x = (w - wy * nwx) * ws + (p - py * ws);

        if (y >= (unsigned)H || x >= (unsigned)H) {
#pragma unroll
            for (int i = 0; i < V; i++)
                for (int e = 0; e < 4; e++)
                    yr[256 * i + e] = (TY)0.0f;
            return;
        }
        src = y * (unsigned)H + x;
    }
    const float *xr = X + (long)src * C + 4 * l;
#pragma unroll
    for (int i = 0; i < V; i++)
        v[i] = *(const f32x4 *)(xr + 256 * i);
    if constexpr (EARLY) {
#pragma unroll
        for (int i = 0; i < V; i++) {
            gv[i] = *(const f32x4 *)(g + 4 * l + 256 * i);
            bv[i] = *(const f32x4 *)(bt + 4 * l + 256 * i);
        }
        /* Keeps all loads issued here (the compiler otherwise sinks gamma
         * and beta below the sums). */
#pragma unroll
        for (int i = 0; i < V; i++)
            asm volatile("" : "+v"(v[i]), "+v"(gv[i]), "+v"(bv[i]));
    }
#pragma unroll
    for (int i = 0; i < V; i++)
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    mean = wave_sum_rows(s) / (float)C;
    s = 0.0f;
#pragma unroll
    for (int i = 0; i < V; i++) {
        const f32x4 dv = v[i] - mean;

        s = fmaf(dv.x, dv.x, fmaf(dv.y, dv.y, fmaf(dv.z, dv.z, fmaf(dv.w, dv.w, s))));
    }
    var = wave_sum_rows(s) / (float)C;
    rs = 1.0f / sqrtf(var + eps);
#pragma unroll
    for (int i = 0; i < V; i++) {
        f32x4 o;

        if constexpr (!EARLY) {
            gv[i] = *(const f32x4 *)(g + 4 * l + 256 * i);
            bv[i] = *(const f32x4 *)(bt + 4 * l + 256 * i);
        }
        o.x = act_k(fmaf((v[i].x - mean) * rs, gv[i].x, bv[i].x), act);
        o.y = act_k(fmaf((v[i].y - mean) * rs, gv[i].y, bv[i].y), act);
        o.z = act_k(fmaf((v[i].z - mean) * rs, gv[i].z, bv[i].z), act);
        o.w = act_k(fmaf((v[i].w - mean) * rs, gv[i].w, bv[i].w), act);
        if constexpr (sizeof(TY) == 4)
            *(f32x4 *)(yr + 256 * i) = o;
        else {
            uint2 pk;

            pk.x = pack_bf16x2(o.x, o.y);
            pk.y = pack_bf16x2(o.z, o.w);
            *(uint2 *)(yr + 256 * i) = pk;
        }
    }
}

/* Narrow rows (C = 4 LPR floats, LPR = 8, 16 or 32 lanes per row): 256 / LPR
 * rows per workgroup, a lane holds one float4 of its row, the sums close
 * with butterflies inside the lane group. No window partition. */
template <int LPR>
__global__ __launch_bounds__(256) void k_layernorm_n(const float *__restrict__ X,
                                                     float *__restrict__ Y,
                                                     const float *__restrict__ g,
                                                     const float *__restrict__ bt,
                                                     long rows, float eps, int act)
{
    constexpr int C = 4 * LPR;
    const int t = threadIdx.x, c = 4 * (t % LPR);
    const long r = (long)blockIdx.x * (256 / LPR) + t / LPR;

    if (r >= rows)
        return;
    const f32x4 v = *(const f32x4 *)(X + r * C + c);
    float s = (v.x + v.y) + (v.z + v.w);

    for (int k = 1; k < LPR; k <<= 1)
        s += __shfl_xor(s, k, 64);
    const float mean = s / (float)C;
    const f32x4 d = {v.x - mean, v.y - mean, v.z - mean, v.w - mean};

    s = fmaf(d.w, d.w, fmaf(d.z, d.z, fmaf(d.y, d.y, d.x * d.x)));
    for (int k = 1; k < LPR; k <<= 1)
        s += __shfl_xor(s, k, 64);
    const float rs = 1.0f / sqrtf(s / (float)C + eps);
    const f32x4 gv = *(const f32x4 *)(g + c), bv = *(const f32x4 *)(bt + c);
    f32x4 y;

    y.x = act_k(fmaf(d.x * rs, gv.x, bv.x), act);
    y.y = act_k(fmaf(d.y * rs, gv.y, bv.y), act);
    y.z = act_k(fmaf(d.z * rs, gv.z, bv.z), act);
    y.w = act_k(fmaf(d.w * rs, gv.w, bv.w), act);
    *(f32x4 *)(Y + r * C + c) = y;
}

extern "C" int launch_layernorm(const float *X, void *Y, int ydt,
                                const float *g, const float *b, long rows,
                                int C, float eps, int act, int H, int ws,
                                int nwx, void *stream)
{
    const long out_rows = ws > 0 ? (long)nwx * nwx * ws * ws : rows;
    hipStream_t st = (hipStream_t)stream;

    if (out_rows == 0)
        return hipSuccess;
    if (ws == 0 && ydt == DT_F32 && (C == 32 || C == 64 || C == 128) &&
        (((uintptr_t)X | (uintptr_t)Y | (uintptr_t)g | (uintptr_t)b) & 15) == 0) {
        const int rpw = 1024 / C; /* rows per workgroup: 256 / (C / 4) */
        const dim3 grid((unsigned)((out_rows + rpw - 1) / rpw));

        if (C == 32)
            hipLaunchKernelGGL(k_layernorm_n<8>, grid, dim3(256), 0, st, X,
                               (float *)Y, g, b, out_rows, eps, act);
        else if (C == 64)
            hipLaunchKernelGGL(k_layernorm_n<16>, grid, dim3(256), 0, st, X,
                               (float *)Y, g, b, out_rows, eps, act);
        else
            hipLaunchKernelGGL(k_layernorm_n<32>, grid, dim3(256), 0, st, X,
                               (float *)Y, g, b, out_rows, eps, act);
        return hipGetLastError();
    }
    /* 16-byte rows of the wave-per-row kernel: C a multiple of 256 up to
     * 4096 (the buffers are hipMalloc'd, so rows start 16-byte aligned). */
    if (C % 256 == 0 && C <= 4096 && out_rows <= 0xffffffffL &&
        (ws == 0 || (long)H * H <= 0xffffffffL)) {
        const dim3 grid((unsigned)((out_rows + 3) / 4));

#define LNW(V)                                                                \
    case V:                                                                   \
        if (ydt == DT_BF16)                                                   \
            hipLaunchKernelGGL((k_layernorm_w<__bf16, V>), grid, dim3(256), 0, \
                               st, X, (__bf16 *)Y, g, b, out_rows, eps, act,  \
                               H, ws, nwx);                                   \
        else                                                                  \
            hipLaunchKernelGGL((k_layernorm_w<float, V>), grid, dim3(256), 0,  \
                               st, X, (float *)Y, g, b, out_rows, eps, act,   \
                               H, ws, nwx);                                   \
        return hipGetLastError();
        switch (C / 256) {
            LNW(1) LNW(2) LNW(3) LNW(4) LNW(5) LNW(6) LNW(7) LNW(8) LNW(9)
            LNW(10) LNW(11) LNW(12) LNW(13) LNW(14) LNW(15) LNW(16)
        }
#undef LNW
    }
    if (ydt == DT_BF16)
        hipLaunchKernelGGL(k_layernorm<__bf16>, dim3(out_rows), dim3(256), 0,
                           (hipStream_t)stream, X, (__bf16 *)Y, g, b, C, eps,
                           act, H, ws, nwx);
    else
        hipLaunchKernelGGL(k_layernorm<float>, dim3(out_rows), dim3(256), 0,
                           (hipStream_t)stream, X, (float *)Y, g, b, C, eps,
                           act, H, ws, nwx);
    return hipGetLastError();
}

/* ------------------------------------------------------------ softmax */

/* In-place softmax of one row of L floats per 256-thread workgroup. */
__global__ __launch_bounds__(256) void k_softmax_rows(float *__restrict__ S,
                                                      int L)
{
    __shared__ float red[4];
    float *s = S + (long)blockIdx.x * L;
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    float m = -INFINITY, sum = 0.0f, inv;
    int j;

    for (j = t; j < L; j += 256)
        m = fmaxf(m, s[j]);
    m = wave_max(m);
    __syncthreads();
    if (l == 0)
        red[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (j = t; j < L; j += 256) {
        const float v = expf(s[j] - m);

        s[j] = v;
        sum += v;
    }
    inv = 1.0f / block_sum256(sum, red);
    for (j = t; j < L; j += 256)
        s[j] *= inv;
}

extern "C" int launch_softmax_rows(float *S, long rows, int L, void *stream)
{
    hipLaunchKernelGGL(k_softmax_rows, dim3(rows), dim3(256), 0,
                       (hipStream_t)stream, S, L);
    return hipGetLastError();
}

/* softmax_ext (sam3_kernels.cl:885-921): row = head * Nq + query (heads
 * from h0); each score first gets the causal mask (key j > query i:
 * -inf) or else, with dy, the box relative position bias
 * dy[(i H + j / W) nh + h] + dx[(i W + j % W) nh + h] (H = L / W), stored
 * back; then the softmax of k_softmax_rows. */
__global__ __launch_bounds__(256) void k_softmax_ext(
    float *__restrict__ S, int L, int Nq, int h0, int causal,
    const float *__restrict__ dy, const float *__restrict__ dx, int W, int nh)
{
    __shared__ float red[4];
    const int row = blockIdx.x, i = row % Nq, h = h0 + row / Nq;
    const int H = W > 0 ? L / W : 0;
    float *s = S + (long)row * L;
    const int t = threadIdx.x, w = t >> 6, l = t & 63;
    float m = -INFINITY, sum = 0.0f, inv;
    int j;

    for (j = t; j < L; j += 256) {
        float v = s[j];

        if (causal && j > i)
            v = -INFINITY;
        else if (dy)
            v += dy[((long)i * H + j / W) * nh + h] + dx[((long)i * W + j % W) * nh + h];
        s[j] = v;
        m = fmaxf(m, v);
    }
    m = wave_max(m);
    __syncthreads();
    if (l == 0)
        red[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    for (j = t; j < L; j += 256) {
        const float v = expf(s[j] - m);

        s[j] = v;
        sum += v;
    }
    inv = 1.0f / block_sum256(sum, red);
    for (j = t; j < L; j += 256)
        s[j] *= inv;
}

extern "C" int launch_softmax_ext(float *S, long rows, int L, int Nq, int h0,
                                  int causal, const float *dy, const float *dx,
                                  int W, int nh, void *stream)
{
    hipLaunchKernelGGL(k_softmax_ext, dim3(rows), dim3(256), 0,
                       (hipStream_t)stream, S, L, Nq, h0, causal, dy, dx, W, nh);
    return hipGetLastError();
}

/* ------------------------------------------------------------ RoPE */

/* One thread per (row, q/k, pair): the rotation of rope_apply
 * (sam3_kernels.cl:679-698) at position r % npos. */
__global__ __launch_bounds__(256) void k_rope_apply(
    float *__restrict__ qkv, long total, int E, int hd, int npos,
    const float2 *__restrict__ cs)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;
    const int nf = hd / 2, half = E / 2;

    if (gid >= total)
        return;
    const int pr = (int)(gid % half);
    const long rest = gid / half;
    const int qk = (int)(rest % 2);
    const long r = rest / 2;
    const int h = pr / nf, j = pr % nf;
    float *x = qkv + r * 3 * E + (long)qk * E + (long)h * hd + 2 * j;
    const float2 rot = cs[(r % npos) * nf + j];
    const float a = x[0], b = x[1];

    x[0] = fmaf(a, rot.x, -(b * rot.y));
    x[1] = fmaf(a, rot.y, b * rot.x);
}

extern "C" int launch_rope_apply(float *qkv, long rows, int E, int hd,
                                 int npos, const float *cs, void *stream)
{
    const long total = rows * E;

    if (total == 0)
        return hipSuccess;
    hipLaunchKernelGGL(k_rope_apply, dim3((total + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, qkv, total, E, hd, npos,
                       (const float2 *)cs);
    return hipGetLastError();
}

/* ------------------------------------------------------------ patches */

/* Patch im2col (sam3_kernels.cl:661-672): row t = ty * grid + tx of out
 * (rows ldo apart) holds the 3 x ps x ps patch at (ty, tx), column
 * c * ps^2 + ky * ps + kx, and zeros from column 3 ps^2 to ldo; out is
 * float or bf16 (ydt). One thread per output element, consecutive
 * threads along a patch row read consecutive image floats. */
__global__ __launch_bounds__(256) void k_patch_im2col(
    const float *__restrict__ img, void *__restrict__ out, int ydt,
    long total, int side, int grid, int ps, int ldo)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= total)
        return;
    const int K = 3 * ps * ps;
    const long t = gid / ldo;
    const int col = (int)(gid % ldo);
    float v = 0.0f;

    if (col < K) {
        const int c = col / (ps * ps), ky = (col % (ps * ps)) / ps, kx = col % ps;
        const int ty = (int)(t / grid), tx = (int)(t % grid);

        v = img[((long)c * side + ty * ps + ky) * side + tx * ps + kx];
    }
    if (ydt == DT_BF16)
        ((uint16_t *)out)[gid] = f2bf(v);
    else
        ((float *)out)[gid] = v;
}

/* The same columns as bf16 for an even patch side, one workgroup per
 * (row of patches ty, channel c): the patch row's ps image rows of the
 * channel go to LDS with 16-byte loads (whole rows, coalesced), then
 * each token's ps * ps columns of that channel leave as a contiguous run
 * of bf16 pairs; the channel-2 workgroup also writes the tokens' zero
 * columns K .. ldo - 1. 1024 threads. The launcher checks the shapes
 * (side a multiple of 4, ps * side floats within 64 KiB of LDS, 32-bit
 * indices). */
__global__ __launch_bounds__(1024) void k_patch_im2col_bf16(const float *__restrict__ img,
                                                            uint32_t *__restrict__ out,
                                                            int side, int grid, int ps, int ldo)
{
    extern __shared__ __attribute__((aligned(16))) float rows[];
    const int ty = blockIdx.x, c = blockIdx.y, K = 3 * ps * ps, pp = ps * ps;
    const f32x4 *src = (const f32x4 *)(img + ((size_t)c * side + (size_t)ty * ps) * side);
    const int n4 = ps * side / 4;
    f32x4 v[4];

    /* At most four 16-byte loads per thread (64 KiB), all issued before
     * the first is stored: one trip to memory instead of one per load. */
    for (int k = 0; k < 4; k++)
        if (threadIdx.x + 1024 * k < n4)
            v[k] = src[threadIdx.x + 1024 * k];
    for (int k = 0; k < 4; k++)
        if (threadIdx.x + 1024 * k < n4)
            ((f32x4 *)rows)[threadIdx.x + 1024 * k] = v[k];
    __syncthreads();
    const int half = pp / 2, work = grid * half;

    for (int i = threadIdx.x; i < work; i += 1024) {
        const int tx = i / half, j = 2 * (i - tx * half), ky = j / ps, kx = j - ky * ps;
        const float *r = rows + ky * side + tx * ps + kx;

        out[((size_t)(ty * grid + tx) * ldo + c * pp + j) / 2] = pack_bf16x2(r[0], r[1]);
    }
    if (c == 2) {
        const int zh = (ldo - K) / 2;

        for (int i = threadIdx.x; i < grid * zh; i += 1024) {
            const int tx = i / zh, j = i - tx * zh;

            out[((size_t)(ty * grid + tx) * ldo + K) / 2 + j] = 0u;
        }
    }
}

extern "C" int launch_patch_im2col(const float *img, void *out, int ydt,
                                   int side, int grid, int ps, int ldo,
                                   void *stream)
{
    const long total = (long)grid * grid * ldo;

    if (ldo < 3 * ps * ps)
        return hipErrorInvalidValue;
    if (ydt == DT_BF16 && ps % 2 == 0 && ldo % 2 == 0 && side % 4 == 0 &&
        grid * ps <= side && (size_t)ps * side * sizeof(float) <= 65536 &&
        total < 0x7fffffffL) {
        hipLaunchKernelGGL(k_patch_im2col_bf16, dim3((unsigned)grid, 3), dim3(1024),
                           (size_t)ps * side * sizeof(float), (hipStream_t)stream, img,
                           (uint32_t *)out, side, grid, ps, ldo);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(k_patch_im2col, dim3((total + 255) / 256), dim3(256),
                       0, (hipStream_t)stream, img, out, ydt, total, side,
                       grid, ps, ldo);
    return hipGetLastError();
}

/* rows x K float or bf16 (sdt) -> rows x KP bf16, columns K .. KP - 1
 * zero: a weight matrix padded to the NT GEMM's 64-wide K steps. */
__global__ __launch_bounds__(256) void k_pad_rows_bf16(const void *__restrict__ src, int sdt,
                                                       uint16_t *__restrict__ dst, long total,
                                                       int K, int KP)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= total)
        return;
    const long r = gid / KP;
    const int c = (int)(gid % KP);
    uint16_t v = 0;

    if (c < K)
        v = sdt == DT_BF16 ? ((const uint16_t *)src)[r * K + c]
                           : f2bf(((const float *)src)[r * K + c]);
    dst[gid] = v;
}

extern "C" int launch_pad_rows_bf16(const void *src, int sdt, void *dst, long rows, int K,
                                    int KP, void *stream)
{
    const long total = rows * KP;

    if (KP < K || total == 0)
        return total == 0 ? hipSuccess : hipErrorInvalidValue;
    hipLaunchKernelGGL(k_pad_rows_bf16, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, src, sdt, (uint16_t *)dst, total, K, KP);
    return hipGetLastError();
}

/* ------------------------------------------------------------ windows */

__global__ __launch_bounds__(256) void k_window_partition(
    const float *__restrict__ X, float *__restrict__ out, long total, int H,
    int W, int C, int ws, int nwx)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= total)
        return;
    const long r = gid / C;
    const int c = (int)(gid % C);
    const int w = (int)(r / ((long)ws * ws)), i = (int)(r % ((long)ws * ws));
    const int y = (w / nwx) * ws + i / ws, x = (w % nwx) * ws + i % ws;

    out[gid] = (y < H && x < W) ? X[((long)y * W + x) * C + c] : 0.0f;
}

extern "C" int launch_window_partition(const float *X, float *out, int H,
                                       int W, int C, int ws, int nwx,
                                       void *stream)
{
    const long total = (long)nwx * nwx * ws * ws * C;

    hipLaunchKernelGGL(k_window_partition, dim3((total + 255) / 256),
                       dim3(256), 0, (hipStream_t)stream, X, out, total, H, W,
                       C, ws, nwx);
    return hipGetLastError();
}

__global__ __launch_bounds__(256) void k_window_unpartition_add(
    float *__restrict__ X, const float *__restrict__ Wd, long total, int W,
    int C, int ws, int nwx)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= total)
        return;
    const long t = gid / C;
    const int c = (int)(gid % C);
    const int y = (int)(t / W), x = (int)(t % W);
    const long w = (long)(y / ws) * nwx + x / ws;
    const long i = (long)(y % ws) * ws + x % ws;

    X[gid] += Wd[(w * ws * ws + i) * C + c];
}

extern "C" int launch_window_unpartition_add(float *X, const float *Wd, int H,
                                             int W, int C, int ws, int nwx,
                                             void *stream)
{
    const long total = (long)H * W * C;

    hipLaunchKernelGGL(k_window_unpartition_add, dim3((total + 255) / 256),
                       dim3(256), 0, (hipStream_t)stream, X, Wd, total, W, C,
                       ws, nwx);
    return hipGetLastError();
}

/* ------------------------------------------------------------ add_bcast */

__global__ __launch_bounds__(256) void k_add_bcast(float *out,
                                                   const float *a,
                                                   const float *b, long n,
                                                   long bmod)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;

    if (i < n)
        out[i] = a[i] + b[i % bmod];
}

extern "C" int launch_add_bcast(float *out, const float *a, const float *b,
                                long n, long bmod, void *stream)
{
    hipLaunchKernelGGL(k_add_bcast, dim3((n + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, out, a, b, n, bmod);
    return hipGetLastError();
}

/* ------------------------------------------------------------ convert */

__global__ __launch_bounds__(256) void k_convert(const float *__restrict__ s,
                                                 uint16_t *__restrict__ d,
                                                 int dt, long n)
{
    const long i = (long)blockIdx.x * 256 + threadIdx.x;

    if (i >= n)
        return;
    if (dt == DT_BF16)
        d[i] = f2bf(s[i]);
    else
        d[i] = __builtin_bit_cast(uint16_t, (_Float16)s[i]);
}

extern "C" int launch_convert(const float *src, void *dst, int dst_dt,
                              size_t count, void *stream)
{
    if (count == 0)
        return hipSuccess;
    hipLaunchKernelGGL(k_convert, dim3((count + 255) / 256), dim3(256), 0,
                       (hipStream_t)stream, src, (uint16_t *)dst, dst_dt,
                       (long)count);
    return hipGetLastError();
}
