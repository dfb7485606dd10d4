/* SPDX-License-Identifier: Unlicense
 *
 * Mask decoder output kernels on gfx950: the scatter of the 2x2 /
 * stride-2 transposed convolutions of the output upscaling
 * (sam3_kernels.cl:762-786), the low-resolution mask logits
 * (sam3_kernels.cl:789-805) and the postprocessing resize with its
 * per-mask statistics (sam3_kernels.cl:807-883).
 */
#include "k_common.h"

/* One thread per (prompt, input pixel, output channel co): the four GEMM
 * columns co 4 + dy 2 + dx are one float4 (coalesced across co), and each
 * lands at output pixel (2y + dy, 2x + dx) of the P x 2H x 2W x Co map as
 * act(G + bias[co] (+ add)), consecutive co again consecutive. The add map
 * (2H x 2W x Co) is shared by the prompts. */
__global__ __launch_bounds__(256) void k_convt_scatter(const float *__restrict__ G,
                                                       float *__restrict__ out,
                                                       const float *__restrict__ bias,
                                                       const float *__restrict__ add,
                                                       int H, int W, int Co,
                                                       long total, int act)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= total)
        return;
    const int co = (int)(gid % Co);
    const long pix = gid / Co;
    const int x = (int)(pix % W);
    const long rest = pix / W;
    const int y = (int)(rest % H);
    const long p = rest / H;
    const f32x4 v = *(const f32x4 *)(G + 4 * gid);
    const float bc = bias[co];

    for (int dy = 0; dy < 2; dy++)
        for (int dx = 0; dx < 2; dx++) {
            const long o = ((2 * y + dy) * 2L * W + 2 * x + dx) * Co + co;
            float u = v[2 * dy + dx] + bc;

            if (add)
                u += add[o];
            out[p * 4L * H * W * Co + o] = act_k(u, act);
        }
}

extern "C" int launch_convt_scatter(const float *G, float *out,
                                    const float *bias, const float *add,
                                    int P, int H, int W, int Co, int act,
                                    void *stream)
{
    const long total = (long)P * H * W * Co;

    if (total <= 0)
        return hipSuccess;
    if ((total + 255) / 256 > 0x7fffffffL || ((uintptr_t)G & 15))
        return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_convt_scatter, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, (hipStream_t)stream, G, out, bias, add,
                       H, W, Co, total, act);
    return hipGetLastError();
}

/* The reference's float4 dot as a chain of fused multiply-adds and its
 * dot16 of four quarters summed left to right. */
__device__ __forceinline__ float dot4f(f32x4 a, f32x4 b)
{
    return fmaf(a.w, b.w, fmaf(a.z, b.z, fmaf(a.y, b.y, a.x * b.x)));
}

/* Low-resolution logits: one thread per (prompt, pixel); the pixel's 32
 * channels are 8 float4 loads, the prompt's 96 hypernetwork weights are
 * read through the cache. out [P][3][npix]. */
__global__ __launch_bounds__(256) void k_mask_logits(const float *__restrict__ U,
                                                     const float *__restrict__ hyper,
                                                     float *__restrict__ out,
                                                     int npix, long total)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= total)
        return;
    const long p = gid / npix, pix = gid - p * npix;
    const f32x4 *u = (const f32x4 *)(U + gid * 32);
    const f32x4 *h = (const f32x4 *)(hyper + p * 96);
    f32x4 uv[8];

    for (int i = 0; i < 8; i++)
        uv[i] = u[i];
    for (int k = 0; k < 3; k++) {
        const f32x4 *hk = h + 8 * k;
        const float d0 = ((dot4f(uv[0], hk[0]) + dot4f(uv[1], hk[1])) + dot4f(uv[2], hk[2])) +
                         dot4f(uv[3], hk[3]);
        const float d1 = ((dot4f(uv[4], hk[4]) + dot4f(uv[5], hk[5])) + dot4f(uv[6], hk[6])) +
                         dot4f(uv[7], hk[7]);

        out[(p * 3 + k) * npix + pix] = d0 + d1;
    }
}

extern "C" int launch_mask_logits(const float *U, const float *hyper,
                                  float *out, int P, int npix, void *stream)
{
    const long total = (long)P * npix;

    if (total <= 0)
        return hipSuccess;
    if (((uintptr_t)U | (uintptr_t)hyper) & 15)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_mask_logits, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, (hipStream_t)stream, U, hyper, out, npix,
                       total);
    return hipGetLastError();
}

/* PyTorch bilinear source coordinate, align_corners = False. */
__device__ __forceinline__ float src_coord(float scale, int dst)
{
    const float s = scale * ((float)dst + 0.5f) - 0.5f;

    return s < 0.0f ? 0.0f : s;
}

/* Postprocessing of mask k = blockIdx.z (plane sel[k] of lowres): a
 * workgroup takes a 64 x 16 tile of the out_h x out_w crop, a thread 4
 * consecutive pixels of one row; the bilinear value, binary mask byte,
 * and the counts (v > offset, v > -offset) and bounding box of v > 0
 * reduced per wave (butterfly sums, minima and maxima over lanes), then per
 * workgroup through LDS, then one global atomic per statistic. */
__global__ __launch_bounds__(256) void k_mask_post(const float *__restrict__ lowres,
                                                   const int *__restrict__ sel,
                                                   int L, int out_h, int out_w,
                                                   float offset,
                                                   unsigned char *__restrict__ mask,
                                                   int *__restrict__ stats)
{
    __shared__ int red[4][6];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int oy = blockIdx.y * 16 + (t >> 4);
    const int ox0 = blockIdx.x * 64 + (t & 15) * 4;
    const int k = blockIdx.z;
    const float *lr = lowres + (long)sel[k] * L * L;
    int inter = 0, uni = 0, x0m = 0x7fffffff, y0m = 0x7fffffff, x1m = -1, y1m = -1;

    if (oy < out_h) {
        const float sy = src_coord((float)L / out_h, oy);
        const int y0 = (int)sy, y1 = y0 + (y0 < L - 1);
        const float ly = sy - y0;
        unsigned char *mrow = mask + ((long)k * out_h + oy) * out_w;

        for (int e = 0; e < 4; e++) {
            const int ox = ox0 + e;

            if (ox >= out_w)
                break;
            const float sx = src_coord((float)L / out_w, ox);
            const int x0 = (int)sx, x1 = x0 + (x0 < L - 1);
            const float lx = sx - x0;
            const float top = fmaf(lx, lr[y0 * L + x1], (1.0f - lx) * lr[y0 * L + x0]);
            const float bot = fmaf(lx, lr[y1 * L + x1], (1.0f - lx) * lr[y1 * L + x0]);
            const float v = fmaf(ly, bot, (1.0f - ly) * top);

            mrow[ox] = v > 0.0f;
            inter += v > offset;
            uni += v > -offset;
            if (v > 0.0f) {
                x0m = min(x0m, ox);
                y0m = min(y0m, oy);
                x1m = max(x1m, ox);
                y1m = max(y1m, oy);
            }
        }
    }
    for (int s = 32; s >= 1; s >>= 1) {
        inter += __shfl_xor(inter, s, 64);
        uni += __shfl_xor(uni, s, 64);
        x0m = min(x0m, __shfl_xor(x0m, s, 64));
        y0m = min(y0m, __shfl_xor(y0m, s, 64));
        x1m = max(x1m, __shfl_xor(x1m, s, 64));
        y1m = max(y1m, __shfl_xor(y1m, s, 64));
    }
    if (lane == 0) {
        red[w][0] = inter;
        red[w][1] = uni;
        red[w][2] = x0m;
        red[w][3] = y0m;
        red[w][4] = x1m;
        red[w][5] = y1m;
    }
    __syncthreads();
    if (t == 0) {
        for (int i = 1; i < 4; i++) {
            inter += red[i][0];
            uni += red[i][1];
            x0m = min(x0m, red[i][2]);
            y0m = min(y0m, red[i][3]);
            x1m = max(x1m, red[i][4]);
            y1m = max(y1m, red[i][5]);
        }
        int *st = stats + 6 * k;

        if (inter)
            atomicAdd(&st[0], inter);
        if (uni)
            atomicAdd(&st[1], uni);
        if (x1m >= 0) {
            atomicMin(&st[2], x0m);
            atomicMin(&st[3], y0m);
            atomicMax(&st[4], x1m);
            atomicMax(&st[5], y1m);
        }
    }
}

extern "C" int launch_mask_post(const float *lowres, const int *sel, int n,
                                int L, int out_h, int out_w, float offset,
                                unsigned char *mask, int *stats, void *stream)
{
    if (n <= 0 || out_h <= 0 || out_w <= 0)
        return hipSuccess;
    if (n > 65535 || (out_h + 15) / 16 > 65535)
        return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL(k_mask_post, dim3((out_w + 63) / 64, (out_h + 15) / 16, n),
                       dim3(256), 0, (hipStream_t)stream, lowres, sel, L,
                       out_h, out_w, offset, mask, stats);
    return hipGetLastError();
}
