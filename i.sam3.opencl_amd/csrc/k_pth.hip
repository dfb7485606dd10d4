/* SPDX-License-Identifier: Unlicense
 *
 * Checkpoint tensor conversion on gfx950: a storage span copied raw into
 * device memory becomes the C-order tensor in the element type the model
 * keeps (float32, half or bfloat16), gathering strided views on the way.
 * Replaces the host-side conversion and gather of the reference's
 * pth_read_f32 / pth_read_c64 (pth_loader.c:915-1012) followed by
 * ocl_upload_weight's float -> half rounding (ocl_backend.c:520-587).
 */
#include "k_common.h"

#include <hip/hip_fp16.h>

/* Storage element types, enum pth_dtype of pth_loader.h. */
#define SRC_F32 0
#define SRC_F16 1
#define SRC_BF16 2
#define SRC_C64 3

struct pth_geom {
    int ndim;
    long long shape[8], stride[8];
};

__device__ __forceinline__ float src_value(const unsigned char *__restrict__ s,
                                           long long off, int sdt)
{
    if (sdt == SRC_F32 || sdt == SRC_C64)
        return ((const float *)s)[off];
    const unsigned short h = ((const unsigned short *)s)[off];
    if (sdt == SRC_F16)
        return (float)__ushort_as_half(h);
    return __uint_as_float((unsigned)h << 16);
}

/* bfloat16 of x, round to nearest even; NaN stays a (quiet) NaN. */
__device__ __forceinline__ unsigned short to_bf16_bits(float x)
{
    const unsigned u = __float_as_uint(x);

    if ((u & 0x7fffffffu) > 0x7f800000u)
        return (unsigned short)((u >> 16) | 0x40u);
    return (unsigned short)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* One thread per output element (a complex element gives two floats),
 * grid-stride over n. contiguous: element i is storage element i; else
 * the C-order index is split over the dimensions and dotted with the
 * strides. */
__global__ __launch_bounds__(256) void k_pth_convert(
    const unsigned char *__restrict__ src, int sdt, void *__restrict__ dst,
    int ddt, long long n, int contiguous, pth_geom g)
{
    const long long step = (long long)gridDim.x * 256;

    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
         i += step) {
        long long off = i;

        if (!contiguous) {
            long long r = i;

            off = 0;
            for (int d = g.ndim - 1; d >= 0; d--) {
                const long long q = r / g.shape[d];

                off += (r - q * g.shape[d]) * g.stride[d];
                r = q;
            }
        }
        if (sdt == SRC_C64) {
            ((float *)dst)[2 * i] = src_value(src, 2 * off, sdt);
            ((float *)dst)[2 * i + 1] = src_value(src, 2 * off + 1, sdt);
            continue;
        }
        const float v = src_value(src, off, sdt);

        if (ddt == DT_F32)
            ((float *)dst)[i] = v;
        else if (ddt == DT_F16)
            ((__half *)dst)[i] = __float2half_rn(v);
        else
            ((unsigned short *)dst)[i] = to_bf16_bits(v);
    }
}

extern "C" int launch_pth_convert(const void *src, int sdt, void *dst,
                                  int ddt, long long n, int ndim,
                                  const long *shape, const long *stride,
                                  int contiguous, void *stream)
{
    pth_geom g;
    long long blocks;

    if (n <= 0)
        return hipSuccess;
    if (ndim < 0 || ndim > 8 || sdt < SRC_F32 || sdt > SRC_C64 ||
        ddt < DT_F32 || ddt > DT_BF16 || (sdt == SRC_C64 && ddt != DT_F32))
        return hipErrorInvalidValue;
    g.ndim = ndim;
    for (int d = 0; d < 8; d++) {
        g.shape[d] = d < ndim ? shape[d] : 1;
        g.stride[d] = d < ndim ? stride[d] : 0;
    }
    blocks = (n + 255) / 256;
    if (blocks > 8192)
        blocks = 8192;
    hipLaunchKernelGGL(k_pth_convert, dim3((unsigned)blocks), dim3(256), 0,
                       (hipStream_t)stream, (const unsigned char *)src, sdt,
                       dst, ddt, n, contiguous, g);
    return hipGetLastError();
}
