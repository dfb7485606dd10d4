/* SPDX-License-Identifier: Unlicense
 *
 * Device-side helpers shared by the gfx950 kernels: vector types of the
 * MFMA builtins, bf16 / half conversions and wave64 reductions.
 */
#ifndef K_COMMON_H
#define K_COMMON_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sam3_launch.h"

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define LOG2E_F 1.4426950408889634f

/* Activations of the GEMM / LayerNorm epilogues (sam3_kernels.cl:24-26). */
#define ACT_NONE_K 0
#define ACT_GELU_K 1
#define ACT_RELU_K 2

__device__ __forceinline__ float act_k(float v, int act)
{
    if (act == ACT_GELU_K)
        return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f));
    if (act == ACT_RELU_K)
        return fmaxf(v, 0.0f);
    return v;
}

/* fp32 -> bf16 / half, round to nearest even (v_cvt_pk_bf16_f32,
 * v_cvt_f16_f32 on gfx950). */
__device__ __forceinline__ uint16_t f2bf(float x)
{
    __bf16 h = (__bf16)x;
    return __builtin_bit_cast(uint16_t, h);
}

__device__ __forceinline__ float bf2f(uint16_t v)
{
    return __builtin_bit_cast(float, (uint32_t)v << 16);
}

__device__ __forceinline__ float h2f(uint16_t v)
{
    return (float)__builtin_bit_cast(_Float16, v);
}

/* Pack two floats into one dword of two bf16, lo in bits 0-15. */
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi)
{
    bf16x2 p;

    p.x = (__bf16)lo;
    p.y = (__bf16)hi;
    return __builtin_bit_cast(uint32_t, p);
}

/* Element load of any storage type as float. */
template <typename T> __device__ __forceinline__ float ld_f(const T *p);
template <> __device__ __forceinline__ float ld_f<float>(const float *p)
{
    return *p;
}
template <> __device__ __forceinline__ float ld_f<uint16_t>(const uint16_t *p)
{
    return bf2f(*p);
}

/* Wave64 butterfly reductions (ds_swizzle / DPP chosen by the compiler). */
__device__ __forceinline__ float wave_sum(float v)
{
    for (int o = 32; o > 0; o >>= 1)
        v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
    for (int o = 32; o > 0; o >>= 1)
        v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

/* GELU(v) = v Phi(v) with erf from Abramowitz & Stegun, Handbook of
 * Mathematical Functions, formula 7.1.25: erf(z) = 1 - (a1 t + a2 t^2 +
 * a3 t^3) e^{-z^2} + eps, t = 1 / (1 + p z), z >= 0, |eps| <= 2.5e-5.
 * Written as GELU(v) = max(v, 0) - |v| (0.5 (a1 t + a2 t^2 + a3 t^3))
 * e^{-v^2 / 2} with z = |v| / sqrt 2 (v erf(v / sqrt 2) is even in v):
 * 12 instructions, 2 of them transcendental. Absolute error <= 2.6e-5
 * against the exact erf GELU, two orders below the bf16 rounding its
 * results get on the precision=bf16 path, which is the only user. */
__device__ __forceinline__ float gelu_bf16path(float v)
{
    const float av = fabsf(v);
    const float t = __builtin_amdgcn_rcpf(fmaf(0.47047f * 0.70710678118654752f, av, 1.0f));
    const float q = fmaf(fmaf(0.5f * 0.7478556f, t, 0.5f * -0.0958798f), t,
                         0.5f * 0.3480242f) * t;
    const float e = __builtin_amdgcn_exp2f((v * v) * (-0.5f * 1.4426950408889634f));

    return fmaf(-av, q * e, fmaxf(v, 0.0f));
}

/* Compute units of the current device, queried once per library (256 on
 * MI355X; 256 when the query fails). Used to size persistent grids and to
 * pick tile shapes; the host launchers call it. */
static inline int dev_cu_count(void)
{
    static int n;

    if (!n) {
        int dev = 0, c = 0;

        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) !=
                hipSuccess ||
            c < 1)
            c = 256;
        n = c;
    }
    return n;
}

/* Wave issue priority by progress through a loop of `total` steps, `done`
 * of them finished (both wave-uniform): 3 until 40 % are done, then 2, 1
 * from 65 %, 0 from 85 % (`lvl` holds the level set, -1 before the first
 * call). A SIMD otherwise favours its oldest wave, so co-resident waves
 * with equal work finish one after another and the last runs alone at a
 * fraction of the MFMA rate; with the waves that are behind issuing first,
 * the SIMD keeps all of them busy to the end. Measured on the attention
 * kernels (one box, the same operands): bf16 global 113.5 -> 109.8 us,
 * windowed 17.8 -> 16.9 us; fp32 global 1110 -> 1076 us, windowed 140.4 ->
 * 133.2 us; thresholds 25/50/75, 50/75/90 and 15/35/60 % within 1-2 %. The
 * caller resets the priority with s_setprio(0) after the loop. */
__device__ __forceinline__ void prio_by_progress(int done, int total, int &lvl)
{
    const int pc = 100 * done / total;
    const int nl = (pc >= 40) + (pc >= 65) + (pc >= 85);

    if (nl == lvl)
        return;
    lvl = nl;
    if (nl == 0)
        __builtin_amdgcn_s_setprio(3);
    else if (nl == 1)
        __builtin_amdgcn_s_setprio(2);
    else if (nl == 2)
        __builtin_amdgcn_s_setprio(1);
    else
        __builtin_amdgcn_s_setprio(0);
}

#endif /* K_COMMON_H */
