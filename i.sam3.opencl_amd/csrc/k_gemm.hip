/* SPDX-License-Identifier: Unlicense
 *
 * Batched GEMM of the reference's contract on gfx950 MFMA:
 *   C = act(alpha * A * op(B) + bias) + R     (sam3_kernels.cl:57-69)
 * batch b = blockIdx.z split as (b / nb1, b % nb1) with per-operand
 * strides, element offsets, transb for B stored N x K (the Linear weight
 * layout) or K x N, R possibly aliasing C.
 *
 * One 256-thread workgroup (4 waves, 2 x 2) computes a 128 x 128 tile of
 * C; each wave owns 64 x 64 as 2 x 2 blocks of 32 x 32 MFMA
 * accumulators (64 f32 per lane).
 *  - MODE_F32:  v_mfma_f32_32x32x2_f32; K tiles of 16 staged in LDS as
 *    [k][m] / [k][n] floats (row stride 132: conflict-free lane reads).
 *  - MODE_BF16: v_mfma_f32_32x32x16_bf16 with f32 accumulation; K tiles
 *    of 64 staged as [m][k] / [n][k] bf16 rows of 72 elements (144 B:
 *    16-lane groups of 16-byte reads hit distinct banks).
 * Operands may be float, half (B only) or bf16; they are converted while
 * being staged. Loads are 16-byte vectors when the host has checked the
 * alignment of every row start, else guarded scalar loads. Rows and
 * columns outside the matrices read as zero and are not stored.
 *
 * MFMA 32x32 lane layouts (64 lanes, l = lane, h = l / 32):
 *   A operand:  lane l holds A[l % 32][k-slice of half h]
 *   B operand:  lane l holds B[k-slice of half h][l % 32]
 *   D (16 f32): reg r of lane l is D[8 (r / 4) + 4 h + r % 4][l % 32]
 */
#include "k_common.h"

/* Up to 8 consecutive elements of type dt at base[idx], as float; the
 * first `valid` are read, the rest are zero. vec: the 8 elements are
 * 16-byte aligned (float: two 16-byte loads). */
__device__ __forceinline__ void load8(const void *base, int dt, long idx,
                                      int valid, bool vec, float f[8])
{
    if (vec && valid >= 8) {
        if (dt == DT_F32) {
            const f32x4 *p = (const f32x4 *)((const float *)base + idx);
            const f32x4 x = p[0], y = p[1];

            f[0] = x[0]; f[1] = x[1]; f[2] = x[2]; f[3] = x[3];
            f[4] = y[0]; f[5] = y[1]; f[6] = y[2]; f[7] = y[3];
        }
        else {
            const u32x4 v = *(const u32x4 *)((const uint16_t *)base + idx);

            for (int e = 0; e < 4; e++) {
                const uint16_t lo = (uint16_t)(v[e] & 0xffffu);
                const uint16_t hi = (uint16_t)(v[e] >> 16);

                f[2 * e] = dt == DT_BF16 ? bf2f(lo) : h2f(lo);
                f[2 * e + 1] = dt == DT_BF16 ? bf2f(hi) : h2f(hi);
            }
        }
        return;
    }
    for (int e = 0; e < 8; e++) {
        float v = 0.0f;

        if (e < valid) {
            if (dt == DT_F32)
                v = ((const float *)base)[idx + e];
            else if (dt == DT_BF16)
                v = bf2f(((const uint16_t *)base)[idx + e]);
            else
                v = h2f(((const uint16_t *)base)[idx + e]);
        }
        f[e] = v;
    }
}

__device__ __forceinline__ int clamp8(long n)
{
    return n <= 0 ? 0 : n >= 8 ? 8 : (int)n;
}

/* Epilogue of one 32 x 32 accumulator block at tile rows mb, cols nb0:
 * alpha, bias, activation, residual, store (store_one,
 * sam3_kernels.cl:306-319). */
__device__ __forceinline__ void store_block(const gemm_desc &d, void *C,
                                           const void *R, f32x16 acc, int mb,
                                           int ncol)
{
    const int l = threadIdx.x & 63, h = l >> 5;

    if (ncol >= d.N)
        return;
    for (int r = 0; r < 16; r++) {
        const int m = mb + 8 * (r >> 2) + 4 * h + (r & 3);
        float v;
        long idx;

        if (m >= d.M)
            continue;
        idx = (long)m * d.ldc + ncol;
        v = d.alpha * acc[r];
        if (d.bias)
            v += d.bias[ncol];
        v = act_k(v, d.act);
        if (d.cdt == DT_F32) {
            if (R)
                v += ((const float *)R)[idx];
            ((float *)C)[idx] = v;
        }
        else {
            if (R)
                v += bf2f(((const uint16_t *)R)[idx]);
            ((uint16_t *)C)[idx] = f2bf(v);
        }
    }
}

/* Operand base of batch b (bytes depend on the element type). */
__device__ __forceinline__ long batch_off(long off, long s0, long s1, long b0,
                                          long b1)
{
    return off + b0 * s0 + b1 * s1;
}

template <bool TRANSB>
__global__ __launch_bounds__(256) void k_gemm_f32(gemm_desc d, int avec,
                                                  int bvec)
{
    __shared__ float As[16][132];
    __shared__ float Bs[16][132];
    const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5,
              l32 = l & 31;
    const int wm = w >> 1, wn = w & 1;
    const int n0 = blockIdx.x * 128, m0 = blockIdx.y * 128;
    const long b0 = blockIdx.z / d.nb1, b1 = blockIdx.z % d.nb1;
    const long abase = batch_off(d.aoff, d.sa0, d.sa1, b0, b1);
    const long bbase = batch_off(d.boff, d.sb0, d.sb1, b0, b1);
    const long cbase = batch_off(d.coff, d.sc0, d.sc1, b0, b1);
    const long rbase = batch_off(d.roff, d.sc0, d.sc1, b0, b1);
    f32x16 acc[2][2];

    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++)
                acc[i][j][r] = 0.0f;

    for (int k0 = 0; k0 < d.K; k0 += 16) {
        float f[8];

        {
            const int row = t >> 1, kk = (t & 1) * 8;
            const int gm = m0 + row, gk = k0 + kk;

            load8(d.A, d.adt, abase + (long)gm * d.lda + gk, gm < d.M ? clamp8(d.K - gk) : 0,
                  avec, f);
            for (int e = 0; e < 8; e++)
                As[kk + e][row] = f[e];
        }
        if (TRANSB) {
            const int row = t >> 1, kk = (t & 1) * 8;
            const int gn = n0 + row, gk = k0 + kk;

            load8(d.B, d.bdt, bbase + (long)gn * d.ldb + gk,
                  gn < d.N ? clamp8(d.K - gk) : 0, bvec, f);
            for (int e = 0; e < 8; e++)
                Bs[kk + e][row] = f[e];
        }
        else {
            const int kr = t >> 4, ns = (t & 15) * 8;
            const int gk = k0 + kr, gn = n0 + ns;

            load8(d.B, d.bdt, bbase + (long)gk * d.ldb + gn,
                  gk < d.K ? clamp8(d.N - gn) : 0, bvec, f);
            for (int e = 0; e < 8; e++)
                Bs[kr][ns + e] = f[e];
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 8; s++) {
            const float a0 = As[2 * s + h][wm * 64 + l32];
            const float a1 = As[2 * s + h][wm * 64 + 32 + l32];
            const float c0 = Bs[2 * s + h][wn * 64 + l32];
            const float c1 = Bs[2 * s + h][wn * 64 + 32 + l32];

            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, c0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0, c1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, c0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1, c1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
    }

    {
        char *C = (char *)d.C + cbase * (d.cdt == DT_F32 ? 4 : 2);
        const char *R = d.R ? (const char *)d.R + rbase * (d.cdt == DT_F32 ? 4 : 2)
                            : NULL;

        for (int i = 0; i < 2; i++)
            for (int j = 0; j < 2; j++)
                store_block(d, C, R, acc[i][j], m0 + wm * 64 + i * 32,
                            n0 + wn * 64 + j * 32 + l32);
    }
}

template <bool TRANSB>
__global__ __launch_bounds__(256) void k_gemm_bf16(gemm_desc d, int avec,
                                                   int bvec)
{
    __shared__ __attribute__((aligned(16))) uint16_t As[128][72];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[128][72];
    const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5,
              l32 = l & 31;
    const int wm = w >> 1, wn = w & 1;
    const int n0 = blockIdx.x * 128, m0 = blockIdx.y * 128;
    const long b0 = blockIdx.z / d.nb1, b1 = blockIdx.z % d.nb1;
    const long abase = batch_off(d.aoff, d.sa0, d.sa1, b0, b1);
    const long bbase = batch_off(d.boff, d.sb0, d.sb1, b0, b1);
    const long cbase = batch_off(d.coff, d.sc0, d.sc1, b0, b1);
    const long rbase = batch_off(d.roff, d.sc0, d.sc1, b0, b1);
    f32x16 acc[2][2];

    for (int i = 0; i < 2; i++)
        for (int j = 0; j < 2; j++)
            for (int r = 0; r < 16; r++)
                acc[i][j][r] = 0.0f;

    for (int k0 = 0; k0 < d.K; k0 += 64) {
        float f[8];

#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = t + 256 * j, row = c >> 3, kk = (c & 7) * 8;
            const int gm = m0 + row, gk = k0 + kk;
            u32x4 v;

            load8(d.A, d.adt, abase + (long)gm * d.lda + gk,
                  gm < d.M ? clamp8(d.K - gk) : 0, avec, f);
            for (int e = 0; e < 4; e++)
                v[e] = pack_bf16x2(f[2 * e], f[2 * e + 1]);
            *(u32x4 *)&As[row][kk] = v;
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int c = t + 256 * j;

            if (TRANSB) {
                const int row = c >> 3, kk = (c & 7) * 8;
                const int gn = n0 + row, gk = k0 + kk;
                u32x4 v;

                load8(d.B, d.bdt, bbase + (long)gn * d.ldb + gk,
                      gn < d.N ? clamp8(d.K - gk) : 0, bvec, f);
                for (int e = 0; e < 4; e++)
                    v[e] = pack_bf16x2(f[2 * e], f[2 * e + 1]);
                *(u32x4 *)&Bs[row][kk] = v;
            }
            else {
                const int kr = c >> 4, ns = (c & 15) * 8;
                const int gk = k0 + kr, gn = n0 + ns;

                load8(d.B, d.bdt, bbase + (long)gk * d.ldb + gn,
                      gk < d.K ? clamp8(d.N - gn) : 0, bvec, f);
                for (int e = 0; e < 8; e++)
                    Bs[ns + e][kr] = f2bf(f[e]);
            }
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const bf16x8 a0 = *(const bf16x8 *)&As[wm * 64 + l32][16 * s + 8 * h];
            const bf16x8 a1 = *(const bf16x8 *)&As[wm * 64 + 32 + l32][16 * s + 8 * h];
            const bf16x8 c0 = *(const bf16x8 *)&Bs[wn * 64 + l32][16 * s + 8 * h];
            const bf16x8 c1 = *(const bf16x8 *)&Bs[wn * 64 + 32 + l32][16 * s + 8 * h];

            acc[0][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, c0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a0, c1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, c0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a1, c1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
    }

    {
        char *C = (char *)d.C + cbase * (d.cdt == DT_F32 ? 4 : 2);
        const char *R = d.R ? (const char *)d.R + rbase * (d.cdt == DT_F32 ? 4 : 2)
                            : NULL;

        for (int i = 0; i < 2; i++)
            for (int j = 0; j < 2; j++)
                store_block(d, C, R, acc[i][j], m0 + wm * 64 + i * 32,
                            n0 + wn * 64 + j * 32 + l32);
    }
}

/* 16-byte alignment of every 8-element load: offset, batch strides and
 * leading dimension are multiples of the elements per 16 bytes (the
 * buffers themselves come from hipMalloc, 256-byte aligned). */
/* Small GEMMs (a few 128 x 128 tiles: the decoder's per-token linears of
 * 8 P rows): a workgroup per 32 x 32 tile whose 4 waves split K four
 * ways; no operand staging: each lane loads its MFMA fragments straight
 * from memory (A row m = lane % 32 and B row n = lane % 32 of the Linear
 * weight, 8 consecutive k per lane half), bf16 MFMA with f32 accumulation;
 * the four partial tiles are summed through LDS, then the usual epilogue.
 * Unbatched, B stored N x K, K % 64 == 0, 16-byte aligned operand rows
 * (checked by the launcher). Rows / columns past M / N read row 0 and are
 * not stored. */
/* Eight consecutive elements of an operand of element type DT (a
 * compile-time constant, so that the loads of a batch of k steps are
 * issued together) as an MFMA fragment. */
template <int DT> __device__ __forceinline__ bf16x8 frag8(const void *base, long idx)
{
    bf16x8 r;

    if constexpr (DT == DT_F32) {
        const f32x4 *p = (const f32x4 *)((const float *)base + idx);
        const f32x4 x = p[0], y = p[1];

        for (int e = 0; e < 4; e++) {
            r[e] = (__bf16)x[e];
            r[4 + e] = (__bf16)y[e];
        }
    }
    else if constexpr (DT == DT_BF16) {
        r = *(const bf16x8 *)((const uint16_t *)base + idx);
    }
    else {
        const u32x4 v = *(const u32x4 *)((const uint16_t *)base + idx);

        for (int e = 0; e < 4; e++) {
            r[2 * e] = (__bf16)h2f((uint16_t)(v[e] & 0xffffu));
            r[2 * e + 1] = (__bf16)h2f((uint16_t)(v[e] >> 16));
        }
    }
    return r;
}

/* Batches of SMALL_BATCH k steps: all their loads, then their MFMAs, so a
 * wave waits for memory once per batch (once in all for K <= 512). */
#define SMALL_BATCH 8

template <int ADT, int BDT>
__global__ __launch_bounds__(256) void k_gemm_small(gemm_desc d)
{
    __shared__ float red[3][16][64];
    const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5, l32 = l & 31;
    const int m0 = blockIdx.y * 32, n0 = blockIdx.x * 32;
    const int m = m0 + l32 < d.M ? m0 + l32 : 0, n = n0 + l32 < d.N ? n0 + l32 : 0;
    const int kq = d.K / 4; /* a multiple of 16 */
    const int nst = kq / 16;
    const long arow = d.aoff + (long)m * d.lda + w * kq + 8 * h;
    const long brow = d.boff + (long)n * d.ldb + w * kq + 8 * h;
    const bool f32c = d.cdt == DT_F32;
    const void *R = d.R ? (const void *)((f32c ? 4 : 2) * d.roff + (const char *)d.R) : nullptr;
    f32x16 acc = {}, res = {};
    float bn = 0.0f;

    /* Wave 0 stores the tile: its bias and residual loads go out with the
     * operand loads instead of after the reduction. */
    if (w == 0 && n0 + l32 < d.N) {
        if (d.bias)
            bn = d.bias[n0 + l32];
        if (R)
            for (int r = 0; r < 16; r++) {
                const int mr = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
                const long idx = (long)(mr < d.M ? mr : 0) * d.ldc + n0 + l32;

                res[r] = f32c ? ((const float *)R)[idx] : bf2f(((const uint16_t *)R)[idx]);
            }
    }

    for (int s0 = 0; s0 < nst; s0 += SMALL_BATCH) {
        bf16x8 a[SMALL_BATCH], b[SMALL_BATCH];

#pragma unroll
        for (int u = 0; u < SMALL_BATCH; u++)
            if (s0 + u < nst) {
                a[u] = frag8<ADT>(d.A, arow + 16 * (s0 + u));
                b[u] = frag8<BDT>(d.B, brow + 16 * (s0 + u));
            }
#pragma unroll
        for (int u = 0; u < SMALL_BATCH; u++)
            if (s0 + u < nst)
                /* D = A B^T tile: rows m (A operand), columns n (B operand). */
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[u], b[u], acc, 0, 0, 0);
    }
    if (w > 0)
        for (int r = 0; r < 16; r++)
            red[w - 1][r][l] = acc[r];
    __syncthreads();
    if (w > 0)
        return;
    for (int r = 0; r < 16; r++)
        acc[r] += (red[0][r][l] + red[1][r][l]) + red[2][r][l];
    void *C = (char *)d.C + (f32c ? 4 : 2) * d.coff;

    if (n0 + l32 >= d.N)
        return;
    /* store_block's epilogue with the preloaded bias and residual. */
    for (int r = 0; r < 16; r++) {
        const int mr = m0 + 8 * (r >> 2) + 4 * h + (r & 3);
        const long idx = (long)mr * d.ldc + n0 + l32;
        float v = act_k(d.alpha * acc[r] + bn, d.act);

        if (mr >= d.M)
            continue;
        if (R)
            v += res[r];
        if (f32c)
            ((float *)C)[idx] = v;
        else
            ((uint16_t *)C)[idx] = f2bf(v);
    }
}

template <int ADT>
static void launch_small_b(const gemm_desc *d, dim3 grid, hipStream_t s)
{
    if (d->bdt == DT_F32)
        hipLaunchKernelGGL((k_gemm_small<ADT, DT_F32>), grid, dim3(256), 0, s, *d);
    else if (d->bdt == DT_BF16)
        hipLaunchKernelGGL((k_gemm_small<ADT, DT_BF16>), grid, dim3(256), 0, s, *d);
    else
        hipLaunchKernelGGL((k_gemm_small<ADT, DT_F16>), grid, dim3(256), 0, s, *d);
}

static int vec_ok(int dt, long off, long s0, long s1, int ld)
{
    const long q = dt == DT_F32 ? 4 : 8;

    return off % q == 0 && s0 % q == 0 && s1 % q == 0 && ld % q == 0;
}

extern "C" int launch_gemm(const gemm_desc *d, void *stream)
{
    const dim3 grid((d->N + 127) / 128, (d->M + 127) / 128, d->nb);
    const int avec = vec_ok(d->adt, d->aoff, d->sa0, d->sa1, d->lda);
    const int bvec = vec_ok(d->bdt, d->boff, d->sb0, d->sb1, d->ldb);
    hipStream_t s = (hipStream_t)stream;

    if (d->nb > 65535 || grid.y > 65535)
        return hipErrorInvalidConfiguration;
    {
        const int r = launch_gemm_nt(d, stream);

        if (r != -1)
            return r;
    }
    if (d->unpart_ws > 0)
        return hipErrorInvalidValue; /* row remap: NT kernel only */
    if (d->mode == MODE_BF16 && d->transb && d->nb == 1 && d->K % 64 == 0 &&
        avec && bvec && (long)grid.x * grid.y <= 64 &&
        ((uintptr_t)d->A & 15) == 0 && ((uintptr_t)d->B & 15) == 0) {
        const dim3 sg((d->N + 31) / 32, (d->M + 31) / 32);

        /* A is never half (the gemm wrapper rejects it). */
        if (d->adt == DT_F32)
            launch_small_b<DT_F32>(d, sg, s);
        else
            launch_small_b<DT_BF16>(d, sg, s);
        return hipGetLastError();
    }
    if (d->mode == MODE_BF16) {
        if (d->transb)
            hipLaunchKernelGGL(k_gemm_bf16<true>, grid, dim3(256), 0, s, *d,
                               avec, bvec);
        else
            hipLaunchKernelGGL(k_gemm_bf16<false>, grid, dim3(256), 0, s, *d,
                               avec, bvec);
    }
    else {
        if (d->transb)
            hipLaunchKernelGGL(k_gemm_f32<true>, grid, dim3(256), 0, s, *d,
                               avec, bvec);
        else
            hipLaunchKernelGGL(k_gemm_f32<false>, grid, dim3(256), 0, s, *d,
                               avec, bvec);
    }
    return hipGetLastError();
}
