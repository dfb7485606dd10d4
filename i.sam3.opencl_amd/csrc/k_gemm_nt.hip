/* SPDX-License-Identifier: Unlicense
 *
 * bf16 "NT" GEMM of the precision=bf16 path on gfx950:
 *   C = act(alpha * A B^T + bias) + R      (sam3_kernels.cl:57-69)
 * with A [M][K] bf16 activations and B [N][K] bf16 weight rows (the
 * Linear layout, transb), float or bf16 C, R possibly aliasing C. This is
 * the shape of every projection of the image encoder (QKV 1024 -> 3072,
 * attention projection 1024 -> 1024, MLP 1024 -> 4096 -> 1024 over the
 * 5184 tokens), so it gets its own kernel; other shapes and types take
 * the general kernels of k_gemm.hip.
 *
 * A workgroup owns a BM x BN tile of C; each wave a WM x WN sub-tile as
 * (WM / 32) x (WN / 32) blocks of 32 x 32 v_mfma_f32_32x32x16_bf16
 * accumulators (the AGPRs hold them when they exceed the VGPRs). K moves
 * in stages of 64: the BM + BN rows of the stage (128 bytes each) go HBM
 * -> LDS with asynchronous global_load_lds_dwordx4 (no staging registers,
 * no conversion) into one of two slots, 16-byte chunk c of row r stored
 * at chunk c ^ ((r >> 1) & 7) so that the MFMA operand reads (16 bytes of
 * one chunk from 16 different rows per 16-lane group) hit distinct
 * banks. One barrier per stage hands a slot from the readers back to the
 * copy of the stage after next.
 *
 * LDS operand bytes per MFMA: (WM + WN) / 32 fragments of 1 KiB per
 * WM WN / 1024 MFMAs: 0.75 KiB for 128 x 64, 1 KiB for 64 x 64, against
 * the 1 KiB per MFMA the LDS can deliver to four SIMDs at the MFMA peak.
 */
#include "k_common.h"

#include <type_traits>

#define NT_KS 64 /* K per stage */

/* XCDs (L2 domains) of an MI355X. */
#define NT_NXCD 8

__device__ __forceinline__ int nt_swz(int row, int chunk)
{
    return 8 * (chunk ^ ((row >> 1) & 7));
}

/* Asynchronous 16-byte global -> LDS copy (global_load_lds_dwordx4, saddr
 * form): lane i of the wave reads base + voff_i and writes lds + 16 i
 * (base and lds wave-uniform, lds via M0). Inline assembly so the compiler
 * does not wait for it before unrelated LDS reads; the kernel waits
 * itself (s_waitcnt vmcnt(0)) before the barrier that publishes the slot.
 */
__device__ __forceinline__ void nt_g2lds16_s(const void *base, unsigned voff, unsigned lds)
{
    asm volatile("s_mov_b32 m0, %0\n\t"
                 "global_load_lds_dwordx4 %1, %2"
                 :
                 : "s"(lds), "v"(voff), "s"(base)
                 : "memory", "m0");
}

/* Store of a 128 x 128 tile of a QKV projection as packed attention
 * operands (gemm_desc pack_*), from the float tile E [128][132] in LDS:
 * the tile's columns are two 64-wide heads of one third. Wave w takes
 * head w / 2 and tile rows 64 (w % 2) .. +63, one 64-key block of one
 * unit (pack_N and the row count are multiples of 64), in eight passes of
 * eight rows: lane l handles 16-byte chunk l % 8 of row l / 8, so eight
 * lanes write one whole 128-byte output row. q / k: RoPE on the chunk's
 * four pairs (2j, 2j + 1), q times scale log2 e, bf16; for k the block's
 * largest |k| over the bf16 values, rounded up by 2^-10. v (V^T rows of
 * 64 keys): lane l takes channel 8 pass + l / 8 and keys 8 (l % 8) .. +7.
 * The arithmetic is k_qkv_pack's, so the operands are the same bits. */
__device__ __forceinline__ void nt_pack_rope(const gemm_desc &d, int m0, int n0, int t,
                                             float2 (&rot)[8][4])
{
    const int third = n0 / d.pack_E, w = t >> 6, l = t & 63, mw = m0 + (w & 1) * 64;

    if (third < 2 && d.pack_rope && mw < d.M)
        for (int pass = 0; pass < 8; pass++) {
            const int p = (mw + 8 * pass + (l >> 3)) % d.pack_N;
            const float4 *src = (const float4 *)((const float2 *)d.pack_rope +
                                                 (long)(p % d.pack_npos) * 32 + 4 * (l & 7));
            const float4 r0 = src[0], r1 = src[1];

            rot[pass][0] = make_float2(r0.x, r0.y);
            rot[pass][1] = make_float2(r0.z, r0.w);
            rot[pass][2] = make_float2(r1.x, r1.y);
            rot[pass][3] = make_float2(r1.z, r1.w);
        }
}

__device__ void nt_pack_store(const gemm_desc &d, const float *E, int m0, int n0, int t,
                              const float2 (&rot)[8][4])
{
    constexpr int LD = 132;
    const int Np = d.pack_N, heads = d.pack_E / 64;
    const int third = n0 / d.pack_E, head0 = (n0 - third * d.pack_E) / 64;
    const int w = t >> 6, l = t & 63, hh = w >> 1, rbase = (w & 1) * 64;
    const int mw = m0 + rbase, c8 = l & 7, r8 = l >> 3;

    if (mw >= d.M)
        return;
    const int win = mw / Np, p0 = mw - win * Np;
    const long unit = (long)win * heads + head0 + hh;

    if (third < 2) {
        uint16_t *dst = (uint16_t *)(third == 0 ? d.pack_q16 : d.pack_k16) +
                        (unit * Np + p0) * 64 + 8 * c8;
        float mx = 0.0f; /* largest row |k|^2 seen, of the bf16 values */

        for (int pass = 0; pass < 8; pass++) {
            const int row = 8 * pass + r8;
            const float *src = E + (rbase + row) * LD + hh * 64 + 8 * c8;
            const f32x4 x0 = *(const f32x4 *)src, x1 = *(const f32x4 *)(src + 4);
            float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            float ps = 0.0f;
            u32x4 pk;

            if (d.pack_rope)
                for (int j = 0; j < 4; j++) {
                    const float2 r = rot[pass][j];
                    const float a = v[2 * j], b = v[2 * j + 1];

                    v[2 * j] = fmaf(a, r.x, -(b * r.y));
                    v[2 * j + 1] = fmaf(a, r.y, b * r.x);
                }
            if (third == 0)
                for (int e = 0; e < 8; e++)
                    v[e] *= d.pack_scale * LOG2E_F;
            for (int e = 0; e < 4; e++) {
                pk[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
                if (third == 1) {
                    /* Squares of the two bf16 values as floats, with FMAs:
                     * v_dot2_f32_bf16 would wait for the MFMA pipe, busy
                     * with the other workgroup's K loop. */
                    const uint32_t u = pk[e];
                    const float lo = __builtin_bit_cast(float, u << 16),
                                hi = __builtin_bit_cast(float, u & 0xffff0000u);

                    ps = fmaf(hi, hi, fmaf(lo, lo, ps));
                }
            }
            *(u32x4 *)(dst + (long)row * 64) = pk;
            if (third == 1) {
                /* The row's |k|^2: its 8 lanes' chunk sums. */
                ps += __shfl_xor(ps, 1, 64);
                ps += __shfl_xor(ps, 2, 64);
                ps += __shfl_xor(ps, 4, 64);
                mx = fmaxf(mx, ps);
            }
        }
        if (third == 1) {
            mx = wave_max(mx);
            if (l == 0)
                d.pack_knorm[unit * (Np / 64) + p0 / 64] = sqrtf(mx) * (1.0f + 0x1p-10f);
        }
    }
    else {
        /* E's V tile is staged with columns XOR 4 ((row / 8) % 8) (see
         * the staging in k_gemm_nt): the eight rows 8 c8 .. +7 a lane reads
         * for one channel then sit on banks apart from the other lanes'
         * rows instead of all on one bank (row stride 132 floats, 8 x 132
         * = 0 mod 32 banks). */
        for (int pass = 0; pass < 8; pass++) {
            const int ch = 8 * pass + r8;
            const float *src = E + (rbase + 8 * c8) * LD + ((hh * 64 + ch) ^ (c8 << 2));
            u32x4 pk;

            for (int e = 0; e < 4; e++)
                pk[e] = pack_bf16x2(src[(2 * e) * LD], src[(2 * e + 1) * LD]);
            *(u32x4 *)((uint16_t *)d.pack_vt16 + (unit * 64 + ch) * Np + p0 + 8 * c8) = pk;
        }
    }
}

/* Epilogue activation of the bf16 products: GELU through gelu_bf16path
 * (erf within 2.5e-5, below the bf16 rounding of fc1's stored output; its
 * short straight-line code leaves the K loop more registers than the
 * library erff). */
__device__ __forceinline__ float nt_act(float v, int act)
{
    if (act == ACT_GELU_K)
        return gelu_bf16path(v);
    return act == ACT_RELU_K ? fmaxf(v, 0.0f) : v;
}

template <int BM, int BN, int WM, int WN>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, 1) void
k_gemm_nt(gemm_desc d)
{
    /* Epilogue rows staged per pass, and the LDS that needs. */
    constexpr int EPI_ROWS = BM <= 128 ? BM : 64;
    constexpr int EPI_BYTES = EPI_ROWS * (BN + 4) * 4;
    constexpr int NW = (BM / WM) * (BN / WN);
    constexpr int NA = WM / 32;             /* 32-row blocks per wave */
    constexpr int NB = WN / 32;             /* 32-column blocks per wave */
    constexpr int ROWS = BM + BN;           /* LDS rows per stage */
    constexpr int SLOT_BYTES = ROWS * NT_KS * 2;
    constexpr int LPW = ROWS / (8 * NW);    /* copies per wave per stage */
    constexpr int LDS_BYTES = 2 * SLOT_BYTES > EPI_BYTES ? 2 * SLOT_BYTES : EPI_BYTES;
    /* Two operand slots during the K loop, the output tile in the
     * epilogue (which may need a little more). */
    __shared__ __attribute__((aligned(16))) uint16_t S_raw[LDS_BYTES / 2];
    const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5,
              l32 = l & 31;
    const int wm = w / (BN / WN), wn = w % (BN / WN);
    const int tiles_n = (d.N + BN - 1) / BN;
    const long total = (long)tiles_n * ((d.M + BM - 1) / BM);
    const long per_xcd = (total + NT_NXCD - 1) / NT_NXCD;
    /* Workgroup g runs on XCD g % 8: give each XCD a contiguous run of
     * tiles (row-major over the tile grid), so its L2 sees the same A rows
     * and a window of B rows. */
    const long tile = (blockIdx.x % NT_NXCD) * per_xcd + blockIdx.x / NT_NXCD;
    if (tile >= total)
        return;
    const int m0 = (int)(tile / tiles_n) * BM, n0 = (int)(tile % tiles_n) * BN;
    /* The tile's first A and B rows: wave-uniform bases (SGPRs) that the
     * K loop advances by 128 bytes per stage. */
    const char *Ab = (const char *)((const uint16_t *)d.A + d.aoff + (long)m0 * d.lda);
    const char *Bb = (const char *)((const uint16_t *)d.B + d.boff + (long)n0 * d.ldb);
    const int nk = d.K / NT_KS;
    const int wu = __builtin_amdgcn_readfirstlane(w);
    f32x16 acc[NA][NB];
    unsigned goff[LPW];

#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int j = 0; j < NB; j++)
            acc[i][j] = (f32x16){};

    /* Copy j of wave w fills stage rows 8 (w LPW + j) .. +7; lane i lands
     * on row + i / 8, physical chunk i % 8 and so fetches logical chunk
     * (i % 8) ^ ((row >> 1) & 7). Rows past M or N read the last row
     * (their products are never stored). Byte offsets from the tile's
     * first row of A or B. */
    for (int j = 0; j < LPW; j++) {
        const int row = 8 * (w * LPW + j) + (l >> 3);
        const int chunk = (l & 7) ^ ((row >> 1) & 7);

        if (row < BM)
            goff[j] = 2u * ((unsigned)(min(m0 + row, d.M - 1) - m0) * d.lda + 8 * chunk);
        else
            goff[j] = 2u * ((unsigned)(min(n0 + row - BM, d.N - 1) - n0) * d.ldb + 8 * chunk);
    }
    const unsigned lds0 = (unsigned)(uintptr_t)S_raw + 1024u * LPW * wu;
    auto load_stage = [&](int ks, int slot) {
        for (int j = 0; j < LPW; j++) {
            /* Whether copy j is of A or of B is the same for the wave. */
            const bool isa = 8 * (wu * LPW + j) < BM;

            nt_g2lds16_s((isa ? Ab : Bb) + 128L * ks, goff[j],
                         lds0 + (unsigned)SLOT_BYTES * slot + 1024u * j);
        }
    };
    /* Byte offsets of this lane's MFMA operand fragments in a slot, per
     * 16-wide K step s: A rows wm WM + 32 i + l32 and B rows BM + wn WN +
     * 32 j + l32 (i, j add 4096 B each); the swizzle depends only on row
     * bits 1..3, which the 32-row blocks leave alone. */
    unsigned aro[4], bro[4];
    for (int s4 = 0; s4 < 4; s4++) {
        const int ra = wm * WM + l32, rb = BM + wn * WN + l32;

        aro[s4] = 2u * (ra * NT_KS + nt_swz(ra, 2 * s4 + h));
        bro[s4] = 2u * (rb * NT_KS + nt_swz(rb, 2 * s4 + h));
    }
    const char *Sb = (const char *)S_raw;
    /* One K stage from slot `slot` (a constant: the loop is unrolled by
     * two, so every fragment address is a register plus an immediate). */
    auto stage = [&](int ks, auto slot_c) {
        constexpr int slot = decltype(slot_c)::value;

        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (ks + 1 < nk)
            load_stage(ks + 1, slot ^ 1);
#pragma unroll
        for (int s4 = 0; s4 < NT_KS / 16; s4++) {
            bf16x8 a[NA], b[NB];

#pragma unroll
            for (int i = 0; i < NA; i++)
                a[i] = *(const bf16x8 *)(Sb + SLOT_BYTES * slot + 4096 * i + aro[s4]);
#pragma unroll
            for (int j = 0; j < NB; j++)
                b[j] = *(const bf16x8 *)(Sb + SLOT_BYTES * slot + 4096 * j + bro[s4]);
#pragma unroll
            for (int i = 0; i < NA; i++)
#pragma unroll
                for (int j = 0; j < NB; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };

    /* 128 x 64 tiles are taken where 128 x 128 would give fewer than two
     * per CU: the launch is one round of three workgroups per CU, whose
     * waves then issue by progress (prio_by_progress: those behind first)
     * rather than oldest first, so that a CU's workgroups finish together
     * (projection 450 -> 466, fc2 690 -> 708 TFLOP/s; the multi-round
     * 128 x 128 launches gain nothing from it). */
    constexpr bool PRIO = BM == 128 && BN == 64;
    int lvl = -1;

    load_stage(0, 0);
    for (int ks = 0; ks + 1 < nk; ks += 2) {
        if (PRIO)
            prio_by_progress(ks, nk, lvl);
        stage(ks, std::integral_constant<int, 0>());
        stage(ks + 1, std::integral_constant<int, 1>());
    }
    if (nk & 1)
        stage(nk - 1, std::integral_constant<int, 0>());
    if (PRIO)
        __builtin_amdgcn_s_setprio(0);

    /* Epilogue (store_one, sam3_kernels.cl:306-319), through LDS: in
     * chunks of 64 rows, the waves owning the rows write alpha acc + bias
     * (activation applied) into the freed operand slots as a row-major
     * float tile (row stride BN + 4: the two 32-lane halves of a write
     * fall on different banks), then every thread takes four consecutive
     * columns of a row: one 16-byte LDS read, the residual and the store
     * as 16-byte (float) or 8-byte (bf16) accesses. With the window row
     * remap each row's grid token costs three divisions. */
    constexpr int CR = EPI_ROWS, LD = BN + 4, T = NW * 64, RPI = T * 4 / BN;
    float *E = (float *)S_raw;
    const bool vec = d.ldc % 4 == 0 && d.coff % 4 == 0 && d.roff % 4 == 0;
    float2 rot[8][4];

    if constexpr (BM == 128 && BN == 128) {
        if (d.pack_N > 0)
            nt_pack_rope(d, m0, n0, t, rot);
    }

    /* The V third of a packed QKV tile stages its columns XOR 4 ((row / 8)
     * % 8) for the V^T store's column reads (nt_pack_store); vmask is 0
     * otherwise. */
    const int vmask = BM == 128 && BN == 128 && d.pack_N > 0 && n0 >= 2 * d.pack_E ? 0x1c : 0;

    /* The activation is chosen once, outside the element loops: a
     * per-element switch on d.act costs more than the K loop's tail. */
    auto stage_out = [&](int c, auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
#pragma clang loop unroll(full)
        for (int i = 0; i < NA; i++) {
            const int rb = wm * WM + 32 * i - c * CR; /* block row in chunk */

            if (rb < 0 || rb >= CR)
                continue;
#pragma clang loop unroll(full)
            for (int j = 0; j < NB; j++) {
                const int col = wn * WN + 32 * j + l32, n = n0 + col;
                const float bn = d.bias && n < d.N ? d.bias[n] : 0.0f;
                const f32x16 cv = acc[i][j];

#pragma clang loop unroll(full)
                for (int r = 0; r < 16; r++) {
                    /* Row rb + 8 (r / 4) + 4 h + r % 4, rb a multiple of 32:
                     * its (row / 8) % 8 is (rb / 8 + r / 4) % 8. */
                    const int sw = ((((rb >> 3) + (r >> 2)) & 7) << 2) & vmask;

                    E[(rb + 8 * (r >> 2) + 4 * h + (r & 3)) * LD + (col ^ sw)] =
                        nt_act(d.alpha * cv[r] + bn, ACT);
                }
            }
        }
    };

    __syncthreads();
#pragma clang loop unroll(full)
    for (int c = 0; c < BM / CR; c++) {
        if (d.act == ACT_GELU_K)
            stage_out(c, std::integral_constant<int, ACT_GELU_K>());
        else if (d.act == ACT_RELU_K)
            stage_out(c, std::integral_constant<int, ACT_RELU_K>());
        else
            stage_out(c, std::integral_constant<int, ACT_NONE_K>());
        __syncthreads();
        if constexpr (BM == 128 && BN == 128) {
            if (d.pack_N > 0) {
                nt_pack_store(d, E, m0, n0, t, rot);
                return;
            }
        }
        /* Output type, residual and window remap chosen once per chunk. */
        auto store_rows = [&](auto f32_c, auto res_c, auto unpart_c) {
            constexpr bool F32 = decltype(f32_c)::value, RES = decltype(res_c)::value,
                           UNPART = decltype(unpart_c)::value;

            for (int it = 0; it < CR / RPI; it++) {
                const int row = it * RPI + t / (BN / 4), col = (t % (BN / 4)) * 4;
                const int m = m0 + c * CR + row, n = n0 + col;
                long crow = m;
                bool keep = m < d.M && n < d.N;

                if (UNPART) {
                    const int ws = d.unpart_ws, wsz = ws * ws;
                    const int w = m / wsz, p = m - w * wsz;
                    const int py = p / ws, wy = w / d.unpart_nwx;
                    const int y = wy * ws + py;
                    const int x = (w - wy * d.unpart_nwx) * ws + (p - py * ws);

                    keep = keep && y < d.unpart_H && x < d.unpart_H;
                    crow = (long)y * d.unpart_H + x;
                }
                if (!keep)
                    continue;
                const f32x4 v4 = *(const f32x4 *)&E[row * LD + col];
                const long idx = d.coff + crow * d.ldc + n;
                const long ridx = d.roff + crow * d.ldc + n;

                if (vec && n + 3 < d.N) {
                    if (F32) {
                        f32x4 o = v4;

                        if (RES)
                            o += *(const f32x4 *)((const float *)d.R + ridx);
                        *(f32x4 *)((float *)d.C + idx) = o;
                    }
                    else {
                        f32x4 o = v4;
                        uint2 pk;

                        if (RES) {
                            const uint2 rv = *(const uint2 *)((const uint16_t *)d.R + ridx);

                            o.x += __builtin_bit_cast(float, rv.x << 16);
                            o.y += __builtin_bit_cast(float, rv.x & 0xffff0000u);
                            o.z += __builtin_bit_cast(float, rv.y << 16);
                            o.w += __builtin_bit_cast(float, rv.y & 0xffff0000u);
                        }
                        pk.x = pack_bf16x2(o.x, o.y);
                        pk.y = pack_bf16x2(o.z, o.w);
                        *(uint2 *)((uint16_t *)d.C + idx) = pk;
                    }
                }
                else
                    for (int e = 0; e < 4 && n + e < d.N; e++) {
                        float v = v4[e];

                        if (F32) {
                            if (RES)
                                v += ((const float *)d.R)[ridx + e];
                            ((float *)d.C)[idx + e] = v;
                        }
                        else {
                            if (RES)
                                v += bf2f(((const uint16_t *)d.R)[ridx + e]);
                            ((uint16_t *)d.C)[idx + e] = f2bf(v);
                        }
                    }
            }
        };
        using T_ = std::true_type;
        using F_ = std::false_type;
        const bool f32 = d.cdt == DT_F32, res = d.R != nullptr, unp = d.unpart_ws > 0;

        if (f32 && res && unp)
            store_rows(T_(), T_(), T_());
        else if (f32 && res)
            store_rows(T_(), T_(), F_());
        else if (f32 && unp)
            store_rows(T_(), F_(), T_());
        else if (f32)
            store_rows(T_(), F_(), F_());
        else if (res && unp)
            store_rows(F_(), T_(), T_());
        else if (res)
            store_rows(F_(), T_(), F_());
        else if (unp)
            store_rows(F_(), F_(), T_());
        else
            store_rows(F_(), F_(), F_());
        __syncthreads();
    }
}

/* ------------------------------------------------------------ big tiles */

/* Wait until at most N_ vector memory operations of this wave are in
 * flight (the global -> LDS copies of the stages issued after the one
 * about to be read). */
template <int N_> __device__ __forceinline__ void nt_vmwait()
{
    static_assert(N_ >= 0 && N_ < 64, "vmcnt");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

/* Big-tile variant of k_gemm_nt: one workgroup per CU, BM x BN tiles of
 * NW = (BM / WM) (BN / WN) waves with WN = 64 (a wave's columns are one
 * 64-wide head of a packed QKV product), K stages of 64 in NSLOT LDS
 * slots, and fragments read one 16-wide K step ahead: the barrier of
 * stage ks + 1 sits before the last K step of stage ks, so the next
 * stage's first fragments load under the current stage's last products
 * and the copy of stage ks + NSLOT (into the slot stage ks leaves) goes
 * out right after it. A wave's WM / 32 + WN / 32 operand fragments of
 * 1 KiB per 16-wide K step feed (WM / 32) (WN / 32) MFMAs: 0.75 KiB of LDS
 * reads per MFMA for 128 x 64 waves, 0.83 KiB for 96 x 64 (1 KiB for the
 * 64 x 64 waves of k_gemm_nt's 128 x 128 tiles). The epilogue stages each
 * wave's tile in its own share of the freed slots and writes whole rows
 * with 16-byte stores: bf16 C in one pass of bf16 rows, fp32 C in passes
 * of PR rows of fp32 (16-byte chunks swizzled by row: sidx),
 * or (packed QKV, 256 x 256 tiles) the attention operands of one 64-key
 * block and head per pass. Products with a residual or a window remap
 * stay on k_gemm_nt. SCH interleaves one fragment read between
 * consecutive products (the 4-wave configuration, one wave per SIMD). */
template <int BM, int BN, int WM, int WN, int NSLOT, bool SCH, bool PACK = false>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64, 1) void
k_gemm_nt2(gemm_desc d)
{
    constexpr int NW = (BM / WM) * (BN / WN);
    constexpr int NA = WM / 32, NB = WN / 32, NS = NT_KS / 16;
    constexpr int ROWS = BM + BN;
    constexpr int SLOT = ROWS * NT_KS * 2;
    constexpr int LPW = ROWS / (8 * NW);
    constexpr int SHARE = NSLOT * SLOT / NW;
    constexpr int PR = SHARE >= WM * WN * 4 ? WM : SHARE >= 64 * WN * 4 ? 64 : 32;
    static_assert(ROWS % (8 * NW) == 0 && WN == 64 && WM % PR == 0 && WM % 32 == 0, "shape");
    static_assert(PR * WN * 4 <= SHARE, "staging");
    __shared__ __attribute__((aligned(16))) uint16_t S[NSLOT * SLOT / 2];
    const int t = threadIdx.x, l = t & 63, w = t >> 6, h = l >> 5, l32 = l & 31;
    const int wu = __builtin_amdgcn_readfirstlane(w);
    const int wm = wu / (BN / WN), wn = wu % (BN / WN);
    const int tm = (d.M + BM - 1) / BM, tn = (d.N + BN - 1) / BN;
    const int total = tm * tn, per_xcd = (total + NT_NXCD - 1) / NT_NXCD;
    /* XCD-aware: XCD x takes tiles [x per_xcd, (x + 1) per_xcd) of an
     * order that walks groups of four tile rows column by column, so the
     * tiles an XCD runs at once share a few A and B panels in its L2. */
    const int tile = (int)(blockIdx.x % NT_NXCD) * per_xcd + (int)(blockIdx.x / NT_NXCD);
    if (tile >= total)
        return;
    constexpr int GR = 4;
    const int grp = tile / (GR * tn), in = tile - grp * GR * tn;
    const int rows_g = min(GR, tm - grp * GR);
    const int m0 = (grp * GR + in % rows_g) * BM, n0 = (in / rows_g) * BN;
    const char *Ab = (const char *)((const uint16_t *)d.A + d.aoff + (long)m0 * d.lda);
    const char *Bb = (const char *)((const uint16_t *)d.B + d.boff + (long)n0 * d.ldb);
    const int nk = d.K / NT_KS;
    unsigned goff[LPW];

    /* Copy j of wave w fills stage rows 8 (w LPW + j) .. +7 (all of A or
     * all of B: BM is a multiple of 8); lane i lands on row + i / 8,
     * physical chunk i % 8, fetching logical chunk (i % 8) ^ ((row >> 1)
     * & 7). Rows past M or N read the last row (never stored). */
    for (int j = 0; j < LPW; j++) {
        const int row = 8 * (wu * LPW + j) + (l >> 3);
        const int chunk = (l & 7) ^ ((row >> 1) & 7);

        if (row < BM)
            goff[j] = 2u * ((unsigned)(min(m0 + row, d.M - 1) - m0) * d.lda + 8 * chunk);
        else
            goff[j] = 2u * ((unsigned)(min(n0 + row - BM, d.N - 1) - n0) * d.ldb + 8 * chunk);
    }
    const unsigned lds0 = (unsigned)(uintptr_t)S + 1024u * LPW * wu;
    auto load_stage = [&](int ks, int slot) {
#pragma unroll
        for (int j = 0; j < LPW; j++)
            nt_g2lds16_s((8 * (wu * LPW + j) < BM ? Ab : Bb) + 128L * ks, goff[j],
                         lds0 + (unsigned)SLOT * slot + 1024u * j);
    };
    /* Fragment byte offsets per K step s: A rows wm WM + 32 i + l32, B
     * rows BM + wn WN + 32 j + l32 (i, j add 4096 B; the swizzle depends on
     * row bits 1..3 only). */
    unsigned aro[NS], bro[NS];
    for (int s = 0; s < NS; s++) {
        const int ra = wm * WM + l32, rb = BM + wn * WN + l32;

        aro[s] = 2u * (ra * NT_KS + nt_swz(ra, 2 * s + h));
        bro[s] = 2u * (rb * NT_KS + nt_swz(rb, 2 * s + h));
    }
    f32x16 acc[NA][NB];
#pragma unroll
    for (int i = 0; i < NA; i++)
#pragma unroll
        for (int j = 0; j < NB; j++)
            acc[i][j] = (f32x16){};
    const char *Sb = (const char *)S;
    bf16x8 fa[2][NA], fb[2][NB];
    auto rd = [&](int ks, int s, int buf) {
        const char *sl = Sb + SLOT * (ks % NSLOT);
#pragma unroll
        for (int i = 0; i < NA; i++)
            fa[buf][i] = *(const bf16x8 *)(sl + 4096 * i + aro[s]);
#pragma unroll
        for (int j = 0; j < NB; j++)
            fb[buf][j] = *(const bf16x8 *)(sl + 4096 * j + bro[s]);
    };
    /* Stage ks landed for this wave: the stages issued after it (at most
     * NSLOT - 2, fewer near the end) may still be in flight. */
    auto wait_stage = [&](int ks) {
        const int young = min(NSLOT - 2, nk - 1 - ks);

        if (young >= NSLOT - 2)
            nt_vmwait<LPW * (NSLOT - 2)>();
        else if (young == 1)
            nt_vmwait<LPW>();
        else
            nt_vmwait<0>();
    };

#pragma unroll
    for (int s = 0; s < NSLOT - 1; s++)
        if (s < nk)
            load_stage(s, s);
    wait_stage(0);
    __syncthreads();
    if (NSLOT - 1 < nk)
        load_stage(NSLOT - 1, NSLOT - 1);
    rd(0, 0, 0);
    for (int ks = 0; ks < nk; ks++) {
#pragma unroll
        for (int s = 0; s < NS; s++) {
            const int buf = s & 1;

            if (s + 1 < NS)
                rd(ks, s + 1, buf ^ 1);
            else if (ks + 1 < nk) {
                wait_stage(ks + 1);
                __syncthreads();
                if (ks + NSLOT < nk)
                    load_stage(ks + NSLOT, (ks + NSLOT) % NSLOT);
                rd(ks + 1, 0, buf ^ 1);
            }
#pragma unroll
            for (int i = 0; i < NA; i++)
#pragma unroll
                for (int j = 0; j < NB; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[buf][i], fb[buf][j],
                                                                        acc[i][j], 0, 0, 0);
            if constexpr (SCH) {
#pragma unroll
                for (int q = 0; q < NA + NB; q++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
                }
                __builtin_amdgcn_sched_group_barrier(0x008, NA * NB - NA - NB, 0);
            }
        }
    }

    /* Epilogue. Every wave is past its last fragment read of every slot. */
    __syncthreads();
    float *st = (float *)((char *)S + wu * SHARE);
    const int mw = m0 + wm * WM, nw = n0 + wn * WN;
    /* Staged element (row, col) of the wave's pass: 16-byte chunk col / 4
     * of the 256-byte row at chunk (col / 4) ^ sw(row), sw(row) = bit 0 of
     * row, then bits 3..5 of row with bit 2 of row folded into the top:
     * the accumulator writes (rows r and r + 4 from the two lane halves,
     * 32 columns each) fill all 64 banks, two rows of 16-byte reads take
     * complementary chunks, and the V^T column reads (eight rows 8 apart,
     * eight columns) touch 64 distinct banks. */
    auto sidx = [](int row, int col) {
        const int sw = (row & 1) | ((((row >> 3) & 7) ^ (((row >> 2) & 1) << 2)) << 1);

        return row * 64 + (((col >> 2) ^ sw) << 2) + (col & 3);
    };
    /* The raw accumulators of rows [p0, p0 + PR): alpha, the bias and the
     * activation are applied as the rows are read back (applying them
     * here would let the compiler hoist every product of alpha out of the
     * pass loop and spill). */
    auto stage_pass = [&](int p0) {
#pragma unroll
        for (int i = 0; i < NA; i++) {
            if (32 * i < p0 || 32 * i >= p0 + PR)
                continue;
#pragma unroll
            for (int j = 0; j < NB; j++)
#pragma unroll
                for (int r = 0; r < 16; r++)
                    st[sidx(32 * i - p0 + 8 * (r >> 2) + 4 * h + (r & 3), 32 * j + l32)] =
                        acc[i][j][r];
        }
        __builtin_amdgcn_s_waitcnt(0xc07f); /* lgkmcnt(0): the wave's own rows */
    };
    /* act(alpha v + bias) for 4 staged columns, the bias values loaded
     * once per lane before any store (reloading them per row would wait
     * on memory each time: the stores may alias the bias). */
    auto finish4 = [&](f32x4 v, f32x4 bv, auto act_c) {
        constexpr int ACT = decltype(act_c)::value;
        f32x4 o;

        for (int e = 0; e < 4; e++)
            o[e] = nt_act(d.alpha * v[e] + bv[e], ACT);
        return o;
    };
    auto bias4 = [&](int n) {
        f32x4 b;

        for (int e = 0; e < 4; e++)
            b[e] = d.bias && n + e < d.N ? d.bias[n + e] : 0.0f;
        return b;
    };

    if constexpr (PACK) {
        static_assert(BM == 256 && BN == 256 && WM == 128, "packed store tiles");
        {
            /* Packed QKV: the wave's columns are head `head` of one third,
             * each 64-row pass one 64-key block of one unit (pack_N is a
             * multiple of 64 and M of pack_N, so a block is whole or past
             * M). The arithmetic is k_qkv_pack's (same bits). */
            static_assert(PR == 64, "one key block per pass");
            const int third = n0 / d.pack_E, heads = d.pack_E / 64, Np = d.pack_N;
            const int head = (nw - third * d.pack_E) / 64;
            const int c8 = l & 7, r8 = l >> 3;
            const f32x4 bq0 = bias4(nw + 8 * c8), bq1 = bias4(nw + 8 * c8 + 4);
            float bvt[8];

            for (int it = 0; it < 8; it++)
                bvt[it] = d.bias ? d.bias[nw + 8 * it + r8] : 0.0f;

#pragma unroll
            for (int p0 = 0; p0 < WM; p0 += 64) {
                const int mb = mw + p0;

                if (mb >= d.M)
                    break;
                const int win = mb / Np, pb = mb - win * Np;
                const long unit = (long)win * heads + head;
                stage_pass(p0);
                /* The pass's RoPE rows (position pb + 8 it + l / 8, pairs
                 * 4 (l % 8) .. +3), all read before the first is used (once
                 * the pass's accumulators are staged), so that the row groups
                 * wait for the table once rather than once each. */
                f32x4 rv[8][2];

                if (third < 2 && d.pack_rope)
#pragma unroll
                    for (int it = 0; it < 8; it++) {
                        const f32x4 *src = (const f32x4 *)((const float2 *)d.pack_rope +
                                                           (long)((pb + 8 * it + r8) % d.pack_npos) * 32 +
                                                           4 * c8);

                        rv[it][0] = src[0];
                        rv[it][1] = src[1];
                    }

                if (third < 2) {
                    uint16_t *dst = (uint16_t *)(third == 0 ? d.pack_q16 : d.pack_k16) +
                                    (unit * Np + pb) * 64 + 8 * c8;
                    float mx = 0.0f; /* largest row |k|^2 of the bf16 values */

#pragma unroll
                    for (int it = 0; it < 8; it++) {
                        const int row = 8 * it + r8;
                        const f32x4 x0 = finish4(*(const f32x4 *)&st[sidx(row, 8 * c8)], bq0,
                                                 std::integral_constant<int, ACT_NONE_K>());
                        const f32x4 x1 = finish4(*(const f32x4 *)&st[sidx(row, 8 * c8 + 4)], bq1,
                                                 std::integral_constant<int, ACT_NONE_K>());
                        float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
                        float ps = 0.0f;
                        u32x4 pk;

                        if (d.pack_rope) {
                            const f32x4 r0 = rv[it][0], r1 = rv[it][1];
                            const float2 rot[4] = {make_float2(r0.x, r0.y), make_float2(r0.z, r0.w),
                                                   make_float2(r1.x, r1.y), make_float2(r1.z, r1.w)};

                            for (int jj = 0; jj < 4; jj++) {
                                const float a = v[2 * jj], b = v[2 * jj + 1];

                                v[2 * jj] = fmaf(a, rot[jj].x, -(b * rot[jj].y));
                                v[2 * jj + 1] = fmaf(a, rot[jj].y, b * rot[jj].x);
                            }
                        }
                        if (third == 0)
                            for (int e = 0; e < 8; e++)
                                v[e] *= d.pack_scale * LOG2E_F;
                        for (int e = 0; e < 4; e++) {
                            pk[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
                            if (third == 1) {
                                const uint32_t u = pk[e];
                                const float lo = __builtin_bit_cast(float, u << 16),
                                            hi = __builtin_bit_cast(float, u & 0xffff0000u);

                                ps = fmaf(hi, hi, fmaf(lo, lo, ps));
                            }
                        }
                        *(u32x4 *)(dst + (long)row * 64) = pk;
                        if (third == 1) {
                            ps += __shfl_xor(ps, 1, 64);
                            ps += __shfl_xor(ps, 2, 64);
                            ps += __shfl_xor(ps, 4, 64);
                            mx = fmaxf(mx, ps);
                        }
                    }
                    if (third == 1) {
                        mx = wave_max(mx);
                        if (l == 0)
                            d.pack_knorm[unit * (Np / 64) + pb / 64] = sqrtf(mx) * (1.0f + 0x1p-10f);
                    }
                }
                else {
                    /* V^T: lane l takes channel 8 it + l / 8 and keys 8 (l % 8)
                     * .. +7, read down the staged column (rows 8 apart of eight
                     * columns: distinct banks under sidx's swizzle). */
                    for (int it = 0; it < 8; it++) {
                        const int ch = 8 * it + r8;
                        const float bc = bvt[it];
                        u32x4 pk;

                        for (int e = 0; e < 4; e++)
                            pk[e] = pack_bf16x2(d.alpha * st[sidx(8 * c8 + 2 * e, ch)] + bc,
                                                d.alpha * st[sidx(8 * c8 + 2 * e + 1, ch)] + bc);
                        *(u32x4 *)((uint16_t *)d.pack_vt16 + (unit * 64 + ch) * Np + pb + 8 * c8) = pk;
                    }
                }
                __builtin_amdgcn_s_waitcnt(0xc07f);
            }
            return;
        }
    }

    /* Generic store (no residual and no window remap: launch_gemm_nt keeps
     * those products on k_gemm_nt): act(alpha acc + bias) into C. */
    static_assert(WM * WN * 2 <= SHARE, "one bf16 staging pass");
    const bool vec = ((d.ldc | d.coff) & (d.cdt == DT_F32 ? 3 : 7)) == 0;

    if (d.cdt != DT_F32) {
        /* bf16 C: rounded once, staged in one pass as 128-byte rows
         * (16-byte chunk c of row r at chunk c ^ (r & 7); lanes l and l ^ 1
         * trade values so each writes two adjacent columns), then 16-byte
         * stores of whole rows. */
        uint16_t *sb = (uint16_t *)st;
        const bool odd = l & 1;
        auto stage16 = [&](auto act_c) {
            constexpr int ACT = decltype(act_c)::value;
#pragma unroll
            for (int j = 0; j < NB; j++) {
                const int cl = 32 * j + (l32 & ~1), n = nw + cl;
                const float b0 = d.bias && n < d.N ? d.bias[n] : 0.0f;
                const float b1 = d.bias && n + 1 < d.N ? d.bias[n + 1] : 0.0f;
#pragma unroll
                for (int i = 0; i < NA; i++)
#pragma unroll
                    for (int r = 0; r < 16; r += 2) {
                        /* even lane: rows r, r + 1 of column cl; odd: of cl + 1 */
                        const float x0 = acc[i][j][r], x1 = acc[i][j][r + 1];
                        const float got = __shfl_xor(odd ? x0 : x1, 1, 64);
                        const float lo = odd ? got : x0, hi = odd ? x1 : got;
                        const int rr = odd ? r + 1 : r;
                        const int row = 32 * i + 8 * (rr >> 2) + 4 * h + (rr & 3);

                        *(uint32_t *)(sb + row * 64 + (((cl >> 3) ^ (row & 7)) << 3) + (cl & 7)) =
                            pack_bf16x2(nt_act(d.alpha * lo + b0, ACT), nt_act(d.alpha * hi + b1, ACT));
                    }
            }
        };
        if (d.act == ACT_GELU_K)
            stage16(std::integral_constant<int, ACT_GELU_K>());
        else if (d.act == ACT_RELU_K)
            stage16(std::integral_constant<int, ACT_RELU_K>());
        else
            stage16(std::integral_constant<int, ACT_NONE_K>());
        __builtin_amdgcn_s_waitcnt(0xc07f); /* lgkmcnt(0): the wave's own rows */
#pragma unroll
        for (int it = 0; it < WM / 8; it++) {
            const int row = 8 * it + (l >> 3), c8 = 8 * (l & 7), m = mw + row, n = nw + c8;

            if (m >= d.M || n >= d.N)
                continue;
            const u32x4 v = *(const u32x4 *)(sb + row * 64 + (((c8 >> 3) ^ (row & 7)) << 3));
            uint16_t *cp = (uint16_t *)d.C + d.coff + (long)m * d.ldc + n;

            if (vec && n + 7 < d.N)
                *(u32x4 *)cp = v;
            else
                for (int e = 0; e < 8 && n + e < d.N; e++)
                    cp[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
        }
        return;
    }
    /* fp32 C: passes of PR rows of raw accumulators, finished as they are
     * read back; lane l writes columns 4 (l % 16) .. +3 of row l / 16 of
     * each 4-row group. */
    const f32x4 bg = bias4(nw + 4 * (l & 15));
    auto store_pass = [&](int p0, auto act_c) {
#pragma unroll
        for (int it = 0; it < PR / 4; it++) {
            const int row = 4 * it + (l >> 4), c4 = 4 * (l & 15), m = mw + p0 + row, n = nw + c4;

            if (m >= d.M || n >= d.N)
                continue;
            const f32x4 v = finish4(*(const f32x4 *)&st[sidx(row, c4)], bg, act_c);
            float *cp = (float *)d.C + d.coff + (long)m * d.ldc + n;

            if (vec && n + 3 < d.N)
                *(f32x4 *)cp = v;
            else
                for (int e = 0; e < 4 && n + e < d.N; e++)
                    cp[e] = v[e];
        }
    };
#pragma unroll
    for (int p0 = 0; p0 < WM; p0 += PR) {
        if (mw + p0 >= d.M)
            break;
        stage_pass(p0);
        if (d.act == ACT_GELU_K)
            store_pass(p0, std::integral_constant<int, ACT_GELU_K>());
        else if (d.act == ACT_RELU_K)
            store_pass(p0, std::integral_constant<int, ACT_RELU_K>());
        else
            store_pass(p0, std::integral_constant<int, ACT_NONE_K>());
        __builtin_amdgcn_s_waitcnt(0xc07f);
    }
}

/* The NT kernel applies to unbatched bf16 x bf16 (weights as [N][K])
 * products with K a multiple of 64 and 16-byte aligned rows. */
extern "C" int gemm_nt_ok(const gemm_desc *d)
{
    return d->mode == MODE_BF16 && d->adt == DT_BF16 && d->bdt == DT_BF16 &&
           d->transb && d->nb == 1 && d->K >= NT_KS && d->K % NT_KS == 0 &&
           d->lda % 8 == 0 && d->ldb % 8 == 0 && d->aoff % 8 == 0 &&
           d->boff % 8 == 0 && d->M >= 1 && d->N >= 1 &&
           (d->pack_N == 0 ||
            (d->pack_N % 64 == 0 && d->pack_E % 128 == 0 && d->N == 3 * d->pack_E &&
             d->M % d->pack_N == 0 && d->alpha == 1.0f && d->act == ACT_NONE_K && !d->R &&
             d->unpart_ws == 0 && d->pack_npos >= 1));
}

/* Big-tile configuration for d (k_gemm_nt2), or 0 for the k_gemm_nt
 * tiles: 1 = 256 x 256 (8 waves of 128 x 64), 2 = 192 x 256 (8 waves of
 * 96 x 64), 3 = 192 x 128 (4 waves of 96 x 64). The packed QKV store
 * takes 1 when a tile's 256 columns are four heads of one third. Other
 * products without a residual take the configuration of least rounds x
 * tile area / rate (K-loop rates measured on random operands at M = 5184:
 * 1150, 1070 and 870 TFLOP/s), if they are large enough to fill the
 * device: either K >= 2048 or the chosen tiles cover >= 90 % of the CUs.
 * On N(0, 1) operands at M = 5184: fc1 (GELU, bf16) 708 against 616
 * TFLOP/s on the 128 x 128 tiles, the QKV product with fp32 C 707 against
 * 668. */
static int nt2_config(const gemm_desc *d)
{
    const long cus = dev_cu_count();
    static const int bm[4] = {0, 256, 192, 192}, bn[4] = {0, 256, 256, 128};
    static const double rate[4] = {0.0, 1.0, 0.93, 0.76};
    int best = 0;
    double cost = 0.0;

    if (d->pack_N > 0)
        return d->pack_E % 256 == 0 ? 1 : 0;
    /* A residual (the attention projection and fc2, fp32 x += ...) keeps
     * the 128 x 64 tiles: three workgroups per CU overlap one's residual
     * traffic with the others' products (fc2 698 against 681-691 TFLOP/s
     * with 192 x 128 tiles). */
    if ((long)d->M * d->N < (1L << 21) || d->K < 512 || d->R)
        return 0;
    for (int c = 1; c <= 3; c++) {
        const long tiles = (long)((d->M + bm[c] - 1) / bm[c]) * ((d->N + bn[c] - 1) / bn[c]);
        const double k = (double)((tiles + cus - 1) / cus) * bm[c] * bn[c] / rate[c];

        if (best == 0 || k < cost) {
            best = c;
            cost = k;
        }
    }
    {
        const long tiles = (long)((d->M + bm[best] - 1) / bm[best]) *
                           ((d->N + bn[best] - 1) / bn[best]);

        if (d->K < 2048 && tiles * 10 < cus * 9)
            return 0;
    }
    return best;
}

/* Returns -1 when the NT kernel does not apply, else a hipError_t. */
extern "C" int launch_gemm_nt(const gemm_desc *d, void *stream)
{
    hipStream_t s = (hipStream_t)stream;
    long t256;
    int bm, bn, big;

    if (!gemm_nt_ok(d))
        return -1;
    big = nt2_config(d);
    if (big) {
        static const int bm2[4] = {0, 256, 192, 192}, bn2[4] = {0, 256, 256, 128};
        const long tiles = (long)((d->M + bm2[big] - 1) / bm2[big]) *
                           ((d->N + bn2[big] - 1) / bn2[big]);
        const long grid = (tiles + NT_NXCD - 1) / NT_NXCD * NT_NXCD;

        if (grid > 0x7fffffffL)
            return hipErrorInvalidConfiguration;
        if (big == 1 && d->pack_N > 0)
            hipLaunchKernelGGL((k_gemm_nt2<256, 256, 128, 64, 2, false, true>),
                               dim3((unsigned)grid), dim3(512), 0, s, *d);
        else if (big == 1)
            hipLaunchKernelGGL((k_gemm_nt2<256, 256, 128, 64, 2, false>), dim3((unsigned)grid),
                               dim3(512), 0, s, *d);
        else if (big == 2)
            hipLaunchKernelGGL((k_gemm_nt2<192, 256, 96, 64, 2, false>), dim3((unsigned)grid),
                               dim3(512), 0, s, *d);
        else
            hipLaunchKernelGGL((k_gemm_nt2<192, 128, 96, 64, 3, true>), dim3((unsigned)grid),
                               dim3(256), 0, s, *d);
        return hipGetLastError();
    }
    /* 128 x 128 tiles (4 waves of 64 x 64, two workgroups per CU, so one
     * workgroup's pipeline fill and output drain overlap the other's
     * products); 256 x 256 tiles (8 waves of 128 x 64, half the operand
     * traffic per product) only for long reductions that still give
     * (nearly) every CU a tile. Measured at M = 5184: K = 1024 runs at
     * 646 vs 691 TFLOP/s (N = 3072) and 460 vs 585 (N = 4096), K = 4096
     * at 1145 vs 1070 (N = 3072). 128 x 64 tiles (4 waves of 64 x 32)
     * where 128 x 128 tiles would give fewer than two per CU: at M = 5184,
     * N = 1024 they run 518 vs 408 TFLOP/s (K = 1024) and 810 vs 732
     * (K = 4096); everywhere else they are slower. */
    t256 = (long)((d->M + 255) / 256) * ((d->N + 255) / 256);
    /* The packed-operand store exists for 128 x 128 tiles only. */
    bm = t256 >= dev_cu_count() * 9 / 10 && d->K >= 2048 && d->pack_N == 0 ? 256 : 128;
    bn = bm;
    if (bm == 128 && d->pack_N == 0 &&
        (long)((d->M + 127) / 128) * ((d->N + 127) / 128) < 2L * dev_cu_count())
        bn = 64;
    {
        const long tiles = (long)((d->M + bm - 1) / bm) * ((d->N + bn - 1) / bn);
        const long grid = (tiles + NT_NXCD - 1) / NT_NXCD * NT_NXCD;

        if (grid > 0x7fffffffL)
            return hipErrorInvalidConfiguration;
        if (bm == 256)
            hipLaunchKernelGGL((k_gemm_nt<256, 256, 128, 64>),
                               dim3((unsigned)grid), dim3(512), 0, s, *d);
        else if (bn == 64)
            hipLaunchKernelGGL((k_gemm_nt<128, 64, 64, 32>),
                               dim3((unsigned)grid), dim3(256), 0, s, *d);
        else
            hipLaunchKernelGGL((k_gemm_nt<128, 128, 64, 64>),
                               dim3((unsigned)grid), dim3(256), 0, s, *d);
    }
    return hipGetLastError();
}
