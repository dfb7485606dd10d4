/* SPDX-License-Identifier: Unlicense
 *
 * Fused image -> token attention of the mask decoder (the block
 * sam3_model.c:1298-1312 / 1330-1345: image-query projection, attention
 * over the 8 prompt tokens, output projection, residual, norm4) on bf16
 * MFMA, for the bf16 path.
 *
 * The projections are folded into per-prompt matrices so the per-token
 * work is two small products against the prompt's 8 tokens. For image
 * token j with input x_j (kin_j = keys_j + PE_j in layer 1, the shared
 * projected query qp0_j in layer 0), head h and prompt token t:
 *
 *   score(j, h, t) = s (Wq_h x_j + bq_h) . k_{t,h}
 *                  = x_j . Wt[h,t] + bt[h,t],
 *       Wt[h,t] = s Wq_h^T k_{t,h} (256 wide; layer 0, where x_j is already
 *       projected: s k_{t,h} on head h's 16 columns of 128), bt[h,t] =
 *       s bq_h . k_{t,h} (0 in layer 0), s = log2(e) / sqrt(16);
 *   out_j = Wo (concat_h sum_t a(j,h,t) v_{t,h}) + bo
 *         = sum_{h,t} a(j,h,t) Y[h,t] + bo,   Y[h,t] = Wo_h v_{t,h},
 *
 * with a the softmax over t per head (exp2 domain). In layer 1 the
 * position encoding enters the scores only through its projection:
 *
 *   score(j, h, t) = keys_j . Wt[h,t] + s k_{t,h} . PQ_{j,h} + bt[h,t],
 *       PQ_j = Wq PE_j (128 wide, head h = columns 16 h .. 16 h + 15),
 *
 * so the kernel reads PQ (bf16, 256 bytes per image token, shared by the
 * prompts) instead of PE (1 KB per token). k_i2t_fold builds Wt, bt, Y^T
 * and the compact rows Kc[h,t] = s k_{t,h} (16 wide) per prompt;
 * k_i2t_fused runs a wave per 32 image tokens: S^T = Wt X^T (+ Kc PQ^T,
 * block diagonal over the heads; 64 rows (h, t) x 32 tokens), the grouped
 * softmax in registers, U^T = Y^T A^T (256 channels x 32 tokens), then +
 * bo + residual and the LayerNorm over the 256 channels, written once.
 *
 * MFMA 32x32x16 bf16 lane layouts (l = lane, hh = l / 32): A operand lane
 * l holds A[l % 32][8 hh .. 8 hh + 7 of the k step]; B operand B[same k
 * slice][l % 32]; D register r of lane l is D[8 (r / 4) + 4 hh + r % 4][l % 32].
 */
#include "k_common.h"

#define FOLD_ROWS 64 /* (head, prompt token) pairs: 8 x 8 */

__device__ __forceinline__ float wld(const void *p, int dt, long i)
{
    if (dt == DT_BF16)
        return bf2f(((const uint16_t *)p)[i]);
    if (dt == DT_F16)
        return h2f(((const uint16_t *)p)[i]);
    return ((const float *)p)[i];
}

/* Column kappa of Y^T (the k index of the second product) holds Y row
 * rho(kappa) = kappa with bits 2 and 3 swapped: k step s, lane half hh
 * and element e = 4 e2 + e10 of the B operand are D register 8 (s % 2) +
 * e of score tile s / 2, whose row is 16 s + 8 e2 + 4 hh + e10. */
__device__ __forceinline__ int yt_row(int kappa)
{
    return (kappa & ~12) | ((kappa & 4) << 1) | ((kappa & 8) >> 1);
}

/* One workgroup per prompt p. sk / sv [P][8][128] (token keys and values
 * of the image -> token attention), Wq [128][256] (layer 1) with bias bq,
 * Wo [256][128]. Writes Wt16 [P][64][K] (bf16), bt [P][64] (when bq is
 * given), YT16 [P][256][64] (bf16, columns in yt_row order; when Wo is
 * given) and, in layer 1 when Kc16 is given, Kc16 [P][64][16] (bf16, row
 * (h, t) = s k_{t,h}: the factor of the projected position encoding's
 * score term). Row r of Wt is (h, t) = (r / 8, r % 8). The token -> image
 * attention uses the same fold for its queries (sk = projected queries,
 * Wq = the key projection, no bq or Wo). */
__global__ __launch_bounds__(256) void k_i2t_fold(const float *__restrict__ sk,
                                                  const float *__restrict__ sv,
                                                  int layer, const void *Wq,
                                                  int wq_dt,
                                                  const float *__restrict__ bq,
                                                  const void *Wo, int wo_dt,
                                                  float s,
                                                  uint16_t *__restrict__ Wt16,
                                                  float *__restrict__ bt,
                                                  uint16_t *__restrict__ YT16,
                                                  uint16_t *__restrict__ Kc16)
{
    /* Workgroup (p, h): head h's 16 columns of the 8 tokens' keys and
     * values, rows 8 h .. 8 h + 7 of Wt and bt, those columns of Y^T. */
    __shared__ float ks[8][16], vs[8][16];
    const int p = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const int K = layer ? 256 : 128;

    if (t < 128) {
        const int tk = t / 16, c = t % 16;

        ks[tk][c] = sk[(long)p * 1024 + tk * 128 + 16 * h + c];
        if (Wo)
            vs[tk][c] = sv[(long)p * 1024 + tk * 128 + 16 * h + c];
    }
    __syncthreads();
    uint16_t *wt = Wt16 + ((long)p * FOLD_ROWS + 8 * h) * K;
    if (layer) {
        /* Thread t = input column d of the 256. */
        float w[16];

        for (int c = 0; c < 16; c++)
            w[c] = wld(Wq, wq_dt, (long)(16 * h + c) * 256 + t);
        for (int tk = 0; tk < 8; tk++) {
            float acc = 0.0f;

            for (int c = 0; c < 16; c++)
                acc = fmaf(ks[tk][c], w[c], acc);
            wt[tk * K + t] = f2bf(s * acc);
        }
        if (bq && t < 8) {
            float acc = 0.0f;

            for (int c = 0; c < 16; c++)
                acc = fmaf(ks[t][c], bq[16 * h + c], acc);
            bt[p * FOLD_ROWS + 8 * h + t] = s * acc;
        }
        if (Kc16 && t < 128)
            Kc16[((long)p * FOLD_ROWS + 8 * h + t / 16) * 16 + t % 16] =
                f2bf(s * ks[t / 16][t % 16]);
    }
    else {
        /* Block diagonal: row (h, tk) holds s k_{tk,h} on columns 16 h ..
         * 16 h + 15 of 128, zero elsewhere. */
        for (int i = t; i < 8 * 128; i += 256) {
            const int tk = i / 128, d = i % 128;

            wt[i] = f2bf(d / 16 == h ? s * ks[tk][d % 16] : 0.0f);
        }
        if (t < 8)
            bt[p * FOLD_ROWS + 8 * h + t] = 0.0f;
    }
    /* Y^T: thread t = output channel ch (skipped without Wo); Y row
     * 8 h + tk lands in column yt_row(8 h + tk) (yt_row is its own
     * inverse). */
    if (Wo) {
        uint16_t *yt = YT16 + (long)p * 256 * FOLD_ROWS + (long)t * FOLD_ROWS;
        float wo[16];

        for (int c = 0; c < 16; c++)
            wo[c] = wld(Wo, wo_dt, (long)t * 128 + 16 * h + c);
        for (int tk = 0; tk < 8; tk++) {
            float acc = 0.0f;

            for (int c = 0; c < 16; c++)
                acc = fmaf(wo[c], vs[tk][c], acc);
            yt[yt_row(8 * h + tk)] = f2bf(acc);
        }
    }
}

extern "C" int launch_i2t_fold(const float *sk, const float *sv, int layer,
                               const void *Wq, int wq_dt, const float *bq,
                               const void *Wo, int wo_dt, float s, int P,
                               void *Wt16, float *bt, void *YT16, void *Kc16,
                               void *stream)
{
    if (P < 1 || (layer && !Wq) || (!layer && !Wo) || (!layer && Kc16))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_i2t_fold, dim3(P, 8), dim3(256), 0, (hipStream_t)stream,
                       sk, sv, layer, Wq, wq_dt, bq, Wo, wo_dt, s,
                       (uint16_t *)Wt16, bt, (uint16_t *)YT16, (uint16_t *)Kc16);
    return hipGetLastError();
}

/* Byte offset of 16-byte chunk `chunk` of row `row` in an LDS tile with
 * rows of `rowbytes`: XOR-swizzled so that the 16 rows one ds_read_b128
 * phase reads fall on distinct banks. */
__device__ __forceinline__ unsigned swz_off(int row, int chunk, int rowbytes)
{
    const int nch = rowbytes / 16;
    const int sw = rowbytes >= 256 ? (row & 15) : ((row >> 1) & 7);

    return (unsigned)(row * rowbytes + 16 * ((chunk ^ sw) & (nch - 1)));
}

/* Work split of the (prompt, 128-token chunk) items over the 8 XCDs
 * (workgroup b runs on XCD b % 8): XCD x owns prompts [x P / 8, (x + 1) P
 * / 8) with all C chunks when P >= 8, else all prompts with chunks [x C /
 * 8, (x + 1) C / 8): pa, np (first prompt, count), ca, nc (first chunk,
 * count). */
/* Item (prompt p, 128-token chunk c) of workgroup b, which runs on XCD
 * b % 8. Both orders take blocks of 8 chunks x a set of prompts, chunk
 * fastest, so that the workgroups in flight on an XCD share each prompt's
 * fold (Wt, Y^T, fetched by the block's first workgroup of the prompt)
 * and each chunk's shared rows (read by the block's prompts together).
 * Layer 1 (XR): XCD x owns a region, prompts [x P / 8, (x + 1) P / 8)
 * with all C chunks when P >= 8 (else all prompts, chunks [x C / 8, (x +
 * 1) C / 8)), so that its prompts' folds and the whole shared PQ (1.3 MB)
 * stay in its L2 from block to block: 1.11 x the bytes of keys + PE
 * fetched at P = 64, against 1.22 x in the order below. Layer 0: XCD x
 * takes the x-th eighth of all items in block order, which runs ~5 %
 * faster there (its shared rows, qp0 and src, are 1.5 KB a token). Grid:
 * 8 x ceil(P / 8) C or 8 x P ceil(C / 8) (layer 1), P C rounded up to a
 * multiple of 8 (layer 0). */
template <bool XR>
__device__ __forceinline__ bool i2t_item(int P, int C, unsigned b, int &p, int &c)
{
    unsigned pa, np, ca, nc, s;

    if constexpr (XR) {
        const int x = (int)(b % 8);

        if (P >= 8) {
            pa = (unsigned)(x * P / 8);
            np = (unsigned)((x + 1) * P / 8) - pa;
            ca = 0;
            nc = (unsigned)C;
        }
        else {
            pa = 0;
            np = (unsigned)P;
            ca = (unsigned)(x * C / 8);
            nc = (unsigned)((x + 1) * C / 8) - ca;
        }
        s = b / 8;
    }
    else {
        const unsigned total = (unsigned)P * (unsigned)C;

        pa = ca = 0;
        np = (unsigned)P;
        nc = (unsigned)C;
        s = (b % 8) * ((total + 7) / 8) + b / 8;
    }
    if (s >= np * nc)
        return false;
    const unsigned blk = s / (8 * np), r = s % (8 * np);
    const unsigned nb = nc - 8 * blk < 8 ? nc - 8 * blk : 8;

    p = (int)(pa + r / nb);
    c = (int)(ca + 8 * blk + r % nb);
    return true;
}

/* Workgroup = 4 waves = 128 image tokens of one prompt (i2t_item). X rows
 * of K floats (per-prompt stride xs, 0 = shared); residual R (stride rs,
 * 0 = shared); out [P][T][256] may alias R. */
/* RX (layer 1): the residual R is the input X itself (the keys), and the
 * scores take the position term Kc PQ^T (pq [T][128] bf16, kc [P][64][16]
 * bf16). The S^T loop drops each token's loaded keys into the output
 * accumulators U^T in their channel layout (an exchange with lane l ^ 32
 * per step), so the U^T product adds onto the residual and the keys are
 * read from HBM once. */
template <int K, bool RX>
__global__ __launch_bounds__(256, 2) void k_i2t_fused(
    const float *X, long xs, const uint16_t *__restrict__ pq,
    const uint16_t *__restrict__ kc,
    const uint16_t *__restrict__ Wt16, const float *__restrict__ bt,
    const uint16_t *__restrict__ YT16, const float *__restrict__ bo,
    const float *R, long rs, const float *__restrict__ g,
    const float *__restrict__ bln, float *out, int T, int P, float eps)
{
    __shared__ __attribute__((aligned(16))) char Ws[FOLD_ROWS * K * 2];
    __shared__ __attribute__((aligned(16))) char Ys[256 * FOLD_ROWS * 2];
    __shared__ float bts[FOLD_ROWS];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, hh = l >> 5,
              l32 = l & 31;
    int p, c;

    if (!i2t_item<RX>(P, (T + 127) / 128, blockIdx.x, p, c))
        return;
    const int ch0 = 128 * c;

    /* Stage the prompt's Wt (64 x K) and Y^T (256 x 64) in LDS. */
    {
        const uint16_t *wt = Wt16 + (long)p * FOLD_ROWS * K;
        const uint16_t *yt = YT16 + (long)p * 256 * FOLD_ROWS;

        for (int i = tid; i < FOLD_ROWS * K / 8; i += 256) {
            const int row = i / (K / 8), c = i % (K / 8);

            *(u32x4 *)(Ws + swz_off(row, c, 2 * K)) = *(const u32x4 *)(wt + 8 * i);
        }
        for (int i = tid; i < 256 * FOLD_ROWS / 8; i += 256) {
            const int row = i / 8, c = i % 8;

            *(u32x4 *)(Ys + swz_off(row, c, 2 * FOLD_ROWS)) = *(const u32x4 *)(yt + 8 * i);
        }
        if (tid < FOLD_ROWS)
            bts[tid] = bt[p * FOLD_ROWS + tid];
    }
    __syncthreads();

    const int j = ch0 + 32 * w + l32;
    const bool valid = j < T;
    const float *xr = X + (long)p * xs + (long)(valid ? j : 0) * K;
    f32x16 s0 = {}, s1 = {};
    /* U^T accumulators (8 tiles of 32 channels x 32 tokens): register r of
     * tile c is channel 32 c + 8 (r / 4) + 4 hh + r % 4 of token l32. With
     * RX they start as the residual. */
    f32x16 u[8];

    for (int c = 0; c < 8; c++)
        u[c] = (f32x16){};

    if constexpr (RX) {
        /* S^T = Kc PQ^T first (while U^T holds nothing), one k step per
         * head: step i of tile T_ contracts head 4 T_ + i's 16 columns of
         * PQ (B operand: 8 of them for the lane's token), against A rows
         * (h, t) that are s k_{t,h} where h is that head and zero for the
         * other heads (rows 8 i .. 8 i + 7 of the tile, lanes l32 / 8 ==
         * i). */
        const uint16_t *pr = pq + (long)(valid ? j : 0) * 128 + 8 * hh;
        const bf16x8 k0 = *(const bf16x8 *)(kc + ((long)p * FOLD_ROWS + l32) * 16 + 8 * hh);
        const bf16x8 k1 = *(const bf16x8 *)(kc + ((long)p * FOLD_ROWS + 32 + l32) * 16 + 8 * hh);
        const bf16x8 zero = {};

        for (int i = 0; i < 4; i++) {
            const bf16x8 b0 = *(const bf16x8 *)(pr + 16 * i);
            const bf16x8 b1 = *(const bf16x8 *)(pr + 64 + 16 * i);
            const bool mine = (l32 >> 3) == i;

            s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mine ? k0 : zero, b0, s0, 0, 0, 0);
            s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(mine ? k1 : zero, b1, s1, 0, 0, 0);
        }
    }

    /* S^T = Wt X^T over K / 16 steps; the lane's B operand is 8
     * consecutive inputs of its token, converted to bf16. */
#pragma unroll(RX ? K / 16 : 4)
    for (int st = 0; st < K / 16; st++) {
        const int c0 = 16 * st + 8 * hh;
        f32x4 a0 = *(const f32x4 *)(xr + c0), a1 = *(const f32x4 *)(xr + c0 + 4);
        bf16x8 bx;

        if constexpr (RX) {
            /* Lane hh holds channels 16 st + 8 hh .. +7 of its token; U^T
             * wants channels 16 st + 4 hh .. +3 and 16 st + 8 + 4 hh .. +3
             * in lane hh: lane 0 keeps a0 and takes lane 1's a0, lane 1
             * keeps a1 and takes lane 0's a1. */
            f32x4 give = hh ? a0 : a1, got;

            for (int e = 0; e < 4; e++)
                got[e] = __shfl_xor(give[e], 32, 64);
            const f32x4 lo = hh ? got : a0, hi = hh ? a1 : got;

            for (int e = 0; e < 4; e++) {
                u[st / 2][8 * (st & 1) + e] = lo[e];
                u[st / 2][8 * (st & 1) + 4 + e] = hi[e];
            }
        }
        for (int e = 0; e < 4; e++) {
            bx[e] = (__bf16)a0[e];
            bx[4 + e] = (__bf16)a1[e];
        }
        const bf16x8 w0 = *(const bf16x8 *)(Ws + swz_off(l32, 2 * st + hh, 2 * K));
        const bf16x8 w1 = *(const bf16x8 *)(Ws + swz_off(32 + l32, 2 * st + hh, 2 * K));

        s0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w0, bx, s0, 0, 0, 0);
        s1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(w1, bx, s1, 0, 0, 0);
    }
    /* Every wave's reads of Wt are done past this point: the epilogue
     * reuses its LDS for staging. */
    __syncthreads();

    /* Grouped softmax: register r of tile T_ is row 32 T_ + 8 (r / 4) +
     * 4 hh + r % 4, i.e. head 4 T_ + r / 4 and prompt token 4 hh + r % 4:
     * each head's 8 scores are 4 registers here and 4 in lane l ^ 32. */
    for (int tt = 0; tt < 2; tt++) {
        f32x16 &sc = tt ? s1 : s0;

        for (int q = 0; q < 4; q++) {
            float m = -INFINITY, sum = 0.0f;

            for (int i = 0; i < 4; i++) {
                sc[4 * q + i] += bts[32 * tt + 8 * q + 4 * hh + i];
                m = fmaxf(m, sc[4 * q + i]);
            }
            m = fmaxf(m, __shfl_xor(m, 32, 64));
            for (int i = 0; i < 4; i++) {
                sc[4 * q + i] = __builtin_amdgcn_exp2f(sc[4 * q + i] - m);
                sum += sc[4 * q + i];
            }
            sum += __shfl_xor(sum, 32, 64);
            const float inv = 1.0f / sum;

            for (int i = 0; i < 4; i++)
                sc[4 * q + i] *= inv;
        }
    }

    /* U^T = Y^T A^T: 8 channel tiles x 4 k steps; the B operand of step st
     * is registers 8 (st % 2) .. + 7 of score tile st / 2. */
    for (int st = 0; st < 4; st++) {
        const f32x16 &sc = st < 2 ? s0 : s1;
        bf16x8 pb;

        for (int e = 0; e < 8; e++)
            pb[e] = (__bf16)sc[8 * (st & 1) + e];
        for (int c = 0; c < 8; c++) {
            const bf16x8 y = *(const bf16x8 *)(Ys + swz_off(32 * c + l32, 2 * st + hh, 2 * FOLD_ROWS));

            u[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(y, pb, u[c], 0, 0, 0);
        }
    }

    /* Epilogue through a per-wave [32 tokens][32 channels] fp32 staging
     * tile in the (now free) Wt area, so that the residual is read and the
     * output written as whole 128-byte row segments: in the coalesced
     * phase lane L takes token 8 k + L / 8, 16-byte chunk L % 8 of the
     * tile; chunk c of staging row r sits at c ^ (r & 7). Register r of
     * U^T tile c is channel 32 c + 8 (r / 4) + 4 hh + r % 4, i.e. chunk
     * 2 (r / 4) + hh of the tile's row l32. The barrier after the S^T
     * product guarantees every wave is done reading Wt. */
    /* Nothing of the epilogue is scheduled into the products above (its
     * loads would stay live across them and spill). */
    __builtin_amdgcn_sched_barrier(0);
    char *stg = Ws + 4096 * w;
    const int j0 = ch0 + 32 * w;
    const float *rbase = R + (long)p * rs;

    float sum = 0.0f;

#pragma unroll
    for (int c = 0; c < 8; c++) {
        if constexpr (RX) {
            /* The residual is already in u. */
            for (int q = 0; q < 4; q++) {
                const f32x4 b4 = *(const f32x4 *)(bo + 32 * c + 8 * q + 4 * hh);

                for (int i = 0; i < 4; i++) {
                    u[c][4 * q + i] += b4[i];
                    sum += u[c][4 * q + i];
                }
            }
            continue;
        }
        for (int k = 0; k < 4; k++) {
            /* Rows past T read row T - 1 (no branch around the load). */
            const int tok = 8 * k + (l >> 3), ck = l & 7;
            const int jr = j0 + tok < T ? j0 + tok : T - 1;
            const f32x4 v = *(const f32x4 *)(rbase + (long)jr * 256 + 32 * c + 4 * ck);

            *(f32x4 *)(stg + 128 * tok + 16 * (ck ^ (tok & 7))) = v;
        }
        for (int q = 0; q < 4; q++) {
            const f32x4 r4 = *(const f32x4 *)(stg + 128 * l32 + 16 * ((2 * q + hh) ^ (l32 & 7)));
            const f32x4 b4 = *(const f32x4 *)(bo + 32 * c + 8 * q + 4 * hh);

            for (int i = 0; i < 4; i++) {
                u[c][4 * q + i] += b4[i] + r4[i];
                sum += u[c][4 * q + i];
            }
        }
    }
    sum += __shfl_xor(sum, 32, 64);
    const float mean = sum * (1.0f / 256.0f);
    float var = 0.0f;

    for (int c = 0; c < 8; c++)
        for (int r = 0; r < 16; r++) {
            const float d = u[c][r] - mean;

            var = fmaf(d, d, var);
        }
    var += __shfl_xor(var, 32, 64);
    const float rsd = __builtin_amdgcn_rsqf(var * (1.0f / 256.0f) + eps);
    float *obase = out + (long)p * T * 256;

#pragma unroll
    for (int c = 0; c < 8; c++) {
        asm volatile("" ::: "memory");
        for (int q = 0; q < 4; q++) {
            const int ch = 32 * c + 8 * q + 4 * hh;
            const f32x4 g4 = *(const f32x4 *)(g + ch), b4 = *(const f32x4 *)(bln + ch);
            f32x4 y;

            for (int i = 0; i < 4; i++)
                y[i] = fmaf((u[c][4 * q + i] - mean) * rsd, g4[i], b4[i]);
            *(f32x4 *)(stg + 128 * l32 + 16 * ((2 * q + hh) ^ (l32 & 7))) = y;
        }
        for (int k = 0; k < 4; k++) {
            const int tok = 8 * k + (l >> 3), ck = l & 7;
            const f32x4 v = *(const f32x4 *)(stg + 128 * tok + 16 * (ck ^ (tok & 7)));

            if (j0 + tok < T)
                *(f32x4 *)(obase + (long)(j0 + tok) * 256 + 32 * c + 4 * ck) = v;
        }
    }
}

extern "C" int launch_i2t_fused(const float *X, long xs, int K, const void *pq16,
                                const void *Kc16, const void *Wt16, const float *bt,
                                const void *YT16, const float *bo,
                                const float *R, long rs, const float *g,
                                const float *b, float *out, int T, int P,
                                float eps, void *stream)
{
    /* K = 256 is layer 1 (residual = input, position term); K = 128 is
     * layer 0 (shared image queries, separate residual, no position
     * term). The grids of i2t_item, in 64-bit arithmetic so that sizes
     * past the grid limit are refused rather than wrapped. */
    const bool l1 = K == 256;
    const long C = T > 0 ? (T + 127) / 128 : 0;
    const long grid = P < 1 ? 0
                      : !l1 ? ((long)P * C + 7) / 8 * 8
                      : 8L * (P >= 8 ? (P + 7L) / 8 * C : P * ((C + 7) / 8));

    if (P < 1 || T < 1 || grid > 0x7fffffffL || (K != 128 && K != 256) ||
        ((xs | rs) & 3) || (l1 && (R != X || rs != xs || !pq16 || !Kc16)) ||
        (!l1 && (pq16 || Kc16)) ||
        (((uintptr_t)X | (uintptr_t)R | (uintptr_t)out | (uintptr_t)bo | (uintptr_t)bt |
          (uintptr_t)g | (uintptr_t)b | (uintptr_t)(l1 ? pq16 : X) |
          (uintptr_t)(l1 ? Kc16 : X) | (uintptr_t)Wt16 | (uintptr_t)YT16) & 15))
        return hipErrorInvalidValue;
    if (l1)
        hipLaunchKernelGGL((k_i2t_fused<256, true>), dim3((unsigned)grid), dim3(256), 0,
                           (hipStream_t)stream, X, xs, (const uint16_t *)pq16,
                           (const uint16_t *)Kc16, (const uint16_t *)Wt16, bt,
                           (const uint16_t *)YT16, bo, R, rs, g, b, out, T, P, eps);
    else
        hipLaunchKernelGGL((k_i2t_fused<128, false>), dim3((unsigned)grid), dim3(256), 0,
                           (hipStream_t)stream, X, xs, nullptr, nullptr,
                           (const uint16_t *)Wt16, bt, (const uint16_t *)YT16, bo, R,
                           rs, g, b, out, T, P, eps);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ */
/* Output upscaling and mask logits, fused                             */
/* ------------------------------------------------------------------ */

/* Per image token (y, x) of prompt p, from keys [P][T][256]:
 *   G1 = keys_j up0w (256 -> 64 channels x 4 pixels (dy, dx)),
 *   u1 = GELU(LN2d(G1 + up0b + feat_s1[2y + dy][2x + dx]))   (per pixel, 64 ch),
 *   G2 = u1 up3w (64 -> 32 channels x 4 sub-pixels (dy', dx')),
 *   u2 = GELU(G2 + up3b + feat_s0[4y + 2dy + dy'][4x + 2dx + dx']),
 *   lowres[p][k][4y + 2dy + dy'][4x + 2dx + dx'] = hyper[p][k] . u2 (k < 3),
 * the sequence of sam3_model.c:1357-1366 and mask_logits with none of the
 * [P][144][144][64] / [P][288][288][32] maps written.
 *
 * Products on bf16 MFMA, a wave per 32 tokens. G1^T = W1T keys^T: physical
 * output row 32 c + 8 q + 4 hh + i (tile c, D register 4 q + i, lane half
 * hh) is pixel dydx = c / 2, channel co = 32 (c % 2) + 16 (q / 2) + 8 hh +
 * 4 (q % 2) + i, so that registers 8 (s % 2) .. + 7 of tile 2 dydx + s / 2
 * are exactly the B operand (channels 16 s + 8 hh .. + 7) of k step s of
 * G2^T = W2T u1^T. G2 row 32 c2 + 8 q2 + 4 hh + i2 is sub-pixel dydx' = c2,
 * channel co' = 8 q2 + 4 hh + i2. */
__device__ __forceinline__ int up1_col(int row)
{
    const int c = row >> 5, q = (row >> 3) & 3, hh = (row >> 2) & 1, i = row & 3;
    const int co = 32 * (c & 1) + 16 * (q >> 1) + 8 * hh + 4 * (q & 1) + i;

    return co * 4 + (c >> 1);
}

/* G2 row 32 c2 + 8 q2 + 4 hh + i2 is sub-pixel c2, channel co' = 16 (q2 /
 * 2) + 8 hh + 4 (q2 % 2) + i2: registers 8 s .. 8 s + 7 of the tile are
 * then the B operand (channels 16 s + 8 hh .. + 7) of k step s of the
 * logits product. */
__device__ __forceinline__ int up2_col(int r2)
{
    const int c2 = r2 >> 5, q2 = (r2 >> 3) & 3, hh = (r2 >> 2) & 1, i2 = r2 & 3;

    return (16 * (q2 >> 1) + 8 * hh + 4 * (q2 & 1) + i2) * 4 + c2;
}

/* W1T16 [256][256] bf16: row r = up0w column up1_col(r) (over the 256
 * inputs); W2T16 [128][64]: row r2 = up3w column up2_col(r2). */
__global__ __launch_bounds__(256) void k_upscale_prep(const void *up0w, int dt0,
                                                      const void *up3w, int dt3,
                                                      uint16_t *__restrict__ W1T16,
                                                      uint16_t *__restrict__ W2T16)
{
    const int r = blockIdx.x, t = threadIdx.x;

    if (r < 256) {
        W1T16[r * 256 + t] = f2bf(wld(up0w, dt0, (long)t * 256 + up1_col(r)));
    }
    else {
        const int r2 = r - 256;

        if (t < 64)
            W2T16[r2 * 64 + t] = f2bf(wld(up3w, dt3, (long)t * 128 + up2_col(r2)));
    }
}

extern "C" int launch_upscale_prep(const void *up0w, int dt0, const void *up3w,
                                   int dt3, void *W1T16, void *W2T16,
                                   void *stream)
{
    hipLaunchKernelGGL(k_upscale_prep, dim3(256 + 128), dim3(256), 0,
                       (hipStream_t)stream, up0w, dt0, up3w, dt3,
                       (uint16_t *)W1T16, (uint16_t *)W2T16);
    return hipGetLastError();
}

/* Persistent: one 8-wave workgroup per CU keeps W1T (128 KB) and W2T
 * (16 KB) in LDS, XOR-swizzled by 16-byte chunk, and each wave walks the
 * (prompt, 32-token group) items with stride 8 x gridDim.x. */
__global__ __launch_bounds__(512, 1) void k_upscale_fused(
    const float *__restrict__ keys, const uint16_t *__restrict__ W1T16,
    const uint16_t *__restrict__ W2T16, const float *__restrict__ b0,
    const float *__restrict__ lnw, const float *__restrict__ lnb,
    const float *__restrict__ b3, const float *__restrict__ fs1,
    const float *__restrict__ fs0, const float *__restrict__ hyper,
    float *__restrict__ lowres, int G, int P, float eps)
{
    __shared__ __attribute__((aligned(16))) char W1s[256 * 512];
    __shared__ __attribute__((aligned(16))) char W2s[128 * 128];
    __shared__ __attribute__((aligned(16))) float vec[64 * 3 + 32];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, hh = l >> 5,
              l32 = l & 31;
    const int T = G * G, groups = (T + 31) / 32, L = 4 * G;
    const unsigned items = (unsigned)P * groups; /* < 2^31 (launcher) */

    for (int i = tid; i < 256 * 32; i += 512)
        *(u32x4 *)(W1s + swz_off(i / 32, i % 32, 512)) = *(const u32x4 *)(W1T16 + 8 * i);
    for (int i = tid; i < 128 * 8; i += 512)
        *(u32x4 *)(W2s + swz_off(i / 8, i % 8, 128)) = *(const u32x4 *)(W2T16 + 8 * i);
    if (tid < 64) {
        vec[tid] = b0[tid];
        vec[64 + tid] = lnw[tid];
        vec[128 + tid] = lnb[tid];
        if (tid < 32)
            vec[192 + tid] = b3[tid];
    }
    __syncthreads();
    const float *vb0 = vec, *vlw = vec + 64, *vlb = vec + 128, *vb3 = vec + 192;

    /* Items (32-token group, prompt) with the prompt fastest; XCD x (the
     * workgroups b with b % 8 == x) walks the x-th eighth of that list, so
     * the feature rows of a group, shared by the prompts, stay in its L2. */
    const unsigned per_xcd = (items + 7) / 8, ranks = gridDim.x / 8;
    const unsigned lo = (blockIdx.x % 8) * per_xcd;
    const unsigned hi = lo + per_xcd < items ? lo + per_xcd : items;

    for (unsigned item = lo + (blockIdx.x / 8) * 8 + w; item < hi; item += ranks * 8) {
        const int p = (int)(item % (unsigned)P);
        const int j = (int)(item / (unsigned)P) * 32 + l32;
        const bool valid = j < T;
        const int jj = valid ? j : 0, y = jj / G, x = jj % G;
        const float *kr = keys + ((long)p * T + jj) * 256;
        float *lr = lowres + (long)p * 3 * (16L * T);
        /* The token's 256 inputs as the 16 bf16 B operands of G1^T, read
         * once for the four pixels. */
        bf16x8 kb[16];

#pragma unroll
        for (int st = 0; st < 16; st++) {
            const int c0 = 16 * st + 8 * hh;
            const f32x4 a0 = *(const f32x4 *)(kr + c0), a1 = *(const f32x4 *)(kr + c0 + 4);

            for (int e = 0; e < 4; e++) {
                kb[st][e] = (__bf16)a0[e];
                kb[st][4 + e] = (__bf16)a1[e];
            }
        }
        /* A operand of the logits product: row l32 < 3 is mask l32's
         * hypernetwork output, channels 16 s + 8 hh .. + 7; rows 3..31
         * zero. */
        bf16x8 hyb[2];

        for (int s = 0; s < 2; s++) {
            const float *hr = hyper + p * 96 + 32 * (l32 < 3 ? l32 : 0) + 16 * s + 8 * hh;
            const f32x4 h0 = *(const f32x4 *)hr, h1 = *(const f32x4 *)(hr + 4);

            for (int e = 0; e < 4; e++) {
                hyb[s][e] = (__bf16)(l32 < 3 ? h0[e] : 0.0f);
                hyb[s][4 + e] = (__bf16)(l32 < 3 ? h1[e] : 0.0f);
            }
        }

        #pragma unroll 1
        for (int dy = 0; dy < 2; dy++) {
            /* Logits of this lane's two output rows' 4 columns per mask,
             * collected over dx, dx': lg[dy'][k][2 dx + dx']. */
            float lg[2][3][4];

            #pragma unroll
            for (int dx = 0; dx < 2; dx++) {
                asm volatile("" ::: "memory");
                const int px = 2 * dy + dx;
                const float *f1 = fs1 + ((long)(2 * y + dy) * (2 * G) + 2 * x + dx) * 64;
                float sum = 0.0f;
                /* G1^T tiles 2 px, 2 px + 1: this pixel's 64 channels. */
                f32x16 g1[2] = {};

                #pragma unroll
                for (int st = 0; st < 16; st++) {
                    #pragma unroll
                    for (int half = 0; half < 2; half++) {
                        const bf16x8 wa = *(const bf16x8 *)(W1s + swz_off(64 * px + 32 * half + l32,
                                                                          2 * st + hh, 512));

                        g1[half] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa, kb[st], g1[half], 0, 0, 0);
                    }
                }

                /* + up0b + feat_s1, LayerNorm2d over the pixel's 64
                 * channels. */
                #pragma unroll
                for (int half = 0; half < 2; half++) {
                    f32x16 &v = g1[half];

                    #pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int co = 32 * half + 16 * (q >> 1) + 8 * hh + 4 * (q & 1);
                        const f32x4 bb = *(const f32x4 *)(vb0 + co), ff = *(const f32x4 *)(f1 + co);

                        #pragma unroll
                        for (int i = 0; i < 4; i++) {
                            v[4 * q + i] += bb[i] + ff[i];
                            sum += v[4 * q + i];
                        }
                    }
                }
                sum += __shfl_xor(sum, 32, 64);
                const float mean = sum * (1.0f / 64.0f);
                float var = 0.0f;

                #pragma unroll
                for (int half = 0; half < 2; half++)
                    #pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const float d = g1[half][r] - mean;

                        var = fmaf(d, d, var);
                    }
                var += __shfl_xor(var, 32, 64);
                const float rs = __builtin_amdgcn_rsqf(var * (1.0f / 64.0f) + eps);
                bf16x8 ub[4];

                #pragma unroll
                for (int half = 0; half < 2; half++) {
                    const f32x16 &v = g1[half];

                    #pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const int co = 32 * half + 16 * (q >> 1) + 8 * hh + 4 * (q & 1);
                        const f32x4 gw = *(const f32x4 *)(vlw + co), gb = *(const f32x4 *)(vlb + co);

                        /* k step s = 2 half + q / 2, element 4 (q % 2) + i. */
                        #pragma unroll
                        for (int i = 0; i < 4; i++)
                            ub[2 * half + (q >> 1)][4 * (q & 1) + i] =
                                (__bf16)gelu_bf16path(fmaf((v[4 * q + i] - mean) * rs, gw[i], gb[i]));
                    }
                }
                /* Per sub-pixel tile c2: G2^T (4 k steps), + up3b + feat_s0,
                 * GELU, then the logits as a product of the prompt's
                 * hypernetwork rows (3 of 32 used) with u2^T. */
                #pragma unroll
                for (int c2 = 0; c2 < 4; c2++) {
                    const int dyp = c2 >> 1, dxp = c2 & 1;
                    const float *f0 = fs0 + ((long)(4 * y + 2 * dy + dyp) * (4 * G) + 4 * x + 2 * dx + dxp) * 32;
                    f32x16 g2 = {}, d3 = {};

                    #pragma unroll
                    for (int s = 0; s < 4; s++) {
                        const bf16x8 wa = *(const bf16x8 *)(W2s + swz_off(32 * c2 + l32, 2 * s + hh, 128));

                        g2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wa, ub[s], g2, 0, 0, 0);
                    }
                    #pragma unroll
                    for (int s = 0; s < 2; s++) {
                        bf16x8 ub2;

                        #pragma unroll
                        for (int h2 = 0; h2 < 2; h2++) {
                            const int co = 16 * s + 8 * hh + 4 * h2;
                            const f32x4 bb = *(const f32x4 *)(vb3 + co), ff = *(const f32x4 *)(f0 + co);

                            #pragma unroll
                            for (int i = 0; i < 4; i++)
                                ub2[4 * h2 + i] = (__bf16)gelu_bf16path(g2[8 * s + 4 * h2 + i] + bb[i] + ff[i]);
                        }
                        d3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(hyb[s], ub2, d3, 0, 0, 0);
                    }
                    /* Rows 0..2 (the masks) are registers 0..2 of lanes
                     * 0..31. */
                    #pragma unroll
                    for (int k = 0; k < 3; k++)
                        lg[dyp][k][2 * dx + dxp] = d3[k];
                }
            }
            /* Lanes 0..31 store output rows 4 y + 2 dy + dy' of each mask. */
            if (valid && hh == 0)
                #pragma unroll
                for (int dyp = 0; dyp < 2; dyp++) {
                    const int Y = 4 * y + 2 * dy + dyp;

                    #pragma unroll
                    for (int k = 0; k < 3; k++) {
                        const f32x4 o = {lg[dyp][k][0], lg[dyp][k][1], lg[dyp][k][2], lg[dyp][k][3]};

                        *(f32x4 *)(lr + (long)k * 16 * T + (long)Y * L + 4 * x) = o;
                    }
                }
        }
    }
}

extern "C" int launch_upscale_fused(const float *keys, const void *W1T16,
                                    const void *W2T16, const float *b0,
                                    const float *lnw, const float *lnb,
                                    const float *b3, const float *fs1,
                                    const float *fs0, const float *hyper,
                                    float *lowres, int G, int P, float eps,
                                    int cus, void *stream)
{
    const long T = (long)G * G, items = (long)P * ((T + 31) / 32);
    /* A multiple of 8 workgroups (the XCD split of the item list), at most
     * one per CU. */
    const long fill = ((items + 7) / 8 < cus ? (items + 7) / 8 : cus) / 8 * 8;
    const long grid = fill > 8 ? fill : 8;

    if (P < 1 || G < 1 || cus < 1 || items + 8L * cus > 0x7fffffffL ||
        ((uintptr_t)hyper & 15) ||
        (((uintptr_t)keys | (uintptr_t)W1T16 | (uintptr_t)W2T16 |
          (uintptr_t)b0 | (uintptr_t)lnw | (uintptr_t)lnb | (uintptr_t)b3 |
          (uintptr_t)fs1 | (uintptr_t)fs0 | (uintptr_t)lowres) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_upscale_fused, dim3((unsigned)grid), dim3(512), 0,
                       (hipStream_t)stream, keys, (const uint16_t *)W1T16,
                       (const uint16_t *)W2T16, b0, lnw, lnb, b3, fs1, fs0,
                       hyper, lowres, G, P, eps);
    return hipGetLastError();
}


/* ------------------------------------------------------------------ */
/* Token -> image attention on per-prompt keys, fused                  */
/* ------------------------------------------------------------------ */

/* For prompt p, head h, prompt token i (row r = 8 h + i):
 *   score(r, j) = s q_{i,h} . (Wk_h (keys_j + PE_j) + bk_h)
 *               = U[r] . keys_j + Qc[r] . PK_{j,h} + const(r),
 *   U[r] = s Wk_h^T q_{i,h} (k_i2t_fold on the projected queries),
 *   Qc[r] = s q_{i,h} (16 wide), PK_j = Wk PE_j (128 wide, per image),
 *   o_{i,h} = Wv_h (sum_j a(r, j) keys_j) + bv_h = Wv_h Z[r] + bv_h;
 * the constant drops out of the softmax. k_t2i_fused: workgroup =
 * (prompt, key split), 4 waves = 2 row tiles x 2 key streams; per 64-key
 * block the workgroup stages keys [64 keys][256] and keys^T [256][64
 * keys] in LDS as bf16, and each wave does S^T = keys U^T + PK Qc^T (32
 * keys x 32 rows, rows = lanes; PK straight from global memory, 256 bytes
 * per key instead of PE's 1 KB), the online softmax, and Z^T += keys^T
 * P^T (256 x 32). The two streams of a row tile merge through LDS; each
 * split leaves (Z, m, l) partials for k_t2i_merge; k_t2i_unfold applies
 * Wv and bv. */

/* Byte offset of keys^T element (dim d, key k) in a [256][64] bf16 tile:
 * rows of 128 B, 16-byte chunk k / 8 at chunk (k / 8) ^ ((d >> 1) & 7). */
__device__ __forceinline__ unsigned vt_off(int d, int k)
{
    return (unsigned)(d * 128 + 16 * ((k >> 3) ^ ((d >> 1) & 7)) + 2 * (k & 7));
}

__global__ __launch_bounds__(256, 2) void k_t2i_fused(
    const float *__restrict__ keys, const uint16_t *__restrict__ pk,
    const uint16_t *__restrict__ U16, const uint16_t *__restrict__ Qc16,
    float *__restrict__ part, int T, int P, int nsplit)
{
    __shared__ __attribute__((aligned(16))) char Ks[64 * 512];
    __shared__ __attribute__((aligned(16))) char Vs[256 * 128];
    const int tid = threadIdx.x, l = tid & 63, w = tid >> 6, hh = l >> 5,
              l32 = l & 31;
    const int rt = w & 1, kh = w >> 1;
    /* XCD-contiguous items, split fastest: one XCD's workgroups take
     * whole prompts (1/8 of them), so the U rows each block re-reads stay
     * in that XCD's L2 (a few prompts' worth), and the shared PK rows
     * (256 bytes a key) of a split are read by the XCD's prompts
     * together. */
    const unsigned total = (unsigned)P * nsplit, per_xcd = (total + 7) / 8;
    const unsigned item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;

    if (item >= total)
        return;
    const int p = (int)(item / (unsigned)nsplit), sp = (int)(item % (unsigned)nsplit);
    const int nblk = (T + 63) / 64;
    const int kb0 = sp * nblk / nsplit, kb1 = (sp + 1) * nblk / nsplit;
    const float *kp = keys + (long)p * T * 256;
    const int row = 32 * rt + l32;

    /* U^T B operands of this lane's row come from the cache each block. */
    const uint16_t *ur = U16 + ((long)p * FOLD_ROWS + row) * 256 + 8 * hh;
    f32x16 z[8];
    for (int dt = 0; dt < 8; dt++)
        z[dt] = (f32x16){};
    float m = -INFINITY, lsum = 0.0f;
    const int krow = 32 * kh + ((l32 & ~12) | ((l32 & 4) << 1) | ((l32 & 8) >> 1));
    /* Qc^T B operands (8 of the 16 values of the lane's row) and whether
     * the row's head is that of k step i (head 4 rt + i): l32 / 8 == i. */
    const bf16x8 qc = *(const bf16x8 *)(Qc16 + ((long)p * FOLD_ROWS + row) * 16 + 8 * hh);
    const int qstep = l32 >> 3;

    for (int kb = kb0; kb < kb1; kb++) {
        /* PK A operands of this wave's 32 keys (kperm order) on the row
         * tile's four heads; rows past T read row T - 1 (their scores are
         * masked below). Issued before the staging so the loads overlap
         * it. */
        bf16x8 pka[4];
        {
            const int key = kb * 64 + krow;
            const uint16_t *pr = pk + (long)(key < T ? key : T - 1) * 128 + 64 * rt + 8 * hh;

            for (int i = 0; i < 4; i++)
                pka[i] = *(const bf16x8 *)(pr + 16 * i);
        }
        /* Stage: task = (8-dim chunk c, key pair) with c fastest, so a
         * wave reads two contiguous 1 KB rows; keys past T are zero. */
        for (int task = tid; task < 32 * 32; task += 256) {
            const int c = task & 31, k0 = 2 * (task >> 5);
            f32x4 a[2][2];

            for (int e = 0; e < 2; e++) {
                const int key = kb * 64 + k0 + e;

                if (key < T) {
                    const float *kr = kp + (long)key * 256 + 8 * c;

                    a[e][0] = *(const f32x4 *)kr;
                    a[e][1] = *(const f32x4 *)(kr + 4);
                }
                else {
                    a[e][0] = a[e][1] = (f32x4){};
                }
            }
            for (int e = 0; e < 2; e++) {
                bf16x8 kin;

                for (int i = 0; i < 4; i++) {
                    kin[i] = (__bf16)a[e][0][i];
                    kin[4 + i] = (__bf16)a[e][1][i];
                }
                *(bf16x8 *)(Ks + swz_off(k0 + e, c, 512)) = kin;
            }
            for (int i = 0; i < 8; i++) {
                const float v0 = i < 4 ? a[0][0][i] : a[0][1][i - 4];
                const float v1 = i < 4 ? a[1][0][i] : a[1][1][i - 4];

                *(uint32_t *)(Vs + vt_off(8 * c + i, k0)) = pack_bf16x2(v0, v1);
            }
        }
        __syncthreads();

        /* S^T for this wave's 32 keys (A rows in kperm order) x 32 rows;
         * the fence keeps the U loads here rather than hoisted into 64
         * registers for the whole loop. */
        asm volatile("" ::: "memory");
        f32x16 sc = {};

        for (int st = 0; st < 16; st++) {
            const bf16x8 ka = *(const bf16x8 *)(Ks + swz_off(krow, 2 * st + hh, 512));
            const bf16x8 ub = *(const bf16x8 *)(ur + 16 * st);

            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka, ub, sc, 0, 0, 0);
        }
        {
            const bf16x8 zero = {};

            for (int i = 0; i < 4; i++)
                sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pka[i], qstep == i ? qc : zero,
                                                            sc, 0, 0, 0);
        }
        /* Register r of lane half hh is key 32 kh + 16 (r / 8) + 8 hh + r % 8. */
        for (int r = 0; r < 16; r++) {
            const int key = kb * 64 + 32 * kh + 16 * (r >> 3) + 8 * hh + (r & 7);

            if (key >= T)
                sc[r] = -INFINITY;
        }
        float bm = -INFINITY;

        for (int r = 0; r < 16; r++)
            bm = __builtin_fmaxf(bm, sc[r]);
        bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
        /* Lazy rescale: m moves only when a score passes it by 2^8. */
        if (bm > m + 8.0f) {
            const float corr = __builtin_amdgcn_exp2f(m - bm);

            lsum *= corr;
            for (int dt = 0; dt < 8; dt++)
                for (int r = 0; r < 16; r++)
                    z[dt][r] *= corr;
            m = bm;
        }
        bf16x8 pb[2];
        /* No finite score in this stream yet: every exp2 below is 0. */
        const float mref = m == -INFINITY ? 0.0f : m;

        for (int r = 0; r < 16; r++) {
            const float e = __builtin_amdgcn_exp2f(sc[r] - mref);

            lsum += e;
            pb[r >> 3][r & 7] = (__bf16)e;
        }
        /* Z^T += keys^T P^T: 8 dim tiles x 2 k steps of 16 keys. */
        for (int a = 0; a < 2; a++)
            for (int dt = 0; dt < 8; dt++) {
                const bf16x8 va = *(const bf16x8 *)(Vs + vt_off(32 * dt + l32, 32 * kh + 16 * a + 8 * hh));

                z[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb[a], z[dt], 0, 0, 0);
            }
        __syncthreads();
    }
    lsum += __shfl_xor(lsum, 32, 64);

    /* Merge the key streams of each row tile through LDS (the staging
     * tiles are free after the last barrier; row l32's 256 values are
     * stored with their float4 slots XOR 4 l32): stream 1 writes (m, l,
     * Z^T), stream 0 combines and stores the split's partial record:
     * part [p][split][64 rows][256] then [p][split][64][2]. */
    float *zs = (float *)(rt ? Vs : Ks); /* 32 rows x 256 = 32 KB per tile */
    __shared__ float mls[2][32][2];

    if (kh == 1) {
        for (int dt = 0; dt < 8; dt++)
            for (int q = 0; q < 4; q++) {
                const int d = 32 * dt + 8 * q + 4 * hh;
                const f32x4 v = {z[dt][4 * q], z[dt][4 * q + 1], z[dt][4 * q + 2], z[dt][4 * q + 3]};

                *(f32x4 *)(zs + l32 * 256 + (d ^ (4 * l32))) = v;
            }
        if (hh == 0) {
            mls[rt][l32][0] = m;
            mls[rt][l32][1] = lsum;
        }
    }
    __syncthreads();
    if (kh == 0) {
        const float m1 = mls[rt][l32][0], l1 = mls[rt][l32][1];
        const float mm = fmaxf(m, m1);
        const float c0 = m == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m - mm);
        const float c1 = m1 == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m1 - mm);
        const long rec = ((long)p * nsplit + sp) * FOLD_ROWS + row;
        float *zo = part + rec * 256;

        for (int dt = 0; dt < 8; dt++)
            for (int q = 0; q < 4; q++) {
                const int d = 32 * dt + 8 * q + 4 * hh;
                const f32x4 v1 = *(const f32x4 *)(zs + l32 * 256 + (d ^ (4 * l32)));
                f32x4 o;

                for (int i = 0; i < 4; i++)
                    o[i] = z[dt][4 * q + i] * c0 + v1[i] * c1;
                *(f32x4 *)(zo + d) = o;
            }
        if (hh == 0) {
            float *ml = part + (long)P * nsplit * FOLD_ROWS * 256 + rec * 2;

            ml[0] = mm;
            ml[1] = lsum * c0 + l1 * c1;
        }
    }
}

/* Z [P][64][256] from the nsplit partial records: thread per (p, row, d). */
__global__ __launch_bounds__(256) void k_t2i_merge(const float *__restrict__ part,
                                                   float *__restrict__ Z, int P,
                                                   int nsplit)
{
    const long gid = (long)blockIdx.x * 256 + threadIdx.x;

    if (gid >= (long)P * FOLD_ROWS * 256)
        return;
    const int d = (int)(gid & 255);
    const long pr = gid >> 8; /* p * 64 + row */
    const int p = (int)(pr / FOLD_ROWS), row = (int)(pr % FOLD_ROWS);
    const float *ml = part + (long)P * nsplit * FOLD_ROWS * 256;
    float M = -INFINITY;

    for (int s = 0; s < nsplit; s++)
        M = fmaxf(M, ml[(((long)p * nsplit + s) * FOLD_ROWS + row) * 2]);
    float num = 0.0f, den = 0.0f;

    for (int s = 0; s < nsplit; s++) {
        const long rec = ((long)p * nsplit + s) * FOLD_ROWS + row;
        const float ms = ml[rec * 2];
        const float wgt = ms == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ms - M);

        num = fmaf(wgt, part[rec * 256 + d], num);
        den = fmaf(wgt, ml[rec * 2 + 1], den);
    }
    Z[gid] = num / den;
}

/* o [P][8][128]: o[p][i][16 h + c] = Wv[16 h + c] . Z[p][8 h + i] + bv.
 * Workgroup (p, h): Z rows 8 h .. + 7 and Wv rows 16 h .. + 15 staged in
 * LDS (Wv rows padded to 257 floats), thread (i, c) one dot product. */
__global__ __launch_bounds__(128) void k_t2i_unfold(const float *__restrict__ Z,
                                                    const void *Wv, int wv_dt,
                                                    const float *__restrict__ bv,
                                                    float *__restrict__ o, int P)
{
    __shared__ float zs[8][256], ws[16][257];
    const int p = blockIdx.x, h = blockIdx.y, t = threadIdx.x;
    const float *zr = Z + ((long)p * FOLD_ROWS + 8 * h) * 256;

    for (int x = t; x < 8 * 256; x += 128)
        zs[x / 256][x % 256] = zr[x];
    for (int x = t; x < 16 * 256; x += 128)
        ws[x / 256][x % 256] = wld(Wv, wv_dt, (long)16 * h * 256 + x);
    __syncthreads();
    const int i = t / 16, c = t % 16;
    float acc = bv[16 * h + c];

    for (int d = 0; d < 256; d++)
        acc = fmaf(ws[c][d], zs[i][d], acc);
    o[((long)p * 8 + i) * 128 + 16 * h + c] = acc;
}

extern "C" int launch_t2i_fused(const float *keys, const void *pk16,
                                const void *U16, const void *Qc16, float *part,
                                float *Z, const void *Wv, int wv_dt,
                                const float *bv, float *o, int T, int P,
                                int nsplit, void *stream)
{
    const int nblk = (T + 63) / 64;
    const long n = (long)P * FOLD_ROWS * 256;

    if (P < 1 || T < 1 || nsplit < 1 || nsplit > nblk ||
        (long)P * nsplit > 0x7fffffffL || !pk16 || !Qc16 ||
        (((uintptr_t)keys | (uintptr_t)pk16 | (uintptr_t)U16 | (uintptr_t)Qc16 |
          (uintptr_t)part) & 15))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_t2i_fused, dim3((unsigned)((P * nsplit + 7) / 8 * 8)),
                       dim3(256), 0, (hipStream_t)stream, keys,
                       (const uint16_t *)pk16, (const uint16_t *)U16,
                       (const uint16_t *)Qc16, part, T, P, nsplit);
    hipLaunchKernelGGL(k_t2i_merge, dim3((unsigned)((n + 255) / 256)), dim3(256),
                       0, (hipStream_t)stream, part, Z, P, nsplit);
    hipLaunchKernelGGL(k_t2i_unfold, dim3(P, 8), dim3(128), 0, (hipStream_t)stream,
                       Z, Wv, wv_dt, bv, o, P);
    return hipGetLastError();
}

/* ------------------------------------------------------------------ */
/* Hypernetwork MLPs and IoU head                                      */
/* ------------------------------------------------------------------ */

/* Workgroup (prompt p, head k): k = 0 the IoU head on token 1 (4 raw
 * outputs into iou [P][4]), k = 1..3 the hypernetwork MLP of mask token
 * k on token 2 + k (32 outputs into hyper [P][3][32]); three Linear
 * layers 256 -> 256 (ReLU) -> 256 (ReLU) -> nout, the layer input in LDS,
 * thread o one output. W*[k] are [256][256], [256][256], [nout][256]. */
struct dec_heads_w {
    const void *w0[4], *w1[4], *w2[4];
    const float *b0[4], *b1[4], *b2[4];
    int dt;
};

/* Output o = thread: its weight row as 16-byte loads, all independent
 * (bf16 rows: 32 loads of 8; fp32 rows: 64 loads of 4), against the layer
 * input in LDS. */
__device__ __forceinline__ float row_dot(const void *W, int dt, int o,
                                         const float *x)
{
    float acc = 0.0f;

    if (dt == DT_BF16) {
        const bf16x8 *r = (const bf16x8 *)((const uint16_t *)W + (long)o * 256);

#pragma unroll 8
        for (int c = 0; c < 32; c++) {
            const bf16x8 v = r[c];

            for (int e = 0; e < 8; e++)
                acc = fmaf((float)v[e], x[8 * c + e], acc);
        }
    }
    else
        for (int i = 0; i < 256; i++)
            acc = fmaf(wld(W, dt, (long)o * 256 + i), x[i], acc);
    return acc;
}

__global__ __launch_bounds__(256) void k_dec_heads(const float *__restrict__ qry,
                                                   dec_heads_w hw,
                                                   float *__restrict__ hyper,
                                                   float *__restrict__ iou)
{
    __shared__ float xa[256], xb[256];
    const int p = blockIdx.x, k = blockIdx.y, t = threadIdx.x;
    const int tok = k ? 2 + k : 1, nout = k ? 32 : 4;

    xa[t] = qry[((long)p * 8 + tok) * 256 + t];
    __syncthreads();
    xb[t] = fmaxf(row_dot(hw.w0[k], hw.dt, t, xa) + hw.b0[k][t], 0.0f);
    __syncthreads();
    xa[t] = fmaxf(row_dot(hw.w1[k], hw.dt, t, xb) + hw.b1[k][t], 0.0f);
    __syncthreads();
    if (t < nout) {
        const float v = row_dot(hw.w2[k], hw.dt, t, xa) + hw.b2[k][t];

        if (k)
            hyper[(long)p * 96 + (k - 1) * 32 + t] = v;
        else
            iou[(long)p * 4 + t] = v;
    }
}

extern "C" int launch_dec_heads(const float *qry, const void *const w0[4],
                                const void *const w1[4], const void *const w2[4],
                                const float *const b0[4], const float *const b1[4],
                                const float *const b2[4], int dt, float *hyper,
                                float *iou, int P, void *stream)
{
    dec_heads_w hw;

    for (int k = 0; k < 4; k++) {
        hw.w0[k] = w0[k];
        hw.w1[k] = w1[k];
        hw.w2[k] = w2[k];
        hw.b0[k] = b0[k];
        hw.b1[k] = b1[k];
        hw.b2[k] = b2[k];
    }
    hw.dt = dt;
    if (P < 1)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_dec_heads, dim3(P, 4), dim3(256), 0, (hipStream_t)stream,
                       qry, hw, hyper, iou);
    return hipGetLastError();
}
