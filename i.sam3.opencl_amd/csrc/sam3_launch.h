/* SPDX-License-Identifier: Unlicense
 *
 * Internal interface between the C host layer (hip_backend.c,
 * sam3_ops.c) and the HIP kernels (*.hip). Every launcher is extern "C",
 * takes device pointers, sizes and a hipStream_t (as void *), queues its
 * kernel(s) on that stream and returns the hipError_t of the launch
 * (0 = hipSuccess). Shapes are validated by the callers.
 */
#ifndef SAM3_LAUNCH_H
#define SAM3_LAUNCH_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types, the HIPB_* values of sam3_hip.h. */
#define DT_F32 0
#define DT_F16 1
#define DT_BF16 2

/* MFMA arithmetic of a GEMM or attention launch. */
#define MODE_F32 0  /* v_mfma_f32_32x32x2_f32, fp32 operands */
#define MODE_BF16 1 /* v_mfma_f32_32x32x16_bf16, f32 accumulation */

/* Batched GEMM with the reference contract (sam3_kernels.cl:57-69). */
struct gemm_desc {
    int M, N, K;
    const void *A;
    long aoff;
    int lda;
    long sa0, sa1;
    int adt;
    const void *B;
    long boff;
    int ldb;
    long sb0, sb1;
    int bdt, transb;
    void *C;
    long coff;
    int ldc;
    long sc0, sc1;
    int cdt;
    int nb, nb1;
    const float *bias;
    const void *R; /* same type and layout as C */
    long roff;
    float alpha;
    int act;
    int mode;
    /* NT kernel only: with ws > 0, output row m is window-partition
     * position m of an H x H grid (nwx windows per side) and C / R rows
     * are its grid token (padding rows are dropped): the projection's
     * window_unpartition_add fused into the store. */
    int unpart_H, unpart_ws, unpart_nwx;
    /* NT kernel only: with pack_N > 0 the product is a QKV projection
     * (N = 3 pack_E columns, q | k | v thirds of 64-wide heads; rows are
     * units of pack_N tokens, pack_N % 64 == 0) and the store writes the
     * attention operands of launch_qkv_pack instead of C: q16 / k16
     * [unit][pack_N][64] bf16 with RoPE (pack_rope, pack_npos positions;
     * q also scaled by pack_scale log2 e), vt16 [unit][64][pack_N], and
     * knorm per 64-key block; unit = row / pack_N * heads + head. */
    int pack_N, pack_E, pack_npos;
    float pack_scale;
    const float *pack_rope;
    void *pack_q16, *pack_k16, *pack_vt16;
    float *pack_knorm;
};
int launch_gemm(const struct gemm_desc *d, void *stream);
/* The bf16 x bf16 "NT" kernel (A [M][K], B [N][K], K % 64 == 0,
 * unbatched); -1 if d does not have that form, else a hipError_t. */
int launch_gemm_nt(const struct gemm_desc *d, void *stream);
int gemm_nt_ok(const struct gemm_desc *d);

/* Row LayerNorm of rows x C floats into Y (float or bf16). With ws > 0
 * the output rows are the window-partitioned order of an H x H grid
 * (nwx windows per side, zero rows for padding): row count nwx^2 ws^2. */
int launch_layernorm(const float *X, void *Y, int ydt, const float *g,
                     const float *b, long rows, int C, float eps, int act,
                     int H, int ws, int nwx, void *stream);

int launch_softmax_rows(float *S, long rows, int L, void *stream);
/* softmax_ext: causal mask or box bias, then the row softmax; rows =
 * heads x Nq, heads from h0 (dy / dx NULL for no bias). */
int launch_softmax_ext(float *S, long rows, int L, int Nq, int h0, int causal,
                       const float *dy, const float *dx, int W, int nh,
                       void *stream);
int launch_rope_apply(float *qkv, long rows, int E, int hd, int npos,
                      const float *cs, void *stream);
int launch_window_partition(const float *X, float *out, int H, int W, int C,
                            int ws, int nwx, void *stream);
int launch_window_unpartition_add(float *X, const float *Wd, int H, int W,
                                  int C, int ws, int nwx, void *stream);
int launch_add_bcast(float *out, const float *a, const float *b, long n,
                     long bmod, void *stream);
/* Patch im2col of a 3 x side x side image into grid^2 rows of 3 ps^2
 * float (ydt DT_F32) or bf16 (DT_BF16) columns, rows ldo >= 3 ps^2 apart
 * with the columns past 3 ps^2 zero. */
int launch_patch_im2col(const float *img, void *out, int ydt, int side,
                        int grid, int ps, int ldo, void *stream);
/* rows x K float or bf16 (sdt) into rows x KP bf16, columns K.. zero. */
int launch_pad_rows_bf16(const void *src, int sdt, void *dst, long rows, int K,
                         int KP, void *stream);

/* Fused attention over nb units of N tokens, head width 64. */
struct attn_desc {
    int N, nb, nb1;
    const void *Q;
    long qoff;
    int ldq;
    long sq0, sq1;
    const void *K;
    long koff;
    int ldk;
    long sk0, sk1;
    const void *V;
    long voff;
    int ldv;
    long sv0, sv1;
    void *O;
    long ooff;
    int ldo;
    long so0, so1;
    int odt;
    const float *rope; /* (cos, sin) x 32 per position, or NULL */
    int npos;
    float scale;
    /* Head width: 64, or 32 on the bf16 path (packed with zero channels
     * 32..63, so the 64-wide kernel applies; 32 output columns stored). */
    int hd;
    /* Keys per unit (N queries, Nk keys; K and V rows count Nk); beyond
     * Nk == N: the box bias as rows [unit][N][H + W] of dy then dx values
     * (launch_box_rows, H = Nk / bW; bW >= 64 a multiple of 8, H of 4;
     * on the bf16 path at head width 32 only), each key
     * j biased by dy[j / bW] + dx[j % bW], or with bW = 0 as a table
     * [unit][N][Nk padded to 64] (launch_box_bias), on the bf16 path
     * scaled to its exp2 domain; or NULL; and the
     * causal mask (key j > query i excluded). */
    int Nk;
    const float *bias;
    int bW;
    int causal;
};

/* fp32 operands, f32 MFMA, RoPE applied on the Q/K loads, the scale to
 * the scores; N queries over Nk keys, head width 64 or 32 (no RoPE), the
 * causal mask or the box bias (d->bias rows, d->bW) in natural units. With 1 < nsplit <= 64 the 32-key blocks
 * are split nsplit ways in the same launch: `part` (nb ceil(N / 128)
 * SPLIT_RECS(nsplit) 9216 floats) holds the records and `cnt` (nb
 * ceil(N / 128) SPLIT_CNT counts) the arrival counts. */
int launch_attn_f32(const struct attn_desc *d, float *part, unsigned *cnt, int nsplit,
                    void *stream);

/* Packed bf16 staging of the fast path, Np = N rounded up to 64:
 * q16/k16 [nb][Np][64] (RoPE applied, q scaled), vt16 [nb][64][Np],
 * zero in the padding; knorm [nb][Np / 64] floats, the largest |k| of
 * each 64-key block (of the bf16 keys, rounded up). */
int launch_qkv_pack(const struct attn_desc *d, void *q16, void *k16,
                    void *vt16, float *knorm, void *stream);

/* Key splits merged inside their launch (both attention paths): per
 * 128-query tile SPLIT_RECS(nsplit) records of 9216 floats (the splits',
 * then one per group of SPLIT_GROUP splits) and SPLIT_CNT arrival counts,
 * zero before a launch and left zero by it. */
#define SPLIT_GROUP 8
#define SPLIT_CNT (SPLIT_GROUP + 1)
#define SPLIT_RECS(ns) ((ns) + ((ns) + SPLIT_GROUP - 1) / SPLIT_GROUP)

/* bf16 MFMA attention on the packed operands; O addressed as in d. With
 * 1 < nsplit <= 64 the key blocks are split nsplit ways and merged inside
 * the launch: `part` (nb ceil(N / 128) SPLIT_RECS(nsplit) 9216 floats)
 * holds the records and skcnt the counts (nb ceil(N / 128) SPLIT_CNT).
 * With skG > 0 (nsplit 1, head width 64 without
 * bias or causal mask) the tiles of each XCD's share (the tile list in
 * eight contiguous parts) go to skdp whole-tile workgroups and skG
 * workgroups that share the rest's (tile, key block) pairs evenly:
 * skrec holds ATTN_SK_REC_FLOATS floats per stream-K workgroup (8 skG of
 * them), skcnt one counter per 128-query tile (nb ceil(N / 128)), zero
 * before the first launch and left zero by every launch. */
#define ATTN_SK_REC_FLOATS (2 * 4 * 34 * 64)
int launch_attn_bf16(const struct attn_desc *d, const void *q16,
                     const void *k16, const void *vt16, const float *knorm,
                     float *part, int nsplit, float *skrec, unsigned *skcnt,
                     int skG, int skdp, void *stream);
/* The same attention in one launch for shapes with too few query tiles
 * to fill the device: ng (2 or 4) groups of waves in each workgroup take
 * contiguous key ranges and merge in LDS (head width 64, no bias or causal
 * mask, at least ng key blocks). */
int launch_attn_bf16_grp(const struct attn_desc *d, const void *q16, const void *k16,
                         const void *vt16, const float *knorm, int ng, void *stream);
/* Zero the n counters of launch_attn_bf16's balanced launch. */
int launch_attn_sk_zero(unsigned *cnt, long n, void *stream);

/* Additive bias table of the fused attention from the box relative
 * position bias of softmax_ext, for grids the bias rows do not take:
 * out [heads][Nq][Nk padded to 64] = unit_scale (dy[(i H + j / W) nh + h]
 * + dx[(i W + j % W) nh + h]), -inf in the padding (H = Nk / W);
 * unit_scale log2(e) for the bf16 kernel, 1 for the exact path. */
int launch_box_bias(float *out, const float *dy, const float *dx, int heads,
                    int Nq, int Nk, int W, int nh, float unit_scale, void *stream);

/* Bias rows of the fused attention from the box relative position bias
 * of softmax_ext: out [heads][Nq][H + W] = unit_scale dy[(i H + y) nh + h]
 * (y < H), then unit_scale dx[(i W + x) nh + h] (x < W), H = Nk / W;
 * unit_scale 1 for the exact path, log2(e) for the bf16 kernel. */
int launch_box_rows(float *out, const float *dy, const float *dx, int heads, int Nq,
                    int Nk, int W, int nh, float unit_scale, void *stream);

/* Decoder attention (8 heads, head width c = dint / 8). */
int launch_mha_fewkeys(const float *Q, long sq, const float *K, long sk,
                       const float *V, long sv, float *O, int P, int Nq,
                       int Nk, int dint, float scale, void *stream);
/* precision=bf16 few-keys attention for dint 256 (head width 32), Nk <= 8,
 * 16-byte aligned rows: four lanes per (prompt, query, head). */
int launch_mha_few32x4(const float *Q, long sq, const float *K, long sk,
                       const float *V, long sv, float *O, int P, int Nq,
                       int Nk, int dint, float scale, void *stream);
/* Split-K token->image attention for c == 16; scratch holds the
 * partial results, mha_manykeys_scratch() bytes (0 when the key range is
 * not split: scratch may then be NULL). */
size_t mha_manykeys_scratch(int P, int Nq, int Nk);
/* Bytes of the static device scratch mha_noalloc uses for those partials
 * (8 MiB: more than the many-keys split rule ever asks, about 4.7 MB at
 * most); dec_scratch_init(device), with that device current, resolves
 * its address on that device (hipb_init calls it), dec_scratch(device)
 * returns it (NULL before). */
#define MHA_NOALLOC_BYTES ((size_t)8 << 20)
int dec_scratch_init(int device);
void *dec_scratch(int device);
int launch_mha_manykeys(const float *Q, long sq, const float *K, long sk,
                        const float *V, long sv, float *O, int P, int Nq,
                        int Nk, int dint, float scale, void *scratch,
                        void *stream);

/* Output upscaling scatter of a 2x2 / stride-2 transposed convolution:
 * G [(P H W)][Co 4] -> out [P][2H][2W][Co] = act(G + bias[co] (+ add,
 * [2H][2W][Co] shared by the prompts)). */
int launch_convt_scatter(const float *G, float *out, const float *bias,
                         const float *add, int P, int H, int W, int Co,
                         int act, void *stream);
/* Low-resolution logits out [P][3][npix] = hyper [P][3][32] . U [P][npix][32]. */
int launch_mask_logits(const float *U, const float *hyper, float *out, int P,
                       int npix, void *stream);
/* Bilinear resize of n selected L x L logit planes to out_h x out_w
 * binary masks, with per-mask counts and bounding boxes accumulated into
 * stats [n][6] (initialised by the caller). */
int launch_mask_post(const float *lowres, const int *sel, int n, int L,
                     int out_h, int out_w, float offset, unsigned char *mask,
                     int *stats, void *stream);

/* Checkpoint tensor from its raw storage span src (element type sdt:
 * enum pth_dtype, 3 = complex64) to n C-order elements of type ddt at
 * dst (complex64 only to DT_F32, two floats per element); element i of
 * a non-contiguous tensor is at storage element sum_d idx_d stride[d]
 * of src. */
int launch_pth_convert(const void *src, int sdt, void *dst, int ddt,
                       long long n, int ndim, const long *shape,
                       const long *stride, int contiguous, void *stream);

/* Image -> token attention folded per prompt (bf16 path): k_i2t_fold
 * builds Wt16 [P][64][K] (bf16), bt [P][64] and YT16 [P][256][64] from
 * the token keys / values sk, sv [P][8][128], the image-query projection
 * Wq [128][256] + bq (layer 1; NULL in layer 0, K = 128) and the output
 * projection Wo [256][128]; s = log2(e) / sqrt(head width). In layer 1
 * Kc16 (optional) receives the compact rows s k_{t,h}, [P][64][16] bf16. */
int launch_i2t_fold(const float *sk, const float *sv, int layer,
                    const void *Wq, int wq_dt, const float *bq,
                    const void *Wo, int wo_dt, float s, int P, void *Wt16,
                    float *bt, void *YT16, void *Kc16, void *stream);
/* out [P][T][256] = LayerNorm(R + bo + attention of X over the folded
 * prompt tokens). K = 256 (layer 1): X = R = the keys (xs == rs), whose
 * image queries are keys + PE: the PE part enters as pq16 [T][128] bf16
 * (PE through the image-query projection, no bias) against Kc16 (the
 * fold's compact rows). K = 128 (layer 0): X = the shared projected image
 * queries (xs = 0), R with stride rs (0 = shared), pq16 = Kc16 = NULL.
 * out may alias R. */
int launch_i2t_fused(const float *X, long xs, int K, const void *pq16,
                     const void *Kc16, const void *Wt16, const float *bt,
                     const void *YT16, const float *bo, const float *R,
                     long rs, const float *g, const float *b, float *out,
                     int T, int P, float eps, void *stream);

/* Output upscaling fused with the mask logits (bf16 path): prep writes
 * the permuted bf16 transposes W1T16 [256][256] of up0w [256][64 4] and
 * W2T16 [128][64] of up3w [64][32 4]; the fused kernel maps keys
 * [P][G^2][256] to lowres [P][3][4G][4G] (feat_s1 [(2G)^2][64], feat_s0
 * [(4G)^2][32], hyper [P][3][32]). */
int launch_upscale_prep(const void *up0w, int dt0, const void *up3w, int dt3,
                        void *W1T16, void *W2T16, void *stream);
int launch_upscale_fused(const float *keys, const void *W1T16,
                         const void *W2T16, const float *b0, const float *lnw,
                         const float *lnb, const float *b3, const float *fs1,
                         const float *fs0, const float *hyper, float *lowres,
                         int G, int P, float eps, int cus, void *stream);

/* Token -> image attention on per-prompt keys (bf16 path): keys [P][T]
 * [256] + PE against the folded queries U16 [P][64][256] (bf16,
 * k_i2t_fold on the projected queries with the key projection), the PE
 * part as pk16 [T][128] bf16 (PE through the key projection, no bias)
 * against Qc16 (the fold's compact rows s q_{i,h}), nsplit key splits
 * with partials in part (P nsplit 64 258 floats), merged into Z [P][64]
 * [256], then o [P][8][128] = Wv Z + bv per head. */
int launch_t2i_fused(const float *keys, const void *pk16, const void *U16,
                     const void *Qc16, float *part, float *Z, const void *Wv,
                     int wv_dt, const float *bv, float *o, int T, int P,
                     int nsplit, void *stream);

/* The decoder's IoU head (head 0, token 1, 4 raw outputs into iou [P][4])
 * and hypernetwork MLPs (heads 1..3, tokens 3..5, into hyper [P][3][32])
 * on qry [P][8][256]: three Linear layers each, weights of element type
 * dt. */
int launch_dec_heads(const float *qry, const void *const w0[4],
                     const void *const w1[4], const void *const w2[4],
                     const float *const b0[4], const float *const b1[4],
                     const float *const b2[4], int dt, float *hyper,
                     float *iou, int P, void *stream);

/* fp32 -> bf16 / half conversion of count elements (weight uploads). */
int launch_convert(const float *src, void *dst, int dst_dt, size_t count,
                   void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SAM3_LAUNCH_H */
