/* CPU oracle for the SAM 3 attention path of i.sam3.opencl.
 *
 * TEST INFRASTRUCTURE ONLY. This library restates, in plain C on the
 * host, the arithmetic of the reference OpenCL kernels (sam3_kernels.cl)
 * and of their host dispatch (sam3_model.c) for the attention path. It
 * is the checker of the HIP path and the CPU baseline of bench.py; it is
 * never linked into, loaded by or called from the product library.
 *
 * Conventions follow the reference: activations are token-major fp32,
 * GEMM operands are (pointer, element offset, leading dimension, two
 * batch strides) with batch index b split into (b / nb1, b % nb1)
 * (sam3_kernels.cl:57-69). mad()/contracted a * b + c is taken as a
 * fused multiply-add, the form clang emits for OpenCL C on both PoCL and
 * ROCm; the runtime's exp/erf/rsqrt are taken from the C library. Both
 * choices are only visible at the level of the last bit and are listed
 * as unpinned where the oracle's tests document them.
 */
#ifndef SAM3_ORACLE_H
#define SAM3_ORACLE_H

#ifdef __cplusplus
extern "C" {
#endif

#define OR_ACT_NONE 0
#define OR_ACT_GELU 1
#define OR_ACT_RELU 2

/* GEMM arithmetic variants of the reference. */
#define OR_GEMM_SEQ 0   /* gemm, gemm_big, gemm_cpu_n: sequential mad over k */
#define OR_GEMM_CPU_T 1 /* gemm_cpu_t: 8 float lanes along k, hsum8, tail */

/* Batched C = act(alpha * A * op(B) + bias) + R with the reference's
 * operand contract (sam3_kernels.cl:57-69). kind selects the arithmetic
 * (OR_GEMM_SEQ / OR_GEMM_CPU_T). R may alias C. */
void or_gemm(int kind, int M, int N, int K, const float *A, long aoff, int lda,
             long sa0, long sa1, const float *B, long boff, int ldb, long sb0,
             long sb1, int transb, float *C, long coff, int ldc, long sc0,
             long sc1, int nb, int nb1, const float *bias, const float *R,
             long roff, float alpha, int act);

/* The host dispatcher gemm() of sam3_model.c:230-302: with profile=cpu
 * (cpu != 0) gemm_cpu_t for transb, gemm_cpu_n otherwise; on a GPU
 * profile gemm or gemm_big, which share the sequential arithmetic. */
void or_gemm_dispatch(int cpu, int M, int N, int K, const float *A, long aoff,
                      int lda, long sa0, long sa1, const float *B, long boff,
                      int ldb, long sb0, long sb1, int transb, float *C,
                      long coff, int ldc, long sc0, long sc1, int nb, int nb1,
                      const float *bias, const float *R, long roff,
                      float alpha, int act);

/* In-place row softmax, one reference work-group of ls items per row
 * (sam3_kernels.cl:637-656, host sam3_model.c:332-341). */
void or_softmax_rows(float *S, long rows, int L);

/* softmax_ext (sam3_kernels.cl:885-921) as attend() launches it
 * (sam3_text.c:320-335, ls = L >= 256 ? 256 : 64 items per row): in
 * place over `rows` rows of L scores, row = head * Nq + query with heads
 * counted from h0. Each score first gets the causal mask (key j > query i
 * becomes -inf) or else, when dy is given, SAM 3's box relative position
 * bias dy[(i H + j / W) nh + h] + dx[(i W + j % W) nh + h] with H = L / W;
 * then the strided max / exp / sum of softmax_rows. */
void or_softmax_ext(float *S, long rows, int L, int Nq, int h0, int causal,
                    const float *dy, const float *dx, int W, int nh);

/* attend() (sam3_text.c:305-343): `heads` heads of width hd at columns
 * h hd of Q [Nq][ldq], K [Nk][ldk], V [Nk][ldv], O [Nq][ldo]; per chunk of
 * hc = min(heads, score_cap / (Nq Nk)) heads: scores = Q K^T / sqrt(hd)
 * (gemm dispatch, cpu as in or_gemm_dispatch), softmax_ext with the mask or
 * bias (nh = heads), O = P V. Returns hc, or -1 if one head's scores do
 * not fit (the reference's fatal error). */
int or_attend(int cpu, int Nq, int Nk, int heads, int hd, const float *Q,
              int ldq, const float *K, int ldk, const float *V, int ldv,
              float *O, int ldo, int causal, const float *dy, const float *dx,
              int W, long score_cap);

/* Row LayerNorm, Y may alias X (sam3_kernels.cl:489-514, host
 * sam3_model.c:314-330). */
void or_layernorm(const float *X, float *Y, long rows, int C, const float *g,
                  const float *b, float eps, int act);

/* In-place 2D RoPE of the q and k thirds of fused qkv rows
 * (sam3_kernels.cl:679-698, host sam3_model.c:965-978). cs holds
 * (cos, sin) pairs, hd / 2 per position. */
void or_rope_apply(float *qkv, long rows, int E, int hd, int npos,
                   const float *cs);

/* Window partition / inverse with residual add (sam3_kernels.cl:712-741,
 * host sam3_model.c:360-392). */
void or_window_partition(const float *X, float *out, int H, int W, int C,
                         int ws, int nwx);
void or_window_unpartition_add(float *X, const float *Wd, int H, int W, int C,
                               int ws, int nwx);

/* out[i] = a[i] + b[i % bmod] (sam3_kernels.cl:700-708). */
void or_add_bcast(float *out, const float *a, const float *b, long n,
                  long bmod);

/* Decoder attention kernels (sam3_kernels.cl:527-633) and their
 * dispatcher mha() (sam3_model.c:413-451); 8 heads, head width
 * c = dint / 8. Returns 0, or -1 for the shape mha() rejects. */
void or_attn_fewkeys(const float *Q, long sq, const float *K, long sk,
                     const float *V, long sv, float *O, int P, int Nq, int Nk,
                     int dint, int c, float scale);
void or_attn_manykeys(const float *Q, long sq, const float *K, long sk,
                      const float *V, long sv, float *O, int P, int Nq,
                      int Nk, int dint, int c, float scale);
int or_mha(int P, int Nq, int Nk, int dint, const float *qp, long sq,
           const float *kp, long sk, const float *vp, long sv, float *o);

/* Attention region of one ViT block (sam3_model.c:981-1013):
 * layernorm(norm1) -> [window_partition] -> linear(qkv) -> rope_apply ->
 * per head chunk {gemm(Q K^T, alpha 1/sqrt(hd)) -> softmax_rows ->
 * gemm(P V)}. x is the grid x grid x E token map; ws = 0 is global
 * attention. Writes the attention output (rows x E, window-partitioned
 * order for windowed blocks) to attn and, if qkv_out is not NULL, the
 * post-RoPE qkv rows (rows x 3E). score_cap is the score buffer size in
 * floats (sam3_model.c:826-828). Returns the head chunk used, or -1 if
 * one head does not fit. */
int or_vit_attention(int cpu, const float *x, int grid, int E, int heads,
                     int hd, int ws, const float *n1w, const float *n1b,
                     const float *qkvw, const float *qkvb, const float *rope,
                     long score_cap, float *attn, float *qkv_out);

/* Patch im2col of a 3 x side x side channel-major image into grid^2
 * rows of 3 * ps * ps columns, column order c * ps^2 + ky * ps + kx
 * (sam3_kernels.cl:661-672). */
void or_patch_im2col(const float *img, float *out, int side, int grid, int ps);

/* Weights of one ViT block (struct vit_block, sam3_model.h); window is
 * the window side, 0 for a global block. */
struct or_block_w {
    const float *n1w, *n1b, *qkvw, *qkvb, *projw, *projb;
    const float *n2w, *n2b, *l1w, *l1b, *l2w, *l2b;
    int window;
};

/* One ViT block on x [grid^2, E] in place (vit_block,
 * sam3_model.c:981-1028): the attention region of or_vit_attention, the
 * projection with residual (windowed: into a temporary, then
 * window_unpartition_add), norm2 and the erf-GELU MLP with residual.
 * rope is the block's table (windowed: window^2 positions, global:
 * grid^2). Returns the heads per score chunk, or -1. */
int or_vit_block(int cpu, float *x, int grid, int E, int heads, int hd,
                 int mlp, const struct or_block_w *b, const float *rope,
                 long score_cap);

/* Trunk of the image encoder (sam_encode_trunk, sam3_model.c:1112-1135):
 * patch im2col of img (3 x side x side, side = grid * ps) and the patch
 * GEMM without bias, + pos [grid^2, E], ln_pre in place, then `depth`
 * blocks (windowed blocks use rope_win, global ones rope_glob). x [grid^2,
 * E] receives the result. Returns 0, or -1 for an unsupported shape. */
int or_encode_trunk(int cpu, const float *img, int grid, int ps, int E,
                    int heads, int hd, int mlp, const float *pe_w,
                    const float *pos, const float *lnpw, const float *lnpb,
                    const struct or_block_w *blocks, int depth,
                    const float *rope_win, const float *rope_glob,
                    long score_cap, float *x);

/* Brute-force scaled dot-product attention in double precision,
 * O[i, :] = sum_j softmax_j(scale * q_i . k_j) v_j, for pinning. */
void or_sdpa_f64(int Nq, int Nk, int d, const double *Q, int ldq,
                 const double *K, int ldk, const double *V, int ldv, double *O,
                 int ldo, double scale);

/* Activation epilogue of the reference kernels (exact-erf GELU, ReLU;
 * sam3_kernels.cl:43-55) and its dot16 of two float16 vectors
 * (sam3_kernels.cl:516-520). */
float or_act(float v, int act);
float or_dot16(const float *a, const float *b);

/* ------------------------------------------------------------------ */
/* Mask decoder (sam3_oracle_dec.c)                                    */
/* ------------------------------------------------------------------ */

/* Weights of one decoder attention (struct sam_attn_w, sam3_model.h:16):
 * q/k/v [dint][256], o [256][dint], biases. */
struct or_attn_w {
    const float *qw, *qb, *kw, *kb, *vw, *vb, *ow, *ob;
    int dint;
};

/* One two-way transformer layer (struct sam_dec_layer, sam3_model.h:28):
 * mlp lin1 [2048][256], lin2 [256][2048]. */
struct or_dec_layer {
    struct or_attn_w self, t2i, i2t;
    const float *n1w, *n1b, *n2w, *n2b, *n3w, *n3b, *n4w, *n4b;
    const float *m1w, *m1b, *m2w, *m2b;
};

/* The point-prompt head's prompt encoder and mask decoder (the decoder
 * fields of struct sam_model, sam3_model.h:55-75). grid: embedding side
 * (SAM_GRID), img: encoder input side (SAM_IMG). gauss [2][128],
 * point_emb [4][256], up0w [256][64 * 4], up3w [64][32 * 4], hyper_w[i]
 * {[256][256], [256][256], [32][256]}, iou_w {.., .., [4][256]}. */
struct or_decoder {
    int grid, img;
    const float *gauss, *point_emb, *not_a_point, *no_mask;
    struct or_dec_layer layers[2];
    struct or_attn_w final_t2i;
    const float *nfw, *nfb;
    const float *up0w, *up0b, *up1w, *up1b, *up3w, *up3b;
    const float *obj_token, *iou_token, *mask_tokens;
    const float *hyper_w[4][3], *hyper_b[4][3];
    const float *iou_w[3], *iou_b[3];
};

void or_pe_encode(const float *gauss, float x, float y, float *out);
void or_host_linear(const float *W, const float *b, const float *x, int nin,
                    int nout, int relu, float *y);
void or_convt_scatter(const float *G, float *out, const float *bias,
                      const float *add, int P, int H, int W, int Co, int act);
void or_mask_logits(const float *U, const float *hyper, float *out, int P,
                    int npix);
void or_mask_post(const float *lowres, const int *sel, int n, int L,
                  int out_h, int out_w, float offset, unsigned char *mask,
                  int *stats);
int or_fill_holes(float *v, int L, int max_area);
void or_postprocess(float *lowres, int L, int n, const int *sel, int out_h,
                    int out_w, float offset, int fill, int max_area,
                    unsigned char *mask, int *stats);
void or_dec_prepare(const struct or_decoder *d, const float *emb, float *pe,
                    float *src, float *srcpe, float *kp0, float *vp0,
                    float *qp0);
void or_t2i_attention(int P, int T, float *qry, const float *qpe,
                      const float *keys, const float *pe,
                      const struct or_attn_w *a, float *kin);
void or_i2t_attention(int layer, int P, int T, const float *qry,
                      const float *qpe, float *keys, const float *kin,
                      const float *qp0, const float *src,
                      const struct or_dec_layer *L);
void or_prompt_tokens(const struct or_decoder *d, int P, const float *points,
                      float *tok);
void or_sam_decode(const struct or_decoder *d, int P, const float *points,
                   const float *pe, const float *src, const float *kp0,
                   const float *vp0, const float *qp0, const float *feat_s0,
                   const float *feat_s1, float *iou, float *lowres,
                   float *tokens, float *hyper_out);

/* Number of OpenMP threads the oracle runs on. */
int or_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* SAM3_ORACLE_H */
