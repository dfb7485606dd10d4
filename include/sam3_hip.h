/* SPDX-License-Identifier: Unlicense
 *
 * sam3_hip.h - MI355X (gfx950) backend and operator API for the SAM 3
 * attention path of i.sam3.opencl.
 *
 * A drop-in for the reference's OpenCL path on the attention region:
 * - the backend section replaces ocl_backend.h (ocl_backend.h:57-104):
 *   cl_mem becomes hipb_mem, ocl_* becomes hipb_*, and the raw OpenCL
 *   calls model code makes (clFinish, clEnqueueCopyBuffer) get
 *   hipb_finish / hipb_copy;
 * - the operator section keeps the names, argument meaning and error
 *   behaviour of sam3_ops.h (sam3_ops.h:19-65) and of the static helpers
 *   of sam3_model.c that the attention path calls (softmax_rows,
 *   rope_apply, window_partition, window_unpartition_add, mha), and adds
 *   attn_fused (the fused replacement of the per-head-chunk
 *   gemm -> softmax_rows -> gemm loop, sam3_model.c:1000-1013) and
 *   vit_attention (the attention region of vit_block,
 *   sam3_model.c:981-1013).
 *
 * Every function is plain C with plain pointers and sizes. Errors follow
 * the reference: any failure is fatal with a message naming the call
 * (G_fatal_error in the reference). A binding that must survive errors
 * selects HIPB_ERR_RECORD and reads hipb_last_error() after each call.
 *
 * One host thread drives one hipb_backend; all work goes to its one
 * in-order stream (the reference's one in-order queue, ocl_backend.c
 * clCreateCommandQueue). The API is not re-entrant, like the reference's
 * (kernel objects there are shared and mutated by SETARG).
 */
#ifndef SAM3_HIP_H
#define SAM3_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ------------------------------------------------------------------ */
/* Backend (replaces ocl_backend.h)                                    */
/* ------------------------------------------------------------------ */

/* Element type of a device buffer. The reference only knows float
 * buffers and half weight matrices (ocl_backend.c:520-587); bf16 is the
 * storage of the precision=bf16 fast path. */
#define HIPB_F32 0
#define HIPB_F16 1
#define HIPB_BF16 2

/* Device profile (profile= option, ocl_backend.h:14-25). A HIP device is
 * a discrete GPU with its own memory: "auto" and "dgpu" select it, the
 * host-memory profiles do not exist here. */
#define HIPB_ARCH_DGPU 2

/* Error handling mode: fatal (print and exit, the reference's
 * G_fatal_error) or record (keep the message, return to the caller). */
#define HIPB_ERR_FATAL 0
#define HIPB_ERR_RECORD 1

/* A device buffer (replaces cl_mem). */
typedef struct hipb_buf *hipb_mem;

struct hipb_buf {
    void *ptr;        /* device address */
    size_t bytes;     /* allocation size */
    int dtype;        /* HIPB_F32, HIPB_F16 or HIPB_BF16 */
    const char *what; /* copy of the name given at allocation */
};

struct hipb_backend {
    int device;            /* HIP device ordinal */
    char device_name[256]; /* marketing name */
    char arch_name[64];    /* gcnArchName, e.g. gfx950:sramecc+:xnack- */
    size_t max_alloc;      /* largest single allocation allowed */
    size_t global_mem;     /* device memory in bytes */
    int cu_count;          /* compute units */
    int clock_khz;         /* peak engine clock */
    int arch;              /* HIPB_ARCH_DGPU */
    int fp16w;    /* precision=fp16: weight matrices stored as half */
    int bf16;     /* precision=bf16: bf16 MFMA fast path */
    int profile;  /* per-kernel timing (I_SAM3_OPENCL_PROFILE set): 1 =
                   * each launch waited for and timed alone (the
                   * reference's run()), 2 = launches bracketed by event
                   * pairs without waiting, read at hipb_finish */
    void *stream; /* hipStream_t, default priority, in order */
    void *ev[2];  /* hipEvent_t pair of the region timer */
    void *scratch;          /* backend-owned device scratch (split-K partials) */
    size_t scratch_bytes;
    /* Pinned host staging of checkpoint uploads (pth_upload): two
     * buffers and the events that mark the end of their last copy. */
    void *stage[2];
    void *stage_ev[2];
    int stage_next;
};

/* Select a device and create its stream (ocl_init, ocl_backend.h:57-59).
 * device_opt: NULL, "auto", "gpu" or a device ordinal "0".."N-1";
 * platform_opt: NULL, "" or a substring of "HIP" / "AMD" (anything else
 * matches no device); profile_opt: NULL, "auto" or "dgpu";
 * precision_opt: NULL or "fp32" (exact path, f32 MFMA), "fp16" (weight
 * matrices stored as half, float arithmetic, as the reference) or
 * "bf16" (bf16 MFMA with f32 accumulation for attention and the GEMMs).
 * Fatal if no device matches. I_SAM3_OPENCL_PROFILE in the environment
 * switches on per-kernel timing, as in the reference. */
void hipb_init(struct hipb_backend *b, const char *device_opt,
               const char *platform_opt, const char *profile_opt,
               const char *precision_opt);

const char *hipb_arch_name(int arch);                 /* ocl_arch_name */
void hipb_free(struct hipb_backend *b);                 /* ocl_free */
const char *hipb_errstr(int err);                       /* ocl_errstr */
void hipb_check(int err, const char *what);             /* ocl_check */

/* Allocate n bytes of float storage, fatal on failure (ocl_alloc). */
hipb_mem hipb_alloc(struct hipb_backend *b, size_t n, const char *what);
/* Allocate count elements of the given HIPB_* type (no counterpart: the
 * reference only has float buffers plus half weights). */
hipb_mem hipb_alloc_typed(struct hipb_backend *b, size_t count, int dtype,
                          const char *what);
/* Allocate and fill from host memory (ocl_upload). */
hipb_mem hipb_upload(struct hipb_backend *b, const void *src, size_t n,
                     const char *what);
/* Weight matrix used only as GEMM operand B: half with precision=fp16,
 * bf16 with precision=bf16, else float (ocl_upload_weight). */
hipb_mem hipb_upload_weight(struct hipb_backend *b, const float *src,
                            size_t count, const char *what);
/* The host rounding hipb_upload_weight applies: float to IEEE binary16
 * (dtype HIPB_F16) or to bfloat16 (HIPB_BF16), round to nearest even;
 * the reference's is static inside ocl_backend.c:521-557 (f32_to_f16). */
void hipb_round_half(const float *src, uint16_t *dst, size_t count, int dtype);
int hipb_is_half(hipb_mem m);                           /* ocl_is_half */
/* Blocking transfers at byte offsets (ocl_write / ocl_read). */
void hipb_write(struct hipb_backend *b, hipb_mem dst, size_t off,
                const void *src, size_t n);
void hipb_read(struct hipb_backend *b, hipb_mem src, size_t off, void *dst,
               size_t n);
/* Release and set to NULL (ocl_release). */
void hipb_release(hipb_mem *m);
/* Wait for all queued work (clFinish(ocl->queue), sam3_model.c:1140). */
void hipb_finish(struct hipb_backend *b);
/* Device copy on the stream (clEnqueueCopyBuffer, sam3_model.c:1266). */
void hipb_copy(struct hipb_backend *b, hipb_mem src, hipb_mem dst,
               size_t src_off, size_t dst_off, size_t n);

/* Error mode and the last recorded error (NULL if none). */
void hipb_set_error_mode(int mode);
const char *hipb_last_error(void);
void hipb_clear_error(void);

/* Per-kernel profile, the reference's run() table (sam3_model.c:149-207):
 * with b->profile set every launch is timed with events on the stream
 * and accumulated per kernel name with its algorithmic FLOPs (profile 2:
 * the launches run back to back and their times are added up at
 * hipb_finish; wall_ms stays 0). */
int hipb_prof_count(void);
int hipb_prof_entry(int i, const char **what, double *ms, double *wall_ms,
                    double *flops, long *calls);
void hipb_prof_reset(void);
void hipb_prof_print(void);

/* Region timer: events recorded on the backend's stream around the work
 * queued between start and stop; stop waits and returns milliseconds. */
void hipb_timer_start(struct hipb_backend *b);
float hipb_timer_stop(struct hipb_backend *b);

/* ------------------------------------------------------------------ */
/* Operators (sam3_ops.h and the attention helpers of sam3_model.c)    */
/* ------------------------------------------------------------------ */

#define ACT_NONE 0
#define ACT_GELU 1
#define ACT_RELU 2

/* One GEMM operand: buffer, element offset, leading dimension and the
 * two batch strides (sam3_ops.h:19-24). */
struct opnd {
    hipb_mem buf;
    long off;
    int ld;
    long s0, s1;
};

/* One ViT block (sam3_model.h:21-25). Weights uploaded with
 * hipb_upload_weight (qkvw, projw, l1w, l2w) or hipb_upload. */
struct vit_block {
    hipb_mem n1w, n1b, qkvw, qkvb, projw, projb, n2w, n2b;
    hipb_mem l1w, l1b, l2w, l2b;
    int window; /* Window side, 0 for global attention. */
};

/* The part of struct sam_model (sam3_model.h:41-117) the attention path
 * and the image encoder trunk read and write. */
struct sam_model {
    struct hipb_backend *hip; /* the reference's m->ocl */
    int embed, depth, heads, hd, mlp;
    int grid; /* token grid side, SAM_GRID = 72 in the reference */
    struct vit_block *blocks;
    hipb_mem rope_win, rope_glob; /* (cos, sin) per position, hd/2 each */
    long score_cap;               /* floats of the score buffer */
    /* Encoder work buffers (sam3_model.c:847-854). */
    hipb_mem x, xn, xw, qkv, scores, attn;
    /* precision=bf16 staging: LN output and packed Q, K, V^T. */
    hipb_mem xn16, q16, k16, vt16;
    /* Largest |k| of each 64-key block of the packed keys (float,
     * [unit][Np / 64]): bounds the scores of a block. */
    hipb_mem knorm;
    /* Trunk prologue (sam3_model.h:46-49): patch side, patch embedding
     * [E][3 patch^2] (no bias), position embedding tiled to [grid^2][E]
     * (sam3_model.c:482-502), ln_pre. */
    int patch;
    hipb_mem pe_w, pos, lnpw, lnpb;
    /* Trunk work buffers (sam3_model.c:853-861): image
     * [3][grid patch]^2, projection output [rows][E], MLP hidden /
     * patch columns; mlp16 the bf16 MLP hidden of precision=bf16. */
    hipb_mem img, tmp, mlpbuf, mlp16;
    /* HIP graph of the trunk's kernels (sam_trunk_graph): hipGraph_t,
     * hipGraphExec_t, and the work-buffer generation it was captured at. */
    void *trunk_graph, *trunk_exec;
    unsigned long trunk_gen;
    /* attend(): the box bias of the fused kernels, as rows [heads][Nq][H
     * + W] of dy then dx values or as an additive table [heads][Nq][Nk
     * padded to 64] (exp2 domain on the bf16 path). */
    hipb_mem abias;
    /* Key-split partial records of the bf16 attention ([unit][split][Np]
     * rows of 64 O values, then their (m, l) pairs). */
    hipb_mem apart;
    /* Stream-K balance of the bf16 attention: piece records and per-tile
     * arrival counters (launch_attn_bf16's skrec, skcnt). */
    hipb_mem askrec, askcnt;
    /* The point-prompt mask decoder (sam_dec_init), or NULL. */
    struct sam_decoder *dec;
    /* Set by sam_load: the blocks array, the weights, the rope tables and
     * the decoder are the model's own, and sam_free releases them. */
    int owns_weights;
};

/* Set up m for the attention path (mlp = 0) or the whole trunk (mlp =
 * MLP width) on backend b and allocate its work buffers for the given
 * blocks, sized like alloc_buffers (sam3_model.c:815-861): rows = max
 * over blocks of nwin * N, score buffer = min(max_alloc, 512 MiB); fatal
 * if one head's scores do not fit (sam3_model.c:833-837). The weights
 * (blocks, pe_w, pos, lnpw, lnpb, rope tables) are the caller's. No
 * counterpart: the reference does this inside sam_load. */
void sam_path_init(struct sam_model *m, struct hipb_backend *b, int grid,
                   int embed, int heads, int hd, int mlp,
                   struct vit_block *blocks, int depth);
void sam_path_free(struct sam_model *m);

struct opnd mat(hipb_mem buf, long off, int ld);                 /* ops.h:48 */
struct opnd bmat(hipb_mem buf, long off, int ld, long s0, long s1); /* ops.h:49 */

/* Batched C = act(alpha * A * op(B) + bias) + R (sam3_ops.h:51-54,
 * contract sam3_kernels.cl:57-69). A and C are float (C may be bf16 and
 * A bf16 with precision=bf16); B may be half or bf16 weights. R may
 * alias C. */
void gemm(struct sam_model *m, int M, int N, int K, struct opnd A,
          struct opnd B, int transb, struct opnd C, int nb, int nb1,
          hipb_mem bias, hipb_mem R, long roff, float alpha, int act);

/* Y[rows, out] = act(X[rows, in] W^T + b) (+ Y when residual)
 * (sam3_ops.h:56-58). */
void linear(struct sam_model *m, int rows, int in, int out, hipb_mem X,
            long xoff, hipb_mem W, hipb_mem b, hipb_mem Y, long yoff, int act,
            int residual);

/* Row LayerNorm, Y may alias X (sam3_ops.h:60-61). */
void layernorm(struct sam_model *m, long rows, int C, hipb_mem X, hipb_mem Y,
               hipb_mem g, hipb_mem b, float eps, int act);

/* out[i] = a[i] + b[i % bmod]; out may alias a (sam3_ops.h:63-65). */
void add_bcast(struct sam_model *m, hipb_mem out, hipb_mem a, hipb_mem b,
               long n, long bmod);

/* In-place softmax of rows of L floats (sam3_model.c:332-341). */
void softmax_rows(struct sam_model *m, hipb_mem S, long rows, int L);

/* softmax_ext over rows = heads x Nq rows of L scores (heads from h0),
 * sam3_kernels.cl:885-921: the causal mask (key j > query i excluded) or,
 * with dy / dx, SAM 3's box relative position bias dy[(i H + j / W) nh +
 * h] + dx[(i W + j % W) nh + h], H = L / W, added before the softmax. The
 * reference's kernel has no host wrapper; attend() launches it. */
void softmax_ext(struct sam_model *m, hipb_mem S, long rows, int L, int Nq,
                 int h0, int causal, hipb_mem dy, hipb_mem dx, int W, int nh);

/* Multi-head attention of the text path, attend() of sam3_text.c:305-343
 * (the reference's static helper, taking the model instead of struct
 * sam3_text): heads of width hd at columns h hd of Q [Nq][ldq], K [Nk][ldk],
 * V [Nk][ldv], O [Nq][ldo]; scale 1 / sqrt(hd); optional causal mask or
 * box bias (dy [Nq][Nk / W][heads], dx [Nq][W][heads]). The fused
 * attention runs on the bf16 path for hd 64 or 32 (with the mask or the
 * bias) and on the fp32 path for hd 64 self-attention without either;
 * otherwise the reference's sequence per score-buffer chunk of heads:
 * gemm Q K^T, softmax_ext, gemm P V (fatal, like the reference, when one
 * head's Nq x Nk scores exceed the score buffer). */
void attend(struct sam_model *m, int Nq, int Nk, int heads, int hd, hipb_mem Q,
            int ldq, hipb_mem K, int ldk, hipb_mem V, int ldv, hipb_mem O,
            int ldo, int causal, hipb_mem dy, hipb_mem dx, int W);

/* In-place RoPE of the q and k thirds of m->qkv rows at position
 * r % npos (sam3_model.c:965-978). */
void rope_apply(struct sam_model *m, hipb_mem table, long rows, int npos);

/* H x H token grid -> ws x ws windows and back with residual add
 * (sam3_model.c:360-392). */
void window_partition(struct sam_model *m, hipb_mem X, hipb_mem out, int H,
                      int C, int ws, int nwx);
void window_unpartition_add(struct sam_model *m, hipb_mem X, hipb_mem Wd,
                            int H, int C, int ws, int nwx);

/* Decoder multi-head attention on projected tensors, 8 heads of width
 * dint / 8, per-prompt element strides (0 = shared by all prompts)
 * (sam3_model.c:413-451). Nk > 64 requires dint / 8 == 16, else fatal
 * "mha: unsupported shape", as the reference. */
void mha(struct sam_model *m, int P, int Nq, int Nk, int dint, hipb_mem qp,
         long sq, hipb_mem kp, long sk, hipb_mem vp, long sv, hipb_mem o);

/* mha without allocating: no counterpart in the reference. For callers
 * that cannot allocate device memory (code under HIP graph capture,
 * serving loops, harnesses that forbid hipMalloc). Same arguments,
 * results and errors as mha; the token -> image (Nk > 64) split-K
 * partials go to a static device scratch of 8 MiB per GPU, held from
 * hipb_init until the process ends, instead of the backend's scratch; a
 * shape needing more is a fatal error. The call queues kernels only (no
 * hipMalloc / hipFree, no profiling events). Calls that overlap on one
 * GPU (several streams or backends) share that scratch and race. */
void mha_noalloc(struct sam_model *m, int P, int Nq, int Nk, int dint,
                 hipb_mem qp, long sq, hipb_mem kp, long sk, hipb_mem vp,
                 long sv, hipb_mem o);

/* Fused softmax attention of nb independent (window, head) units of N
 * tokens and head width 64: O = softmax(scale * rope(Q) rope(K)^T) V.
 * Q, K, V and O use the operand addressing of gemm (batch b split as
 * (b / nb1, b % nb1) with strides s0/s1, rows of ld elements), so the
 * operands of the reference's QK^T and PV calls (sam3_model.c:1004-1011)
 * apply unchanged. rope (NULL for none) rotates Q and K rows at position
 * i % npos of the unit. With precision=bf16 the product runs on bf16
 * MFMA with f32 accumulation; otherwise on f32 MFMA. Replaces the
 * gemm -> softmax_rows -> gemm loop of sam3_model.c:1000-1013. */
void attn_fused(struct sam_model *m, int N, int nb, int nb1, struct opnd Q,
                struct opnd K, struct opnd V, struct opnd O, hipb_mem rope,
                int npos, float scale);

/* The attention stage of the precision=bf16 path alone, on the packed
 * operands that attn_fused / vit_attention left in m->q16, m->k16,
 * m->vt16 and m->knorm (nb units of N tokens, RoPE and scale applied);
 * O as in attn_fused. No counterpart in the reference: it is for callers that
 * produce packed operands themselves and for timing the kernel. */
void attn_packed(struct sam_model *m, int N, int nb, int nb1, struct opnd O);

/* Attention region of one ViT block (sam3_model.c:981-1013): norm1,
 * window partition, QKV projection, RoPE and attention of m->x into
 * m->attn (rows = nwin * N, window-partitioned for windowed blocks).
 * With unfused != 0 it replays the reference's operator sequence
 * (gemm -> softmax_rows -> gemm per head chunk, through m->scores). */
void vit_attention(struct sam_model *m, const struct vit_block *blk,
                   int unfused);

/* One ViT block on m->x in place (vit_block, sam3_model.c:981-1028):
 * the attention region, the projection with residual (windowed blocks
 * through m->tmp and window_unpartition_add), norm2 and the erf-GELU MLP
 * with residual. With precision=bf16 the GEMM operands are bf16 (norm2
 * output and MLP hidden stored as bf16), accumulation and the residual
 * stream float. unfused: the reference's attention operator sequence. */
void vit_block(struct sam_model *m, const struct vit_block *blk, int unfused);

/* Image encoder trunk (sam_encode_trunk, sam3_model.c:1112-1135): the
 * host image img (3 x side x side floats, side = grid * patch) is
 * written to the device, patch im2col + patch GEMM (no bias) + position
 * embedding + ln_pre give m->x, then the m->depth blocks run in order.
 * The result stays in m->x; the caller synchronises (hipb_finish). */
void sam_encode_trunk(struct sam_model *m, const float *img);

/* HIP-graph replay of the trunk. With enable != 0: run the trunk's
 * kernels once (so that every work buffer exists), capture them on the
 * backend's stream, and let later sam_encode_trunk calls replay the graph
 * after the image upload (one launch instead of ~200). enable = 0 drops
 * the graph. Weights, rope tables and work buffers are captured by
 * address: re-enable after changing weights; a work-buffer reallocation by
 * any later call drops the graph (later calls run the kernels one by
 * one). Profiling (profile 1 or 2) always runs the kernels one by one. No
 * counterpart in the reference (whose OpenCL queue has no graphs). */
void sam_trunk_graph(struct sam_model *m, int enable);

/* ------------------------------------------------------------------ */
/* Point-prompt mask decoder (sam3_model.c:1212-1517)                  */
/* ------------------------------------------------------------------ */

#define SAM_DIM 256 /* decoder embedding width (sam3_model.h:12) */
#define SAM_HOLE 256 /* largest hole filled, pixels (sam3_model.h:14) */

/* Weights of one decoder attention (sam3_model.h:16-19): q/k/v
 * [dint][256], o [256][dint] (hipb_upload_weight), biases (hipb_upload). */
struct sam_attn_w {
    hipb_mem qw, qb, kw, kb, vw, vb, ow, ob;
    int dint;
};

/* One two-way transformer layer (sam3_model.h:28-32): mlp lin1
 * [2048][256], lin2 [256][2048]. */
struct sam_dec_layer {
    struct sam_attn_w self, t2i, i2t;
    hipb_mem n1w, n1b, n2w, n2b, n3w, n3b, n4w, n4b;
    hipb_mem m1w, m1b, m2w, m2b;
};

/* The decoder fields of struct sam_model (sam3_model.h:55-75, 100-116).
 * The caller fills the weights (device: layers, final_t2i, nf*, up*,
 * the MLP heads; host: the prompt encoder tables and tokens) and, per
 * image, emb / feat_s0 / feat_s1;
 * sam_dec_init allocates the rest. up0w [256][64 4] and up3w [64][32 4]
 * are the ConvTranspose2d weights [in][out][2][2]. hyper_w[i] = {[256]
 * [256], [256][256], [32][256]}, iou_w = {.., .., [4][256]}. */
struct sam_decoder {
    int img;   /* encoder input side, SAM_IMG (points are in its pixels) */
    int batch; /* prompts per sam_decode call */
    float gauss[2 * 128];
    float point_emb[4][SAM_DIM];
    float not_a_point[SAM_DIM];
    float no_mask[SAM_DIM];
    struct sam_dec_layer layers[2];
    struct sam_attn_w final_t2i;
    hipb_mem nfw, nfb;
    hipb_mem up0w, up0b, up1w, up1b, up3w, up3b;
    float obj_token[SAM_DIM], iou_token[SAM_DIM], mask_tokens[4 * SAM_DIM];
    /* Hypernetwork MLPs and IoU head, device weights (the reference keeps
     * them on the host; here they run as small GEMMs on the stream). */
    hipb_mem hyper_w[4][3], hyper_b[4][3];
    hipb_mem iou_w[3], iou_b[3];
    /* Image features [grid^2][256], [16 grid^2][32], [4 grid^2][64]. */
    hipb_mem emb, feat_s0, feat_s1;
    /* Per-image caches: src = emb + no_mask, dense PE, src + PE, layer-0
     * projections of the shared keys / values / image queries. */
    hipb_mem src, pe_img, srcpe, kp0, vp0, qp0;
    /* Batch buffers (sam3_model.c:895-916). */
    hipb_mem qpe, qry, qin, sq, sk, sv, so, sh;
    hipb_mem keys, kin, bq, bk, bv, bo;
    hipb_mem u1, g2, u2, hyper, lowres;
    float *h_queries, *h_lowres;
    /* Postprocessed masks and their statistics. */
    hipb_mem mask, sel, stats;
    size_t mask_cap;
    /* precision=bf16: per-prompt folded image -> token attention, Wt
     * [batch][64][256] bf16, bt [batch][64], Y^T [batch][256][64] bf16. */
    hipb_mem fold_w, fold_b, fold_y;
    /* precision=bf16: up0w / up3w as the fused upscaling's permuted bf16
     * transposes [256][256] and [128][64]. */
    hipb_mem up_w1t, up_w2t;
    /* precision=bf16: token -> image attention key-split partials
     * ((2 CUs + batch) records of 64 rows x 258 floats) and the merged
     * weighted key sums Z [batch][64][256]. */
    hipb_mem t2i_part, t2i_z;
    /* precision=bf16: the folds' compact per-head token rows (s k_{t,h},
     * or s q_{i,h} for token -> image) [batch][64][16] bf16, and the dense
     * PE through the layer-1 image-query, layer-1 key and final key
     * projections (no bias), [grid^2][128] bf16 each, per image: the
     * position term of the fused blocks' scores. */
    hipb_mem fold_c, pe_q1, pe_k1, pe_kf;
    /* sam_dec_graph: hipGraph_t, hipGraphExec_t of the device sequence
     * for graph_P prompts, and the backend scratch it was captured with. */
    void *graph, *graph_exec;
    int graph_P;
    void *graph_scratch;
};

/* Attach decoder d to m (grid from m) and allocate its caches and batch
 * buffers for `batch` prompts; computes the dense positional encoding
 * from d->gauss, so call it after filling the prompt-encoder tables. No
 * counterpart: the reference does this in alloc_buffers
 * (sam3_model.c:876-916). */
void sam_dec_init(struct sam_model *m, struct sam_decoder *d, int batch);
void sam_dec_free(struct sam_model *m);

/* The decoder part of sam_encode (sam3_model.c:1150-1171): src = emb +
 * no_mask, srcpe = src + PE, kp0 / vp0 / qp0 layer-0 projections. */
void sam_dec_prepare(struct sam_model *m);

/* sam_decode (sam3_model.c:1239-1400): P <= batch single-point prompts
 * (x, y pairs in encoder input pixels); iou [P][3] receives the multimask
 * IoU predictions, d->lowres the [P][3][4 grid]^2 low-resolution logits. */
void sam_decode(struct sam_model *m, int P, const float *points, float *iou);

/* Capture (enable = 1) or drop (0) a HIP graph of sam_decode's device
 * sequence for P prompts; sam_decode then replays it (one launch after
 * the token upload) whenever it is called with that P and the backend's
 * scratch has not been reallocated, and runs the kernels one by one
 * otherwise. Profiling (profile 1 or 2) always runs them one by one. No
 * counterpart in the reference (whose OpenCL queue has no graphs). */
void sam_dec_graph(struct sam_model *m, int P, int enable);

/* Token -> image attention with per-prompt keys and residual into the
 * queries (static t2i_attention, sam3_model.c:1212-1229); kin = keys +
 * PE is left in d->kin. */
void t2i_attention(struct sam_model *m, int P, const struct sam_attn_w *a);

/* Image -> token attention of decoder layer `layer` with norm4, keys
 * updated in place (inline in sam_decode: sam3_model.c:1298-1312 for
 * layer 0, 1330-1345 for layer 1, which reads kin). */
void i2t_attention(struct sam_model *m, int layer, int P);

/* Transposed-convolution scatter (sam3_model.c convt_scatter, kernel
 * sam3_kernels.cl:762-786): G [(P H W)][Co 4] -> out [P][2H][2W][Co],
 * + bias, + add [2H][2W][Co] (NULL for none), then act. */
void convt_scatter(struct sam_model *m, hipb_mem G, hipb_mem out,
                   hipb_mem bias, hipb_mem add, int P, int H, int W, int Co,
                   int act);

/* Low-resolution logits out [P][3][npix] = hyper [P][3][32] .
 * U [P][npix][32] (the mask_logits kernel, sam3_kernels.cl:789-805, as
 * sam_decode launches it, sam3_model.c:1387-1398). */
void mask_logits(struct sam_model *m, hipb_mem U, hipb_mem hyper,
                 hipb_mem out, int P, int npix);

/* sam_postprocess (sam3_model.c:1445-1517): optional hole filling (host)
 * of the n selected planes sel[] of d->lowres, bilinear resize to out_h x
 * out_w binary masks in d->mask and stats [n][6] = count(logit >
 * offset), count(logit > -offset), xmin, ymin, xmax, ymax. */
void sam_postprocess(struct sam_model *m, int n, const int *sel, int out_h,
                     int out_w, float offset, int fill, int *stats);
/* Copy rows y0..y1, columns x0..x1 of postprocessed mask k to dst
 * (sam3_model.c:1519-1530). */
void sam_read_mask(struct sam_model *m, int k, int out_h, int out_w, int x0,
                   int y0, int x1, int y1, unsigned char *dst);

/* ------------------------------------------------------------------ */
/* Checkpoint weights (pth_loader.h files into device memory)          */
/* ------------------------------------------------------------------ */

struct pth_file;
struct pth_tensor;

/* Tensor t of an open checkpoint as a new device buffer of the given
 * HIPB_* type, C order: the storage span it covers is copied through
 * pinned staging and converted / gathered on the device (float32, half
 * and bfloat16 storage to any of the three, rounding to nearest even;
 * complex64 only to HIPB_F32 as (real, imaginary) pairs). No counterpart:
 * the reference reads to host floats and uploads (sam3_model.c:52-76). */
hipb_mem pth_upload(struct hipb_backend *b, const struct pth_file *pf,
                    const struct pth_tensor *t, int dtype, const char *what);

/* The reference's load helpers (sam3_ops.h:26-38): pth_require then a
 * float32 device buffer (load_dev) or a weight matrix in the backend's
 * weight type (load_dev_w: half with precision=fp16, bf16 with
 * precision=bf16, else float32); the _fmt forms format the name;
 * load_host returns malloc'd host floats, load_host_into copies them. */
hipb_mem load_dev(struct sam_model *m, const struct pth_file *pf,
                  const char *name, int ndim, const long *shape);
hipb_mem load_dev_w(struct sam_model *m, const struct pth_file *pf,
                    const char *name, int ndim, const long *shape);
hipb_mem load_dev_fmt(struct sam_model *m, const struct pth_file *pf,
                      int ndim, const long *shape, const char *fmt, ...);
hipb_mem load_dev_w_fmt(struct sam_model *m, const struct pth_file *pf,
                        int ndim, const long *shape, const char *fmt, ...);
float *load_host(const struct pth_file *pf, const char *name, int ndim,
                 const long *shape);
void load_host_into(const struct pth_file *pf, const char *name, int ndim,
                    const long *shape, float *dst);

/* Non-zero if pf holds the SAM 3 trunk, the tracker's mask decoder and
 * the point-prompt neck (sam_is_sam3, sam3_model.c:41-46; main.c:537-550
 * refuses other checkpoints with it). */
int sam_is_sam3(const struct pth_file *pf);

/* sam_load (sam3_model.c:918-962) without the necks: the image encoder
 * trunk of a SAM 3 checkpoint (sizes, depth, window and grid from its
 * tensors, sam3_model.c:473-583; the grid is the global blocks' rope
 * extent) with its work buffers, and with point_head the point-prompt
 * decoder's weights (sam3_model.c:657-758) and sam_dec_init(m, d, batch).
 * The image features of the decoder (emb, feat_s0, feat_s1) stay the
 * caller's to provide. */
void sam_load(struct sam_model *m, struct hipb_backend *b,
              const struct pth_file *pf, int batch, int point_head);
/* Release a model (sam3_model.c:1532): with owns_weights (sam_load) its
 * weights, rope tables, blocks and decoder too; else sam_path_free. */
void sam_free(struct sam_model *m);

#ifdef __cplusplus
}
#endif

#endif /* SAM3_HIP_H */
