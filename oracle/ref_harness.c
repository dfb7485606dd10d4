/* Runner of the reference's own OpenCL kernels (TEST INFRASTRUCTURE ONLY).
 *
 * oracle/ref.mk compiles /root/reference/sam3_kernels.cl, unchanged,
 * into a gfx950 code object under oracle/_ref/ and builds this file into
 * oracle/_ref/libsam3ref.so. Each ref_* function uploads host arrays,
 * launches one reference kernel with the argument order and NDRange
 * geometry the reference host code uses for it, and reads the result
 * back. It is used only to produce golden vectors (tests/golden/) and as
 * a live cross-check in GPU tests; nothing in the product calls it.
 *
 * Host launch code followed: gemm() sam3_model.c:230-302, layernorm()
 * sam3_model.c:314-330, softmax_rows() sam3_model.c:332-341,
 * window_partition() / window_unpartition_add() sam3_model.c:360-392,
 * mha() sam3_model.c:413-451, rope_apply() sam3_model.c:965-978,
 * run1d() sam3_model.c:209-214, softmax_ext in attend() sam3_text.c:320-335,
 * convt_scatter() sam3_model.c:394-411, mask_logits in sam_decode()
 * sam3_model.c:1387-1398, mask_post in sam_postprocess()
 * sam3_model.c:1500-1515.
 */
#define CL_TARGET_OPENCL_VERSION 120
#define CL_USE_DEPRECATED_OPENCL_1_2_APIS
#include <CL/cl.h>

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static cl_context ctx;
static cl_command_queue q;
static cl_program prog;
static cl_device_id dev;
static char devname[256];
static char errbuf[512];

const char *ref_error(void)
{
    return errbuf;
}

const char *ref_device(void)
{
    return devname;
}

#define CHECK(e, what)                                                         \
    do {                                                                       \
        cl_int e_ = (e);                                                       \
        if (e_ != CL_SUCCESS) {                                                \
            snprintf(errbuf, sizeof(errbuf), "%s failed (%d)", what, e_);      \
            return -1;                                                         \
        }                                                                      \
    } while (0)

int ref_init(const char *code_object)
{
    cl_platform_id plats[8];
    cl_uint np = 0, nd = 0, i;
    cl_int err, st;
    FILE *f;
    long n;
    unsigned char *bin;

    CHECK(clGetPlatformIDs(8, plats, &np), "clGetPlatformIDs");
    for (i = 0; i < np; i++)
        if (clGetDeviceIDs(plats[i], CL_DEVICE_TYPE_GPU, 1, &dev, &nd) ==
                CL_SUCCESS &&
            nd > 0)
            break;
    if (i == np) {
        snprintf(errbuf, sizeof(errbuf), "no OpenCL GPU device");
        return -1;
    }
    clGetDeviceInfo(dev, CL_DEVICE_NAME, sizeof(devname), devname, NULL);
    ctx = clCreateContext(NULL, 1, &dev, NULL, NULL, &err);
    CHECK(err, "clCreateContext");
    q = clCreateCommandQueue(ctx, dev, 0, &err);
    CHECK(err, "clCreateCommandQueue");
    f = fopen(code_object, "rb");
    if (!f) {
        snprintf(errbuf, sizeof(errbuf), "cannot open %s", code_object);
        return -1;
    }
    fseek(f, 0, SEEK_END);
    n = ftell(f);
    fseek(f, 0, SEEK_SET);
    bin = malloc(n);
    if (fread(bin, 1, n, f) != (size_t)n) {
        fclose(f);
        free(bin);
        snprintf(errbuf, sizeof(errbuf), "short read of %s", code_object);
        return -1;
    }
    fclose(f);
    {
        const size_t len = (size_t)n;
        const unsigned char *b = bin;

        prog = clCreateProgramWithBinary(ctx, 1, &dev, &len, &b, &st, &err);
    }
    free(bin);
    CHECK(err, "clCreateProgramWithBinary");
    CHECK(clBuildProgram(prog, 1, &dev, "", NULL, NULL), "clBuildProgram");
    return 0;
}

void ref_free(void)
{
    if (prog)
        clReleaseProgram(prog);
    if (q)
        clReleaseCommandQueue(q);
    if (ctx)
        clReleaseContext(ctx);
    prog = NULL;
    q = NULL;
    ctx = NULL;
}

static cl_mem buf_in(const void *h, size_t bytes, cl_int *err)
{
    if (!h) {
        *err = CL_SUCCESS;
        return NULL;
    }
    return clCreateBuffer(ctx, CL_MEM_READ_WRITE | CL_MEM_COPY_HOST_PTR,
                          bytes ? bytes : 4, (void *)h, err);
}

static int launch(cl_kernel k, int dim, const size_t *g, const size_t *l,
                  const char *what)
{
    CHECK(clEnqueueNDRangeKernel(q, k, dim, NULL, g, l, 0, NULL, NULL), what);
    CHECK(clFinish(q), "clFinish");
    return 0;
}

/* run1d: 256 items per group, global rounded up (sam3_model.c:209-214). */
static int run1d(cl_kernel k, size_t n, const char *what)
{
    size_t l = 256, g = (n + l - 1) / l * l;

    return launch(k, 1, &g, &l, what);
}

#define ARG(k, i, v) CHECK(clSetKernelArg(k, i, sizeof(v), &(v)), "clSetKernelArg")

/* kernel: 0 gemm, 1 gemm_big, 2 gemm_cpu_t, 3 gemm_cpu_n. A/B/C/bias are
 * host arrays of alen/blen/clen/N floats; C is updated in place; with
 * use_r, R is C itself at roff. */
int ref_gemm(int kernel, int M, int N, int K, const float *A, long alen,
             long aoff, int lda, long sa0, long sa1, const float *B, long blen,
             long boff, int ldb, long sb0, long sb1, int transb, float *C,
             long clen, long coff, int ldc, long sc0, long sc1, int nb,
             int nb1, const float *bias, int use_r, long roff, float alpha,
             int act)
{
    static const char *names[4] = {"gemm", "gemm_big", "gemm_cpu_t",
                                   "gemm_cpu_n"};
    cl_int err, cM = M, cN = N, cK = K, clda = lda, cldb = ldb, ct = transb,
                cldc = ldc, cnb1 = nb1, cact = act;
    cl_long caoff = aoff, csa0 = sa0, csa1 = sa1, cboff = boff, csb0 = sb0,
            csb1 = sb1, ccoff = coff, csc0 = sc0, csc1 = sc1, croff = roff;
    cl_float calpha = alpha;
    cl_mem dA, dB, dC, dbias, dR;
    cl_kernel k;
    size_t g[3], l[3] = {16, 16, 1};
    int rc;

    if (kernel < 0 || kernel > 3)
        return -1;
    /* gemm_big's preconditions (sam3_model.c:240-242). */
    if (kernel == 1 &&
        !(M >= 128 && N >= 64 && K % 4 == 0 && lda % 4 == 0 && aoff % 4 == 0 &&
          sa0 % 4 == 0 && sa1 % 4 == 0 && ldb % 4 == 0 && boff % 4 == 0 &&
          sb0 % 4 == 0 && sb1 % 4 == 0)) {
        snprintf(errbuf, sizeof(errbuf), "gemm_big preconditions not met");
        return -1;
    }
    k = clCreateKernel(prog, names[kernel], &err);
    CHECK(err, "clCreateKernel");
    dA = buf_in(A, alen * 4, &err);
    CHECK(err, "A");
    dB = buf_in(B, blen * 4, &err);
    CHECK(err, "B");
    dC = buf_in(C, clen * 4, &err);
    CHECK(err, "C");
    dbias = buf_in(bias, (size_t)N * 4, &err);
    CHECK(err, "bias");
    dR = use_r ? dC : NULL;
    ARG(k, 0, cM);
    ARG(k, 1, cN);
    ARG(k, 2, cK);
    ARG(k, 3, dA);
    ARG(k, 4, caoff);
    ARG(k, 5, clda);
    ARG(k, 6, csa0);
    ARG(k, 7, csa1);
    ARG(k, 8, dB);
    ARG(k, 9, cboff);
    ARG(k, 10, cldb);
    ARG(k, 11, csb0);
    ARG(k, 12, csb1);
    ARG(k, 13, ct);
    ARG(k, 14, dC);
    ARG(k, 15, ccoff);
    ARG(k, 16, cldc);
    ARG(k, 17, csc0);
    ARG(k, 18, csc1);
    ARG(k, 19, cnb1);
    ARG(k, 20, dbias);
    ARG(k, 21, dR);
    ARG(k, 22, croff);
    ARG(k, 23, calpha);
    ARG(k, 24, cact);
    if (kernel >= 2) {
        g[0] = transb ? (size_t)(N + 3) / 4 : (size_t)(N + 7) / 8;
        g[1] = transb ? (size_t)(M + 1) / 2 : (size_t)(M + 3) / 4;
        g[2] = nb;
        rc = launch(k, 3, g, NULL, names[kernel]);
    }
    else {
        const int tile = kernel == 1 ? 128 : 64;

        g[0] = (size_t)((N + tile - 1) / tile) * 16;
        g[1] = (size_t)((M + tile - 1) / tile) * 16;
        g[2] = nb;
        rc = launch(k, 3, g, l, names[kernel]);
    }
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, dC, CL_TRUE, 0, clen * 4, C, 0, NULL, NULL),
              "read C");
    clReleaseMemObject(dA);
    clReleaseMemObject(dB);
    clReleaseMemObject(dC);
    if (dbias)
        clReleaseMemObject(dbias);
    clReleaseKernel(k);
    return rc;
}

int ref_softmax_rows(float *S, long rows, int L)
{
    cl_int err, cL = L;
    cl_mem d;
    cl_kernel k = clCreateKernel(prog, "softmax_rows", &err);
    size_t ls = L >= 256 ? 256 : 64, gs = rows * ls;
    int rc;

    CHECK(err, "clCreateKernel");
    d = buf_in(S, (size_t)rows * L * 4, &err);
    CHECK(err, "S");
    ARG(k, 0, d);
    ARG(k, 1, cL);
    rc = launch(k, 1, &gs, &ls, "softmax_rows");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, d, CL_TRUE, 0, (size_t)rows * L * 4, S, 0,
                                  NULL, NULL),
              "read S");
    clReleaseMemObject(d);
    clReleaseKernel(k);
    return rc;
}

/* softmax_ext as attend() launches it (sam3_text.c:320-335): one
 * work-group of 256 (L >= 256) or 64 items per row; dy / dx may be NULL
 * (a NULL cl_mem argument, as the reference passes for no bias). */
int ref_softmax_ext(float *S, long rows, int L, int Nq, int h0, int causal,
                    const float *dy, long ndy, const float *dx, long ndx, int W,
                    int nh)
{
    cl_int err, cL = L, cNq = Nq, ch0 = h0, cc = causal, cW = W, cnh = nh;
    cl_mem d, ddy = NULL, ddx = NULL;
    cl_kernel k = clCreateKernel(prog, "softmax_ext", &err);
    size_t ls = L >= 256 ? 256 : 64, gs = rows * ls;
    int rc;

    CHECK(err, "clCreateKernel");
    d = buf_in(S, (size_t)rows * L * 4, &err);
    CHECK(err, "S");
    if (dy) {
        ddy = buf_in(dy, (size_t)ndy * 4, &err);
        CHECK(err, "dy");
        ddx = buf_in(dx, (size_t)ndx * 4, &err);
        CHECK(err, "dx");
    }
    ARG(k, 0, d);
    ARG(k, 1, cL);
    ARG(k, 2, cNq);
    ARG(k, 3, ch0);
    ARG(k, 4, cc);
    ARG(k, 5, ddy);
    ARG(k, 6, ddx);
    ARG(k, 7, cW);
    ARG(k, 8, cnh);
    rc = launch(k, 1, &gs, &ls, "softmax_ext");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, d, CL_TRUE, 0, (size_t)rows * L * 4, S, 0,
                                  NULL, NULL),
              "read S");
    clReleaseMemObject(d);
    if (ddy) {
        clReleaseMemObject(ddy);
        clReleaseMemObject(ddx);
    }
    clReleaseKernel(k);
    return rc;
}

int ref_layernorm(const float *X, float *Y, long rows, int C, const float *g,
                  const float *b, float eps, int act)
{
    cl_int err, cC = C, cact = act;
    cl_float ceps = eps;
    cl_mem dX, dY, dg, db;
    cl_kernel k = clCreateKernel(prog, "layernorm", &err);
    size_t ls = C >= 1024 ? 256 : 64, gs = rows * ls;
    int rc;

    CHECK(err, "clCreateKernel");
    dX = buf_in(X, (size_t)rows * C * 4, &err);
    CHECK(err, "X");
    dY = buf_in(Y, (size_t)rows * C * 4, &err);
    CHECK(err, "Y");
    dg = buf_in(g, (size_t)C * 4, &err);
    CHECK(err, "g");
    db = buf_in(b, (size_t)C * 4, &err);
    CHECK(err, "b");
    ARG(k, 0, dX);
    ARG(k, 1, dY);
    ARG(k, 2, dg);
    ARG(k, 3, db);
    ARG(k, 4, cC);
    ARG(k, 5, ceps);
    ARG(k, 6, cact);
    rc = launch(k, 1, &gs, &ls, "layernorm");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, dY, CL_TRUE, 0, (size_t)rows * C * 4, Y, 0,
                                  NULL, NULL),
              "read Y");
    clReleaseMemObject(dX);
    clReleaseMemObject(dY);
    clReleaseMemObject(dg);
    clReleaseMemObject(db);
    clReleaseKernel(k);
    return rc;
}

int ref_rope_apply(float *qkv, long rows, int E, int hd, int npos,
                   const float *cs)
{
    cl_int err, cE = E, chd = hd, cnpos = npos, total = (cl_int)(rows * E);
    cl_mem d, dcs;
    cl_kernel k = clCreateKernel(prog, "rope_apply", &err);
    int rc;

    CHECK(err, "clCreateKernel");
    d = buf_in(qkv, (size_t)rows * 3 * E * 4, &err);
    CHECK(err, "qkv");
    dcs = buf_in(cs, (size_t)npos * hd * 4, &err);
    CHECK(err, "cs");
    ARG(k, 0, d);
    ARG(k, 1, cE);
    ARG(k, 2, chd);
    ARG(k, 3, cnpos);
    ARG(k, 4, dcs);
    ARG(k, 5, total);
    rc = run1d(k, (size_t)total, "rope_apply");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, d, CL_TRUE, 0, (size_t)rows * 3 * E * 4,
                                  qkv, 0, NULL, NULL),
              "read qkv");
    clReleaseMemObject(d);
    clReleaseMemObject(dcs);
    clReleaseKernel(k);
    return rc;
}

int ref_window_partition(const float *X, float *out, int H, int C, int ws,
                         int nwx)
{
    cl_int err, cH = H, cC = C, cws = ws, cnwx = nwx;
    cl_int total = nwx * nwx * ws * ws * C;
    cl_mem dX, dO;
    cl_kernel k = clCreateKernel(prog, "window_partition", &err);
    int rc;

    CHECK(err, "clCreateKernel");
    dX = buf_in(X, (size_t)H * H * C * 4, &err);
    CHECK(err, "X");
    dO = buf_in(out, (size_t)total * 4, &err);
    CHECK(err, "out");
    ARG(k, 0, dX);
    ARG(k, 1, dO);
    ARG(k, 2, cH);
    ARG(k, 3, cH);
    ARG(k, 4, cC);
    ARG(k, 5, cws);
    ARG(k, 6, cnwx);
    ARG(k, 7, total);
    rc = run1d(k, (size_t)total, "window_partition");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, dO, CL_TRUE, 0, (size_t)total * 4, out, 0,
                                  NULL, NULL),
              "read out");
    clReleaseMemObject(dX);
    clReleaseMemObject(dO);
    clReleaseKernel(k);
    return rc;
}

int ref_window_unpartition_add(float *X, const float *Wd, int H, int C, int ws,
                               int nwx)
{
    cl_int err, cH = H, cC = C, cws = ws, cnwx = nwx;
    cl_mem dX, dW;
    cl_kernel k = clCreateKernel(prog, "window_unpartition_add", &err);
    int rc;

    CHECK(err, "clCreateKernel");
    dX = buf_in(X, (size_t)H * H * C * 4, &err);
    CHECK(err, "X");
    dW = buf_in(Wd, (size_t)nwx * nwx * ws * ws * C * 4, &err);
    CHECK(err, "Wd");
    ARG(k, 0, dX);
    ARG(k, 1, dW);
    ARG(k, 2, cH);
    ARG(k, 3, cH);
    ARG(k, 4, cC);
    ARG(k, 5, cws);
    ARG(k, 6, cnwx);
    rc = run1d(k, (size_t)H * H * C, "window_unpartition_add");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, dX, CL_TRUE, 0, (size_t)H * H * C * 4, X, 0,
                                  NULL, NULL),
              "read X");
    clReleaseMemObject(dX);
    clReleaseMemObject(dW);
    clReleaseKernel(k);
    return rc;
}

/* mha() on projected tensors: 8 heads, c = dint / 8, scale 1 / sqrt(c);
 * Nk > 64 runs attn_manykeys (c must be 16), else attn_fewkeys. */
int ref_mha(int P, int Nq, int Nk, int dint, const float *Q, long qlen,
            long sq, const float *K, long klen, long sk, const float *V,
            long vlen, long sv, float *O)
{
    cl_int err, c = dint / 8, cNq = Nq, cNk = Nk, cd = dint;
    cl_int csq = (cl_int)sq, csk = (cl_int)sk, csv = (cl_int)sv;
    cl_int total = P * 8 * Nq;
    cl_float scale = 1.0f / sqrtf((float)c);
    const int many = Nk > 64;
    cl_mem dQ, dK, dV, dO;
    cl_kernel k;
    int rc;

    if (many && c != 16) {
        snprintf(errbuf, sizeof(errbuf), "mha: unsupported shape");
        return -1;
    }
    k = clCreateKernel(prog, many ? "attn_manykeys" : "attn_fewkeys", &err);
    CHECK(err, "clCreateKernel");
    dQ = buf_in(Q, qlen * 4, &err);
    CHECK(err, "Q");
    dK = buf_in(K, klen * 4, &err);
    CHECK(err, "K");
    dV = buf_in(V, vlen * 4, &err);
    CHECK(err, "V");
    dO = buf_in(O, (size_t)P * Nq * dint * 4, &err);
    CHECK(err, "O");
    ARG(k, 0, dQ);
    ARG(k, 1, csq);
    ARG(k, 2, dK);
    ARG(k, 3, csk);
    ARG(k, 4, dV);
    ARG(k, 5, csv);
    ARG(k, 6, dO);
    ARG(k, 7, cNq);
    ARG(k, 8, cNk);
    ARG(k, 9, cd);
    ARG(k, 10, c);
    ARG(k, 11, scale);
    ARG(k, 12, total);
    if (many) {
        size_t gs = (size_t)total * 256, ls = 256;

        rc = launch(k, 1, &gs, &ls, "attn_manykeys");
    }
    else
        rc = run1d(k, (size_t)total, "attn_fewkeys");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, dO, CL_TRUE, 0, (size_t)P * Nq * dint * 4, O,
                                  0, NULL, NULL),
              "read O");
    clReleaseMemObject(dQ);
    clReleaseMemObject(dK);
    clReleaseMemObject(dV);
    clReleaseMemObject(dO);
    clReleaseKernel(k);
    return rc;
}

/* convt_scatter (host convt_scatter, sam3_model.c:394-411): G [(P H W)]
 * [Co 4], out [P][2H][2W][Co], add may be NULL. */
int ref_convt_scatter(const float *G, float *out, const float *bias,
                      const float *add, int P, int H, int W, int Co, int act)
{
    cl_int err, cH = H, cW = W, cCo = Co, cact = act;
    cl_int total = P * 4 * H * W * Co;
    cl_mem dG, dO, dB, dA;
    cl_kernel k = clCreateKernel(prog, "convt_scatter", &err);
    int rc;

    CHECK(err, "clCreateKernel");
    dG = buf_in(G, (size_t)total * 4, &err);
    CHECK(err, "G");
    dO = buf_in(out, (size_t)total * 4, &err);
    CHECK(err, "out");
    dB = buf_in(bias, (size_t)Co * 4, &err);
    CHECK(err, "bias");
    dA = buf_in(add, (size_t)4 * H * W * Co * 4, &err);
    CHECK(err, "add");
    ARG(k, 0, dG);
    ARG(k, 1, dO);
    ARG(k, 2, dB);
    ARG(k, 3, dA);
    ARG(k, 4, cH);
    ARG(k, 5, cW);
    ARG(k, 6, cCo);
    ARG(k, 7, total);
    ARG(k, 8, cact);
    rc = run1d(k, (size_t)total, "convt_scatter");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, dO, CL_TRUE, 0, (size_t)total * 4, out, 0,
                                  NULL, NULL),
              "read out");
    clReleaseMemObject(dG);
    clReleaseMemObject(dO);
    clReleaseMemObject(dB);
    if (dA)
        clReleaseMemObject(dA);
    clReleaseKernel(k);
    return rc;
}

/* mask_logits as sam_decode launches it (sam3_model.c:1387-1398): U
 * [P][npix][32], hyper [P][96], out [P][3][npix]. */
int ref_mask_logits(const float *U, const float *hyper, float *out, int P,
                    int npix)
{
    cl_int err, cn = npix, total = P * npix;
    cl_mem dU, dH, dO;
    cl_kernel k = clCreateKernel(prog, "mask_logits", &err);
    int rc;

    CHECK(err, "clCreateKernel");
    dU = buf_in(U, (size_t)total * 32 * 4, &err);
    CHECK(err, "U");
    dH = buf_in(hyper, (size_t)P * 96 * 4, &err);
    CHECK(err, "hyper");
    dO = buf_in(out, (size_t)P * 3 * npix * 4, &err);
    CHECK(err, "out");
    ARG(k, 0, dU);
    ARG(k, 1, dH);
    ARG(k, 2, dO);
    ARG(k, 3, cn);
    ARG(k, 4, total);
    rc = run1d(k, (size_t)total, "mask_logits");
    if (rc == 0)
        CHECK(clEnqueueReadBuffer(q, dO, CL_TRUE, 0, (size_t)P * 3 * npix * 4,
                                  out, 0, NULL, NULL),
              "read out");
    clReleaseMemObject(dU);
    clReleaseMemObject(dH);
    clReleaseMemObject(dO);
    clReleaseKernel(k);
    return rc;
}

/* mask_post as sam_postprocess launches it (sam3_model.c:1500-1515):
 * 16 x 16 groups over (out_w, out_h) rounded up, one plane per z; stats
 * [n][6] hold the initial values on entry. */
int ref_mask_post(const float *lowres, int planes, const int *sel, int n,
                  int L, int out_h, int out_w, float offset,
                  unsigned char *mask, int *stats)
{
    cl_int err, cL = L, coh = out_h, cow = out_w;
    cl_float coff = offset;
    cl_mem dL, dS, dM, dT;
    cl_kernel k = clCreateKernel(prog, "mask_post", &err);
    size_t g[3], l[3] = {16, 16, 1};
    int rc;

    CHECK(err, "clCreateKernel");
    dL = buf_in(lowres, (size_t)planes * L * L * 4, &err);
    CHECK(err, "lowres");
    dS = buf_in(sel, (size_t)n * 4, &err);
    CHECK(err, "sel");
    dM = clCreateBuffer(ctx, CL_MEM_READ_WRITE, (size_t)n * out_h * out_w,
                        NULL, &err);
    CHECK(err, "mask");
    dT = buf_in(stats, (size_t)n * 6 * 4, &err);
    CHECK(err, "stats");
    ARG(k, 0, dL);
    ARG(k, 1, dS);
    ARG(k, 2, cL);
    ARG(k, 3, coh);
    ARG(k, 4, cow);
    ARG(k, 5, coff);
    ARG(k, 6, dM);
    ARG(k, 7, dT);
    g[0] = (size_t)(out_w + 15) / 16 * 16;
    g[1] = (size_t)(out_h + 15) / 16 * 16;
    g[2] = n;
    rc = launch(k, 3, g, l, "mask_post");
    if (rc == 0) {
        CHECK(clEnqueueReadBuffer(q, dM, CL_TRUE, 0, (size_t)n * out_h * out_w,
                                  mask, 0, NULL, NULL),
              "read mask");
        CHECK(clEnqueueReadBuffer(q, dT, CL_TRUE, 0, (size_t)n * 6 * 4, stats,
                                  0, NULL, NULL),
              "read stats");
    }
    clReleaseMemObject(dL);
    clReleaseMemObject(dS);
    clReleaseMemObject(dM);
    clReleaseMemObject(dT);
    clReleaseKernel(k);
    return rc;
}
