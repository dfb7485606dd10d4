/* SPDX-License-Identifier: Unlicense
 *
 * hip_backend.c - device selection, buffers, transfers, errors and the
 * per-kernel profile of the HIP path. Takes the role ocl_backend.c has
 * in the reference (ocl_backend.h:57-104) for one discrete MI355X:
 * one device, one in-order stream, device-resident buffers.
 */
#include "hipb_internal.h"
#include "sam3_launch.h"

#include <hip/hip_runtime_api.h>

#include <ctype.h>
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------ errors */

static int err_mode = HIPB_ERR_FATAL;
static char err_msg[1024];
static int err_set;

void hipb_set_error_mode(int mode)
{
    err_mode = mode == HIPB_ERR_RECORD ? HIPB_ERR_RECORD : HIPB_ERR_FATAL;
}

const char *hipb_last_error(void)
{
    return err_set ? err_msg : NULL;
}

void hipb_clear_error(void)
{
    err_set = 0;
    err_msg[0] = 0;
}

int hipb_failed(void)
{
    return err_set;
}

void hipb_fatal(const char *fmt, ...)
{
    va_list ap;
    char buf[1024];

    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    if (err_mode == HIPB_ERR_FATAL) {
        fprintf(stderr, "ERROR: %s\n", buf);
        exit(EXIT_FAILURE);
    }
    if (!err_set) {
        memcpy(err_msg, buf, sizeof(buf));
        err_set = 1;
    }
}

const char *hipb_errstr(int err)
{
    return hipGetErrorString((hipError_t)err);
}

void hipb_check(int err, const char *what)
{
    if (err != hipSuccess)
        hipb_fatal("HIP: %s failed: %s (%d)", what, hipb_errstr(err), err);
}

/* ------------------------------------------------------------ profile */

static struct {
    const char *what;
    double ms, wall_ms, flops;
    long calls;
} prof[64];
static int nprof;
static void *prof_ev[2];
static double prof_w0;

static double now_ms(void)
{
    struct timespec ts;

    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

/* profile = 2: every launch is bracketed by two events of a pool on the
 * stream, without waiting (the kernels run back to back as they would
 * unprofiled); hipb_finish reads the pairs and adds their durations to
 * the table. A launch beyond the pool is not timed. */
#define FLOW_EV 2048
static void *flow_ev[2 * FLOW_EV];
static struct {
    const char *what;
    double flops;
} flow_op[FLOW_EV];
static int nflow;

static void flow_flush(void)
{
    int k;

    for (k = 0; k < nflow; k++) {
        float ms = 0.0f;
        int i;

        hipEventElapsedTime(&ms, (hipEvent_t)flow_ev[2 * k], (hipEvent_t)flow_ev[2 * k + 1]);
        for (i = 0; i < nprof && strcmp(prof[i].what, flow_op[k].what) != 0; i++)
            ;
        if (i == nprof && nprof < 64)
            prof[nprof++].what = flow_op[k].what;
        if (i < 64) {
            prof[i].ms += ms;
            prof[i].flops += flow_op[k].flops;
            prof[i].calls++;
        }
    }
    nflow = 0;
}

void hipb_run_begin(struct hipb_backend *b)
{
    if (!b->profile)
        return;
    if (b->profile == 2) {
        if (nflow < FLOW_EV) {
            if (!flow_ev[2 * nflow]) {
                hipEventCreate((hipEvent_t *)&flow_ev[2 * nflow]);
                hipEventCreate((hipEvent_t *)&flow_ev[2 * nflow + 1]);
            }
            hipEventRecord((hipEvent_t)flow_ev[2 * nflow], (hipStream_t)b->stream);
        }
        return;
    }
    hipStreamSynchronize((hipStream_t)b->stream);
    if (!prof_ev[0]) {
        hipEventCreate((hipEvent_t *)&prof_ev[0]);
        hipEventCreate((hipEvent_t *)&prof_ev[1]);
    }
    prof_w0 = now_ms();
    hipEventRecord((hipEvent_t)prof_ev[0], (hipStream_t)b->stream);
}

void hipb_run_end(struct hipb_backend *b, int err, const char *what,
                  double flops)
{
    float ms = 0.0f;
    double w1;
    int i;

    if (err != hipSuccess) {
        hipb_fatal("HIP: %s failed: %s (%d)", what, hipb_errstr(err), err);
        return;
    }
    if (!b->profile)
        return;
    if (b->profile == 2) {
        if (nflow < FLOW_EV) {
            hipEventRecord((hipEvent_t)flow_ev[2 * nflow + 1], (hipStream_t)b->stream);
            flow_op[nflow].what = what;
            flow_op[nflow].flops = flops;
            nflow++;
        }
        return;
    }
    hipEventRecord((hipEvent_t)prof_ev[1], (hipStream_t)b->stream);
    hipEventSynchronize((hipEvent_t)prof_ev[1]);
    w1 = now_ms();
    hipEventElapsedTime(&ms, (hipEvent_t)prof_ev[0], (hipEvent_t)prof_ev[1]);
    for (i = 0; i < nprof && strcmp(prof[i].what, what) != 0; i++)
        ;
    if (i == nprof && nprof < 64)
        prof[nprof++].what = what;
    if (i < 64) {
        prof[i].ms += ms;
        prof[i].wall_ms += w1 - prof_w0;
        prof[i].flops += flops;
        prof[i].calls++;
    }
}

int hipb_prof_count(void)
{
    return nprof;
}

int hipb_prof_entry(int i, const char **what, double *ms, double *wall_ms,
                    double *flops, long *calls)
{
    if (i < 0 || i >= nprof)
        return -1;
    *what = prof[i].what;
    *ms = prof[i].ms;
    *wall_ms = prof[i].wall_ms;
    *flops = prof[i].flops;
    *calls = prof[i].calls;
    return 0;
}

void hipb_prof_reset(void)
{
    nprof = 0;
    nflow = 0;
    memset(prof, 0, sizeof(prof));
}

/* Same table as sam_free prints (sam3_model.c:1536-1546). */
void hipb_prof_print(void)
{
    int i;

    fprintf(stderr, "%-24s %10s %10s %8s %10s\n", "kernel", "ms", "wall ms",
            "calls", "GFLOP/s");
    for (i = 0; i < nprof; i++)
        fprintf(stderr, "%-24s %10.3f %10.3f %8ld %10.1f\n", prof[i].what,
                prof[i].ms, prof[i].wall_ms, prof[i].calls,
                prof[i].ms > 0 ? prof[i].flops / (prof[i].ms * 1e6) : 0.0);
}

/* ------------------------------------------------------------ init */

/* Lower-case copy of at most cap - 1 characters of s. */
static void fold_lower(char *dst, const char *s, size_t cap)
{
    size_t i = 0;

    for (; s[i] && i + 1 < cap; i++)
        dst[i] = (char)tolower((unsigned char)s[i]);
    dst[i] = 0;
}

/* Does the platform name hold `want`, ignoring case? Both folded to
 * lower case, then a plain substring search; an empty `want` matches. */
static int name_has(const char *name, const char *want)
{
    char a[512], b[512];

    fold_lower(a, name, sizeof a);
    fold_lower(b, want, sizeof b);
    return strstr(a, b) != NULL;
}

const char *hipb_arch_name(int arch)
{
    return arch == HIPB_ARCH_DGPU ? "dgpu" : "unknown";
}

void hipb_init(struct hipb_backend *b, const char *device_opt,
               const char *platform_opt, const char *profile_opt,
               const char *precision_opt)
{
    static const char platform_name[] = "AMD HIP";
    hipDeviceProp_t prop;
    hipStream_t s;
    int n = 0, dev = 0;
    const char *env;

    memset(b, 0, sizeof(*b));
    if (platform_opt && !*platform_opt)
        platform_opt = NULL;
    if (!precision_opt || strcmp(precision_opt, "fp32") == 0)
        ;
    else if (strcmp(precision_opt, "fp16") == 0)
        b->fp16w = 1;
    else if (strcmp(precision_opt, "bf16") == 0)
        b->bf16 = 1;
    else {
        hipb_fatal("Invalid precision option <%s>", precision_opt);
        return;
    }

    if (!device_opt || strcmp(device_opt, "auto") == 0 ||
        strcmp(device_opt, "gpu") == 0)
        dev = 0;
    else if (isdigit((unsigned char)device_opt[0]))
        dev = atoi(device_opt);
    else if (strcmp(device_opt, "cpu") == 0) {
        hipb_fatal("HIP: no usable cpu device found");
        return;
    }
    else {
        hipb_fatal("Invalid device option <%s>", device_opt);
        return;
    }

    if (hipGetDeviceCount(&n) != hipSuccess)
        n = 0;
    if (platform_opt && !name_has(platform_name, platform_opt))
        n = 0;
    if (n == 0 || dev >= n) {
        hipb_fatal("HIP: no usable %s device found%s%s",
                   device_opt ? device_opt : "auto",
                   platform_opt ? " on platforms matching " : "",
                   platform_opt ? platform_opt : "");
        return;
    }

    if (profile_opt && strcmp(profile_opt, "auto") != 0 &&
        strcmp(profile_opt, "dgpu") != 0) {
        hipb_fatal("Invalid profile option <%s> for a HIP device "
                   "(auto or dgpu)",
                   profile_opt);
        return;
    }
    b->arch = HIPB_ARCH_DGPU;

    hipb_check(hipSetDevice(dev), "hipSetDevice");
    if (hipb_failed())
        return;
    hipb_check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
    if (hipb_failed())
        return;
    b->device = dev;
    snprintf(b->device_name, sizeof(b->device_name), "%.255s", prop.name);
    snprintf(b->arch_name, sizeof(b->arch_name), "%.63s", prop.gcnArchName);
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        hipb_fatal("HIP: device <%s> is %s; this library is built for gfx950 "
                   "only",
                   prop.name, prop.gcnArchName);
        return;
    }
    /* Address of this device's static scratch (mha_noalloc). */
    hipb_check(dec_scratch_init(dev), "hipGetSymbolAddress (device scratch)");
    if (hipb_failed())
        return;
    b->global_mem = prop.totalGlobalMem;
    b->max_alloc = prop.totalGlobalMem / 4 * 3;
    b->cu_count = prop.multiProcessorCount;
    b->clock_khz = prop.clockRate;

    hipb_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking),
               "hipStreamCreate");
    if (hipb_failed())
        return;
    b->stream = s;
    hipb_check(hipEventCreate((hipEvent_t *)&b->ev[0]), "hipEventCreate");
    hipb_check(hipEventCreate((hipEvent_t *)&b->ev[1]), "hipEventCreate");
    env = getenv("I_SAM3_OPENCL_PROFILE");
    b->profile = env && *env;
    if (getenv("SAM3_HIP_VERBOSE"))
        fprintf(stderr,
                "HIP device: %s [%s], %lu MiB, %d CUs, weights in %s, "
                "attention in %s\n",
                b->device_name, b->arch_name,
                (unsigned long)(b->global_mem >> 20), b->cu_count,
                b->fp16w ? "fp16" : b->bf16 ? "bf16" : "fp32",
                b->bf16 ? "bf16 MFMA" : "f32 MFMA");
}

void hipb_free(struct hipb_backend *b)
{
    if (b->stream)
        hipStreamSynchronize((hipStream_t)b->stream);
    if (b->scratch)
        hipFree(b->scratch);
    for (int i = 0; i < 2; i++) {
        if (b->stage[i])
            hipHostFree(b->stage[i]);
        if (b->stage_ev[i])
            hipEventDestroy((hipEvent_t)b->stage_ev[i]);
    }
    if (b->ev[0])
        hipEventDestroy((hipEvent_t)b->ev[0]);
    if (b->ev[1])
        hipEventDestroy((hipEvent_t)b->ev[1]);
    if (b->stream)
        hipStreamDestroy((hipStream_t)b->stream);
    memset(b, 0, sizeof(*b));
}

/* ------------------------------------------------------------ buffers */

static const size_t dt_size[3] = {4, 2, 2};

size_t hipb_count(hipb_mem m)
{
    return m ? m->bytes / dt_size[m->dtype] : 0;
}

hipb_mem hipb_alloc_typed(struct hipb_backend *b, size_t count, int dtype,
                          const char *what)
{
    size_t n;
    hipb_mem m;
    hipError_t e;

    if (dtype < HIPB_F32 || dtype > HIPB_BF16) {
        hipb_fatal("HIP: buffer <%s>: invalid element type %d", what, dtype);
        return NULL;
    }
    n = count * dt_size[dtype];
    if (n == 0)
        n = 4;
    if (n > b->max_alloc) {
        hipb_fatal("HIP: buffer <%s> needs %lu MiB, more than the device "
                   "maximum allocation of %lu MiB (reduce batch= or "
                   "tile_size=)",
                   what, (unsigned long)(n >> 20),
                   (unsigned long)(b->max_alloc >> 20));
        return NULL;
    }
    /* The name is copied behind the descriptor: callers may pass a
     * temporary string (bindings do). */
    {
        const size_t len = what ? strlen(what) : 0;

        m = calloc(1, sizeof(*m) + len + 1);
        if (!m) {
            hipb_fatal("HIP: out of host memory for buffer <%s>", what);
            return NULL;
        }
        if (what)
            memcpy((char *)(m + 1), what, len);
        m->what = (const char *)(m + 1);
    }
    e = hipMalloc(&m->ptr, n);
    if (e != hipSuccess) {
        free(m);
        hipb_fatal("HIP: allocating %lu MiB for <%s> failed: %s",
                   (unsigned long)(n >> 20), what, hipb_errstr(e));
        return NULL;
    }
    m->bytes = n;
    m->dtype = dtype;
    return m;
}

hipb_mem hipb_alloc(struct hipb_backend *b, size_t n, const char *what)
{
    return hipb_alloc_typed(b, (n + 3) / 4, HIPB_F32, what);
}

void hipb_write(struct hipb_backend *b, hipb_mem dst, size_t off,
                const void *src, size_t n)
{
    if (!dst || off + n > dst->bytes) {
        hipb_fatal("HIP: write of %lu bytes at %lu beyond buffer <%s>",
                   (unsigned long)n, (unsigned long)off,
                   dst ? dst->what : "(null)");
        return;
    }
    hipb_check(hipMemcpyAsync((char *)dst->ptr + off, src, n,
                              hipMemcpyHostToDevice, (hipStream_t)b->stream),
               "hipMemcpyAsync (write)");
    hipb_check(hipStreamSynchronize((hipStream_t)b->stream),
               "hipStreamSynchronize (write)");
}

void hipb_read(struct hipb_backend *b, hipb_mem src, size_t off, void *dst,
               size_t n)
{
    if (!src || off + n > src->bytes) {
        hipb_fatal("HIP: read of %lu bytes at %lu beyond buffer <%s>",
                   (unsigned long)n, (unsigned long)off,
                   src ? src->what : "(null)");
        return;
    }
    hipb_check(hipMemcpyAsync(dst, (const char *)src->ptr + off, n,
                              hipMemcpyDeviceToHost, (hipStream_t)b->stream),
               "hipMemcpyAsync (read)");
    hipb_check(hipStreamSynchronize((hipStream_t)b->stream),
               "hipStreamSynchronize (read)");
}

hipb_mem hipb_upload(struct hipb_backend *b, const void *src, size_t n,
                     const char *what)
{
    hipb_mem m = hipb_alloc(b, n, what);

    if (m)
        hipb_write(b, m, 0, src, n);
    return m;
}

/* IEEE 754 binary16 from binary32, round to nearest, ties to even (the
 * weight storage of precision=fp16). Worked on the magnitude's bit
 * pattern: results in binary16's normal range re-bias the exponent
 * (127 -> 15) and round the 13 dropped mantissa bits by adding
 * 0xfff plus the kept low bit before the shift (a carry out of the
 * mantissa moves the exponent up, up to infinity); results below
 * 2^-14 are whole multiples of binary16's subnormal step 2^-24, so the
 * magnitude scaled by 2^24 (exact) and rounded to an integer by rintf
 * (the default mode rounds halves to even) is the subnormal pattern,
 * 0x400 being the smallest normal one. NaN keeps its upper payload bits
 * and is made quiet. */
static uint16_t f32_to_f16(float f)
{
    uint32_t bits, mag, r;
    uint16_t sign;

    memcpy(&bits, &f, 4);
    sign = (uint16_t)((bits >> 16) & 0x8000u);
    mag = bits & 0x7fffffffu;
    if (mag > 0x7f800000u)
        return (uint16_t)(sign | 0x7e00u | (mag >> 13 & 0x3ffu));
    /* 65520 = halfway between binary16's largest finite 65504 and 2^16,
     * which ties to the even 2^16: infinity. */
    if (mag >= 0x477ff000u)
        return (uint16_t)(sign | 0x7c00u);
    if (mag < 0x38800000u) {
        float a;

        memcpy(&a, &mag, 4);
        return (uint16_t)(sign | (uint16_t)rintf(a * 0x1p24f));
    }
    r = mag - (112u << 23);
    r += 0x0fffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}

/* bfloat16, round to nearest even. */
static uint16_t f32_to_bf16(float f)
{
    uint32_t x;

    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u)
        return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

void hipb_round_half(const float *src, uint16_t *dst, size_t count, int dtype)
{
    size_t i;

    if (dtype == HIPB_F16)
        for (i = 0; i < count; i++)
            dst[i] = f32_to_f16(src[i]);
    else
        for (i = 0; i < count; i++)
            dst[i] = f32_to_bf16(src[i]);
}

hipb_mem hipb_upload_weight(struct hipb_backend *b, const float *src,
                            size_t count, const char *what)
{
    int dtype = b->fp16w ? HIPB_F16 : b->bf16 ? HIPB_BF16 : HIPB_F32;
    hipb_mem m;
    uint16_t *h;

    if (dtype == HIPB_F32)
        return hipb_upload(b, src, count * sizeof(float), what);
    m = hipb_alloc_typed(b, count, dtype, what);
    if (!m)
        return NULL;
    h = malloc(count * 2 + 2);
    hipb_round_half(src, h, count, dtype);
    hipb_write(b, m, 0, h, count * 2);
    free(h);
    return m;
}

int hipb_is_half(hipb_mem m)
{
    return m && m->dtype == HIPB_F16;
}

void hipb_release(hipb_mem *m)
{
    if (*m) {
        hipFree((*m)->ptr);
        free(*m);
        *m = NULL;
    }
}

void hipb_finish(struct hipb_backend *b)
{
    hipb_check(hipStreamSynchronize((hipStream_t)b->stream),
               "hipStreamSynchronize");
    if (b->profile == 2)
        flow_flush();
}

void hipb_copy(struct hipb_backend *b, hipb_mem src, hipb_mem dst,
               size_t src_off, size_t dst_off, size_t n)
{
    if (!src || !dst || src_off + n > src->bytes ||
        dst_off + n > dst->bytes) {
        hipb_fatal("HIP: copy of %lu bytes beyond buffer bounds",
                   (unsigned long)n);
        return;
    }
    hipb_check(hipMemcpyAsync((char *)dst->ptr + dst_off,
                              (const char *)src->ptr + src_off, n,
                              hipMemcpyDeviceToDevice, (hipStream_t)b->stream),
               "hipMemcpyAsync (copy)");
}

void *hipb_scratch(struct hipb_backend *b, size_t n)
{
    if (n <= b->scratch_bytes)
        return b->scratch;
    if (b->scratch) {
        hipStreamSynchronize((hipStream_t)b->stream);
        hipFree(b->scratch);
        b->scratch = NULL;
        b->scratch_bytes = 0;
    }
    if (hipMalloc(&b->scratch, n) != hipSuccess) {
        b->scratch = NULL;
        hipb_fatal("HIP: allocating %lu MiB of scratch failed",
                   (unsigned long)(n >> 20));
        return NULL;
    }
    b->scratch_bytes = n;
    return b->scratch;
}

/* ------------------------------------------------------------ timer */

void hipb_timer_start(struct hipb_backend *b)
{
    hipb_check(hipEventRecord((hipEvent_t)b->ev[0], (hipStream_t)b->stream),
               "hipEventRecord");
}

float hipb_timer_stop(struct hipb_backend *b)
{
    float ms = 0.0f;

    hipb_check(hipEventRecord((hipEvent_t)b->ev[1], (hipStream_t)b->stream),
               "hipEventRecord");
    hipb_check(hipEventSynchronize((hipEvent_t)b->ev[1]),
               "hipEventSynchronize");
    hipb_check(hipEventElapsedTime(&ms, (hipEvent_t)b->ev[0],
                                   (hipEvent_t)b->ev[1]),
               "hipEventElapsedTime");
    return ms;
}
