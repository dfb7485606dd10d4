/* SPDX-License-Identifier: Unlicense
 *
 * pth_loader.c - PyTorch checkpoint reader (torch.save zip format) with
 * the API of the reference's pth_loader.h (pth_loader.h:35-65).
 *
 * pth_open maps the whole file read-only, indexes its zip directory
 * (pth_archive.c), runs data.pkl through the pickle machine
 * (pth_unpickle.c) and records every tensor of the state_dict with its
 * storage's place in the file, after checking with overflow-safe
 * arithmetic that every element its strides reach lies inside that
 * storage. Nothing is read from the storages until a pth_read_* call (or
 * the device upload of sam3_load.c) asks for a tensor.
 */
#include "hipb_internal.h"
#include "pth_internal.h"

#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

static size_t elem_bytes(enum pth_dtype d)
{
    return d == PTH_C64 ? 8 : d == PTH_F32 ? 4 : 2;
}

static uint64_t le16(const unsigned char *p)
{
    return (uint64_t)p[0] | (uint64_t)p[1] << 8;
}

/* ------------------------------------------------------------ open */

/* Largest element count of one tensor: its float32 copy must fit a
 * size_t with room to spare. */
#define MAX_NUMEL ((uint64_t)1 << 56)

/* Check the view of entry x over a storage of `bytes` bytes; returns 0,
 * or -1 with the error set. */
static int check_view(const struct pth_entry *x, uint64_t bytes, const char *path,
                      struct pth_err *e)
{
    uint64_t last, numel = 1, end;
    int d;

    if (x->offset < 0)
        goto exceeds;
    last = (uint64_t)x->offset;
    for (d = 0; d < x->ndim; d++) {
        uint64_t reach;

        if (x->shape[d] <= 0)
            return pth_fail(e, "Empty tensor <%s> in checkpoint", x->name);
        if (x->stride[d] < 0 ||
            __builtin_mul_overflow((uint64_t)(x->shape[d] - 1), (uint64_t)x->stride[d],
                                   &reach) ||
            __builtin_add_overflow(last, reach, &last) ||
            __builtin_mul_overflow(numel, (uint64_t)x->shape[d], &numel) ||
            numel > MAX_NUMEL)
            goto exceeds;
    }
    if (__builtin_add_overflow(last, 1, &end) ||
        __builtin_mul_overflow(end, (uint64_t)elem_bytes(x->dtype), &end) || end > bytes)
        goto exceeds;
    return 0;
exceeds:
    return pth_fail(e, "Tensor <%s> exceeds its storage in <%s>", x->name, path);
}

/* The member called data.pkl, at the top or inside the archive's folder
 * (torch.save names the folder after the saved file). */
static const struct pth_member *find_pickle(const struct pth_archive *a)
{
    size_t k;

    for (k = 0; k < a->count; k++) {
        const struct pth_member *m = &a->member[k];
        const uint32_t n = m->name_len;

        if (n >= 8 && !memcmp(m->name + n - 8, "data.pkl", 8) &&
            (n == 8 || m->name[n - 9] == '/'))
            return m;
    }
    return NULL;
}

/* Fill pf->tensors from the entries: each storage is the member
 * "<folder>data/<key>" beside data.pkl. */
static int place_tensors(struct pth_file *pf, const struct pth_archive *a,
                         const struct pth_member *pkl, const struct pth_entry *v,
                         int n, struct pth_err *e)
{
    const int flen = (int)pkl->name_len - 8;
    int k, d;

    pf->tensors = calloc(n ? (size_t)n : 1, sizeof(*pf->tensors));
    if (!pf->tensors)
        return pth_fail(e, "Out of memory reading <%s>", pf->path);
    for (k = 0; k < n; k++) {
        const struct pth_entry *x = &v[k];
        struct pth_tensor *t = &pf->tensors[k];
        const struct pth_member *st;
        char *member;
        uint64_t off;
        int len;

        len = snprintf(NULL, 0, "%.*sdata/%s", flen, pkl->name, x->key);
        member = malloc((size_t)len + 1);
        if (!member)
            return pth_fail(e, "Out of memory reading <%s>", pf->path);
        snprintf(member, (size_t)len + 1, "%.*sdata/%s", flen, pkl->name, x->key);
        st = pth_archive_lookup(a, member, (size_t)len);
        if (!st) {
            pth_fail(e, "Storage <%s> of tensor <%s> missing in <%s>", member, x->name,
                     pf->path);
            free(member);
            return -1;
        }
        free(member);
        if (pth_archive_data(a, st, &off, e) != 0 || check_view(x, st->size, pf->path, e) != 0)
            return -1;
        t->name = strdup(x->name);
        if (!t->name)
            return pth_fail(e, "Out of memory reading <%s>", pf->path);
        pf->ntensors = k + 1;
        t->ndim = x->ndim;
        t->dtype = x->dtype;
        t->storage_offset = (long)x->offset;
        for (d = 0; d < x->ndim; d++) {
            t->shape[d] = (long)x->shape[d];
            t->stride[d] = (long)x->stride[d];
        }
        t->data_offset = (off_t)off;
        t->storage_bytes = (size_t)st->size;
    }
    return 0;
}

void pth_open(struct pth_file *pf, const char *path)
{
    struct pth_err e;
    struct pth_archive a;
    const struct pth_member *pkl;
    struct pth_entry *entries = NULL;
    struct stat st;
    uint64_t off;
    void *map = MAP_FAILED;
    int fd, n = 0, rc = -1;

    memset(pf, 0, sizeof(*pf));
    memset(&e, 0, sizeof(e));
    memset(&a, 0, sizeof(a));
    fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd >= 0 && fstat(fd, &st) == 0 && S_ISREG(st.st_mode) && st.st_size > 0)
        map = mmap(NULL, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (fd < 0 || !S_ISREG(st.st_mode) || (st.st_size > 0 && map == MAP_FAILED)) {
        if (fd >= 0)
            close(fd);
        hipb_fatal("Unable to open checkpoint <%s>", path);
        return;
    }
    close(fd);
    pf->map = map == MAP_FAILED ? NULL : map;
    pf->map_bytes = (size_t)st.st_size;
    pf->path = strdup(path);
    if (!pf->path) {
        pth_close(pf);
        hipb_fatal("Out of memory reading <%s>", path);
        return;
    }
    a.base = pf->map;
    a.bytes = pf->map_bytes;
    a.path = pf->path;
    if (pth_archive_index(&a, &e) != 0)
        goto out;
    pkl = find_pickle(&a);
    if (!pkl) {
        pth_fail(&e, "No data.pkl in <%s>: not a PyTorch checkpoint", pf->path);
        goto out;
    }
    if (pth_archive_data(&a, pkl, &off, &e) != 0 ||
        pth_unpickle(pf->map + off, (size_t)pkl->size, pf->path, &entries, &n, &e) != 0)
        goto out;
    rc = place_tensors(pf, &a, pkl, entries, n, &e);
out:
    pth_entries_free(entries, n);
    pth_archive_free(&a);
    if (rc != 0) {
        char msg[sizeof(e.msg)];

        memcpy(msg, e.msg, sizeof(msg));
        pth_close(pf);
        hipb_fatal("%s", msg);
    }
}

/* ------------------------------------------------------------ lookup */

const struct pth_tensor *pth_find(const struct pth_file *pf, const char *name)
{
    int k;

    for (k = 0; k < pf->ntensors; k++)
        if (!strcmp(pf->tensors[k].name, name))
            return &pf->tensors[k];
    return NULL;
}

const struct pth_tensor *pth_require(const struct pth_file *pf,
                                     const char *name, int ndim,
                                     const long *shape)
{
    const struct pth_tensor *t = pth_find(pf, name);
    int d;

    if (!t) {
        hipb_fatal("Tensor <%s> not found in checkpoint <%s>", name,
                   pf->path ? pf->path : "");
        return NULL;
    }
    if (t->ndim != ndim) {
        hipb_fatal("Tensor <%s> has rank %d, expected %d", name, t->ndim,
                   ndim);
        return NULL;
    }
    for (d = 0; shape && d < ndim; d++)
        if (shape[d] >= 0 && t->shape[d] != shape[d]) {
            hipb_fatal("Tensor <%s> has size %ld along axis %d, expected %ld",
                       name, t->shape[d], d, shape[d]);
            return NULL;
        }
    return t;
}

long pth_numel(const struct pth_tensor *t)
{
    long n = 1;
    int d;

    for (d = 0; d < t->ndim; d++)
        n *= t->shape[d];
    return n;
}

double pth_bytes(const struct pth_file *pf, const char *prefix)
{
    const size_t len = strlen(prefix);
    double sum = 0;
    int k;

    for (k = 0; k < pf->ntensors; k++)
        if (!strncmp(pf->tensors[k].name, prefix, len))
            sum += (double)pth_numel(&pf->tensors[k]) *
                   (double)elem_bytes(pf->tensors[k].dtype);
    return sum;
}

/* ------------------------------------------------------------ reads */

/* IEEE half to float: normal and special values by moving the fields,
 * zeros and subnormals as m 2^-24 (exact in float). */
static float half_bits_to_float(uint16_t h)
{
    const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 31u, man = h & 0x3ffu;
    uint32_t u;
    float f;

    if (e == 31)
        u = s | 0x7f800000u | man << 13;
    else if (e)
        u = s | (e + 112) << 23 | man << 13;
    else {
        f = (float)man * 0x1p-24f;
        memcpy(&u, &f, 4);
        u |= s;
    }
    memcpy(&f, &u, 4);
    return f;
}

static float to_float(const unsigned char *p, enum pth_dtype d)
{
    uint32_t u;
    float f;

    if (d == PTH_F32) {
        memcpy(&f, p, 4);
        return f;
    }
    if (d == PTH_F16)
        return half_bits_to_float((uint16_t)le16(p));
    u = (uint32_t)le16(p) << 16;
    memcpy(&f, &u, 4);
    return f;
}

/* Innermost run of elements that are adjacent in the storage, in C
 * order: the trailing dimensions of unit stride chaining. */
static long contiguous_tail(const struct pth_tensor *t, int *dims)
{
    long run = 1;
    int d = t->ndim;

    while (d > 0 && (t->shape[d - 1] == 1 || t->stride[d - 1] == run)) {
        run *= t->shape[d - 1];
        d--;
    }
    *dims = d;
    return run;
}

/* Visit the tensor in C order as runs of contiguous storage elements:
 * fn(arg, storage element offset, run length, output element index). */
static void for_runs(const struct pth_tensor *t,
                     void (*fn)(void *, long, long, long), void *arg)
{
    long idx[PTH_MAX_DIMS] = {0}, out = 0, n = pth_numel(t), run;
    int outer, d;

    run = contiguous_tail(t, &outer);
    while (out < n) {
        long off = t->storage_offset;

        for (d = 0; d < outer; d++)
            off += idx[d] * t->stride[d];
        fn(arg, off, run, out);
        out += run;
        for (d = outer - 1; d >= 0; d--) {
            if (++idx[d] < t->shape[d])
                break;
            idx[d] = 0;
        }
    }
}

struct runargs {
    const unsigned char *base; /* storage data */
    enum pth_dtype dtype;
    unsigned char *dst;
};

static void run_f32(void *arg, long off, long len, long out)
{
    const struct runargs *a = arg;
    float *dst = (float *)a->dst + out;
    long i;

    if (a->dtype == PTH_F32) {
        memcpy(dst, a->base + (size_t)off * 4, (size_t)len * 4);
        return;
    }
    for (i = 0; i < len; i++)
        dst[i] = to_float(a->base + (size_t)(off + i) * 2, a->dtype);
}

static void run_c64(void *arg, long off, long len, long out)
{
    const struct runargs *a = arg;

    memcpy(a->dst + (size_t)out * 8, a->base + (size_t)off * 8,
           (size_t)len * 8);
}

float *pth_read_f32(const struct pth_file *pf, const struct pth_tensor *t)
{
    struct runargs a;

    if (t->dtype == PTH_C64) {
        hipb_fatal("Tensor <%s> is complex, a real tensor is expected",
                   t->name);
        return NULL;
    }
    a.base = pf->map + t->data_offset;
    a.dtype = t->dtype;
    a.dst = malloc((size_t)pth_numel(t) * sizeof(float));
    if (!a.dst) {
        hipb_fatal("Out of memory reading tensor <%s>", t->name);
        return NULL;
    }
    for_runs(t, run_f32, &a);
    return (float *)a.dst;
}

float *pth_read_c64(const struct pth_file *pf, const struct pth_tensor *t)
{
    struct runargs a;

    if (t->dtype != PTH_C64) {
        hipb_fatal("Tensor <%s> is not complex", t->name);
        return NULL;
    }
    /* Little-endian complex64 elements are (float re, float im). */
    a.base = pf->map + t->data_offset;
    a.dtype = t->dtype;
    a.dst = malloc((size_t)pth_numel(t) * 8);
    if (!a.dst) {
        hipb_fatal("Out of memory reading tensor <%s>", t->name);
        return NULL;
    }
    for_runs(t, run_c64, &a);
    return (float *)a.dst;
}

void pth_read_row_f32(const struct pth_file *pf, const struct pth_tensor *t,
                      long r, float *dst)
{
    if (t->dtype != PTH_F32 || t->ndim != 2 || t->stride[1] != 1 ||
        t->stride[0] != t->shape[1]) {
        hipb_fatal("Tensor <%s> is not a contiguous float32 matrix", t->name);
        return;
    }
    if (r < 0 || r >= t->shape[0]) {
        hipb_fatal("Row %ld out of range in tensor <%s>", r, t->name);
        return;
    }
    memcpy(dst,
           pf->map + t->data_offset +
               (size_t)(t->storage_offset + r * t->stride[0]) * 4,
           (size_t)t->shape[1] * sizeof(float));
}

void pth_close(struct pth_file *pf)
{
    int k;

    if (pf->map)
        munmap((void *)pf->map, pf->map_bytes);
    for (k = 0; k < pf->ntensors; k++)
        free(pf->tensors[k].name);
    free(pf->tensors);
    free(pf->path);
    memset(pf, 0, sizeof(*pf));
}
