/* SPDX-License-Identifier: Unlicense
 *
 * pth_loader.c - PyTorch checkpoint reader (torch.save zip format) with
 * the API of the reference's pth_loader.c (pth_loader.c:709-1052).
 *
 * The whole file is mapped read-only. pth_open walks the zip central
 * directory (classic or zip64 end records, zip64 extra fields), runs the
 * archive's data.pkl through a small pickle machine that knows the
 * opcodes torch.save emits (protocols 2 to 5) and the callables that
 * rebuild tensors and parameters, and records every tensor of the
 * state_dict with its storage's place in the file. Nothing is read from
 * the storages until a pth_read_* call (or the device upload of
 * sam3_load.c) asks for a tensor.
 *
 * Format facts used here (PKWARE APPNOTE 6.3, CPython Lib/pickle.py,
 * torch/serialization.py and torch/_utils.py): torch.save writes stored
 * entries "<archive>/data.pkl" and "<archive>/data/<key>"; a tensor is
 * pickled as REDUCE(torch._utils._rebuild_tensor_v2, (storage, offset,
 * size, stride, requires_grad, hooks)) with the storage a persistent id
 * ("storage", torch.<Type>Storage, key, location, numel).
 */
#include "hipb_internal.h"
#include "pth_loader.h"

#include <fcntl.h>
#include <setjmp.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ------------------------------------------------------------ context */

/* Parse state of one pth_open: a failure formats its message and jumps
 * back to pth_open, which releases everything and reports it. */
struct ctx {
    jmp_buf jb;
    char msg[768];
    const char *path;
    const unsigned char *base;
    size_t size;
};

static void die(struct ctx *c, const char *fmt, ...)
    __attribute__((noreturn, format(printf, 2, 3)));

static void die(struct ctx *c, const char *fmt, ...)
{
    va_list ap;

    va_start(ap, fmt);
    vsnprintf(c->msg, sizeof(c->msg), fmt, ap);
    va_end(ap);
    longjmp(c->jb, 1);
}

/* Little-endian unsigned integer of n bytes. */
static uint64_t le(const unsigned char *p, int n)
{
    uint64_t v = 0;

    while (n-- > 0)
        v = v << 8 | p[n];
    return v;
}

/* File bytes [off, off + n), or a fatal truncation. */
static const unsigned char *at(struct ctx *c, uint64_t off, uint64_t n)
{
    if (off > c->size || n > c->size - off)
        die(c, "Truncated zip structure in <%s>", c->path);
    return c->base + off;
}

/* ------------------------------------------------------------ zip */

struct zent {
    const char *name; /* into the mapping, nlen bytes, not terminated */
    int nlen;
    int method;
    uint64_t size, loff;
};

struct zdir {
    long n;
    struct zent *e;
};

#define SIG_EOCD 0x06054b50u
#define SIG_EOCD64 0x06064b50u
#define SIG_LOC64 0x07064b50u
#define SIG_CDIR 0x02014b50u
#define SIG_LOCAL 0x04034b50u

static void zip_dir(struct ctx *c, struct zdir *z)
{
    const unsigned char *eocd = NULL, *p, *end;
    uint64_t n, cdsize, cdoff;
    size_t i, lo;
    long k;

    /* The end record (22 bytes plus a comment of at most 65535) is the
     * last occurrence of its signature. */
    if (c->size >= 22) {
        lo = c->size > 22 + 65535 ? c->size - 22 - 65535 : 0;
        for (i = c->size - 22 + 1; i-- > lo;)
            if (le(c->base + i, 4) == SIG_EOCD) {
                eocd = c->base + i;
                break;
            }
    }
    if (!eocd)
        die(c, "<%s> is not a zip archive (PyTorch >= 1.6 checkpoint format "
               "expected)", c->path);
    n = le(eocd + 10, 2);
    cdsize = le(eocd + 12, 4);
    cdoff = le(eocd + 16, 4);
    if (n == 0xffff || cdsize == 0xffffffffu || cdoff == 0xffffffffu) {
        const unsigned char *loc, *rec;

        if (eocd - c->base < 20 || le(eocd - 20, 4) != SIG_LOC64)
            die(c, "Corrupt zip64 directory in <%s>", c->path);
        loc = eocd - 20;
        rec = at(c, le(loc + 8, 8), 56);
        if (le(rec, 4) != SIG_EOCD64)
            die(c, "Corrupt zip64 end record in <%s>", c->path);
        n = le(rec + 32, 8);
        cdsize = le(rec + 40, 8);
        cdoff = le(rec + 48, 8);
    }
    p = at(c, cdoff, cdsize);
    end = p + cdsize;
    if (n > cdsize / 46)
        die(c, "Corrupt zip central directory in <%s>", c->path);
    z->e = calloc(n ? n : 1, sizeof(*z->e));
    for (k = 0; k < (long)n; k++) {
        struct zent *e = &z->e[k];
        uint64_t csize, usize, loff;
        unsigned nlen, xlen, clen;
        const unsigned char *x, *xend;

        if (end - p < 46 || le(p, 4) != SIG_CDIR)
            die(c, "Corrupt zip central directory in <%s>", c->path);
        e->method = (int)le(p + 10, 2);
        csize = le(p + 20, 4);
        usize = le(p + 24, 4);
        nlen = (unsigned)le(p + 28, 2);
        xlen = (unsigned)le(p + 30, 2);
        clen = (unsigned)le(p + 32, 2);
        loff = le(p + 42, 4);
        if ((uint64_t)(end - p) < 46ull + nlen + xlen + clen)
            die(c, "Corrupt zip central directory in <%s>", c->path);
        e->name = (const char *)p + 46;
        e->nlen = (int)nlen;
        /* Zip64 extended information: the 8-byte values of the fields
         * whose 4-byte slots hold 0xffffffff, in the order uncompressed
         * size, compressed size, local header offset. */
        for (x = p + 46 + nlen, xend = x + xlen; xend - x >= 4;) {
            unsigned id = (unsigned)le(x, 2), len = (unsigned)le(x + 2, 2);
            const unsigned char *v = x + 4, *vend = v + len;

            if (vend > xend)
                break;
            if (id == 1) {
                if (usize == 0xffffffffu && vend - v >= 8)
                    usize = le(v, 8), v += 8;
                if (csize == 0xffffffffu && vend - v >= 8)
                    csize = le(v, 8), v += 8;
                if (loff == 0xffffffffu && vend - v >= 8)
                    loff = le(v, 8);
            }
            x = vend;
        }
        e->size = usize;
        e->loff = loff;
        (void)csize;
        p += 46 + nlen + xlen + clen;
    }
    z->n = (long)n;
}

static const struct zent *zip_find(const struct zdir *z, const char *name,
                                   size_t len)
{
    long k;

    for (k = 0; k < z->n; k++)
        if ((size_t)z->e[k].nlen == len && !memcmp(z->e[k].name, name, len))
            return &z->e[k];
    return NULL;
}

/* Byte offset of an entry's data: past its local header, whose own
 * extra field (torch pads it to align the data) may differ from the
 * central directory's. */
static uint64_t zip_data(struct ctx *c, const struct zent *e)
{
    const unsigned char *h;
    uint64_t off;

    if (e->method != 0)
        die(c, "Zip entry <%.*s> in <%s> is compressed; only stored entries "
               "(as written by torch.save) are supported",
            e->nlen, e->name, c->path);
    h = at(c, e->loff, 30);
    if (le(h, 4) != SIG_LOCAL)
        die(c, "Corrupt local header for <%.*s> in <%s>", e->nlen, e->name,
            c->path);
    off = e->loff + 30 + le(h + 26, 2) + le(h + 28, 2);
    at(c, off, e->size);
    return off;
}

/* ------------------------------------------------------------ pickle */

enum vkind {
    V_NONE, V_INT, V_FLOAT, V_STR, V_TUPLE, V_LIST, V_DICT, V_GLOBAL,
    V_STORAGE, V_TENSOR, V_OTHER
};

struct tens {
    struct val *storage;
    long offset;
    int ndim;
    long shape[PTH_MAX_DIMS], stride[PTH_MAX_DIMS];
};

struct val {
    enum vkind kind;
    long long i;        /* V_INT */
    const char *s;      /* V_STR text, V_GLOBAL module, V_STORAGE key */
    const char *s2;     /* V_GLOBAL name */
    int n, cap;         /* items: tuple / list; dict as k0 v0 k1 v1 ... */
    struct val **it;
    enum pth_dtype dtype; /* V_STORAGE */
    struct tens *t;       /* V_TENSOR */
};

/* Arena of the machine's values and strings, freed at once. */
struct chunk {
    struct chunk *next;
    size_t used, cap;
    unsigned char mem[];
};

struct vm {
    struct ctx *c;
    const unsigned char *p, *end;
    struct chunk *arena;
    struct val **stack;
    long sp, scap;
    long *marks;
    long nm, mcap;
    struct val **memo;
    long nmemo, memocap;
};

static void *grow(struct vm *m, void *a, long *cap, long need, size_t es)
{
    long nc = *cap ? *cap : 64;
    void *b;

    if (need <= *cap)
        return a;
    while (nc < need)
        nc *= 2;
    b = realloc(a, (size_t)nc * es);
    if (!b)
        die(m->c, "Out of memory reading <%s>", m->c->path);
    *cap = nc;
    return b;
}

static void *alloc(struct vm *m, size_t n)
{
    struct chunk *k = m->arena;
    void *r;

    n = (n + 15) & ~(size_t)15;
    if (!k || k->cap - k->used < n) {
        size_t cap = n > 65536 ? n : 65536;

        k = malloc(sizeof(*k) + cap);
        if (!k)
            die(m->c, "Out of memory reading <%s>", m->c->path);
        k->next = m->arena;
        k->used = 0;
        k->cap = cap;
        m->arena = k;
    }
    r = k->mem + k->used;
    k->used += n;
    memset(r, 0, n);
    return r;
}

static void vm_free(struct vm *m)
{
    while (m->arena) {
        struct chunk *k = m->arena;

        m->arena = k->next;
        free(k);
    }
    free(m->stack);
    free(m->marks);
    free(m->memo);
}

static struct val *mk(struct vm *m, enum vkind kind)
{
    struct val *v = alloc(m, sizeof(*v));

    v->kind = kind;
    return v;
}

static const char *mkstr(struct vm *m, const unsigned char *s, size_t n)
{
    char *d = alloc(m, n + 1);

    memcpy(d, s, n);
    return d;
}

static void add(struct vm *m, struct val *c, struct val *v)
{
    if (c->n == c->cap) {
        int nc = c->cap ? 2 * c->cap : 8;
        struct val **it = alloc(m, (size_t)nc * sizeof(*it));

        if (c->n)
            memcpy(it, c->it, (size_t)c->n * sizeof(*it));
        c->it = it;
        c->cap = nc;
    }
    c->it[c->n++] = v;
}

static const unsigned char *take(struct vm *m, uint64_t n)
{
    const unsigned char *q = m->p;

    if ((uint64_t)(m->end - m->p) < n)
        die(m->c, "Truncated pickle in checkpoint <%s>", m->c->path);
    m->p += n;
    return q;
}

static const char *take_line(struct vm *m)
{
    const unsigned char *q = m->p, *nl = memchr(q, '\n', m->end - q);

    if (!nl)
        die(m->c, "Truncated pickle in checkpoint <%s>", m->c->path);
    m->p = nl + 1;
    return mkstr(m, q, nl - q);
}

static void push(struct vm *m, struct val *v)
{
    m->stack = grow(m, m->stack, &m->scap, m->sp + 1, sizeof(*m->stack));
    m->stack[m->sp++] = v;
}

static struct val *pop(struct vm *m)
{
    if (m->sp <= (m->nm ? m->marks[m->nm - 1] : 0))
        die(m->c, "Pickle stack underflow in checkpoint <%s>", m->c->path);
    return m->stack[--m->sp];
}

static struct val *top(struct vm *m)
{
    if (m->sp <= (m->nm ? m->marks[m->nm - 1] : 0))
        die(m->c, "Pickle stack underflow in checkpoint <%s>", m->c->path);
    return m->stack[m->sp - 1];
}

/* Stack height at the topmost mark, which is removed. */
static long pop_mark(struct vm *m)
{
    if (!m->nm)
        die(m->c, "Pickle mark not found in checkpoint <%s>", m->c->path);
    return m->marks[--m->nm];
}

/* A tuple of the stack items from height h up; the stack drops to h. */
static struct val *tuple_from(struct vm *m, long h)
{
    struct val *v = mk(m, V_TUPLE);
    long k;

    for (k = h; k < m->sp; k++)
        add(m, v, m->stack[k]);
    m->sp = h;
    return v;
}

static void memo_set(struct vm *m, uint64_t idx, struct val *v)
{
    /* torch.save memoizes a few values per tensor; 2^24 slots (128 MiB of
     * pointers) bound what a corrupt index can make this allocate. */
    if (idx >= (uint64_t)1 << 24)
        die(m->c, "Invalid pickle memo index in <%s>", m->c->path);
    if ((long)idx >= m->memocap) {
        long old = m->memocap;

        m->memo = grow(m, m->memo, &m->memocap, (long)idx + 1,
                       sizeof(*m->memo));
        memset(m->memo + old, 0, (size_t)(m->memocap - old) * sizeof(*m->memo));
    }
    m->memo[idx] = v;
    if ((long)idx >= m->nmemo)
        m->nmemo = (long)idx + 1;
}

static struct val *memo_get(struct vm *m, uint64_t idx)
{
    if (idx >= (uint64_t)m->nmemo || !m->memo[idx])
        die(m->c, "Invalid pickle memo reference %llu in <%s>",
            (unsigned long long)idx, m->c->path);
    return m->memo[idx];
}

static long long as_int(struct vm *m, const struct val *v)
{
    if (v->kind != V_INT)
        die(m->c, "Integer expected in checkpoint pickle <%s>", m->c->path);
    return v->i;
}

static int is_global(const struct val *v, const char *mod, const char *name)
{
    return v->kind == V_GLOBAL && !strcmp(v->s, mod) && !strcmp(v->s2, name);
}

/* REDUCE: the tensor and parameter rebuilders and OrderedDict are
 * understood; any other callable gives an opaque object. */
static struct val *reduce(struct vm *m, struct val *fn, struct val *args)
{
    if (args->kind != V_TUPLE)
        die(m->c, "Pickle REDUCE without argument tuple in <%s>", m->c->path);
    if (is_global(fn, "torch._utils", "_rebuild_tensor_v2") ||
        is_global(fn, "torch._utils", "_rebuild_tensor")) {
        const struct val *size, *stride;
        struct val *v;
        int d;

        if (args->n < 4 || args->it[0]->kind != V_STORAGE ||
            args->it[2]->kind != V_TUPLE || args->it[3]->kind != V_TUPLE)
            die(m->c, "Unexpected tensor rebuild arguments in <%s>",
                m->c->path);
        size = args->it[2];
        stride = args->it[3];
        if (size->n > PTH_MAX_DIMS || size->n != stride->n)
            die(m->c, "Unsupported tensor rank %d in <%s>", size->n,
                m->c->path);
        v = mk(m, V_TENSOR);
        v->t = alloc(m, sizeof(*v->t));
        v->t->storage = args->it[0];
        v->t->offset = (long)as_int(m, args->it[1]);
        v->t->ndim = size->n;
        for (d = 0; d < size->n; d++) {
            v->t->shape[d] = (long)as_int(m, size->it[d]);
            v->t->stride[d] = (long)as_int(m, stride->it[d]);
        }
        return v;
    }
    if (is_global(fn, "torch._utils", "_rebuild_parameter") ||
        is_global(fn, "torch._utils", "_rebuild_parameter_with_state")) {
        if (args->n < 1 || args->it[0]->kind != V_TENSOR)
            die(m->c, "Unexpected parameter rebuild arguments in <%s>",
                m->c->path);
        return args->it[0];
    }
    if (is_global(fn, "collections", "OrderedDict"))
        return mk(m, V_DICT);
    return mk(m, V_OTHER);
}

/* BINPERSID: ("storage", torch.<Type>Storage, key, location, numel). */
static struct val *storage(struct vm *m, const struct val *pid)
{
    static const struct {
        const char *name;
        enum pth_dtype dtype;
    } types[] = {{"FloatStorage", PTH_F32},
                 {"HalfStorage", PTH_F16},
                 {"BFloat16Storage", PTH_BF16},
                 {"ComplexFloatStorage", PTH_C64}};
    struct val *v;
    size_t k;

    if (pid->kind != V_TUPLE || pid->n < 5 || pid->it[0]->kind != V_STR ||
        strcmp(pid->it[0]->s, "storage") || pid->it[1]->kind != V_GLOBAL ||
        pid->it[2]->kind != V_STR)
        die(m->c, "Unsupported persistent id in checkpoint <%s>", m->c->path);
    v = mk(m, V_STORAGE);
    v->s = pid->it[2]->s;
    for (k = 0; k < sizeof(types) / sizeof(types[0]); k++)
        if (!strcmp(pid->it[1]->s2, types[k].name)) {
            v->dtype = types[k].dtype;
            return v;
        }
    die(m->c, "Unsupported tensor storage type <%s.%s> in checkpoint "
              "(float32, float16, bfloat16 and complex64 are supported)",
        pid->it[1]->s, pid->it[1]->s2);
}

/* Items from the topmost mark go into the container below it (dict:
 * key, value pairs; list: values; anything else drops them). */
static void extend_from_mark(struct vm *m, int pairs)
{
    long h = pop_mark(m), k;
    struct val *c;

    if (h < 1 || (pairs && (m->sp - h) % 2))
        die(m->c, "Invalid %s in checkpoint pickle <%s>",
            pairs ? "SETITEMS" : "APPENDS", m->c->path);
    c = m->stack[h - 1];
    if (c->kind == (pairs ? V_DICT : V_LIST))
        for (k = h; k < m->sp; k++)
            add(m, c, m->stack[k]);
    m->sp = h;
}

static struct val *run(struct vm *m)
{
    for (;;) {
        const unsigned char op = *take(m, 1);
        const unsigned char *q;
        struct val *a, *b, *v;
        uint64_t n;

        switch (op) {
        case 0x80: /* PROTO */
            take(m, 1);
            break;
        case 0x95: /* FRAME */
            take(m, 8);
            break;
        case '.': /* STOP */
            return pop(m);
        case '(': /* MARK */
            m->marks = grow(m, m->marks, &m->mcap, m->nm + 1,
                            sizeof(*m->marks));
            m->marks[m->nm++] = m->sp;
            break;
        case '0': /* POP */
            if (m->nm && m->sp == m->marks[m->nm - 1])
                m->nm--;
            else
                pop(m);
            break;
        case '1': /* POP_MARK */
            m->sp = pop_mark(m);
            break;
        case '2': /* DUP */
            push(m, top(m));
            break;
        case '}': /* EMPTY_DICT */
            push(m, mk(m, V_DICT));
            break;
        case ']': /* EMPTY_LIST */
            push(m, mk(m, V_LIST));
            break;
        case ')': /* EMPTY_TUPLE */
            push(m, mk(m, V_TUPLE));
            break;
        case 0x8f: /* EMPTY_SET */
            push(m, mk(m, V_OTHER));
            break;
        case 'N': /* NONE */
            push(m, mk(m, V_NONE));
            break;
        case 0x88: /* NEWTRUE */
        case 0x89: /* NEWFALSE */
            v = mk(m, V_INT);
            v->i = op == 0x88;
            push(m, v);
            break;
        case 'J': /* BININT: signed 32-bit */
            v = mk(m, V_INT);
            v->i = (int32_t)(uint32_t)le(take(m, 4), 4);
            push(m, v);
            break;
        case 'K': /* BININT1 */
            v = mk(m, V_INT);
            v->i = *take(m, 1);
            push(m, v);
            break;
        case 'M': /* BININT2 */
            v = mk(m, V_INT);
            v->i = (long long)le(take(m, 2), 2);
            push(m, v);
            break;
        case 0x8a: /* LONG1 */
        case 0x8b: /* LONG4: little-endian two's complement */
            n = op == 0x8a ? *take(m, 1) : le(take(m, 4), 4);
            if (n > 8)
                die(m->c, "Integer too large in checkpoint pickle <%s>",
                    m->c->path);
            q = take(m, n);
            v = mk(m, V_INT);
            v->i = (long long)le(q, (int)n);
            if (n && n < 8 && (q[n - 1] & 0x80))
                v->i -= (long long)1 << (8 * n);
            push(m, v);
            break;
        case 'G': { /* BINFLOAT: big-endian double */
            uint64_t u = 0;
            double d;
            int k;

            q = take(m, 8);
            for (k = 0; k < 8; k++)
                u = u << 8 | q[k];
            memcpy(&d, &u, 8);
            (void)d;
            push(m, mk(m, V_FLOAT));
            break;
        }
        case 'X':    /* BINUNICODE */
        case 'T':    /* BINSTRING */
        case 0x8c:   /* SHORT_BINUNICODE */
        case 'U':    /* SHORT_BINSTRING */
        case 0x8d: { /* BINUNICODE8 */
            n = op == 0x8c || op == 'U' ? *take(m, 1)
                : op == 0x8d            ? le(take(m, 8), 8)
                                        : le(take(m, 4), 4);
            q = take(m, n);
            v = mk(m, V_STR);
            v->s = mkstr(m, q, n);
            push(m, v);
            break;
        }
        case 'B':  /* BINBYTES */
        case 'C':  /* SHORT_BINBYTES */
        case 0x8e: /* BINBYTES8 */
            n = op == 'C' ? *take(m, 1) : op == 'B' ? le(take(m, 4), 4)
                                                    : le(take(m, 8), 8);
            take(m, n);
            push(m, mk(m, V_OTHER));
            break;
        case 'c': /* GLOBAL: module and name lines */
            v = mk(m, V_GLOBAL);
            v->s = take_line(m);
            v->s2 = take_line(m);
            push(m, v);
            break;
        case 0x93: /* STACK_GLOBAL */
            b = pop(m);
            a = pop(m);
            if (a->kind != V_STR || b->kind != V_STR)
                die(m->c, "Invalid STACK_GLOBAL in checkpoint <%s>",
                    m->c->path);
            v = mk(m, V_GLOBAL);
            v->s = a->s;
            v->s2 = b->s;
            push(m, v);
            break;
        case 'q': /* BINPUT */
            memo_set(m, *take(m, 1), top(m));
            break;
        case 'r': /* LONG_BINPUT */
            memo_set(m, le(take(m, 4), 4), top(m));
            break;
        case 0x94: /* MEMOIZE: the next index is the memo's length */
            memo_set(m, (uint64_t)m->nmemo, top(m));
            break;
        case 'h': /* BINGET */
            push(m, memo_get(m, *take(m, 1)));
            break;
        case 'j': /* LONG_BINGET */
            push(m, memo_get(m, le(take(m, 4), 4)));
            break;
        case 't': /* TUPLE */
            push(m, tuple_from(m, pop_mark(m)));
            break;
        case 0x85: /* TUPLE1 */
        case 0x86: /* TUPLE2 */
        case 0x87: /* TUPLE3 */
            n = op - 0x84;
            if ((uint64_t)(m->sp - (m->nm ? m->marks[m->nm - 1] : 0)) < n)
                die(m->c, "Pickle stack underflow in checkpoint <%s>",
                    m->c->path);
            push(m, tuple_from(m, m->sp - (long)n));
            break;
        case 'Q': /* BINPERSID */
            push(m, storage(m, pop(m)));
            break;
        case 'R': /* REDUCE */
            a = pop(m);
            b = pop(m);
            push(m, reduce(m, b, a));
            break;
        case 0x81: /* NEWOBJ */
            pop(m);
            pop(m);
            push(m, mk(m, V_OTHER));
            break;
        case 0x92: /* NEWOBJ_EX */
            pop(m);
            pop(m);
            pop(m);
            push(m, mk(m, V_OTHER));
            break;
        case 'b': /* BUILD: object state plays no part in a state_dict */
            pop(m);
            top(m);
            break;
        case 's': /* SETITEM */
            b = pop(m);
            a = pop(m);
            v = top(m);
            if (v->kind == V_DICT) {
                add(m, v, a);
                add(m, v, b);
            }
            break;
        case 'u': /* SETITEMS */
            extend_from_mark(m, 1);
            break;
        case 'a': /* APPEND */
            a = pop(m);
            v = top(m);
            if (v->kind == V_LIST)
                add(m, v, a);
            break;
        case 'e':  /* APPENDS */
        case 0x90: /* ADDITEMS (sets are opaque) */
            extend_from_mark(m, 0);
            break;
        case 0x91: /* FROZENSET */
            m->sp = pop_mark(m);
            push(m, mk(m, V_OTHER));
            break;
        default:
            die(m->c, "Unsupported pickle opcode 0x%02x in checkpoint <%s>",
                op, m->c->path);
        }
    }
}

static int has_tensors(const struct val *d)
{
    int k;

    for (k = 1; k < d->n; k += 2)
        if (d->it[k]->kind == V_TENSOR)
            return 1;
    return 0;
}

/* The saved dict if it holds tensors, else its "model" or "state_dict"
 * entry (training checkpoints wrap the weights so). */
static const struct val *state_dict(const struct val *root)
{
    int k;

    if (root->kind != V_DICT)
        return NULL;
    if (has_tensors(root))
        return root;
    for (k = 0; k + 1 < root->n; k += 2) {
        const struct val *key = root->it[k], *v = root->it[k + 1];

        if (key->kind == V_STR && v->kind == V_DICT && has_tensors(v) &&
            (!strcmp(key->s, "model") || !strcmp(key->s, "state_dict")))
            return v;
    }
    return NULL;
}

/* ------------------------------------------------------------ open */

static size_t elem_bytes(enum pth_dtype d)
{
    return d == PTH_C64 ? 8 : d == PTH_F32 ? 4 : 2;
}

static void drop_tensors(struct pth_file *pf)
{
    int i;

    for (i = 0; i < pf->ntensors; i++)
        free(pf->tensors[i].name);
    free(pf->tensors);
    pf->tensors = NULL;
    pf->ntensors = 0;
}

/* Index the state_dict sd of the archive whose data.pkl sits under the
 * folder prefix (plen bytes): every (string key, tensor) pair. */
static void index_tensors(struct ctx *c, struct pth_file *pf,
                          const struct zdir *z, const struct val *sd,
                          const char *prefix, size_t plen)
{
    char name[1024];
    int k, nt = 0;

    for (k = 1; k < sd->n; k += 2)
        nt += sd->it[k]->kind == V_TENSOR && sd->it[k - 1]->kind == V_STR;
    pf->tensors = calloc(nt ? nt : 1, sizeof(*pf->tensors));
    for (k = 1; k < sd->n; k += 2) {
        const struct val *key = sd->it[k - 1], *tv = sd->it[k];
        const struct tens *src;
        struct pth_tensor *t;
        const struct zent *ze;
        long long last;
        int d, len;

        if (tv->kind != V_TENSOR || key->kind != V_STR)
            continue;
        src = tv->t;
        t = &pf->tensors[pf->ntensors++];
        t->name = strdup(key->s);
        t->ndim = src->ndim;
        t->storage_offset = src->offset;
        t->dtype = src->storage->dtype;
        for (d = 0; d < src->ndim; d++) {
            t->shape[d] = src->shape[d];
            t->stride[d] = src->stride[d];
        }
        len = snprintf(name, sizeof(name), "%.*sdata/%s", (int)plen, prefix,
                       src->storage->s);
        ze = len < (int)sizeof(name) ? zip_find(z, name, (size_t)len) : NULL;
        if (!ze)
            die(c, "Storage <%s> of tensor <%s> missing in <%s>", name,
                t->name, c->path);
        t->data_offset = (off_t)zip_data(c, ze);
        t->storage_bytes = (size_t)ze->size;
        /* Every element the strides reach lies inside the storage. */
        last = t->storage_offset;
        for (d = 0; d < t->ndim; d++) {
            if (t->shape[d] <= 0)
                die(c, "Empty tensor <%s> in checkpoint", t->name);
            if (t->stride[d] < 0 || t->shape[d] > ((long long)1 << 40) ||
                t->stride[d] > ((long long)1 << 40))
                die(c, "Tensor <%s> exceeds its storage in <%s>", t->name,
                    c->path);
            last += (long long)(t->shape[d] - 1) * t->stride[d];
        }
        if (t->storage_offset < 0 ||
            (unsigned long long)(last + 1) * elem_bytes(t->dtype) >
                t->storage_bytes)
            die(c, "Tensor <%s> exceeds its storage in <%s>", t->name,
                c->path);
    }
}

void pth_open(struct pth_file *pf, const char *path)
{
    struct ctx c;
    struct zdir z = {0, NULL};
    struct vm m;
    const struct zent *pkl = NULL;
    const struct val *sd;
    struct stat st;
    void *map;
    long k;
    int fd;

    memset(pf, 0, sizeof(*pf));
    memset(&m, 0, sizeof(m));
    fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0 || fstat(fd, &st) != 0 || !S_ISREG(st.st_mode)) {
        if (fd >= 0)
            close(fd);
        hipb_fatal("Unable to open checkpoint <%s>", path);
        return;
    }
    map = st.st_size > 0 ? mmap(NULL, (size_t)st.st_size, PROT_READ,
                                MAP_PRIVATE, fd, 0)
                         : MAP_FAILED;
    close(fd);
    if (st.st_size > 0 && map == MAP_FAILED) {
        hipb_fatal("Unable to open checkpoint <%s>", path);
        return;
    }
    pf->map = map == MAP_FAILED ? NULL : map;
    pf->map_bytes = (size_t)st.st_size;
    pf->path = strdup(path);
    c.path = pf->path;
    c.base = pf->map;
    c.size = pf->map_bytes;
    m.c = &c;

    if (setjmp(c.jb)) {
        free(z.e);
        vm_free(&m);
        pth_close(pf);
        hipb_fatal("%s", c.msg);
        return;
    }
    zip_dir(&c, &z);
    /* data.pkl sits in a folder named after the saved file. */
    for (k = 0; k < z.n && !pkl; k++) {
        const struct zent *e = &z.e[k];

        if (e->nlen >= 8 && !memcmp(e->name + e->nlen - 8, "data.pkl", 8) &&
            (e->nlen == 8 || e->name[e->nlen - 9] == '/'))
            pkl = e;
    }
    if (!pkl)
        die(&c, "No data.pkl in <%s>: not a PyTorch checkpoint", path);
    m.p = c.base + zip_data(&c, pkl);
    m.end = m.p + pkl->size;
    sd = state_dict(run(&m));
    if (!sd)
        die(&c, "No state_dict of tensors found in <%s>", path);
    index_tensors(&c, pf, &z, sd, pkl->name, (size_t)pkl->nlen - 8);
    free(z.e);
    vm_free(&m);
}

/* ------------------------------------------------------------ lookup */

const struct pth_tensor *pth_find(const struct pth_file *pf, const char *name)
{
    int i;

    for (i = 0; i < pf->ntensors; i++)
        if (!strcmp(pf->tensors[i].name, name))
            return &pf->tensors[i];
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
    int i;

    for (i = 0; i < pf->ntensors; i++)
        if (!strncmp(pf->tensors[i].name, prefix, len))
            sum += (double)pth_numel(&pf->tensors[i]) *
                   (double)elem_bytes(pf->tensors[i].dtype);
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
        return half_bits_to_float((uint16_t)le(p, 2));
    u = (uint32_t)le(p, 2) << 16;
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
    if (pf->map)
        munmap((void *)pf->map, pf->map_bytes);
    drop_tensors(pf);
    free(pf->path);
    memset(pf, 0, sizeof(*pf));
}
