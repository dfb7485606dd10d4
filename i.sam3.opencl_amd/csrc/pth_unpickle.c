/* SPDX-License-Identifier: Unlicense
 *
 * pth_unpickle.c - the pickle machine of the checkpoint reader: runs a
 * checkpoint's data.pkl far enough to know which tensors its state_dict
 * holds and how each one views which storage.
 *
 * Format facts (CPython Lib/pickle.py and pickletools.py for the opcodes
 * of protocols 2-5; torch/serialization.py and torch/_utils.py for what
 * torch.save pickles): a tensor is REDUCE(torch._utils._rebuild_tensor_v2,
 * (storage, offset, size, stride, requires_grad, hooks[, metadata])), a
 * Parameter REDUCE(torch._utils._rebuild_parameter[_with_state], (tensor,
 * ...)), and a storage the persistent id ("storage", torch.<Type>Storage,
 * key, location, numel) resolved by BINPERSID.
 *
 * Design. Objects live in one pool and are named by 32-bit indices
 * (index 0 is never an object, so 0 marks an unset memo slot). A
 * container keeps its items as a chain of link cells, so the same object
 * can sit in several containers, as memo references make it do. Texts go
 * to one arena. A global is resolved to its role (tensor rebuild,
 * parameter rebuild, OrderedDict, storage type, anything else) when
 * GLOBAL / STACK_GLOBAL runs, and REDUCE applies the role. Opcodes
 * dispatch through a table of handlers; an opcode without one is an
 * error. Everything this reader cannot use (floats, bytes, objects of
 * other classes, sets) is kept only as an opaque placeholder.
 */
#include "pth_internal.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

enum kind {
    K_NONE, K_BOOL, K_INT, K_FLOAT, K_STR, K_BYTES, K_TUPLE, K_LIST, K_DICT,
    K_SET, K_GLOBAL, K_STORAGE, K_TENSOR, K_OPAQUE
};

/* What a global stands for. */
enum role { R_OTHER, R_TENSOR, R_PARAMETER, R_ORDERED_DICT, R_STORAGE_TYPE };

struct obj {
    uint8_t kind;
    uint8_t role;     /* K_GLOBAL */
    uint8_t dtype;    /* K_GLOBAL storage type, K_STORAGE */
    uint8_t usable;   /* K_GLOBAL storage type: a dtype this reader reads */
    uint32_t a, b;    /* K_STR / K_BYTES: text, length; K_GLOBAL: module,
                         name texts; K_STORAGE: key text; K_TENSOR: view */
    int64_t i;        /* K_INT, K_BOOL */
    uint32_t head, tail, count; /* containers: link chain */
};

struct link {
    uint32_t obj, next;
};

struct view {
    uint32_t storage;
    int ndim;
    int64_t offset;
    int64_t shape[PTH_MAX_DIMS], stride[PTH_MAX_DIMS];
};

struct machine {
    const unsigned char *p, *end;
    const char *path;
    struct pth_err *e;
    struct obj *obj;
    uint32_t nobj, cobj;
    struct link *link;
    uint32_t nlink, clink;
    char *text;
    uint32_t ntext, ctext;
    struct view *view;
    uint32_t nview, cview;
    uint32_t *stack;
    uint32_t sp, cstack;
    uint32_t *mark;
    uint32_t nmark, cmark;
    uint32_t *memo;
    uint32_t cmemo, memo_used;
    uint32_t result;
    int stopped;
};

/* Largest memo index accepted: far more objects than any checkpoint's
 * pickle holds, small enough that the slot table stays modest. */
#define MEMO_LIMIT (1u << 24)
#define ITEM_LIMIT 0x7fffffffu

typedef int (*op_fn)(struct machine *m, unsigned char op);

/* ------------------------------------------------------------ storage */

static int oom(struct machine *m)
{
    return pth_fail(m->e, "Out of memory reading <%s>", m->path);
}

/* Make room for `need` elements of `size` bytes in *arr (capacity *cap). */
static int reserve(struct machine *m, void **arr, uint32_t *cap, uint64_t need,
                   size_t size)
{
    uint64_t n = *cap ? *cap : 64;
    void *p;

    if (need <= *cap)
        return 0;
    if (need > ITEM_LIMIT)
        return oom(m);
    while (n < need)
        n *= 2;
    if (n > ITEM_LIMIT)
        n = ITEM_LIMIT;
    p = realloc(*arr, n * size);
    if (!p)
        return oom(m);
    *arr = p;
    *cap = (uint32_t)n;
    return 0;
}

#define RESERVE(m, arr, cap, need) \
    reserve(m, (void **)&(arr), &(cap), (need), sizeof(*(arr)))

/* New object of `kind`; 0 on failure (object 0 is the reserved null). */
static uint32_t new_obj(struct machine *m, enum kind kind)
{
    struct obj *o;

    if (RESERVE(m, m->obj, m->cobj, (uint64_t)m->nobj + 1) != 0)
        return 0;
    o = &m->obj[m->nobj];
    memset(o, 0, sizeof(*o));
    o->kind = (uint8_t)kind;
    return m->nobj++;
}

/* Copy n bytes into the text arena (NUL-terminated); returns the offset
 * or -1. */
static int64_t add_text(struct machine *m, const void *s, size_t n)
{
    uint32_t at;

    if (n >= ITEM_LIMIT || RESERVE(m, m->text, m->ctext, (uint64_t)m->ntext + n + 1) != 0)
        return -1;
    at = m->ntext;
    memcpy(m->text + at, s, n);
    m->text[at + n] = 0;
    m->ntext += (uint32_t)n + 1;
    return at;
}

static const char *text_of(const struct machine *m, uint32_t at)
{
    return m->text + at;
}

/* Append item to container c. */
static int chain(struct machine *m, uint32_t c, uint32_t item)
{
    struct obj *o;
    uint32_t l;

    if (RESERVE(m, m->link, m->clink, (uint64_t)m->nlink + 1) != 0)
        return -1;
    l = m->nlink++;
    m->link[l].obj = item;
    m->link[l].next = 0;
    o = &m->obj[c];
    if (o->count)
        m->link[o->tail].next = l;
    else
        o->head = l;
    o->tail = l;
    o->count++;
    return 0;
}

/* Item k of container c (k < count). */
static uint32_t item(const struct machine *m, uint32_t c, uint32_t k)
{
    uint32_t l = m->obj[c].head;

    while (k--)
        l = m->link[l].next;
    return m->link[l].obj;
}

static int is_str(const struct machine *m, uint32_t o, const char *s)
{
    return m->obj[o].kind == K_STR && !strcmp(text_of(m, m->obj[o].a), s);
}

/* Dict insert with Python's semantics: a string key already present
 * keeps its place and takes the new value. */
static int dict_set(struct machine *m, uint32_t d, uint32_t key, uint32_t val)
{
    if (m->obj[key].kind == K_STR) {
        uint32_t l = m->obj[d].head, k;

        for (k = 0; k < m->obj[d].count; k += 2, l = m->link[m->link[l].next].next)
            if (is_str(m, m->link[l].obj, text_of(m, m->obj[key].a))) {
                m->link[m->link[l].next].obj = val;
                return 0;
            }
    }
    if (chain(m, d, key) != 0 || chain(m, d, val) != 0)
        return -1;
    return 0;
}

/* ------------------------------------------------------------ stack */

static int push(struct machine *m, uint32_t o)
{
    if (!o || RESERVE(m, m->stack, m->cstack, (uint64_t)m->sp + 1) != 0)
        return -1;
    m->stack[m->sp++] = o;
    return 0;
}

static int underflow(struct machine *m)
{
    return pth_fail(m->e, "Pickle stack underflow in checkpoint <%s>", m->path);
}

/* Pop into *o; the items above the innermost mark are the only ones
 * reachable. */
static int pop(struct machine *m, uint32_t *o)
{
    if (m->sp == 0 || (m->nmark && m->sp <= m->mark[m->nmark - 1]))
        return underflow(m);
    *o = m->stack[--m->sp];
    return 0;
}

static int peek(struct machine *m, uint32_t *o)
{
    if (m->sp == 0 || (m->nmark && m->sp <= m->mark[m->nmark - 1]))
        return underflow(m);
    *o = m->stack[m->sp - 1];
    return 0;
}

/* Remove the innermost mark; *from = the stack depth it recorded. */
static int unmark(struct machine *m, uint32_t *from)
{
    if (!m->nmark)
        return pth_fail(m->e, "Pickle mark not found in checkpoint <%s>", m->path);
    *from = m->mark[--m->nmark];
    return 0;
}

/* New container of `kind` holding stack items [from, sp), popped. */
static uint32_t collect(struct machine *m, enum kind kind, uint32_t from)
{
    const uint32_t c = new_obj(m, kind);
    uint32_t k;

    if (!c)
        return 0;
    for (k = from; k < m->sp; k++)
        if (chain(m, c, m->stack[k]) != 0)
            return 0;
    m->sp = from;
    return c;
}

/* Bytes of the opcode's argument. */
static int take(struct machine *m, uint64_t n, const unsigned char **q)
{
    if ((uint64_t)(m->end - m->p) < n)
        return pth_fail(m->e, "Truncated pickle in checkpoint <%s>", m->path);
    *q = m->p;
    m->p += n;
    return 0;
}

static uint64_t le_field(const unsigned char *q, int n)
{
    uint64_t v = 0;

    while (n-- > 0)
        v = v << 8 | q[n];
    return v;
}

/* A newline-terminated argument line (GLOBAL). */
static int take_line(struct machine *m, int64_t *at)
{
    const unsigned char *nl = memchr(m->p, '\n', (size_t)(m->end - m->p));

    if (!nl)
        return pth_fail(m->e, "Truncated pickle in checkpoint <%s>", m->path);
    *at = add_text(m, m->p, (size_t)(nl - m->p));
    m->p = nl + 1;
    return *at < 0 ? -1 : 0;
}

/* ------------------------------------------------------------ globals */

static const struct {
    const char *module, *name;
    enum role role;
} ROLES[] = {
    {"torch._utils", "_rebuild_tensor", R_TENSOR},
    {"torch._utils", "_rebuild_tensor_v2", R_TENSOR},
    {"torch._utils", "_rebuild_parameter", R_PARAMETER},
    {"torch._utils", "_rebuild_parameter_with_state", R_PARAMETER},
    {"collections", "OrderedDict", R_ORDERED_DICT},
};

static const struct {
    const char *name;
    enum pth_dtype dtype;
} STORAGES[] = {
    {"FloatStorage", PTH_F32},
    {"HalfStorage", PTH_F16},
    {"BFloat16Storage", PTH_BF16},
    {"ComplexFloatStorage", PTH_C64},
};

/* The global module.name as an object with its role. */
static uint32_t make_global(struct machine *m, uint32_t module, uint32_t name)
{
    const char *mod = text_of(m, module), *nm = text_of(m, name);
    const size_t len = strlen(nm);
    const uint32_t g = new_obj(m, K_GLOBAL);
    struct obj *o;
    size_t k;

    if (!g)
        return 0;
    o = &m->obj[g];
    o->a = module;
    o->b = name;
    o->role = R_OTHER;
    for (k = 0; k < sizeof(ROLES) / sizeof(ROLES[0]); k++)
        if (!strcmp(ROLES[k].module, mod) && !strcmp(ROLES[k].name, nm))
            o->role = (uint8_t)ROLES[k].role;
    if (!strcmp(mod, "torch") && len > 7 && !strcmp(nm + len - 7, "Storage")) {
        o->role = R_STORAGE_TYPE;
        for (k = 0; k < sizeof(STORAGES) / sizeof(STORAGES[0]); k++)
            if (!strcmp(STORAGES[k].name, nm)) {
                o->dtype = (uint8_t)STORAGES[k].dtype;
                o->usable = 1;
            }
    }
    return g;
}

/* ------------------------------------------------------------ values */

static int want_int(struct machine *m, uint32_t o, int64_t *v)
{
    if (m->obj[o].kind != K_INT && m->obj[o].kind != K_BOOL)
        return pth_fail(m->e, "Integer expected in checkpoint pickle <%s>", m->path);
    *v = m->obj[o].i;
    return 0;
}

/* REDUCE of a tensor rebuild: (storage, offset, size, stride, ...). */
static uint32_t rebuild_tensor(struct machine *m, uint32_t args)
{
    uint32_t st, size, stride, t;
    struct view *v;
    int d, n;

    if (m->obj[args].count < 4)
        goto bad;
    st = item(m, args, 0);
    size = item(m, args, 2);
    stride = item(m, args, 3);
    if (m->obj[st].kind != K_STORAGE || m->obj[size].kind != K_TUPLE ||
        m->obj[stride].kind != K_TUPLE || m->obj[size].count != m->obj[stride].count)
        goto bad;
    n = (int)m->obj[size].count;
    if (n > PTH_MAX_DIMS) {
        pth_fail(m->e, "Unsupported tensor rank %d in <%s>", n, m->path);
        return 0;
    }
    if (RESERVE(m, m->view, m->cview, (uint64_t)m->nview + 1) != 0)
        return 0;
    v = &m->view[m->nview];
    v->storage = st;
    v->ndim = n;
    if (want_int(m, item(m, args, 1), &v->offset) != 0)
        return 0;
    for (d = 0; d < n; d++)
        if (want_int(m, item(m, size, (uint32_t)d), &v->shape[d]) != 0 ||
            want_int(m, item(m, stride, (uint32_t)d), &v->stride[d]) != 0)
            return 0;
    t = new_obj(m, K_TENSOR);
    if (t)
        m->obj[t].a = m->nview++;
    return t;
bad:
    pth_fail(m->e, "Unexpected tensor rebuild arguments in <%s>", m->path);
    return 0;
}

/* REDUCE of a parameter rebuild: the parameter is its tensor. */
static uint32_t rebuild_parameter(struct machine *m, uint32_t args)
{
    uint32_t t;

    if (m->obj[args].count < 1 || m->obj[t = item(m, args, 0)].kind != K_TENSOR) {
        pth_fail(m->e, "Unexpected parameter rebuild arguments in <%s>", m->path);
        return 0;
    }
    return t;
}

/* ("storage", torch.<Type>Storage, key, location, numel) -> storage. */
static uint32_t load_persistent(struct machine *m, uint32_t pid)
{
    uint32_t type, key, s;
    const struct obj *g;
    int64_t at;
    char num[32];

    if (m->obj[pid].kind != K_TUPLE || m->obj[pid].count != 5 ||
        !is_str(m, item(m, pid, 0), "storage"))
        goto bad;
    type = item(m, pid, 1);
    key = item(m, pid, 2);
    g = &m->obj[type];
    if (g->kind != K_GLOBAL || g->role != R_STORAGE_TYPE)
        goto bad;
    if (!g->usable) {
        pth_fail(m->e, "Unsupported tensor storage type <%s.%s> in checkpoint "
                       "(float32, float16, bfloat16 and complex64 are supported)",
                 text_of(m, g->a), text_of(m, g->b));
        return 0;
    }
    if (m->obj[key].kind == K_STR)
        at = m->obj[key].a;
    else if (m->obj[key].kind == K_INT) {
        snprintf(num, sizeof(num), "%lld", (long long)m->obj[key].i);
        at = add_text(m, num, strlen(num));
    }
    else
        goto bad;
    if (at < 0 || !(s = new_obj(m, K_STORAGE)))
        return 0;
    m->obj[s].a = (uint32_t)at;
    m->obj[s].dtype = m->obj[type].dtype;
    return s;
bad:
    pth_fail(m->e, "Unsupported persistent id in checkpoint <%s>", m->path);
    return 0;
}

/* ------------------------------------------------------------ opcodes */

static int op_proto(struct machine *m, unsigned char op)
{
    const unsigned char *q = NULL;

    return take(m, 1, &q);
}

static int op_frame(struct machine *m, unsigned char op)
{
    const unsigned char *q = NULL;

    return take(m, 8, &q); /* framing only groups opcodes */
}

static int op_stop(struct machine *m, unsigned char op)
{
    if (pop(m, &m->result) != 0)
        return -1;
    m->stopped = 1;
    return 0;
}

static int op_mark(struct machine *m, unsigned char op)
{
    if (RESERVE(m, m->mark, m->cmark, (uint64_t)m->nmark + 1) != 0)
        return -1;
    m->mark[m->nmark++] = m->sp;
    return 0;
}

static int op_pop(struct machine *m, unsigned char op)
{
    uint32_t o = 0, from = 0;

    if (m->nmark && m->sp == m->mark[m->nmark - 1])
        return unmark(m, &from); /* POP of a bare mark drops the mark */
    return pop(m, &o);
}

static int op_pop_mark(struct machine *m, unsigned char op)
{
    uint32_t from = 0;

    if (unmark(m, &from) != 0)
        return -1;
    m->sp = from;
    return 0;
}

static int op_dup(struct machine *m, unsigned char op)
{
    uint32_t o = 0;

    return peek(m, &o) != 0 ? -1 : push(m, o);
}

static int op_empty(struct machine *m, unsigned char op)
{
    const enum kind kind = op == '}' ? K_DICT : op == ']' ? K_LIST : op == ')' ? K_TUPLE : K_SET;

    return push(m, new_obj(m, kind));
}

static int op_const(struct machine *m, unsigned char op)
{
    const uint32_t o = new_obj(m, op == 'N' ? K_NONE : K_BOOL);

    if (o)
        m->obj[o].i = op == 0x88;
    return push(m, o);
}

/* BININT (signed 32-bit), BININT1 (unsigned 8-bit), BININT2 (unsigned
 * 16-bit). */
static int op_int(struct machine *m, unsigned char op)
{
    const int n = op == 'J' ? 4 : op == 'K' ? 1 : 2;
    const unsigned char *q = NULL;
    uint32_t o = 0;

    if (take(m, (uint64_t)n, &q) != 0 || !(o = new_obj(m, K_INT)))
        return -1;
    m->obj[o].i = n == 4 ? (int64_t)(int32_t)le_field(q, 4) : (int64_t)le_field(q, n);
    return push(m, o);
}

/* LONG1 / LONG4: little-endian two's complement of a stated length. */
static int op_long(struct machine *m, unsigned char op)
{
    const unsigned char *q = NULL;
    uint64_t n, v;
    uint32_t o = 0;

    if (take(m, op == 0x8a ? 1 : 4, &q) != 0)
        return -1;
    n = le_field(q, op == 0x8a ? 1 : 4);
    if (n > 8)
        return pth_fail(m->e, "Integer too large in checkpoint pickle <%s>", m->path);
    if (take(m, n, &q) != 0 || !(o = new_obj(m, K_INT)))
        return -1;
    v = le_field(q, (int)n);
    if (n && n < 8 && (q[n - 1] & 0x80))
        v |= ~(uint64_t)0 << (8 * n);
    m->obj[o].i = (int64_t)v;
    return push(m, o);
}

static int op_float(struct machine *m, unsigned char op)
{
    const unsigned char *q = NULL;

    return take(m, 8, &q) != 0 ? -1 : push(m, new_obj(m, K_FLOAT));
}

/* Length-prefixed text or bytes: the prefix width and the kind by
 * opcode. */
static int op_text(struct machine *m, unsigned char op)
{
    int width;
    enum kind kind = K_STR;
    const unsigned char *q = NULL;
    uint64_t n;
    int64_t at;
    uint32_t o = 0;

    switch (op) {
    case 'X': case 'T': width = 4; break;
    case 0x8c: case 'U': width = 1; break;
    case 0x8d: width = 8; break;
    case 'B': width = 4; kind = K_BYTES; break;
    case 'C': width = 1; kind = K_BYTES; break;
    default: width = 8; kind = K_BYTES; break; /* BINBYTES8 */
    }
    if (take(m, (uint64_t)width, &q) != 0)
        return -1;
    n = le_field(q, width);
    if (take(m, n, &q) != 0)
        return -1;
    if (kind == K_BYTES)
        return push(m, new_obj(m, K_BYTES));
    if ((at = add_text(m, q, (size_t)n)) < 0 || !(o = new_obj(m, K_STR)))
        return -1;
    m->obj[o].a = (uint32_t)at;
    m->obj[o].b = (uint32_t)n;
    return push(m, o);
}

static int op_global(struct machine *m, unsigned char op)
{
    int64_t mod = 0, name = 0;

    if (take_line(m, &mod) != 0 || take_line(m, &name) != 0)
        return -1;
    return push(m, make_global(m, (uint32_t)mod, (uint32_t)name));
}

static int op_stack_global(struct machine *m, unsigned char op)
{
    uint32_t mod = 0, name = 0;

    if (pop(m, &name) != 0 || pop(m, &mod) != 0)
        return -1;
    if (m->obj[mod].kind != K_STR || m->obj[name].kind != K_STR)
        return pth_fail(m->e, "Invalid STACK_GLOBAL in checkpoint <%s>", m->path);
    return push(m, make_global(m, m->obj[mod].a, m->obj[name].a));
}

static int memo_store(struct machine *m, uint64_t idx)
{
    uint32_t o = 0;

    if (idx >= MEMO_LIMIT)
        return pth_fail(m->e, "Invalid pickle memo index in <%s>", m->path);
    if (peek(m, &o) != 0)
        return -1;
    if (idx >= m->cmemo) {
        const uint32_t old = m->cmemo;

        if (RESERVE(m, m->memo, m->cmemo, idx + 1) != 0)
            return -1;
        memset(m->memo + old, 0, (size_t)(m->cmemo - old) * sizeof(*m->memo));
    }
    m->memo_used += !m->memo[idx];
    m->memo[idx] = o;
    return 0;
}

/* BINPUT (8-bit index), LONG_BINPUT (32-bit), MEMOIZE (the next index:
 * the number of entries so far). */
static int op_put(struct machine *m, unsigned char op)
{
    const unsigned char *q = NULL;

    if (op == 0x94)
        return memo_store(m, m->memo_used);
    if (take(m, op == 'q' ? 1 : 4, &q) != 0)
        return -1;
    return memo_store(m, le_field(q, op == 'q' ? 1 : 4));
}

static int op_get(struct machine *m, unsigned char op)
{
    const unsigned char *q = NULL;
    uint64_t idx;

    if (take(m, op == 'h' ? 1 : 4, &q) != 0)
        return -1;
    idx = le_field(q, op == 'h' ? 1 : 4);
    if (idx >= m->cmemo || !m->memo[idx])
        return pth_fail(m->e, "Invalid pickle memo reference %llu in <%s>",
                        (unsigned long long)idx, m->path);
    return push(m, m->memo[idx]);
}

/* TUPLE (items above the mark), TUPLE1..3 (the top one to three). */
static int op_tuple(struct machine *m, unsigned char op)
{
    uint32_t from = 0;

    if (op == 't') {
        if (unmark(m, &from) != 0)
            return -1;
    }
    else {
        const uint32_t n = op - 0x84u;
        const uint32_t floor = m->nmark ? m->mark[m->nmark - 1] : 0;

        if (m->sp < floor + n)
            return underflow(m);
        from = m->sp - n;
    }
    return push(m, collect(m, K_TUPLE, from));
}

static int op_persid(struct machine *m, unsigned char op)
{
    uint32_t pid = 0;

    return pop(m, &pid) != 0 ? -1 : push(m, load_persistent(m, pid));
}

static int op_reduce(struct machine *m, unsigned char op)
{
    uint32_t fn = 0, args = 0, out;

    if (pop(m, &args) != 0 || pop(m, &fn) != 0)
        return -1;
    if (m->obj[args].kind != K_TUPLE)
        return pth_fail(m->e, "Pickle REDUCE without argument tuple in <%s>", m->path);
    switch (m->obj[fn].kind == K_GLOBAL ? m->obj[fn].role : R_OTHER) {
    case R_TENSOR: out = rebuild_tensor(m, args); break;
    case R_PARAMETER: out = rebuild_parameter(m, args); break;
    case R_ORDERED_DICT: out = new_obj(m, K_DICT); break;
    default: out = new_obj(m, K_OPAQUE); break;
    }
    return push(m, out);
}

/* NEWOBJ (cls, args) and NEWOBJ_EX (cls, args, kwargs): an instance of a
 * class this reader does not model. */
static int op_newobj(struct machine *m, unsigned char op)
{
    uint32_t x = 0;
    int k;

    for (k = 0; k < (op == 0x92 ? 3 : 2); k++)
        if (pop(m, &x) != 0)
            return -1;
    return push(m, new_obj(m, K_OPAQUE));
}

/* BUILD: the state of the object below (an OrderedDict's _metadata, a
 * Parameter's attributes) plays no part in a state_dict. */
static int op_build(struct machine *m, unsigned char op)
{
    uint32_t state = 0, o = 0;

    return pop(m, &state) != 0 ? -1 : peek(m, &o);
}

/* Items [from, sp) into the container below them. */
static int fill(struct machine *m, uint32_t from, const char *what, enum kind want,
                int pairs)
{
    uint32_t target, k;
    enum kind kind;

    if (from == 0 || (m->nmark && from <= m->mark[m->nmark - 1]))
        return underflow(m);
    target = m->stack[from - 1];
    kind = (enum kind)m->obj[target].kind;
    if ((kind != want && kind != K_OPAQUE) || (pairs && (m->sp - from) % 2))
        return pth_fail(m->e, "Invalid %s in checkpoint pickle <%s>", what, m->path);
    if (kind == want && want != K_SET)
        for (k = from; k < m->sp; k += pairs ? 2 : 1)
            if ((pairs ? dict_set(m, target, m->stack[k], m->stack[k + 1])
                       : chain(m, target, m->stack[k])) != 0)
                return -1;
    m->sp = from;
    return 0;
}

static int op_fill(struct machine *m, unsigned char op)
{
    uint32_t from = 0;

    switch (op) {
    case 's': /* SETITEM */
        return m->sp < 2 ? underflow(m) : fill(m, m->sp - 2, "SETITEM", K_DICT, 1);
    case 'a': /* APPEND */
        return m->sp < 1 ? underflow(m) : fill(m, m->sp - 1, "APPEND", K_LIST, 0);
    default:
        break;
    }
    if (unmark(m, &from) != 0)
        return -1;
    switch (op) {
    case 'u': return fill(m, from, "SETITEMS", K_DICT, 1);
    case 'e': return fill(m, from, "APPENDS", K_LIST, 0);
    default: return fill(m, from, "ADDITEMS", K_SET, 0);
    }
}

static int op_frozenset(struct machine *m, unsigned char op)
{
    uint32_t from = 0;

    if (unmark(m, &from) != 0)
        return -1;
    m->sp = from;
    return push(m, new_obj(m, K_SET));
}

static const op_fn OPS[256] = {
    [0x80] = op_proto, [0x95] = op_frame, ['.'] = op_stop,
    ['('] = op_mark, ['0'] = op_pop, ['1'] = op_pop_mark, ['2'] = op_dup,
    ['}'] = op_empty, [']'] = op_empty, [')'] = op_empty, [0x8f] = op_empty,
    ['N'] = op_const, [0x88] = op_const, [0x89] = op_const,
    ['J'] = op_int, ['K'] = op_int, ['M'] = op_int,
    [0x8a] = op_long, [0x8b] = op_long, ['G'] = op_float,
    ['X'] = op_text, ['T'] = op_text, [0x8c] = op_text, ['U'] = op_text,
    [0x8d] = op_text, ['B'] = op_text, ['C'] = op_text, [0x8e] = op_text,
    ['c'] = op_global, [0x93] = op_stack_global,
    ['q'] = op_put, ['r'] = op_put, [0x94] = op_put,
    ['h'] = op_get, ['j'] = op_get,
    ['t'] = op_tuple, [0x85] = op_tuple, [0x86] = op_tuple, [0x87] = op_tuple,
    ['Q'] = op_persid, ['R'] = op_reduce, [0x81] = op_newobj, [0x92] = op_newobj,
    ['b'] = op_build,
    ['s'] = op_fill, ['u'] = op_fill, ['a'] = op_fill, ['e'] = op_fill,
    [0x90] = op_fill, [0x91] = op_frozenset,
};

/* ------------------------------------------------------------ state */

static uint32_t tensors_in(const struct machine *m, uint32_t d)
{
    uint32_t n = 0, l = m->obj[d].head, k;

    for (k = 0; k + 1 < m->obj[d].count; k += 2, l = m->link[m->link[l].next].next)
        n += m->obj[m->link[m->link[l].next].obj].kind == K_TENSOR;
    return n;
}

/* Value of the string key `key` in dict d, or 0. */
static uint32_t dict_get(const struct machine *m, uint32_t d, const char *key)
{
    uint32_t l = m->obj[d].head, k;

    for (k = 0; k + 1 < m->obj[d].count; k += 2, l = m->link[m->link[l].next].next)
        if (is_str(m, m->link[l].obj, key))
            return m->link[m->link[l].next].obj;
    return 0;
}

/* The dict of tensors: the root itself, else its "model" or
 * "state_dict" entry (how training checkpoints wrap their weights). */
static uint32_t state_dict(const struct machine *m)
{
    static const char *const wraps[] = {"model", "state_dict"};
    const uint32_t root = m->result;
    size_t k;

    if (m->obj[root].kind != K_DICT)
        return 0;
    if (tensors_in(m, root))
        return root;
    for (k = 0; k < sizeof(wraps) / sizeof(wraps[0]); k++) {
        const uint32_t d = dict_get(m, root, wraps[k]);

        if (d && m->obj[d].kind == K_DICT && tensors_in(m, d))
            return d;
    }
    return 0;
}

static int export_entries(struct machine *m, uint32_t d, struct pth_entry **out,
                          int *count)
{
    const uint32_t n = tensors_in(m, d);
    struct pth_entry *v = calloc(n ? n : 1, sizeof(*v));
    uint32_t l = m->obj[d].head, k;
    int used = 0;

    if (!v)
        return oom(m);
    for (k = 0; k + 1 < m->obj[d].count; k += 2, l = m->link[m->link[l].next].next) {
        const struct obj *key = &m->obj[m->link[l].obj];
        const struct obj *t = &m->obj[m->link[m->link[l].next].obj];
        const struct view *w;
        struct pth_entry *x;

        if (t->kind != K_TENSOR || key->kind != K_STR)
            continue;
        w = &m->view[t->a];
        x = &v[used++];
        x->name = strdup(text_of(m, key->a));
        x->key = strdup(text_of(m, m->obj[w->storage].a));
        if (!x->name || !x->key) {
            pth_entries_free(v, used);
            return oom(m);
        }
        x->dtype = (enum pth_dtype)m->obj[w->storage].dtype;
        x->ndim = w->ndim;
        x->offset = w->offset;
        memcpy(x->shape, w->shape, sizeof(x->shape));
        memcpy(x->stride, w->stride, sizeof(x->stride));
    }
    *out = v;
    *count = used;
    return 0;
}

static void release(struct machine *m)
{
    free(m->obj);
    free(m->link);
    free(m->text);
    free(m->view);
    free(m->stack);
    free(m->mark);
    free(m->memo);
}

int pth_unpickle(const unsigned char *p, size_t n, const char *path,
                 struct pth_entry **out, int *count, struct pth_err *e)
{
    struct machine m;
    uint32_t sd;
    int rc = -1;

    memset(&m, 0, sizeof(m));
    m.p = p;
    m.end = p + n;
    m.path = path;
    m.e = e;
    *out = NULL;
    *count = 0;
    /* Object 0 and link cell 0 are never used: index 0 is "none" (an
     * unset memo slot, the end of a chain). */
    if (new_obj(&m, K_NONE) != 0 || RESERVE(&m, m.link, m.clink, 1) != 0)
        goto done;
    m.nlink = 1;
    while (!m.stopped) {
        const unsigned char *q = NULL;
        op_fn fn;

        if (take(&m, 1, &q) != 0)
            goto done;
        fn = OPS[*q];
        if (!fn) {
            pth_fail(e, "Unsupported pickle opcode 0x%02x in checkpoint <%s>", *q, path);
            goto done;
        }
        if (fn(&m, *q) != 0) {
            if (!e->set) /* every handler records its failure; defensive */
                oom(&m);
            goto done;
        }
    }
    sd = state_dict(&m);
    if (!sd) {
        pth_fail(e, "No state_dict of tensors found in <%s>", path);
        goto done;
    }
    rc = export_entries(&m, sd, out, count);
done:
    release(&m);
    return rc;
}

void pth_entries_free(struct pth_entry *v, int count)
{
    int k;

    for (k = 0; k < count; k++) {
        free(v[k].name);
        free(v[k].key);
    }
    free(v);
}
