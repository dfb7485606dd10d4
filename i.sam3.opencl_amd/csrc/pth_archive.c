/* SPDX-License-Identifier: Unlicense
 *
 * pth_archive.c - index of the zip archive a PyTorch >= 1.6 checkpoint is
 * (torch.save writes stored members "<folder>/data.pkl" and
 * "<folder>/data/<key>"), over the read-only mapping of the file.
 *
 * Layout facts from PKWARE APPNOTE 6.3: the end of central directory
 * record (4.3.16, signature 0x06054b50, 22 bytes plus a comment of up to
 * 65535) closes the file; when one of its counts, sizes or offsets holds
 * the all-ones sentinel, the zip64 locator (4.3.15, 0x07064b50, 20 bytes)
 * right before it gives the zip64 end record (4.3.14, 0x06064b50) with
 * the 64-bit values. Central directory headers (4.3.12, 0x02014b50, 46
 * bytes + name + extra + comment) carry the method, sizes and local
 * header offset, any sentinel of which is replaced, in the fixed order
 * uncompressed size, compressed size, offset, by the 8-byte fields of the
 * zip64 extended information extra block (4.5.3, tag 0x0001). A member's
 * bytes follow its local header (4.3.7, 0x04034b50, 30 bytes + name +
 * extra; that extra may differ from the central one).
 *
 * Every read goes through span(), which refuses ranges outside the file
 * with overflow-safe arithmetic, so a damaged archive is an error, never
 * a read past the mapping.
 */
#include "pth_internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SIG_EOCD 0x06054b50u
#define SIG_LOC64 0x07064b50u
#define SIG_EOCD64 0x06064b50u
#define SIG_CENTRAL 0x02014b50u
#define SIG_LOCAL 0x04034b50u
#define EOCD_BYTES 22u
#define MAX_COMMENT 65535u

int pth_fail(struct pth_err *e, const char *fmt, ...)
{
    va_list ap;

    if (!e->set) {
        va_start(ap, fmt);
        vsnprintf(e->msg, sizeof(e->msg), fmt, ap);
        va_end(ap);
        e->set = 1;
    }
    return -1;
}

/* Little-endian unsigned field of n bytes. */
static uint64_t field(const unsigned char *p, int n)
{
    uint64_t v = 0;

    while (n-- > 0)
        v = v << 8 | p[n];
    return v;
}

/* p = base + off when [off, off + len) lies inside the file. */
static const unsigned char *span(const struct pth_archive *a, uint64_t off,
                                 uint64_t len)
{
    uint64_t end;

    if (__builtin_add_overflow(off, len, &end) || end > a->bytes)
        return NULL;
    return a->base + off;
}

static int truncated(const struct pth_archive *a, struct pth_err *e)
{
    return pth_fail(e, "Truncated zip structure in <%s>", a->path);
}

/* The end of central directory record: the last signature from which a
 * whole record and its stated comment fit before the end of the file. */
static int find_eocd(const struct pth_archive *a, uint64_t *at)
{
    uint64_t lo, pos;

    if (a->bytes < EOCD_BYTES)
        return -1;
    lo = a->bytes > EOCD_BYTES + MAX_COMMENT ? a->bytes - EOCD_BYTES - MAX_COMMENT : 0;
    for (pos = a->bytes - EOCD_BYTES + 1; pos-- > lo;) {
        const unsigned char *r = a->base + pos;

        if (field(r, 4) == SIG_EOCD && pos + EOCD_BYTES + field(r + 20, 2) <= a->bytes) {
            *at = pos;
            return 0;
        }
    }
    return -1;
}

/* Where the central directory lies and how many headers it holds. */
struct directory {
    uint64_t offset, size, entries;
};

static int locate_directory(const struct pth_archive *a, struct directory *dir,
                            struct pth_err *e)
{
    const unsigned char *r, *loc, *r64;
    uint64_t at;

    if (find_eocd(a, &at) != 0)
        return pth_fail(e, "<%s> is not a zip archive (PyTorch >= 1.6 checkpoint "
                           "format expected)", a->path);
    r = a->base + at;
    dir->entries = field(r + 10, 2);
    dir->size = field(r + 12, 4);
    dir->offset = field(r + 16, 4);
    if (dir->entries != 0xffffu && dir->size != 0xffffffffu && dir->offset != 0xffffffffu)
        return 0;
    loc = at >= 20 ? span(a, at - 20, 20) : NULL;
    if (!loc || field(loc, 4) != SIG_LOC64)
        return pth_fail(e, "Corrupt zip64 directory in <%s>", a->path);
    r64 = span(a, field(loc + 8, 8), 56);
    if (!r64 || field(r64, 4) != SIG_EOCD64)
        return pth_fail(e, "Corrupt zip64 end record in <%s>", a->path);
    dir->entries = field(r64 + 32, 8);
    dir->size = field(r64 + 40, 8);
    dir->offset = field(r64 + 48, 8);
    return 0;
}

/* Replace the sentinel fields of a central header by the values of its
 * zip64 extended information block, if it has one. */
static int apply_zip64_extra(const struct pth_archive *a, const unsigned char *x,
                             uint64_t xlen, struct pth_member *m, struct pth_err *e)
{
    uint64_t pos = 0;

    while (pos + 4 <= xlen) {
        const uint64_t tag = field(x + pos, 2), len = field(x + pos + 2, 2);
        const unsigned char *v = x + pos + 4, *vend = v + len;
        uint64_t *slot[3];
        int k, n = 0;

        if (pos + 4 + len > xlen)
            return pth_fail(e, "Corrupt zip central directory in <%s>", a->path);
        if (tag == 1) {
            if (m->size == 0xffffffffu)
                slot[n++] = &m->size;
            if (m->csize == 0xffffffffu)
                slot[n++] = &m->csize;
            if (m->header == 0xffffffffu)
                slot[n++] = &m->header;
            for (k = 0; k < n; k++, v += 8) {
                if (v + 8 > vend)
                    return pth_fail(e, "Corrupt zip central directory in <%s>", a->path);
                *slot[k] = field(v, 8);
            }
            return 0;
        }
        pos += 4 + len;
    }
    return 0;
}

static int by_name(const void *pa, const void *pb)
{
    const struct pth_member *x = pa, *y = pb;
    const uint32_t n = x->name_len < y->name_len ? x->name_len : y->name_len;
    const int c = memcmp(x->name, y->name, n);

    if (c)
        return c;
    return (x->name_len > y->name_len) - (x->name_len < y->name_len);
}

int pth_archive_index(struct pth_archive *a, struct pth_err *e)
{
    struct directory dir = {0, 0, 0};
    uint64_t pos, k;

    a->member = NULL;
    a->count = 0;
    if (locate_directory(a, &dir, e) != 0)
        return -1;
    if (!span(a, dir.offset, dir.size))
        return truncated(a, e);
    /* Each header takes at least 46 bytes of the directory. */
    if (dir.entries > dir.size / 46 + 1)
        return pth_fail(e, "Corrupt zip central directory in <%s>", a->path);
    a->member = calloc(dir.entries ? dir.entries : 1, sizeof(*a->member));
    if (!a->member)
        return pth_fail(e, "Out of memory reading <%s>", a->path);
    pos = dir.offset;
    for (k = 0; k < dir.entries; k++) {
        const unsigned char *h = span(a, pos, 46);
        struct pth_member *m = &a->member[k];
        uint64_t nlen, xlen, clen;

        if (!h || pos + 46 > dir.offset + dir.size || field(h, 4) != SIG_CENTRAL)
            return pth_fail(e, "Corrupt zip central directory in <%s>", a->path);
        nlen = field(h + 28, 2);
        xlen = field(h + 30, 2);
        clen = field(h + 32, 2);
        if (!span(a, pos + 46, nlen + xlen + clen))
            return truncated(a, e);
        m->name = (const char *)h + 46;
        m->name_len = (uint32_t)nlen;
        m->method = (uint16_t)field(h + 10, 2);
        m->csize = field(h + 20, 4);
        m->size = field(h + 24, 4);
        m->header = field(h + 42, 4);
        if (apply_zip64_extra(a, h + 46 + nlen, xlen, m, e) != 0)
            return -1;
        pos += 46 + nlen + xlen + clen;
    }
    a->count = (size_t)dir.entries;
    qsort(a->member, a->count, sizeof(*a->member), by_name);
    return 0;
}

const struct pth_member *pth_archive_lookup(const struct pth_archive *a,
                                            const char *name, size_t len)
{
    struct pth_member key;

    memset(&key, 0, sizeof(key));
    key.name = name;
    key.name_len = (uint32_t)len;
    return a->count ? bsearch(&key, a->member, a->count, sizeof(key), by_name) : NULL;
}

int pth_archive_data(const struct pth_archive *a, const struct pth_member *m,
                     uint64_t *off, struct pth_err *e)
{
    const unsigned char *h = span(a, m->header, 30);
    uint64_t data;

    if (!h || field(h, 4) != SIG_LOCAL)
        return pth_fail(e, "Corrupt local header for <%.*s> in <%s>", (int)m->name_len,
                        m->name, a->path);
    if (m->method != 0 || m->csize != m->size)
        return pth_fail(e, "Zip entry <%.*s> in <%s> is compressed; only stored entries "
                           "(as written by torch.save) are supported",
                        (int)m->name_len, m->name, a->path);
    data = m->header + 30 + field(h + 26, 2) + field(h + 28, 2);
    if (!span(a, data, m->size))
        return truncated(a, e);
    *off = data;
    return 0;
}

void pth_archive_free(struct pth_archive *a)
{
    free(a->member);
    a->member = NULL;
    a->count = 0;
}
