/* SPDX-License-Identifier: Unlicense
 *
 * Internal interfaces of the checkpoint reader (pth_loader.h): the zip
 * archive index over the mapped file (pth_archive.c), the pickle machine
 * that finds the state_dict's tensors (pth_unpickle.c), and the error
 * sink they share. Every function here reports a failure by returning -1
 * after writing the message into the sink; the public calls in
 * pth_loader.c turn it into the library's fatal-with-message error.
 */
#ifndef SAM3_PTH_INTERNAL_H
#define SAM3_PTH_INTERNAL_H

#include <stddef.h>
#include <stdint.h>

#include "pth_loader.h"

/* The first failure of one pth_open. */
struct pth_err {
    char msg[768];
    int set;
};

/* Record the message (the first one wins) and return -1. */
int pth_fail(struct pth_err *e, const char *fmt, ...)
    __attribute__((format(printf, 2, 3)));

/* ------------------------------------------------------------ archive */

/* One member of the zip central directory. */
struct pth_member {
    const char *name;  /* into the mapping, not NUL-terminated */
    uint32_t name_len;
    uint16_t method;   /* 0 = stored */
    uint64_t size;     /* uncompressed bytes */
    uint64_t csize;    /* bytes in the archive */
    uint64_t header;   /* offset of the local header */
};

/* The members of a mapped archive, sorted by name. */
struct pth_archive {
    const unsigned char *base;
    uint64_t bytes;
    const char *path;
    struct pth_member *member;
    size_t count;
};

int pth_archive_index(struct pth_archive *a, struct pth_err *e);
const struct pth_member *pth_archive_lookup(const struct pth_archive *a,
                                            const char *name, size_t len);
/* File offset of a stored member's bytes (all of them inside the file). */
int pth_archive_data(const struct pth_archive *a, const struct pth_member *m,
                     uint64_t *off, struct pth_err *e);
void pth_archive_free(struct pth_archive *a);

/* ------------------------------------------------------------ pickle */

/* A (name, tensor) entry of the state_dict as the pickle describes it:
 * the storage is named by its archive key, the view by offset, shape and
 * strides in elements. */
struct pth_entry {
    char *name;
    char *key;
    enum pth_dtype dtype;
    int ndim;
    int64_t offset;
    int64_t shape[PTH_MAX_DIMS];
    int64_t stride[PTH_MAX_DIMS];
};

/* Run the pickle [p, p + n) of the checkpoint `path` and return its
 * state_dict's tensors in dict order (a bare dict of tensors, or the one
 * under "model" or "state_dict"). */
int pth_unpickle(const unsigned char *p, size_t n, const char *path,
                 struct pth_entry **out, int *count, struct pth_err *e);
void pth_entries_free(struct pth_entry *v, int count);

#endif /* SAM3_PTH_INTERNAL_H */
