/* SPDX-License-Identifier: Unlicense
 *
 * pth_loader.h - reader of PyTorch checkpoints (torch.save zip format,
 * stored entries) and of the state_dict they hold. A drop-in for the
 * reference's pth_loader.h (pth_loader.h:1-67): the same functions,
 * enum, tensor record and error behaviour (every format problem is fatal
 * with a message naming the file, like G_fatal_error there; with
 * hipb_set_error_mode(HIPB_ERR_RECORD) the message is kept for
 * hipb_last_error() and the call returns NULL / 0 / an empty file).
 *
 * The file is mapped read-only once at pth_open; tensor reads copy or
 * convert straight from the mapping. Arrays returned by pth_read_f32 and
 * pth_read_c64 are malloc'd: release them with free().
 */
#ifndef SAM3_PTH_LOADER_H
#define SAM3_PTH_LOADER_H

#include <stddef.h>
#include <sys/types.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PTH_MAX_DIMS 8 /* pth_loader.h:9 */

/* Storage element types (pth_loader.h:11-12). PTH_C64: complex64, two
 * float32 per element (real, imaginary). */
enum pth_dtype { PTH_F32, PTH_F16, PTH_BF16, PTH_C64 };

/* One tensor of the state_dict: where its storage lies in the file and
 * how the tensor is strided over it (pth_loader.h:17-26). */
struct pth_tensor {
    char *name;
    int ndim;
    long shape[PTH_MAX_DIMS];
    long stride[PTH_MAX_DIMS];
    long storage_offset;  /* in elements */
    enum pth_dtype dtype;
    off_t data_offset;    /* byte offset of the storage in the file */
    size_t storage_bytes; /* byte size of the storage entry */
};

/* An open checkpoint (pth_loader.h:28-33). The reference's FILE *fp is
 * replaced by the read-only mapping of the whole file. */
struct pth_file {
    const unsigned char *map;
    size_t map_bytes;
    char *path;
    int ntensors;
    struct pth_tensor *tensors;
};

/* Open and index a checkpoint (pth_loader.h:35-37): a bare state_dict,
 * or one held under "model" or "state_dict" of the saved dict. */
void pth_open(struct pth_file *pf, const char *path);

/* The tensor called name, or NULL (pth_loader.h:39-40). */
const struct pth_tensor *pth_find(const struct pth_file *pf, const char *name);

/* pth_find, fatal if absent or if its rank differs from ndim or a size
 * from shape[d] >= 0; shape may be NULL (pth_loader.h:42-46). */
const struct pth_tensor *pth_require(const struct pth_file *pf,
                                     const char *name, int ndim,
                                     const long *shape);

long pth_numel(const struct pth_tensor *t); /* pth_loader.h:48 */

/* Storage bytes of the tensors whose names start with prefix
 * (pth_loader.h:50-51). */
double pth_bytes(const struct pth_file *pf, const char *prefix);

/* A real tensor as a new C-order float32 array (pth_loader.h:53-54). */
float *pth_read_f32(const struct pth_file *pf, const struct pth_tensor *t);

/* A complex64 tensor as a new C-order array of 2 numel floats, (real,
 * imaginary) pairs (pth_loader.h:56-58). */
float *pth_read_c64(const struct pth_file *pf, const struct pth_tensor *t);

/* Row r of a C-contiguous float32 matrix into dst (shape[1] floats)
 * (pth_loader.h:60-63). */
void pth_read_row_f32(const struct pth_file *pf, const struct pth_tensor *t,
                      long r, float *dst);

void pth_close(struct pth_file *pf); /* pth_loader.h:65 */

#ifdef __cplusplus
}
#endif

#endif /* SAM3_PTH_LOADER_H */
