/* SPDX-License-Identifier: Unlicense
 *
 * Internal helpers shared by hip_backend.c and sam3_ops.c.
 */
#ifndef HIPB_INTERNAL_H
#define HIPB_INTERNAL_H

#include "sam3_hip.h"

/* Fatal error: prints and exits in HIPB_ERR_FATAL mode (the reference's
 * G_fatal_error); in HIPB_ERR_RECORD mode keeps the first message and
 * returns, and the caller returns at once. */
void hipb_fatal(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
/* Non-zero while a recorded error is pending. */
int hipb_failed(void);

/* Launch bracket of the reference's run() (sam3_model.c:167-207): with
 * profiling on, waits for the stream, records events around the launch
 * and accumulates time and flops under what. err is the launcher's
 * hipError_t; a failure is fatal naming what. */
void hipb_run_begin(struct hipb_backend *b);
void hipb_run_end(struct hipb_backend *b, int err, const char *what,
                  double flops);

/* Grow a backend-owned device scratch to at least n bytes. */
void *hipb_scratch(struct hipb_backend *b, size_t n);

/* Elements of a buffer of its own type. */
size_t hipb_count(hipb_mem m);

#endif /* HIPB_INTERNAL_H */
