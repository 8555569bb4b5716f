/* internal.h -- what the other host files of libsepia_hip.so (store.c) use
 * of sepia_hip.c. Not exported. */
#ifndef SEPIA_INTERNAL_H
#define SEPIA_INTERNAL_H

#define __HIP_PLATFORM_AMD__ 1
#include <hip/hip_runtime_api.h>

#include <stddef.h>
#include <stdint.h>

#include "../../include/sepia_gpu.h"

#define SEPIA_HIDDEN __attribute__((visibility("hidden")))

/* One "sepia: hip: ..." line on stderr. */
SEPIA_HIDDEN void sepia_log(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
/* 1 if sepia_gpu_init succeeded (else logs for op). */
SEPIA_HIDDEN int sepia_ready(const char *op);
/* The library's stream. */
SEPIA_HIDDEN hipStream_t sepia_stream(void);
/* A buffer's device address and length. */
SEPIA_HIDDEN uint8_t *sepia_buf_dev(SepiaGpuBuf *b);
SEPIA_HIDDEN size_t sepia_buf_len(const SepiaGpuBuf *b);
/* Bytes of a row of n elements of a ggml type; -1 for an unknown type or an
 * n that is not a whole number of blocks (reference quants_row_bytes,
 * src/quants.c:45-56). */
SEPIA_HIDDEN int64_t sepia_row_bytes(int ggml_type, int64_t n);
/* Count one device or pinned-host allocation (sepia_hip_alloc_count). */
SEPIA_HIDDEN void sepia_count_alloc(void);
/* Release store.c's pinned staging buffers (sepia_gpu_shutdown calls it). */
SEPIA_HIDDEN void sepia_store_shutdown(void);

#endif
