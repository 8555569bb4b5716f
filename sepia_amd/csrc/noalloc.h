/* noalloc.h -- internal interface between sepia_hip.c and noalloc.hip (the
 * fixed device array behind sepia_hip_moe_decode_noalloc). Not exported. */
#ifndef SEPIA_NOALLOC_H
#define SEPIA_NOALLOC_H

/* Bytes of the per-device array: a 64 KiB counter region, then the data
 * region (a C3 layer's decode needs about 300 KB of it). */
#define SEPIA_NOALLOC_BYTES ((size_t)4 << 20)

#ifdef __cplusplus
extern "C" {
#endif

/* With the device to set up current: looks up the device address of the
 * array (hipGetSymbolAddress) once and keeps it for that device. 1 on
 * success. */
__attribute__((visibility("hidden"))) int sepia_noalloc_setup(void);

/* The current device's address of the array, NULL if it was never set up. */
__attribute__((visibility("hidden"))) void *sepia_noalloc_ptr(void);

#ifdef __cplusplus
}
#endif
#endif
