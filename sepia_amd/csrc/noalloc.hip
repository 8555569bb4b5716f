// noalloc.hip -- the device-resident scratch of sepia_hip_moe_decode_noalloc.
//
// A caller that cannot allocate device memory (code under HIP graph
// capture, a serving loop, a harness that forbids hipMalloc) gets its MoE
// decode scratch from this fixed array instead of the library's growable
// region: the counter words the FFN launches use, then router logits, the
// selection, h and the per-slot partial rows. Each GPU the library runs on
// holds its own copy of the array until the process ends.
//
// In host code the name `scratch` is only a host-side stand-in for the
// device variable; passing it to a kernel would make the kernel fault. The
// device address is asked for once per device, with that device current
// (sepia_noalloc_setup, called from sepia_gpu_init), and host code uses only
// that address afterwards.
#include <hip/hip_runtime.h>

#include <stddef.h>
#include <stdint.h>

#include "noalloc.h"

static __device__ __align__(256) uint8_t scratch[SEPIA_NOALLOC_BYTES];

#define NOALLOC_MAX_DEVICES 64
static void *g_ptr[NOALLOC_MAX_DEVICES];

extern "C" int sepia_noalloc_setup(void) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) return 0;
    if (g_ptr[dev]) return 1;
    void *p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return 0;
    g_ptr[dev] = p;
    return 1;
}

extern "C" void *sepia_noalloc_ptr(void) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= NOALLOC_MAX_DEVICES) return nullptr;
    return g_ptr[dev];
}
