// Fixed per-device scratch of the entry points that allocate nothing.
#ifndef NSR_SCRATCH_H
#define NSR_SCRATCH_H

#include <hip/hip_runtime_api.h>

// 1 MiB of f32 per GPU.
#define NSR_NOALLOC_SCRATCH_FLOATS (256 * 1024)

// Device address of `device`'s copy of the scratch array; must be called with
// that device current. Resolved once per device (hipGetSymbolAddress) and
// cached; returns the resolution's status.
hipError_t nsr_scratch_device_ptr(int device, float** out);

#endif
