// noalloc_scratch.h -- size of the device scratch array and the accessor
// defined in noalloc_scratch.hip (built with hipcc, linked into the host
// library).
#pragma once
#include <hip/hip_runtime_api.h>

// 2^21 floats = 8 MiB per device.
#define FORGE_NOALLOC_SCRATCH_FLOATS (1u << 21)

#ifdef __cplusplus
extern "C" {
#endif
hipError_t forge_internal_noalloc_scratch(float** out);
#ifdef __cplusplus
}
#endif
