// noalloc_scratch.h -- size of the device scratch array and the accessor
// defined in noalloc_scratch.hip (built with hipcc, linked into the host
// library).
#pragma once
#include <hip/hip_runtime_api.h>

// (2 * 1024 + 64) * 1024 floats = 8.25 MiB per device: the partial rows of
// the widest shape the LayerNorm backward's looping path can take here (1024
// partial rows from 256 workgroups of four waves on a 256-CU device, times
// 1024 columns, for dgamma and for dbeta) plus the 64 chunk rows of their
// column sums.
#define FORGE_NOALLOC_SCRATCH_FLOATS ((2u * 1024u + 64u) * 1024u)

#ifdef __cplusplus
extern "C" {
#endif
hipError_t forge_internal_noalloc_scratch(float** out);
#ifdef __cplusplus
}
#endif
