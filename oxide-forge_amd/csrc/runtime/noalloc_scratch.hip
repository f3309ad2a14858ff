// noalloc_scratch.hip -- the device scratch of the no-allocation entry point
// (forge_layer_norm_bwd_noalloc in include/oxforge.h).
//
// A file-scope device array of FORGE_NOALLOC_SCRATCH_FLOATS floats (8.25 MiB).
// Every GPU that the library runs on holds its own copy until the process
// ends; the HIP runtime places it when this code object is first used on
// that device.  Host code never passes the array's name to a kernel (on the
// host it is only a stand-in symbol, not a device address): the runtime
// resolves the device address once per device, at forge_runtime_create with
// that device current, through forge_internal_noalloc_scratch below, and
// passes that address to the kernels.
#include <hip/hip_runtime.h>

#include "noalloc_scratch.h"

static __device__ __align__(256) float scratch[FORGE_NOALLOC_SCRATCH_FLOATS];

// Device address of `scratch` on the current device (hipGetSymbolAddress's
// status is returned unchanged; *out is null on failure).
extern "C" hipError_t forge_internal_noalloc_scratch(float** out) {
    *out = nullptr;
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) *out = static_cast<float*>(p);
    return e;
}
