// ee_noalloc.hip -- the device-resident workspace of ee_routed_linear_noalloc.
//
// ee_routed_linear needs a workspace for the activation codes of its INT8 and
// FP8 rows and their scales; its caller allocates it.  Callers that cannot
// allocate (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc) call ee_routed_linear_noalloc instead, which uses this array:
//   bytes [0, EE_NOALLOC_MAX_CODE_BYTES)              codes  [M, K], row stride K
//   bytes [EE_NOALLOC_MAX_CODE_BYTES, + 4 * MAX_ROWS)  f32 scales [M]
// Each GPU the library runs on holds its own copy (about 32 MiB) until the
// process ends.  Every slot a call reads was written earlier in the same call,
// so nothing needs clearing; calls that overlap on one GPU share the array and
// race.  This file is compiled by hipcc (host and device code) into the host
// library; the kernels are the ordinary gfx950 code objects and receive the
// array's device address as their workspace argument.
#include <hip/hip_runtime.h>

#include "entropy_engine.h"

#define EE_NOALLOC_SCRATCH_BYTES (EE_NOALLOC_MAX_CODE_BYTES + 4 * EE_NOALLOC_MAX_ROWS)

static __device__ __align__(256) uint8_t scratch[EE_NOALLOC_SCRATCH_BYTES];

// Device address of the array on the current device (the host-side name is
// only a stand-in for it).  Called once per engine, i.e. once per device the
// caller creates an engine on, with that device current.  Returns the HIP
// error code (0 = success).
extern "C" __attribute__((visibility("hidden"))) int ee_noalloc_scratch_address(void** out, int64_t* bytes) {
    *out = nullptr;
    *bytes = 0;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    *out = p;
    *bytes = EE_NOALLOC_SCRATCH_BYTES;
    return 0;
}
