// The scratch array of qp_dispatch_noalloc: a file-scope device array, so a caller that may not allocate (code
// under HIP graph capture, serving loops, harnesses that forbid hipMalloc) gets the prefill matmul's workspace
// without any allocation.  Every call on a device shares that device's array and finds the last call's contents;
// calls that overlap on one device race.  In host code `scratch` names a host-side stand-in: only the address that
// hipGetSymbolAddress returns (per device) is used to reach the array.
#include <hip/hip_runtime.h>
#include "qp_scratch.h"

static __device__ __align__(256) uint8_t scratch[QP_SCRATCH_BYTES];

namespace qp_scratch {

constexpr int kMaxDevices = 64;
static uint64_t g_ptr[kMaxDevices];  // per device: the array's device address (0: not looked up yet)

int lookup(int device, uint64_t* ptr) {
    if (device < 0 || device >= kMaxDevices) return (int)hipErrorInvalidDevice;
    if (!g_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return (int)e;
        g_ptr[device] = (uint64_t)p;
    }
    *ptr = g_ptr[device];
    return 0;
}

}  // namespace qp_scratch
