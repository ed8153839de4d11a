// The library's fixed device scratch (used by qp_dispatch_noalloc; see include/quipu.h).
#pragma once
#include <stdint.h>

// Bytes of the scratch array each device holds from qp_init until the process ends: the prefill matmul's split
// input planes (4 bytes per input value: up to 512 tokens at K = 14336) and as many split-K partials as fit beside
// them.
#define QP_SCRATCH_BYTES (32u << 20)

namespace qp_scratch {
// Device address of the scratch array on `device`, which must be the current device: looked up with
// hipGetSymbolAddress on the first call for that device, cached afterwards.  Returns a hipError_t value.
__attribute__((visibility("hidden"))) int lookup(int device, uint64_t* ptr);
}  // namespace qp_scratch
