// noalloc.hip -- device-resident scratch of the allocation-free decode step
// (eh_append_decode_batched_noalloc).
//
// The array below lives in this library's own code object: the HIP runtime
// places one copy on every GPU the library runs on, and each copy is held
// until the process ends.  Host code must never pass `scratch` itself to a
// kernel (in host code the name is only a host-side stand-in, not a device
// address): eh_noalloc_scratch_setup looks up the current device's address
// once, when a context is created on that device, and the launcher uses that
// address from then on.

#include <hip/hip_runtime.h>

#include <cstdint>

// 32 MiB: the token-balanced decode's partials need 4 * (grid + batch) *
// n_head * 130 bytes (6.6 MB at batch 32, 12 q heads, 1024 runs).
static __device__ __align__(256) unsigned char scratch[32u << 20];

// With the context's device current: the device address of this device's
// copy of `scratch` and its size.  Returns the hipError_t of the lookup.
extern "C" __attribute__((visibility("hidden"))) int eh_noalloc_scratch_setup(void** ptr,
                                                                               uint64_t* bytes) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
    *ptr = p;
    *bytes = sizeof(scratch);
    return 0;
}
