// fmha_noalloc.hip — the launch for callers that cannot allocate (this
// build's own entry point; no counterpart in the reference).
//
// fmha_fwd_d64_bf16_noalloc() is fmha_fwd_d64_bf16_ws() with the workspace
// taken from `scratch`, a static device array of FMHA_NOALLOC_SCRATCH_BYTES
// that the library holds on every GPU it runs on until the process ends.  Its
// device address comes from hipGetSymbolAddress, once per device with that
// device current (the array's name in host code is only a host-side stand-in,
// never a device address).  The balanced form writes every partial slot it
// reads in the same launch, so nothing in the array needs clearing; calls
// that overlap in time on one GPU share the array and race.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "fmha_fwd.h"

static __device__ __align__(256) char scratch[FMHA_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch[kMaxDevices];

// `scratch`'s device address on the current device (looked up on the first
// call there); hipSuccess or the lookup's error.
hipError_t scratch_here(void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    void* ptr = g_scratch[dev].load(std::memory_order_acquire);
    if (ptr == nullptr) {
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (ptr == nullptr) return hipErrorInvalidSymbol;
        g_scratch[dev].store(ptr, std::memory_order_release);
    }
    *out = ptr;
    return hipSuccess;
}

}  // namespace

extern "C" hipError_t fmha_fwd_d64_bf16_noalloc(const FmhaFwdParams* params, int batch, int causal, int variant,
                                                hipStream_t stream) {
    const int64_t need = fmha_fwd_d64_bf16_workspace_size(params, batch, causal, variant);
    if (need < 0) return hipErrorInvalidValue;                                  // rejected arguments
    if (need > (int64_t)FMHA_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;  // beyond the array
    void* ptr = nullptr;
    if (need > 0) {
        const hipError_t e = scratch_here(&ptr);
        if (e != hipSuccess) return e;
    }
    return fmha_fwd_d64_bf16_ws(params, batch, causal, variant, ptr, need, stream);
}
