// Device scratch of the no-allocation GEMM entry point (mxfp6_gemm_noalloc_async): one
// file-scope device array, MXFP6_NOALLOC_SCRATCH_BYTES long, that holds a call's split-K partials
// and, when it fits beside them, the repacked copy of A. It lives in this translation unit alone,
// so its code object (and with it the array's device memory) is loaded on a GPU only by the first
// no-allocation call there, and stays until the process ends.
//
// In host code `scratch` names a host-side stand-in, not device memory: its device address is read
// once per device with hipGetSymbolAddress (that device current) and only that address is passed
// on. Every call on a GPU shares that GPU's array and leaves its contents behind; nothing in it
// needs to start at zero (each call writes every byte it later reads), and calls that overlap on
// one GPU race.
#include <hip/hip_runtime.h>

#include <mutex>

#include "../hip_layer.h"
#include "mxfp6_gemm.h"

static __device__ __align__(256) uint8_t scratch[MXFP6_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_addr[kMaxDevices];
}  // namespace

extern "C" void* mxfp6_hip_scratch(size_t* bytes) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_addr[dev] == nullptr) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr)
            return nullptr;
        scratch_addr[dev] = p;
    }
    *bytes = sizeof(scratch);
    return scratch_addr[dev];
}
