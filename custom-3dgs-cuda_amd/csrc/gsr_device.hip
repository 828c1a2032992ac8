// gsr_device.hip — the library's per-device globals:
//   - the device status word: kernels that reach their look-back spin bound
//     or find inconsistent counts OR an error bit into it (bit 0: spin
//     bound, bit 2: inconsistent counts).  The one-group kernel behind
//     bin_count moves it to the host with the pair count, so the next forward call reports
//     what any earlier kernel on the device found, without a synchronisation
//     of its own;
//   - `scratch`, the fixed workspace of the allocation-free backward entry
//     point (gsr_rasterize_backward_noalloc).
// Each device holds its own copy of both at its own address.  Host code takes
// those addresses from hipGetSymbolAddress, once per device with that device
// current, and passes them to kernels as arguments; the symbols' names are
// host-side stand-ins and are never used as device addresses.
#include <hip/hip_runtime.h>

#include <mutex>

#include "gsr_internal.h"

namespace gsr {

// Word 0 is the status; the rest pads the word to its own 256-byte block.
static __device__ __align__(256) int status_word[64];

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
DeviceGlobals g_table[kMaxDevices];  // by device ordinal; null until set up

__global__ void raise_status_kernel(int* __restrict__ status, int bits) {
    if (threadIdx.x == 0 && blockIdx.x == 0) atomicOr(status, bits);
}

}  // namespace

hipError_t device_globals(DeviceGlobals* out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_mu);
    DeviceGlobals& g = g_table[dev];
    if (!g.status || !g.scratch) {
        void* st = nullptr;
        void* sc = nullptr;
        e = hipGetSymbolAddress(&st, HIP_SYMBOL(status_word));
        if (e != hipSuccess) return e;
        e = hipGetSymbolAddress(&sc, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!st || !sc) return hipErrorInvalidSymbol;
        g.status = static_cast<int*>(st);
        g.scratch = sc;
    }
    *out = g;
    return hipSuccess;
}

hipError_t launch_raise_status(int* status, int bits, hipStream_t st) {
    hipLaunchKernelGGL(raise_status_kernel, dim3(1), dim3(64), 0, st, status, bits);
    return hipGetLastError();
}

}  // namespace gsr
