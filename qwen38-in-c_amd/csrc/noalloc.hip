// noalloc.hip -- the fixed device scratch of q35mm_matmul_noalloc.
//
// Callers that cannot allocate (code under HIP graph capture, tight serving
// loops) get the scratch their kernels need between launches from one
// file-scope device array instead of library allocations: stream-K arrival
// counters in the first kNoAllocCntBytes (zero between launches: every
// stream-K launch returns the counters it takes to zero), then a region of
// kNoAllocBytes for split partials and staged bf16 activations.
//
// The array's name is a host-side stand-in, not a device address; host code
// uses only the address hipGetSymbolAddress returns, resolved once per
// device at library initialisation with that device current.  Every call on
// a device shares that device's array and keeps the last call's contents;
// calls whose kernels overlap on one device race on it.
#include <hip/hip_runtime.h>

#include "q35mm_internal.h"

namespace {
constexpr size_t kNoAllocTotal = q35mm::kNoAllocCntBytes + q35mm::kNoAllocBytes;
static __device__ __align__(256) uint8_t scratch[kNoAllocTotal];

__global__ __launch_bounds__(256) void zero_u32_kernel(uint32_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
uint8_t *g_ptr[kMaxDevices] = {};
}  // namespace

namespace q35mm {

hipError_t noalloc_setup(int device, hipStream_t stream) {
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    if (g_ptr[device]) return hipSuccess;
    void *ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    // the counters must start at zero; a kernel clears them (the array is
    // zero at load, but that is not something to rely on)
    hipLaunchKernelGGL(zero_u32_kernel, dim3(16), dim3(256), 0, stream, static_cast<uint32_t *>(ptr),
                       kNoAllocCntBytes / 4);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    if (e != hipSuccess) return e;
    g_ptr[device] = static_cast<uint8_t *>(ptr);
    return hipSuccess;
}

uint8_t *noalloc_scratch(int device) { return device >= 0 && device < kMaxDevices ? g_ptr[device] : nullptr; }

}  // namespace q35mm
