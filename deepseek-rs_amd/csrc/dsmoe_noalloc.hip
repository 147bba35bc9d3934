// Static device scratch for dsmoe_forward_noalloc (dsmoe_host.cpp): the
// buffers one decode call (T <= 8) needs between its launches, in a
// file-scope device array instead of hipMalloc'd memory, for callers that
// cannot allocate (code under graph capture, tight serving loops).
//
// Each GPU the library runs on holds its own copy of `scratch` until the
// process ends.  Host code never uses the array's name as an address: at
// set-up (the library's per-device code object load, with that device
// current) hipGetSymbolAddress gives the device address, which is kept per
// device and passed to the kernels as an ordinary pointer.
//
// Every call on one GPU shares that GPU's array and finds the previous
// call's contents in it; calls that overlap on one GPU race.  The only state
// that must start at zero are the mid row counters, which every completed
// call leaves at zero again; set-up clears the whole array once.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

constexpr size_t kNoAllocScratchBytes = size_t(16) << 20;

static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

__global__ void __launch_bounds__(256) clear_words(uint4* p, size_t n) {
  const uint4 z = {0u, 0u, 0u, 0u};
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = z;
}

}  // namespace

// Called once per device with that device current.  Returns 0 and the
// device address and size of this device's array, or a HIP error code.
extern "C" int dsmoe_noalloc_setup(void** ptr, size_t* bytes) {
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) return e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol;
  hipLaunchKernelGGL(clear_words, dim3(1024), dim3(256), 0, nullptr, (uint4*)p, kNoAllocScratchBytes / 16);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
  if (e != hipSuccess) return (int)e;
  *ptr = p;
  *bytes = kNoAllocScratchBytes;
  return 0;
}
