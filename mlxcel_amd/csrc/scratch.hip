// scratch.hip — device scratch of the no-allocation entry point
// (mlxq_quantized_matmul_noalloc): a file-scope device array that every call
// on one GPU shares, so that call needs no hipMalloc.  Each GPU the library
// runs on holds its own copy of the array until the process ends.
#include <hip/hip_runtime.h>

#include <map>
#include <mutex>

#include "kernels.hpp"

namespace {

// Split-K partials of the decode kernels (5-16 rows: K ranges x rows x N
// fp32, e.g. 39 MB for a 151936-wide LM head at 16 rows) and of the prefill
// GEMM fit in 64 MiB at the shapes of 8B-class models.
constexpr size_t kScratchBytes = (size_t)64 << 20;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_mu;
std::map<int, void*> g_ptr;  // device -> address of that device's copy of `scratch`

}  // namespace

namespace mlxq {

size_t static_scratch_bytes() { return kScratchBytes; }

// Device address of `scratch` on the current device, resolved once per device
// with that device current.  In host code the array's name is only a host-side
// stand-in; kernels get this address instead.
hipError_t static_scratch(int dev, void** ptr) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_ptr.find(dev);
  if (it != g_ptr.end()) {
    *ptr = it->second;
    return hipSuccess;
  }
  void* p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  g_ptr[dev] = p;
  *ptr = p;
  return hipSuccess;
}

}  // namespace mlxq
