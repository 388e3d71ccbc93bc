// scratch.hip -- the statically allocated split-K scratch of the
// allocation-free dispatcher entry point (imq_qmm_t_noalloc).
//
// The array lives in the code object's device data: each GPU the library runs
// on holds its own copy, allocated when the code object is loaded there and
// kept until the process ends.  In host code the name `scratch` is only a
// stand-in for the symbol, not a device address; the device address of a
// GPU's copy comes from hipGetSymbolAddress with that GPU current, and only
// that address is ever passed to a kernel.
#include <hip/hip_runtime.h>

#include <mutex>
#include <vector>

#include "imq_kernels.hpp"

static __device__ __align__(256) float scratch[imq::kStaticScratchBytes / sizeof(float)];

namespace imq {

// Device address of `scratch` on `device` (which must be the current device),
// looked up once per device and kept for the process.
hipError_t static_scratch(int device, void** out) {
  static std::mutex mu;
  static std::vector<void*> addr;
  *out = nullptr;
  if (device < 0) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(mu);
  if ((size_t)device >= addr.size()) addr.resize((size_t)device + 1, nullptr);
  if (!addr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    addr[device] = p;
  }
  *out = addr[device];
  return hipSuccess;
}

}  // namespace imq
