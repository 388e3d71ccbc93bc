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

#include <memory>
#include <mutex>
#include <vector>

#include "imq_kernels.hpp"

static __device__ __align__(256) float scratch[imq::kStaticScratchBytes / sizeof(float)];

namespace imq {
namespace {

// Per device: the scratch's address and the event of the last call that
// used it.  Entries are never removed (a GPU's copy of the array lives until
// the process ends), so references to them stay valid.
struct DeviceScratch {
  void* addr = nullptr;
  hipEvent_t last = nullptr;
  bool recorded = false;  // `last` has been recorded at least once
  std::mutex order;       // held from scratch_acquire to scratch_release
};

std::mutex g_mu;
std::vector<std::unique_ptr<DeviceScratch>> g_dev;

DeviceScratch* entry(int device) {
  std::lock_guard<std::mutex> lk(g_mu);
  if (device < 0 || (size_t)device >= g_dev.size()) return nullptr;
  return g_dev[device].get();
}

}  // namespace

// Device address of `scratch` on `device` (which must be the current device),
// looked up once per device and kept for the process; the device's ordering
// event is created with it.
hipError_t static_scratch(int device, void** out) {
  *out = nullptr;
  if (device < 0) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lk(g_mu);
  if ((size_t)device >= g_dev.size()) g_dev.resize((size_t)device + 1);
  if (!g_dev[device]) g_dev[device] = std::make_unique<DeviceScratch>();
  DeviceScratch& d = *g_dev[device];
  if (!d.addr) {
    void* p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e != hipSuccess) return e;
    d.last = ev;
    d.addr = p;
  }
  *out = d.addr;
  return hipSuccess;
}

hipError_t scratch_acquire(int device, hipStream_t stream) {
  DeviceScratch* d = entry(device);
  if (!d || !d->addr) return hipErrorNotInitialized;
  d->order.lock();
  if (d->recorded) {
    const hipError_t e = hipStreamWaitEvent(stream, d->last, 0);
    if (e != hipSuccess) {
      d->order.unlock();
      return e;
    }
  }
  return hipSuccess;
}

hipError_t scratch_release(int device, hipStream_t stream) {
  DeviceScratch* d = entry(device);
  if (!d) return hipErrorNotInitialized;
  const hipError_t e = hipEventRecord(d->last, stream);
  if (e == hipSuccess) d->recorded = true;
  d->order.unlock();
  return e;
}

}  // namespace imq
