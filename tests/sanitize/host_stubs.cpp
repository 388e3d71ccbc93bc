// host_stubs.cpp -- the device-side entry points of libimq for a host-only
// build of its C++ (capi.cpp, weights.cpp, step.cpp) under AddressSanitizer
// and UndefinedBehaviorSanitizer on a machine without a GPU.
//
// TEST INFRASTRUCTURE ONLY.  The kernels live in .hip translation units that
// only hipcc compiles; here every launcher reports hipErrorNoDevice and the
// planners answer as the real ones do for arguments that never reach a
// launch.  What the sanitized build exercises is the host code: the
// safetensors/JSON parser and the argument checks of every C entry point.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "imq_kernels.hpp"

namespace imq {

hipError_t launch_dequant(const uint32_t*, const void*, const void*, void*, int, int, int,
                          hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemv(const uint32_t*, const void*, const void*, const void*, void*, int, int,
                        int, int, hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemv_swiglu(const uint32_t*, const void*, const void*, const void*, void*, int,
                               int, int, int, int, int, int, float, float, int, hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemv_resid_add(const uint32_t*, const void*, const void*, const void*,
                                  const void*, void*, int, int, int, int, hipStream_t) {
  return hipErrorNoDevice;
}
bool qgemv_norm_fits(int, int, int, int, int, const void*, const float*) { return false; }
hipError_t launch_qgemv_norm(const uint32_t*, const void*, const void*, const void*, const float*,
                             float, void*, int, int, int, int, hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemv_swiglu_norm(const uint32_t*, const void*, const void*, const void*,
                                    const float*, float, void*, int, int, int, int, int, int, int,
                                    int, hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemm(const uint32_t*, const void*, const void*, const void*, void*, int, int,
                        int, int, hipStream_t, SplitWs) {
  return hipErrorNoDevice;
}
size_t qgemm_split_bytes(int, int, int, bool) { return 0; }
QgemmPlan qgemm_plan(int k, int n, int m, bool, bool, int, bool) {
  return QgemmPlan{qgemm_big_supported(k, n, m), 128, 1, 0, 256};
}
bool qgemm_big_supported(int k, int n, int m) {
  return (size_t)m * k * 2 < ((size_t)1 << 31) && (size_t)n * k / 2 < ((size_t)1 << 31) &&
         k % 256 == 0;
}
hipError_t launch_qgemm_postscale(const uint32_t*, const void*, const void*, const void*, float*,
                                  int, int, int, float, int, hipStream_t, SplitWs, const float*) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemm_postscale_f16(const uint32_t*, const void*, const void*, const void*,
                                      void*, int, int, int, float, hipStream_t, const float*) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemm_resid_add(const uint32_t*, const void*, const void*, const void*,
                                  const void*, void*, int, int, int, int, hipStream_t, SplitWs) {
  return hipErrorNoDevice;
}
hipError_t launch_rmsnorm_t(const void*, const float*, void*, int, int, float, int, hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemm_gate_add(const uint32_t*, const void*, const void*, const void*,
                                 const float*, const float*, float*, int, int, int, float, int,
                                 hipStream_t, SplitWs, const float*) {
  return hipErrorNoDevice;
}
hipError_t launch_qgemm_swiglu(const uint32_t*, const void*, const void*, const void*, void*, int,
                               int, int, int, int, int, int, float, float, int, hipStream_t,
                               SplitWs) {
  return hipErrorNoDevice;
}
hipError_t launch_prescale(const float*, void*, size_t, float, int, hipStream_t, const float*) {
  return hipErrorNoDevice;
}
hipError_t launch_dynamic_scale(const float*, size_t, float, float*, hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_rmsnorm(const float*, const float*, void*, int, int, float, int, hipStream_t,
                          float) {
  return hipErrorNoDevice;
}
hipError_t launch_fill_f32(float*, float, int, hipStream_t) { return hipErrorNoDevice; }
hipError_t launch_silu_f32(const float*, float*, int, hipStream_t) { return hipErrorNoDevice; }
hipError_t static_scratch(int, void** out) {
  *out = nullptr;
  return hipErrorNoDevice;
}
hipError_t scratch_acquire(int, hipStream_t) { return hipErrorNoDevice; }
hipError_t scratch_release(int, hipStream_t) { return hipErrorNoDevice; }
bool qskinny_supported(int k, int n, int m, int dtype) {
  return m >= 1 && m <= kQskinnyMaxM && n >= 1 && k >= 128 && k % 128 == 0 &&
         (dtype == 0 || dtype == 1) && (size_t)n * k / 2 < ((size_t)1 << 32) &&
         (size_t)m * k * 2 < ((size_t)1 << 31);
}
size_t qskinny_split_bytes(int, int, int) { return 0; }
size_t qskinny_resid_split_bytes(int, int, int) { return 0; }
hipError_t launch_qskinny_swiglu(const uint32_t*, const void*, const void*, const void*, void*,
                                 int, int, int, int, int, float, float, int, hipStream_t,
                                 SplitWs) {
  return hipErrorNoDevice;
}
hipError_t launch_reduce_swiglu(const float*, int, int, int, void*, int, float, float, int,
                                hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_swiglu_t(const void*, int, int, int, void*, int, float, float, int,
                           hipStream_t) {
  return hipErrorNoDevice;
}
int qskinny_splits(int, int, int) { return 1; }
hipError_t launch_dequant_rows(const uint32_t*, const void*, const void*, const int32_t*, int,
                               void*, int, int, int, hipStream_t) {
  return hipErrorNoDevice;
}
hipError_t launch_qskinny(const uint32_t*, const void*, const void*, const void*, void*, int, int,
                          int, int, hipStream_t, SplitWs) {
  return hipErrorNoDevice;
}
hipError_t launch_qskinny_resid_add(const uint32_t*, const void*, const void*, const void*,
                                    const void*, void*, int, int, int, int, hipStream_t, SplitWs) {
  return hipErrorNoDevice;
}
bool qskinny_resid_add_norm_fits(int, int, int, int, const void*, const void*, const float*,
                                 const void*, SplitWs) {
  return false;
}
hipError_t launch_qskinny_resid_add_norm(const uint32_t*, const void*, const void*, const void*,
                                         const void*, void*, const float*, void*, float, int, int,
                                         int, int, hipStream_t, SplitWs) {
  return hipErrorNoDevice;
}

}  // namespace imq
