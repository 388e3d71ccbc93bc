// norm.hip -- row RMSNorm from the fp32 residual stream into a qmm input.
//
// y[r][c] = T(x[r][c] * rsqrt(mean_c(x[r][c]^2) + eps) * w[c]): the RMSNorm
// between the blocks of a DiT step, in the shape of the reference's
// dd_rmsnorm_pitched (Sources/ImarelloDirect/DirectDiTKernels.swift:61-99:
// fp32 sum of squares, rsqrt(mean + eps), times an fp32 weight; eps 1e-5 at
// DirectDiTStep.swift:416).  HBM-bound: one workgroup per row.
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kThreads = 256;

template <int T>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           typename Elem<T>::S* __restrict__ y,
                                                           int cols, float eps) {
  __shared__ float part[kThreads / 64];
  const float* xr = x + (size_t)blockIdx.x * cols;
  float acc = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) acc = __builtin_fmaf(xr[c], xr[c], acc);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) total += part[i];
  const float inv = __frsqrt_rn(total / (float)cols + eps);
  typename Elem<T>::S* yr = y + (size_t)blockIdx.x * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads) yr[c] = Elem<T>::out(xr[c] * inv * w[c]);
}

}  // namespace

hipError_t launch_rmsnorm(const float* x, const float* w, void* y, int rows, int cols, float eps,
                          int dtype, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  switch (dtype) {
    case kBf16:
      hipLaunchKernelGGL(rmsnorm_kernel<kBf16>, dim3(rows), dim3(kThreads), 0, stream, x, w,
                         static_cast<uint16_t*>(y), cols, eps);
      break;
    case kF16:
      hipLaunchKernelGGL(rmsnorm_kernel<kF16>, dim3(rows), dim3(kThreads), 0, stream, x, w,
                         static_cast<uint16_t*>(y), cols, eps);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace imq
