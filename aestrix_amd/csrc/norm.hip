// norm.hip -- row RMSNorm from the fp32 residual stream into a qmm input.
//
// y[r][c] = T(x[r][c] * rsqrt(mean_c(x[r][c]^2) + eps) * w[c] * s): the RMSNorm
// between the blocks of a DiT step, in the shape of the reference's
// dd_rmsnorm_pitched (Sources/ImarelloDirect/DirectDiTKernels.swift:61-99:
// fp32 sum of squares, rsqrt(mean + eps), times an fp32 weight; eps 1e-5 at
// DirectDiTStep.swift:416).  HBM-bound: one workgroup per row.  Rounding to
// T is RNE (the hardware pair conversion in the vector kernel).  s is 1 between
// the blocks and 1/16 before the head's proj_out (the ÷16 of the f16 protocol
// that dd_ln_mod_prescale folds into its output, DirectDiTKernels.swift:16-59);
// a power of two, so it never changes a rounding.
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kThreads = 256;

template <int T>
__global__ __launch_bounds__(kThreads) void rmsnorm_kernel(const float* __restrict__ x,
                                                           const float* __restrict__ w,
                                                           typename Elem<T>::S* __restrict__ y,
                                                           int cols, float eps, float s) {
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
  for (int c = threadIdx.x; c < cols; c += kThreads) yr[c] = Elem<T>::out(xr[c] * inv * w[c] * s);
}

// The same for cols % 4 == 0 and cols <= 1024 * V: each thread loads its V
// float4 pieces of the row once (16-byte loads), keeps them in registers for
// the scaling pass and stores 4 outputs as one 8-byte store.  The row is read
// from memory once instead of twice.
template <int T, int V>
__global__ __launch_bounds__(kThreads) void rmsnorm_vec_kernel(const float* __restrict__ x,
                                                               const float* __restrict__ w,
                                                               typename Elem<T>::S* __restrict__ y,
                                                               int cols, float eps, float s) {
  __shared__ float part[kThreads / 64];
  const int n4 = cols >> 2;
  const float4* xr = reinterpret_cast<const float4*>(x + (size_t)blockIdx.x * cols);
  float4 v[V];
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    v[i] = idx < n4 ? xr[idx] : make_float4(0.f, 0.f, 0.f, 0.f);
    acc = __builtin_fmaf(v[i].x, v[i].x, acc);
    acc = __builtin_fmaf(v[i].y, v[i].y, acc);
    acc = __builtin_fmaf(v[i].z, v[i].z, acc);
    acc = __builtin_fmaf(v[i].w, v[i].w, acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) total += part[i];
  const float inv = __frsqrt_rn(total / (float)cols + eps);
  const float4* wr = reinterpret_cast<const float4*>(w);
  uint2* yr = reinterpret_cast<uint2*>(y + (size_t)blockIdx.x * cols);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    if (idx < n4) {
      const float4 ww = wr[idx];
      yr[idx] = make_uint2(Elem<T>::pack2(v[i].x * inv * ww.x * s, v[i].y * inv * ww.y * s),
                           Elem<T>::pack2(v[i].z * inv * ww.z * s, v[i].w * inv * ww.w * s));
    }
  }
}

template <int T>
hipError_t launch_t(const float* x, const float* w, void* y, int rows, int cols, float eps,
                    float s, hipStream_t stream) {
  auto* yy = static_cast<typename Elem<T>::S*>(y);
  const bool vec = cols % 4 == 0 && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)w & 15u) == 0 &&
                   ((uintptr_t)y & 7u) == 0;
  const int v = (cols / 4 + kThreads - 1) / kThreads;
  const dim3 grid(rows), block(kThreads);
  if (vec && v <= 1)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, 1>), grid, block, 0, stream, x, w, yy, cols, eps, s);
  else if (vec && v == 2)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, 2>), grid, block, 0, stream, x, w, yy, cols, eps, s);
  else if (vec && v == 3)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, 3>), grid, block, 0, stream, x, w, yy, cols, eps, s);
  else if (vec && v == 4)
    hipLaunchKernelGGL((rmsnorm_vec_kernel<T, 4>), grid, block, 0, stream, x, w, yy, cols, eps, s);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<T>, grid, block, 0, stream, x, w, yy, cols, eps, s);
  return hipGetLastError();
}

__global__ __launch_bounds__(kThreads) void fill_f32_kernel(float* __restrict__ p, float v, int n) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < n) p[i] = v;
}

// y[r][c] = T(x[r][c] * rsqrt(mean_c(x[r][c]^2) + eps) * w[c]) on a T row
// (the text encoder's dq_rmsnorm, DirectGlueKernels.swift:14-49: fp32 sum of
// squares, fp32 weight, the residual stream itself in T).  One workgroup per
// row; the row is read twice (the second pass from the cache).
template <int T>
__global__ __launch_bounds__(kThreads) void rmsnorm_tin_kernel(
    const typename Elem<T>::S* __restrict__ x, const float* __restrict__ w,
    typename Elem<T>::S* __restrict__ y, int cols, float eps) {
  __shared__ float part[kThreads / 64];
  const typename Elem<T>::S* xr = x + (size_t)blockIdx.x * cols;
  float acc = 0.f;
  for (int c = threadIdx.x; c < cols; c += kThreads) {
    const float v = Elem<T>::param(xr[c]);
    acc = __builtin_fmaf(v, v, acc);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) total += part[i];
  const float inv = __frsqrt_rn(total / (float)cols + eps);
  typename Elem<T>::S* yr = y + (size_t)blockIdx.x * cols;
  for (int c = threadIdx.x; c < cols; c += kThreads)
    yr[c] = Elem<T>::out(Elem<T>::param(xr[c]) * inv * w[c]);
}

// The same for cols % 8 == 0, cols <= 2048 V, 16-byte aligned rows: each
// thread loads its V 16-byte pieces (8 values) once, keeps them for the
// scaling pass and stores 8 outputs at a time.  The scalar kernel above waits
// for cols / 256 dependent 2-byte load rounds per pass: 14 us for [512 x
// 2560] where this takes a fraction.
template <int T, int V>
__global__ __launch_bounds__(kThreads) void rmsnorm_tin_vec_kernel(
    const typename Elem<T>::S* __restrict__ x, const float* __restrict__ w,
    typename Elem<T>::S* __restrict__ y, int cols, float eps) {
  __shared__ float part[kThreads / 64];
  const int n8 = cols >> 3;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)blockIdx.x * cols);
  const float4* wr = reinterpret_cast<const float4*>(w);
  uint4 v[V];
  float4 wv[V][2];  // the weights load beside the row, not after the sum
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    if (idx < n8) {
      wv[i][0] = wr[2 * idx];
      wv[i][1] = wr[2 * idx + 1];
    }
  }
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    v[i] = idx < n8 ? xr[idx] : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t q[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = Elem<T>::param((uint16_t)(q[e] & 0xFFFFu));
      const float hi = Elem<T>::param((uint16_t)(q[e] >> 16));
      acc = __builtin_fmaf(lo, lo, acc);
      acc = __builtin_fmaf(hi, hi, acc);
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int i = 0; i < kThreads / 64; ++i) total += part[i];
  const float inv = __frsqrt_rn(total / (float)cols + eps);
  uint4* yr = reinterpret_cast<uint4*>(y + (size_t)blockIdx.x * cols);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * kThreads;
    if (idx < n8) {
      const float4 w0 = wv[i][0], w1 = wv[i][1];
      const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      const uint32_t q[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = Elem<T>::pack2(Elem<T>::param((uint16_t)(q[e] & 0xFFFFu)) * inv * ww[2 * e],
                              Elem<T>::param((uint16_t)(q[e] >> 16)) * inv * ww[2 * e + 1]);
      yr[idx] = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// y[i] = v / (1 + exp(-v)), v = x[i], fp32: dd_silu_f32 (DirectDiTKernels.swift:176-184)
// with the device library's expf and an IEEE division.
__global__ __launch_bounds__(kThreads) void silu_f32_kernel(const float* __restrict__ x,
                                                            float* __restrict__ y, int n) {
  const int i = blockIdx.x * kThreads + threadIdx.x;
  if (i < n) {
    const float v = x[i];
    y[i] = v / (1.0f + expf(-v));
  }
}

}  // namespace

hipError_t launch_rmsnorm_t(const void* x, const float* w, void* y, int rows, int cols, float eps,
                            int dtype, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const dim3 grid(rows), block(kThreads);
  const auto* xx = static_cast<const uint16_t*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  const int v = (cols / 8 + kThreads - 1) / kThreads;
  const bool vec = cols % 8 == 0 && v <= 4 && ((uintptr_t)x & 15u) == 0 &&
                   ((uintptr_t)w & 15u) == 0 && ((uintptr_t)y & 15u) == 0;
  if (dtype != kBf16 && dtype != kF16) return hipErrorInvalidValue;
#define IMQ_RMS_TIN(TT)                                                                        \
  do {                                                                                         \
    if (vec && v <= 1)                                                                         \
      hipLaunchKernelGGL((rmsnorm_tin_vec_kernel<TT, 1>), grid, block, 0, stream, xx, w, yy,   \
                         cols, eps);                                                           \
    else if (vec && v == 2)                                                                    \
      hipLaunchKernelGGL((rmsnorm_tin_vec_kernel<TT, 2>), grid, block, 0, stream, xx, w, yy,   \
                         cols, eps);                                                           \
    else if (vec)                                                                              \
      hipLaunchKernelGGL((rmsnorm_tin_vec_kernel<TT, 4>), grid, block, 0, stream, xx, w, yy,   \
                         cols, eps);                                                           \
    else                                                                                       \
      hipLaunchKernelGGL(rmsnorm_tin_kernel<TT>, grid, block, 0, stream, xx, w, yy, cols, eps); \
  } while (0)
  if (dtype == kBf16) IMQ_RMS_TIN(kBf16);
  else IMQ_RMS_TIN(kF16);
#undef IMQ_RMS_TIN
  return hipGetLastError();
}

hipError_t launch_silu_f32(const float* x, float* y, int n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(silu_f32_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, x, y, n);
  return hipGetLastError();
}

hipError_t launch_fill_f32(float* p, float v, int n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(fill_f32_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)),
                     dim3(kThreads), 0, stream, p, v, n);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, void* y, int rows, int cols, float eps,
                          int dtype, hipStream_t stream, float out_scale) {
  if (rows <= 0) return hipSuccess;
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(x, w, y, rows, cols, eps, out_scale, stream);
    case kF16: return launch_t<kF16>(x, w, y, rows, cols, eps, out_scale, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace imq
