// prescale.hip -- the input half of the f16 quantized-linear sandwich.
//
// y[i] = T(x[i] / scale): AttentionUtils.compiledPreScale
// (Sources/ImarelloMLX/AttentionUtils.swift:155-160, `(x / s).asType(.float16)`),
// which applyLinearCore (:198-230) runs before the f16 qmm so that its f16
// accumulation cannot overflow (scale 16, AttentionTuning.linearF16Scale).
// The quotient is the correctly rounded fp32 division and the conversion to
// T rounds to nearest even, as MLX's f32 divide and astype do, so the result
// is bit-exact.  HBM-bound: 4 bytes read and 2 written per element.
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kThreads = 256;

// Eight elements per thread and iteration: two 16-byte loads, one 16-byte
// store.  Requires x and y 16-byte aligned; n8 = count / 8.
template <int T>
__global__ __launch_bounds__(kThreads) void prescale_vec_kernel(const float4* __restrict__ x,
                                                                uint4* __restrict__ y, size_t n8,
                                                                float scale,
                                                                const float* __restrict__ scale_dev) {
  if (scale_dev) scale = *scale_dev;
  const size_t stride = (size_t)gridDim.x * kThreads;
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < n8; i += stride) {
    const float4 a = x[2 * i], b = x[2 * i + 1];
    y[i] = make_uint4(Elem<T>::pack2(__fdiv_rn(a.x, scale), __fdiv_rn(a.y, scale)),
                      Elem<T>::pack2(__fdiv_rn(a.z, scale), __fdiv_rn(a.w, scale)),
                      Elem<T>::pack2(__fdiv_rn(b.x, scale), __fdiv_rn(b.y, scale)),
                      Elem<T>::pack2(__fdiv_rn(b.z, scale), __fdiv_rn(b.w, scale)));
  }
}

// Elements [first, count) one at a time (unaligned buffers, or the tail).
template <int T>
__global__ __launch_bounds__(kThreads) void prescale_kernel(const float* __restrict__ x,
                                                            uint16_t* __restrict__ y, size_t first,
                                                            size_t count, float scale,
                                                            const float* __restrict__ scale_dev) {
  if (scale_dev) scale = *scale_dev;
  const size_t stride = (size_t)gridDim.x * kThreads;
  for (size_t i = first + (size_t)blockIdx.x * kThreads + threadIdx.x; i < count; i += stride)
    y[i] = Elem<T>::out(__fdiv_rn(x[i], scale));
}

// Enough workgroups to fill the device several times over; the kernels loop.
unsigned grid_for(size_t items) {
  const size_t want = (items + kThreads - 1) / kThreads;
  return (unsigned)(want < 4096 ? (want > 0 ? want : 1) : 4096);
}

template <int T>
hipError_t launch_t(const float* x, void* y, size_t count, float scale, const float* scale_dev,
                    hipStream_t stream) {
  auto* yy = static_cast<uint16_t*>(y);
  size_t done = 0;
  if (((uintptr_t)x & 15u) == 0 && ((uintptr_t)y & 15u) == 0) {
    const size_t n8 = count / 8;
    if (n8 > 0) {
      hipLaunchKernelGGL(prescale_vec_kernel<T>, dim3(grid_for(n8)), dim3(kThreads), 0, stream,
                         reinterpret_cast<const float4*>(x), reinterpret_cast<uint4*>(yy), n8,
                         scale, scale_dev);
      const hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
    done = n8 * 8;
  }
  if (done < count)
    hipLaunchKernelGGL(prescale_kernel<T>, dim3(grid_for(count - done)), dim3(kThreads), 0, stream,
                       x, yy, done, count, scale, scale_dev);
  return hipGetLastError();
}

// amax of |x| over count floats into *out (as bits: for non-negative floats
// the integer order is the float order, and a NaN, whose bits exceed
// infinity's, wins like the max of a tensor holding one); *out starts at 0.
__global__ __launch_bounds__(kThreads) void amax_kernel(const float* __restrict__ x, size_t count,
                                                        unsigned int* __restrict__ out) {
  __shared__ unsigned int part[kThreads / 64];
  const size_t stride = (size_t)gridDim.x * kThreads;
  unsigned int m = 0;
  for (size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x; i < count; i += stride)
    m = max(m, __float_as_uint(x[i]) & 0x7FFFFFFFu);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = max(m, (unsigned int)__shfl_xor((int)m, off, 64));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned int b = part[0];
#pragma unroll
    for (int i = 1; i < kThreads / 64; ++i) b = max(b, part[i]);
    atomicMax(out, b);
  }
}

// *s = max(amax / target, 1), the amax read from *s's bits (one thread).
__global__ void scale_from_amax_kernel(float* __restrict__ s, float target) {
  const float amax = __uint_as_float(*reinterpret_cast<unsigned int*>(s));
  const float q = __fdiv_rn(amax, target);
  *s = (q != q) ? q : (q > 1.0f ? q : 1.0f);  // a NaN amax gives a NaN scale
}

__global__ void zero_u32_kernel(unsigned int* __restrict__ p) { *p = 0u; }

}  // namespace

hipError_t launch_prescale(const float* x, void* y, size_t count, float scale, int dtype,
                           hipStream_t stream, const float* scale_dev) {
  if (count == 0) return hipSuccess;
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(x, y, count, scale, scale_dev, stream);
    case kF16: return launch_t<kF16>(x, y, count, scale, scale_dev, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dynamic_scale(const float* x, size_t count, float target, float* out,
                                hipStream_t stream) {
  auto* bits = reinterpret_cast<unsigned int*>(out);
  hipLaunchKernelGGL(zero_u32_kernel, dim3(1), dim3(1), 0, stream, bits);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (count > 0) {
    hipLaunchKernelGGL(amax_kernel, dim3(grid_for(count)), dim3(kThreads), 0, stream, x, count,
                       bits);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  hipLaunchKernelGGL(scale_from_amax_kernel, dim3(1), dim3(1), 0, stream, out, target);
  return hipGetLastError();
}

}  // namespace imq
