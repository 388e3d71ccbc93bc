// dequant.hip -- standalone affine 4-bit dequantize for gfx950.
//
// out[n][k] = RNE_T(fl32(scale[n][k/64] * q[n][k] + bias[n][k/64]))
// Restates MLX `dequantized(..., groupSize: 64, bits: 4)` as used by the
// reference (Sources/ImarelloDirect/DirectTEEncoder.swift:106-134).
//
// HBM-bound: 0.5 B of codes + 4/64 B of scale/bias read and 2 B written per
// element.  One lane owns 32 consecutive codes (a 16-byte load, half a group)
// and writes 64 bytes of output; a wave therefore reads 1 KiB of packed codes
// and writes 4 KiB of contiguous output.  The bf16 rounding uses the integer
// formula so the result is bit-identical to it for every input pattern.
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kThreads = 256;

template <typename T>
struct DeqOut;

template <>
struct DeqOut<uint16_t> {  // bf16 bit patterns
  static __device__ __forceinline__ float load(const uint16_t* p) { return bf16_to_f32(*p); }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    return f32_to_bf16_int(lo) | (f32_to_bf16_int(hi) << 16);
  }
};

struct F16Tag {};
template <>
struct DeqOut<F16Tag> {  // f16 bit patterns
  static __device__ __forceinline__ float load(const uint16_t* p) {
    return (float)__builtin_bit_cast(_Float16, *p);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    // v_cvt_f16_f32 rounds to nearest even (default round mode).
    const uint32_t a = __builtin_bit_cast(uint16_t, (_Float16)lo);
    const uint32_t b = __builtin_bit_cast(uint16_t, (_Float16)hi);
    return a | (b << 16);
  }
};

template <typename Tag>
__global__ __launch_bounds__(kThreads) void dequant_kernel(const u32x4_t* __restrict__ w,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint16_t* __restrict__ biases,
                                                           u32x4_t* __restrict__ out,
                                                           uint32_t total_chunks,
                                                           uint32_t chunks_per_row) {
  const uint32_t c = blockIdx.x * kThreads + threadIdx.x;
  if (c >= total_chunks) return;
  const uint32_t row = c / chunks_per_row;
  const uint32_t j = c - row * chunks_per_row;
  const size_t gi = (size_t)row * (chunks_per_row >> 1) + (j >> 1);
  const float s = DeqOut<Tag>::load(scales + gi);
  const float b = DeqOut<Tag>::load(biases + gi);
  const u32x4_t q = __builtin_nontemporal_load(w + c);
  const uint32_t words[4] = {q.x, q.y, q.z, q.w};
  u32x4_t* dst = out + (size_t)c * 4;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t word = words[i];
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float q0 = (float)((word >> (8 * p)) & 0xFu);
      const float q1 = (float)((word >> (8 * p + 4)) & 0xFu);
      // Two rounded operations, never contracted into an fma: the product is
      // exact unless it overflows, and then it must stay +-inf as in the
      // reference's `scale * q + bias`.
      o[p] = DeqOut<Tag>::pack(__fadd_rn(__fmul_rn(s, q0), b), __fadd_rn(__fmul_rn(s, q1), b));
    }
    __builtin_nontemporal_store(u32x4_t{o[0], o[1], o[2], o[3]}, dst + i);
  }
}

}  // namespace

hipError_t launch_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                          uint16_t* out, int k, int n, bool f16, hipStream_t stream) {
  const uint32_t chunks_per_row = (uint32_t)(k / 32);
  // Keep each launch's flat chunk index inside 31 bits; split by rows.
  const int64_t max_rows = (int64_t)0x7FFFFFFF / chunks_per_row;
  for (int64_t r0 = 0; r0 < n; r0 += max_rows) {
    const int64_t rows = (n - r0 < max_rows) ? (n - r0) : max_rows;
    const uint32_t total = (uint32_t)(rows * chunks_per_row);
    const u32x4_t* wp = reinterpret_cast<const u32x4_t*>(w + r0 * (k / 8));
    const uint16_t* sp = scales + r0 * (k / 64);
    const uint16_t* bp = biases + r0 * (k / 64);
    u32x4_t* op = reinterpret_cast<u32x4_t*>(out + r0 * (int64_t)k);
    const dim3 grid((total + kThreads - 1) / kThreads);
    if (f16)
      hipLaunchKernelGGL(dequant_kernel<F16Tag>, grid, dim3(kThreads), 0, stream, wp, sp, bp, op,
                         total, chunks_per_row);
    else
      hipLaunchKernelGGL(dequant_kernel<uint16_t>, grid, dim3(kThreads), 0, stream, wp, sp, bp,
                         op, total, chunks_per_row);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace imq
