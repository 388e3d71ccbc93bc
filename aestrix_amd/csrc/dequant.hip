// dequant.hip -- standalone affine 4-bit dequantize for gfx950.
//
// out[n][k] = RNE_T(fl32(scale[n][k/64] * q[n][k] + bias[n][k/64]))
// Restates MLX `dequantized(..., groupSize: 64, bits: 4)` as used by the
// reference (Sources/ImarelloDirect/DirectTEEncoder.swift:106-134).
//
// HBM-bound: 0.5 B of codes + 4/64 B of scale/bias read and 2 B written per
// element.  Rows of W and of the output are contiguous, so a flat word index w
// addresses everything: codes word w, group w / 8 (a row of K/8 words holds
// K/64 groups of 8 words), output bytes [16 w, 16 w + 16).  A workgroup owns
// 1024 consecutive words; lane t of it handles words t, t+256, t+512, t+768,
// so every wave instruction loads 256 contiguous bytes of codes and stores
// 1 KiB of contiguous output.  Rounding is v_cvt_pk_bf16_f32 (RNE), which
// equals the integer formula of DirectTEEncoder.swift:39-43 for every non-NaN
// value; a NaN result (possible only when a scale or bias is itself inf or
// NaN) stays a quiet NaN.
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kThreads = 256;
constexpr int kWordsPerThread = 4;
constexpr int kWordsPerBlock = kThreads * kWordsPerThread;

struct Bf16Out {
  static __device__ __forceinline__ float load(uint16_t h) { return bf16_to_f32(h); }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};

struct F16Out {
  static __device__ __forceinline__ float load(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) {
    // v_cvt_f16_f32 rounds to nearest even (default round mode).
    const uint32_t a = __builtin_bit_cast(uint16_t, (_Float16)lo);
    const uint32_t b = __builtin_bit_cast(uint16_t, (_Float16)hi);
    return a | (b << 16);
  }
};

// out = s * q + b as two rounded operations, never contracted into an fma:
// the product is exact unless it overflows, and then it must stay +-inf as in
// the reference's `scale * q + bias` on Float.
__device__ __forceinline__ float affine(float s, float q, float b) {
#pragma clang fp contract(off)
  const float p = s * q;
  return p + b;
}

template <typename Out>
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint32_t* __restrict__ w,
                                                           const uint16_t* __restrict__ scales,
                                                           const uint16_t* __restrict__ biases,
                                                           u32x4_t* __restrict__ out,
                                                           uint32_t total_words) {
  const uint32_t base = blockIdx.x * (uint32_t)kWordsPerBlock + threadIdx.x;
  uint32_t words[kWordsPerThread];
  uint16_t sb[kWordsPerThread][2];
#pragma unroll
  for (int i = 0; i < kWordsPerThread; ++i) {
    const uint32_t wi = base + (uint32_t)(i * kThreads);
    if (wi < total_words) {
      words[i] = __builtin_nontemporal_load(w + wi);
      sb[i][0] = scales[wi >> 3];
      sb[i][1] = biases[wi >> 3];
    }
  }
#pragma unroll
  for (int i = 0; i < kWordsPerThread; ++i) {
    const uint32_t wi = base + (uint32_t)(i * kThreads);
    if (wi >= total_words) continue;
    const float s = Out::load(sb[i][0]);
    const float b = Out::load(sb[i][1]);
    // Even codes sit in the low nibble of each byte, odd codes in the high
    // nibble; each byte converts with one v_cvt_f32_ubyteN.
    const uint32_t lo = words[i] & 0x0F0F0F0Fu;
    const uint32_t hi = (words[i] >> 4) & 0x0F0F0F0Fu;
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float q0 = (float)((lo >> (8 * p)) & 0xFFu);
      const float q1 = (float)((hi >> (8 * p)) & 0xFFu);
      o[p] = Out::pack(affine(s, q0, b), affine(s, q1, b));
    }
    __builtin_nontemporal_store(u32x4_t{o[0], o[1], o[2], o[3]}, out + wi);
  }
}

}  // namespace

hipError_t launch_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                          uint16_t* out, int k, int n, bool f16, hipStream_t stream) {
  const int64_t total = (int64_t)n * (k / 8);
  // Keep each launch's word index inside 31 bits; split at group boundaries.
  const int64_t max_words = (int64_t)1 << 30;
  for (int64_t w0 = 0; w0 < total; w0 += max_words) {
    const uint32_t words = (uint32_t)((total - w0 < max_words) ? (total - w0) : max_words);
    const dim3 grid((words + kWordsPerBlock - 1) / kWordsPerBlock);
    u32x4_t* op = reinterpret_cast<u32x4_t*>(out) + w0;
    if (f16)
      hipLaunchKernelGGL(dequant_kernel<F16Out>, grid, dim3(kThreads), 0, stream, w + w0,
                         scales + w0 / 8, biases + w0 / 8, op, words);
    else
      hipLaunchKernelGGL(dequant_kernel<Bf16Out>, grid, dim3(kThreads), 0, stream, w + w0,
                         scales + w0 / 8, biases + w0 / 8, op, words);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace imq
