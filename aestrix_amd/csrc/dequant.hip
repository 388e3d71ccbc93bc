// dequant.hip -- standalone affine 4-bit dequantize for gfx950.
//
// out[n][k] = RNE_T(fl32(scale[n][k/64] * q[n][k] + bias[n][k/64]))
// Restates MLX `dequantized(..., groupSize: 64, bits: 4)` as used by the
// reference (Sources/ImarelloDirect/DirectTEEncoder.swift:106-134).  T is
// bf16, f16 or f32 (f32: out = fl32(s*q + b)); scales, biases and out share T.
//
// HBM-bound: 0.5 B of codes + 4/64 B of scale/bias read and 2 B written per
// element (bf16/f16).  Rows of W and of the output are contiguous, so a flat word index w
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
  using S = uint16_t;
  static constexpr int kWordBytes = 16;  // output bytes per packed word
  static __device__ __forceinline__ float load(S h) { return bf16_to_f32(h); }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};

struct F16Out {
  using S = uint16_t;
  static constexpr int kWordBytes = 16;
  static __device__ __forceinline__ float load(S h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

struct F32Out {
  using S = float;
  static constexpr int kWordBytes = 32;
  static __device__ __forceinline__ float load(S v) { return v; }
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
                                                           const typename Out::S* __restrict__ scales,
                                                           const typename Out::S* __restrict__ biases,
                                                           u32x4_t* __restrict__ out,
                                                           uint32_t total_words) {
  const uint32_t base = blockIdx.x * (uint32_t)kWordsPerBlock + threadIdx.x;
  uint32_t words[kWordsPerThread];
  typename Out::S sb[kWordsPerThread][2];
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
    if constexpr (Out::kWordBytes == 16) {
      uint32_t o[4];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        const float q0 = (float)((lo >> (8 * p)) & 0xFFu);
        const float q1 = (float)((hi >> (8 * p)) & 0xFFu);
        o[p] = Out::pack(affine(s, q0, b), affine(s, q1, b));
      }
      __builtin_nontemporal_store(u32x4_t{o[0], o[1], o[2], o[3]}, out + wi);
    } else {
      uint32_t o[8];
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        o[2 * p] = __float_as_uint(affine(s, (float)((lo >> (8 * p)) & 0xFFu), b));
        o[2 * p + 1] = __float_as_uint(affine(s, (float)((hi >> (8 * p)) & 0xFFu), b));
      }
      __builtin_nontemporal_store(u32x4_t{o[0], o[1], o[2], o[3]}, out + 2 * wi);
      __builtin_nontemporal_store(u32x4_t{o[4], o[5], o[6], o[7]}, out + 2 * wi + 1);
    }
  }
}

// The same arithmetic with one quantization group per thread (16-bit T): the
// group's 8 packed words in two 16-byte loads and its scale and bias in one
// load each, against twelve loads per 64 output bytes in the per-word form
// (whose texture path was busy for most of the kernel).  A thread's 128
// output bytes are staged in LDS and read back so that each wave store writes
// 1 KiB contiguous; a group's 16-byte piece i sits in slot i ^ (group % 8) of
// its row, so neither the writes (16 lanes: 16 rows, one piece each) nor the
// reads (16 lanes: two rows) meet in a bank.  Groups past the end load a
// clamped duplicate and store nothing.  GATHER: output group g is group
// g % gpr of W's row rows[g / gpr] (the rows form below), the id clamped to
// [0, n) so that a bad id never reads outside W.
constexpr int kStageRow = 8;  // 16-byte LDS slots per group

template <typename Out, bool GATHER = false>
__global__ __launch_bounds__(kThreads) void dequant_group_kernel(
    const uint32_t* __restrict__ w, const typename Out::S* __restrict__ scales,
    const typename Out::S* __restrict__ biases, u32x4_t* __restrict__ out, uint32_t groups,
    const int32_t* __restrict__ rows = nullptr, uint32_t gpr = 0, int n = 0) {
  static_assert(Out::kWordBytes == 16, "16-bit outputs");
  __shared__ u32x4_t stage[kThreads * kStageRow];
  const uint32_t g0 = blockIdx.x * (uint32_t)kThreads;
  const uint32_t go = min(g0 + threadIdx.x, groups - 1);
  size_t g = go;  // the source group
  if constexpr (GATHER) {
    const uint32_t r = go / gpr;
    const int id = min(max(rows[r], 0), n - 1);
    g = (size_t)id * gpr + (go - r * gpr);
  }
  const u32x4_t* wp = reinterpret_cast<const u32x4_t*>(w) + 2 * g;
  const u32x4_t c0 = __builtin_nontemporal_load(wp);
  const u32x4_t c1 = __builtin_nontemporal_load(wp + 1);
  const float s = Out::load(scales[g]);
  const float b = Out::load(biases[g]);
  const uint32_t words[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  u32x4_t* row = stage + threadIdx.x * kStageRow;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t lo = words[i] & 0x0F0F0F0Fu;
    const uint32_t hi = (words[i] >> 4) & 0x0F0F0F0Fu;
    uint32_t o[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float q0 = (float)((lo >> (8 * p)) & 0xFFu);
      const float q1 = (float)((hi >> (8 * p)) & 0xFFu);
      o[p] = Out::pack(affine(s, q0, b), affine(s, q1, b));
    }
    row[i ^ (threadIdx.x & 7)] = u32x4_t{o[0], o[1], o[2], o[3]};
  }
  __syncthreads();
  // Wave v's 64 groups are 8 KiB of contiguous output; its store j covers
  // bytes [1 KiB j, 1 KiB (j + 1)): lane l takes 16 bytes of group 8 j + l / 8.
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int grp = 64 * wv + 8 * j + (lane >> 3);
    if (g0 + (uint32_t)grp < groups)
      __builtin_nontemporal_store(stage[grp * kStageRow + ((lane ^ grp) & 7)],
                                  out + (size_t)(g0 + (uint32_t)grp) * 8 + (lane & 7));
  }
}

// Rows gathered by index (DirectTEEncoder.embedRow, :106-123, for a batch of
// token ids): output row r is deq(W[rows[r]]); ids are clamped to [0, n) so a
// bad id never reads outside W.  One thread per packed word, as above.
template <typename Out>
__global__ __launch_bounds__(kThreads) void dequant_rows_kernel(
    const uint32_t* __restrict__ w, const typename Out::S* __restrict__ scales,
    const typename Out::S* __restrict__ biases, const int32_t* __restrict__ rows,
    u32x4_t* __restrict__ out, uint32_t total_words, uint32_t wpr, int n) {
  const uint32_t o = blockIdx.x * (uint32_t)kThreads + threadIdx.x;
  if (o >= total_words) return;
  const uint32_t r = o / wpr, j = o - r * wpr;
  const int id = min(max(rows[r], 0), n - 1);
  const size_t wi = (size_t)id * wpr + j;
  const uint32_t word = __builtin_nontemporal_load(w + wi);
  const float s = Out::load(scales[wi >> 3]);
  const float b = Out::load(biases[wi >> 3]);
  const uint32_t lo = word & 0x0F0F0F0Fu;
  const uint32_t hi = (word >> 4) & 0x0F0F0F0Fu;
  if constexpr (Out::kWordBytes == 16) {
    uint32_t v[4];
#pragma unroll
    for (int p = 0; p < 4; ++p)
      v[p] = Out::pack(affine(s, (float)((lo >> (8 * p)) & 0xFFu), b),
                       affine(s, (float)((hi >> (8 * p)) & 0xFFu), b));
    out[o] = u32x4_t{v[0], v[1], v[2], v[3]};
  } else {
    uint32_t v[8];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      v[2 * p] = __float_as_uint(affine(s, (float)((lo >> (8 * p)) & 0xFFu), b));
      v[2 * p + 1] = __float_as_uint(affine(s, (float)((hi >> (8 * p)) & 0xFFu), b));
    }
    out[2 * o] = u32x4_t{v[0], v[1], v[2], v[3]};
    out[2 * o + 1] = u32x4_t{v[4], v[5], v[6], v[7]};
  }
}

template <typename Out>
hipError_t launch_rows_out(const uint32_t* w, const void* scales, const void* biases,
                           const int32_t* rows, int count, void* out, int k, int n,
                           hipStream_t stream) {
  using S = typename Out::S;
  const uint32_t wpr = (uint32_t)(k / 8), total = (uint32_t)count * wpr;
  // The grouped kernel loads 16 bytes of codes at a time: W 16-byte aligned
  // (the entry point asks only for 4).
  if constexpr (Out::kWordBytes == 16) {
    if (((uintptr_t)w & 15u) == 0) {
      const uint32_t gpr = wpr / 8, groups = (uint32_t)count * gpr;  // K % 64 == 0
      hipLaunchKernelGGL((dequant_group_kernel<Out, true>),
                         dim3((groups + kThreads - 1) / kThreads), dim3(kThreads), 0, stream, w,
                         static_cast<const S*>(scales), static_cast<const S*>(biases),
                         static_cast<u32x4_t*>(out), groups, rows, gpr, n);
      return hipGetLastError();
    }
  }
  hipLaunchKernelGGL(dequant_rows_kernel<Out>, dim3((total + kThreads - 1) / kThreads),
                     dim3(kThreads), 0, stream, w, static_cast<const S*>(scales),
                     static_cast<const S*>(biases), rows, static_cast<u32x4_t*>(out), total, wpr, n);
  return hipGetLastError();
}

template <typename Out>
hipError_t launch_out(const uint32_t* w, const void* scales, const void* biases, void* out,
                      int64_t total, hipStream_t stream) {
  using S = typename Out::S;
  // Keep each launch's word index inside 31 bits; split at group boundaries.
  const int64_t max_words = (int64_t)1 << 30;
  for (int64_t w0 = 0; w0 < total; w0 += max_words) {
    const uint32_t words = (uint32_t)((total - w0 < max_words) ? (total - w0) : max_words);
    const dim3 grid((words + kWordsPerBlock - 1) / kWordsPerBlock);
    u32x4_t* op = reinterpret_cast<u32x4_t*>(out) + w0 * (Out::kWordBytes / 16);
    if constexpr (Out::kWordBytes == 16) {
      const uint32_t groups = words / 8;  // rows hold whole groups: K % 64 == 0
      hipLaunchKernelGGL(dequant_group_kernel<Out>, dim3((groups + kThreads - 1) / kThreads),
                         dim3(kThreads), 0, stream, w + w0,
                         static_cast<const S*>(scales) + w0 / 8,
                         static_cast<const S*>(biases) + w0 / 8, op, groups);
    } else {
      hipLaunchKernelGGL(dequant_kernel<Out>, grid, dim3(kThreads), 0, stream, w + w0,
                         static_cast<const S*>(scales) + w0 / 8,
                         static_cast<const S*>(biases) + w0 / 8, op, words);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace

hipError_t launch_dequant_rows(const uint32_t* w, const void* scales, const void* biases,
                               const int32_t* rows, int count, void* out, int k, int n, int dtype,
                               hipStream_t stream) {
  if (count <= 0) return hipSuccess;
  switch (dtype) {
    case kBf16: return launch_rows_out<Bf16Out>(w, scales, biases, rows, count, out, k, n, stream);
    case kF16: return launch_rows_out<F16Out>(w, scales, biases, rows, count, out, k, n, stream);
    case kF32: return launch_rows_out<F32Out>(w, scales, biases, rows, count, out, k, n, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dequant(const uint32_t* w, const void* scales, const void* biases, void* out,
                          int k, int n, int dtype, hipStream_t stream) {
  const int64_t total = (int64_t)n * (k / 8);
  switch (dtype) {
    case kBf16: return launch_out<Bf16Out>(w, scales, biases, out, total, stream);
    case kF16: return launch_out<F16Out>(w, scales, biases, out, total, stream);
    case kF32: return launch_out<F32Out>(w, scales, biases, out, total, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace imq
