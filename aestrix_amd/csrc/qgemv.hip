// qgemv.hip -- skinny quantized matmul (1 <= M <= 16) for gfx950, no MFMA.
//
// y[m][n] = sum_k x[m][k] * deq(W)[n][k], fp32 accumulation, bf16 output:
// the M <= 16 regime of MLX quantizedMM(transpose: true, groupSize: 64,
// bits: 4) (Sources/ImarelloDiT/AttentionUtils.swift:212-221) and of the
// reference's M=1 conditioner qmm (Sources/ImarelloDirect/DirectConditioner.swift:168-213).
//
// Bandwidth-bound on the packed weight (0.5 B/element).  Layout:
//  * a row of W is owned by G consecutive lanes (G in {8,16,32,64}); lane l of
//    the group reads 16-byte chunks l, l+G, l+2G, ... of the row (32 codes,
//    half a quantization group each), so one wave instruction reads 64/G
//    contiguous row segments of G*16 bytes;
//  * x[M][K-tile] is staged once per workgroup in LDS and read as bf16 pairs;
//  * codes are dequantized in registers to bf16 (the same rounding as the
//    dequantize kernel: RNE_bf16(fl32(s*q + b))) and multiplied with
//    v_dot2_f32_bf16 into fp32 accumulators;
//  * the G partial sums of a row are combined with cross-lane shuffles.
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kUnroll = 8;              // 16-byte chunks in flight per lane
constexpr int kLdsBytesMax = 64 * 1024; // x tile budget per workgroup

template <int MR, int G>
__global__ __launch_bounds__(kThreads) void qgemv_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ y, int K, int N,
                                                         int kt) {
  extern __shared__ u32x4_t xs[];  // [MR][kt / 8] u32x4_t (bf16 x tile)
  constexpr int RPW = 64 / G;    // rows per wave
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int gl = lane & (G - 1);
  const int row = (blockIdx.x * kWaves + wave) * RPW + lane / G;
  const bool row_ok = row < N;
  const int wpr = K >> 3;
  const int gpr = K >> 6;
  const int xs_stride = kt >> 3;  // u32x4_t per x row in LDS
  const size_t rsafe = row_ok ? (size_t)row : 0;
  const u32x4_t* wrow = reinterpret_cast<const u32x4_t*>(w + rsafe * wpr);
  const uint16_t* srow = scales + rsafe * gpr;
  const uint16_t* brow = biases + rsafe * gpr;

  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;

  for (int k0 = 0; k0 < K; k0 += kt) {
    const int ktc = (K - k0 < kt) ? (K - k0) : kt;
    if (k0 > 0) __syncthreads();
    const int vpr = ktc >> 3;  // u32x4_t of x per row in this tile
    for (int i = threadIdx.x; i < MR * vpr; i += kThreads) {
      const int m = i / vpr;
      const int v = i - m * vpr;
      xs[m * xs_stride + v] = *reinterpret_cast<const u32x4_t*>(x + (size_t)m * K + k0 + v * 8);
    }
    __syncthreads();
    if (row_ok) {
      const int nch = ktc >> 5;  // 16-byte chunks of this row inside the tile
      const int c0 = k0 >> 5;
      for (int jb = gl; jb < nch; jb += G * kUnroll) {
        u32x4_t q[kUnroll];
        uint32_t sb[kUnroll][2];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int j = jb + u * G;
          if (j < nch) {
            q[u] = __builtin_nontemporal_load(wrow + c0 + j);
            const int g = (c0 + j) >> 1;
            sb[u][0] = srow[g];
            sb[u][1] = brow[g];
          }
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
          const int j = jb + u * G;
          if (j < nch) {
            const float s = bf16_to_f32(sb[u][0]);
            const float b = bf16_to_f32(sb[u][1]);
            const float s24 = s * 0x1p24f;
            const float s20 = s * 0x1p20f;
            uint32_t wp[16];
            dequant_word_bf16(q[u].x, s24, s20, b, wp + 0);
            dequant_word_bf16(q[u].y, s24, s20, b, wp + 4);
            dequant_word_bf16(q[u].z, s24, s20, b, wp + 8);
            dequant_word_bf16(q[u].w, s24, s20, b, wp + 12);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
              const u32x4_t* xv = xs + m * xs_stride + j * 4;
              float a = acc[m];
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const u32x4_t xx = xv[v];
                a = dot2_bf16(wp[4 * v + 0], xx.x, a);
                a = dot2_bf16(wp[4 * v + 1], xx.y, a);
                a = dot2_bf16(wp[4 * v + 2], xx.z, a);
                a = dot2_bf16(wp[4 * v + 3], xx.w, a);
              }
              acc[m] = a;
            }
          }
        }
      }
    }
  }

#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int off = G >> 1; off > 0; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
  }
  if (row_ok && gl == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m) y[(size_t)m * N + row] = (uint16_t)f32_to_bf16_int(acc[m]);
  }
}

template <int MR, int G>
hipError_t launch_g(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                    uint16_t* y, int k, int n, hipStream_t stream) {
  int kt = (kLdsBytesMax / (2 * MR)) / 64 * 64;
  if (kt > k) kt = k;
  const int rows_per_block = kWaves * (64 / G);
  const dim3 grid((n + rows_per_block - 1) / rows_per_block);
  const size_t lds = (size_t)MR * kt * 2;
  hipLaunchKernelGGL((qgemv_kernel<MR, G>), grid, dim3(kThreads), lds, stream, w, s, b, x, y, k,
                     n, kt);
  return hipGetLastError();
}

template <int MR>
hipError_t launch_m(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                    uint16_t* y, int k, int n, hipStream_t stream) {
  // Lanes per row: enough waves to cover the chip (about 2048 waves), but no
  // more lanes than the row has 16-byte chunks.
  const int chunks = k / 32;
  int g = 16;
  if ((int64_t)n * 16 / 64 < 2048) g = 32;
  if ((int64_t)n * 32 / 64 < 2048) g = 64;
  while (g > 8 && g > chunks) g >>= 1;
  switch (g) {
    case 8: return launch_g<MR, 8>(w, s, b, x, y, k, n, stream);
    case 16: return launch_g<MR, 16>(w, s, b, x, y, k, n, stream);
    case 32: return launch_g<MR, 32>(w, s, b, x, y, k, n, stream);
    default: return launch_g<MR, 64>(w, s, b, x, y, k, n, stream);
  }
}

}  // namespace

hipError_t launch_qgemv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                        const uint16_t* x, uint16_t* y, int k, int n, int m, hipStream_t stream) {
  switch (m) {
#define IMQ_QGEMV_CASE(MR) \
  case MR: return launch_m<MR>(w, scales, biases, x, y, k, n, stream);
    IMQ_QGEMV_CASE(1) IMQ_QGEMV_CASE(2) IMQ_QGEMV_CASE(3) IMQ_QGEMV_CASE(4)
    IMQ_QGEMV_CASE(5) IMQ_QGEMV_CASE(6) IMQ_QGEMV_CASE(7) IMQ_QGEMV_CASE(8)
    IMQ_QGEMV_CASE(9) IMQ_QGEMV_CASE(10) IMQ_QGEMV_CASE(11) IMQ_QGEMV_CASE(12)
    IMQ_QGEMV_CASE(13) IMQ_QGEMV_CASE(14) IMQ_QGEMV_CASE(15) IMQ_QGEMV_CASE(16)
#undef IMQ_QGEMV_CASE
    default: return hipErrorInvalidValue;
  }
}

}  // namespace imq
