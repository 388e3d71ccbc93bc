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

#include <algorithm>
#include <cstdlib>

namespace imq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxU = 8;                 // 16-byte chunks in flight per lane
constexpr int kLdsBytesMax = 64 * 1024;  // x tile budget per workgroup

// LDS position of x piece p (16 bytes) of chunk j (32 elements) is
// 4 j + (p ^ ((j >> 2) & 3)).  The lanes of a row group read chunks j, j+1, ...
// in the same instruction; the swizzle spreads their 16-byte reads over all
// bank groups while the piece index p stays a compile-time constant.
__device__ __forceinline__ int xs_swizzle(int slot) {
  const int j = slot >> 2;
  return (j << 2) | ((slot & 3) ^ ((j >> 2) & 3));
}

// x staging slot idx of a tile: row idx / vpr, 16-byte piece idx % vpr.  The
// load is clamped into the tile (never predicated), the store is guarded.
__device__ __forceinline__ u32x4_t load_x_slot(const uint16_t* x, int K, int k0, int vpr,
                                               int total, int idx) {
  const int i = min(idx, total - 1);
  const int m = i / vpr;
  return *reinterpret_cast<const u32x4_t*>(x + (size_t)m * K + k0 + (i - m * vpr) * 8);
}

__device__ __forceinline__ void store_x_slot(u32x4_t* xs, int stride, int vpr, int total, int idx,
                                             u32x4_t v) {
  if (idx < total) {
    const int m = idx / vpr;
    xs[m * stride + xs_swizzle(idx - m * vpr)] = v;
  }
}

// Loads are never predicated: an index past the end is clamped to the last
// valid chunk (a harmless duplicate read).  Predicated loads make the compiler
// merge the register array through a phi and wait on each load in turn.
template <int MR, int G, int U>
__global__ __launch_bounds__(kThreads) void qgemv_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ y, int K, int N,
                                                         int M, int kt) {
  extern __shared__ u32x4_t xs[];  // [MR][kt / 8] bf16 x tile
  constexpr int RPW = 64 / G;      // rows per wave
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int gl = lane & (G - 1);
  const int row = (blockIdx.x * kWaves + wave) * RPW + lane / G;
  const bool row_ok = row < N;
  const int wpr = K >> 3;
  const int gpr = K >> 6;
  const int xs_stride = kt >> 3;  // u32x4_t per x row in LDS
  // Lanes past the last row read row 0 (in bounds) and never store.
  const size_t rsafe = row_ok ? (size_t)row : 0;
  const u32x4_t* wrow = reinterpret_cast<const u32x4_t*>(w + rsafe * wpr);
  const uint16_t* srow = scales + rsafe * gpr;
  const uint16_t* brow = biases + rsafe * gpr;

  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;

  for (int k0 = 0; k0 < K; k0 += kt) {
    const int ktc = (K - k0 < kt) ? (K - k0) : kt;
    const int nch = ktc >> 5;  // 16-byte chunks of a row inside this tile
    const int c0 = k0 >> 5;
    const int batches = (nch + G * U - 1) / (G * U);  // the same for every lane
    const int vpr = ktc >> 3;       // u32x4_t of x per row in this tile
    const int xtotal = M * vpr;     // u32x4_t of x in this tile (<= 4 rounds of 1024)
    for (int it = 0; it < batches; ++it) {
      const int jb = gl + it * G * U;
      // x loads of the first staging round go out first: the LDS writes that
      // need them then do not wait for the weight loads issued after them.
      u32x4_t xv[4];
      if (it == 0) {
        if (k0 > 0) __syncthreads();  // every wave is done with the previous tile
#pragma unroll
        for (int i = 0; i < 4; ++i) xv[i] = load_x_slot(x, K, k0, vpr, xtotal, tid + i * kThreads);
      }
      u32x4_t q[U];
      uint32_t sv[U], bv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = min(jb + u * G, nch - 1);
        q[u] = __builtin_nontemporal_load(wrow + c0 + j);
        const int g = (c0 + j) >> 1;
        sv[u] = srow[g];
        bv[u] = brow[g];
      }
      if (it == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) store_x_slot(xs, xs_stride, vpr, xtotal, tid + i * kThreads, xv[i]);
        // Further rounds (M * tile > 1024 chunks of x): unrolled, no loop back edge.
#pragma unroll
        for (int r = 1; r < 4; ++r) {
          if (r * 4 * kThreads < xtotal) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              xv[i] = load_x_slot(x, K, k0, vpr, xtotal, tid + (4 * r + i) * kThreads);
#pragma unroll
            for (int i = 0; i < 4; ++i)
              store_x_slot(xs, xs_stride, vpr, xtotal, tid + (4 * r + i) * kThreads, xv[i]);
          }
        }
        __syncthreads();
      }
      if (row_ok) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int j = jb + u * G;
          if (j < nch) {
            const float sc = bf16_to_f32(sv[u]);
            const float bi = bf16_to_f32(bv[u]);
            const float s24 = sc * 0x1p24f;
            const float s20 = sc * 0x1p20f;
            const int swz = (j >> 2) & 3;
            uint32_t wp[16];
            dequant_word_bf16(q[u].x, s24, s20, bi, wp + 0);
            dequant_word_bf16(q[u].y, s24, s20, bi, wp + 4);
            dequant_word_bf16(q[u].z, s24, s20, bi, wp + 8);
            dequant_word_bf16(q[u].w, s24, s20, bi, wp + 12);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
              const u32x4_t* xv = xs + m * xs_stride + j * 4;
              float a = acc[m];
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                const u32x4_t xx = xv[v ^ swz];
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
    for (int m = 0; m < MR; ++m)
      if (m < M) y[(size_t)m * N + row] = (uint16_t)f32_to_bf16_int(acc[m]);
  }
}

// Straight-line variant for the common case: x[0:M][0:K] fits the LDS tile
// and one batch of U chunks per lane covers a row (K <= 32 * G * U).  x is
// staged first, by direct buffer->LDS loads (no registers, so the compiler
// inserts no waits for them); then the weight/scale loads go out; one
// `s_waitcnt vmcnt(3U)` (the x loads are the older ones) and a raw barrier
// make x visible while the weights are still in flight, and the dot products
// of chunk u wait only for chunk u's own loads.
template <int MR, int G, int U>
__global__ __launch_bounds__(kThreads) void qgemv_single_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x, uint16_t* __restrict__ y,
    int K, int N, int M) {
  extern __shared__ u32x4_t xs[];  // [MR][K / 8] bf16 x, swizzled; rounded up to 256 slots
  constexpr int RPW = 64 / G;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gl = lane & (G - 1);
  const int row = (blockIdx.x * kWaves + wave) * RPW + lane / G;
  const bool row_ok = row < N;
  const int gpr = K >> 6;
  const int nch = K >> 5;
  const int vpr = K >> 3;
  const int xtotal = M * vpr;
  const size_t rsafe = row_ok ? (size_t)row : 0;
  const u32x4_t* wrow = reinterpret_cast<const u32x4_t*>(w + rsafe * (K >> 3));
  const uint16_t* srow = scales + rsafe * gpr;
  const uint16_t* brow = biases + rsafe * gpr;

  // 1. x -> LDS.  LDS slot s holds x piece (m, idx) = (s / vpr, s % vpr) with
  //    idx the swizzled position xs_swizzle(4 j + p); slots past the end load
  //    a clamped duplicate into the padding.
  {
    const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)((size_t)M * K * 2));
    for (int base = 0; base < xtotal; base += kThreads) {
      const int sl = min(base + tid, xtotal - 1);
      const int m = sl / vpr;
      const int idx = sl - m * vpr;
      const int j = idx >> 2;
      const int pc = (idx & 3) ^ ((j >> 2) & 3);
      const uint32_t off = (uint32_t)((m * K + j * 32 + pc * 8) * 2);
      load_lds16(xr, off, 0u, xs + base + wave * 64);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // 2. weight chunks and their scales/biases.
  u32x4_t q[U];
  uint32_t sv[U], bv[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = min(gl + u * G, nch - 1);
    q[u] = __builtin_nontemporal_load(wrow + j);
    sv[u] = srow[j >> 1];
    bv[u] = brow[j >> 1];
  }
  __builtin_amdgcn_sched_barrier(0);
  // 3. x visible; the weight loads may still be in flight.
  IMQ_WAIT_VMCNT(3 * U);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  float acc[MR];
#pragma unroll
  for (int m = 0; m < MR; ++m) acc[m] = 0.f;
  // Chunks past the row end (possible only in the last batch) were loaded
  // from a clamped index; their sums are computed and dropped by a select, so
  // every load is consumed in straight-line code (a branch would let the
  // compiler sink the loads behind the barrier and break the vmcnt count).
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int j = min(gl + u * G, nch - 1);
    const bool ok = gl + u * G < nch;
    const float sc = bf16_to_f32(sv[u]);
    const float bi = bf16_to_f32(bv[u]);
    const float s24 = sc * 0x1p24f;
    const float s20 = sc * 0x1p20f;
    const int swz = (j >> 2) & 3;
    uint32_t wp[16];
    dequant_word_bf16(q[u].x, s24, s20, bi, wp + 0);
    dequant_word_bf16(q[u].y, s24, s20, bi, wp + 4);
    dequant_word_bf16(q[u].z, s24, s20, bi, wp + 8);
    dequant_word_bf16(q[u].w, s24, s20, bi, wp + 12);
    // Rows m >= M (M rounded up to MR) repeat row M - 1 and are not stored.
#pragma unroll
    for (int m = 0; m < MR; ++m) {
      const u32x4_t* xp = xs + min(m, M - 1) * vpr + j * 4;
      float a = acc[m];
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const u32x4_t xx = xp[v ^ swz];
        a = dot2_bf16(wp[4 * v + 0], xx.x, a);
        a = dot2_bf16(wp[4 * v + 1], xx.y, a);
        a = dot2_bf16(wp[4 * v + 2], xx.z, a);
        a = dot2_bf16(wp[4 * v + 3], xx.w, a);
      }
      acc[m] = ok ? a : acc[m];
    }
  }
#pragma unroll
  for (int m = 0; m < MR; ++m) {
#pragma unroll
    for (int off = G >> 1; off > 0; off >>= 1) acc[m] += __shfl_xor(acc[m], off, 64);
  }
  if (row_ok && gl == 0) {
#pragma unroll
    for (int m = 0; m < MR; ++m)
      if (m < M) y[(size_t)m * N + row] = (uint16_t)f32_to_bf16_int(acc[m]);
  }
}

template <int MR, int G, int U>
hipError_t launch_u(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                    uint16_t* y, int k, int n, int m, int kt, hipStream_t stream) {
  const int rows_per_block = kWaves * (64 / G);
  const dim3 grid((n + rows_per_block - 1) / rows_per_block);
  if (kt == k && k / 32 <= G * U) {
    // x slots rounded up to whole 256-slot rounds (the DMA padding).
    const size_t slots = ((size_t)m * (k / 8) + kThreads - 1) / kThreads * kThreads;
    const size_t lds = slots * 16;
    hipLaunchKernelGGL((qgemv_single_kernel<MR, G, U>), grid, dim3(kThreads), lds, stream, w, s,
                       b, x, y, k, n, m);
  } else {
    const size_t lds = (size_t)MR * kt * 2;
    hipLaunchKernelGGL((qgemv_kernel<MR, G, U>), grid, dim3(kThreads), lds, stream, w, s, b, x, y,
                       k, n, m, kt);
  }
  return hipGetLastError();
}

template <int MR, int G>
hipError_t launch_g(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                    uint16_t* y, int k, int n, int m, hipStream_t stream) {
  int kt = (kLdsBytesMax / (2 * MR)) / 64 * 64;
  if (kt > k) kt = k;
  int u = (kt / 32 + G - 1) / G;  // chunks per lane for one batch covering the tile
  if (u > kMaxU) u = kMaxU;
  switch (u) {
    case 1: return launch_u<MR, G, 1>(w, s, b, x, y, k, n, m, kt, stream);
    case 2: return launch_u<MR, G, 2>(w, s, b, x, y, k, n, m, kt, stream);
    case 3: return launch_u<MR, G, 3>(w, s, b, x, y, k, n, m, kt, stream);
    case 4: return launch_u<MR, G, 4>(w, s, b, x, y, k, n, m, kt, stream);
    case 5: return launch_u<MR, G, 5>(w, s, b, x, y, k, n, m, kt, stream);
    case 6: return launch_u<MR, G, 6>(w, s, b, x, y, k, n, m, kt, stream);
    case 7: return launch_u<MR, G, 7>(w, s, b, x, y, k, n, m, kt, stream);
    default: return launch_u<MR, G, 8>(w, s, b, x, y, k, n, m, kt, stream);
  }
}

// Lanes per row.  Each candidate G in {16, 32, 64} gives n * G / 64 waves
// and uses nch / (G * U) of its lanes' chunk slots (U = ceil(nch / G));
// pick the one with the most useful waves, counting at most 4096 waves (two
// per SIMD at 64 VGPRs is where more waves stopped helping on the two
// shapes measured: 9728 x 2560 and 2560 x 9728), and prefer G values whose
// U fits the straight-line kernel.  IMQ_QGEMV_LANES=16|32|64 overrides.
int pick_lanes(int k, int n) {
  static const int forced = [] {
    const char* e = getenv("IMQ_QGEMV_LANES");
    const int v = e ? atoi(e) : 0;
    return (v == 16 || v == 32 || v == 64) ? v : 0;
  }();
  if (forced) return forced;
  const int nch = k / 32;
  int best = 16;
  double best_score = -1.0;
  for (int g = 16; g <= 64; g *= 2) {
    const int u = (nch + g - 1) / g;
    const double waves = std::min((double)n * g / 64.0, 4096.0);
    double score = waves * nch / (double)(g * u);
    if (u > kMaxU) score *= 0.5;  // looped kernel
    if (score > best_score * 1.02) {
      best = g;
      best_score = score;
    }
  }
  return best;
}

template <int MR>
hipError_t launch_m(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                    uint16_t* y, int k, int n, int m, hipStream_t stream) {
  switch (pick_lanes(k, n)) {
    case 16: return launch_g<MR, 16>(w, s, b, x, y, k, n, m, stream);
    case 32: return launch_g<MR, 32>(w, s, b, x, y, k, n, m, stream);
    default: return launch_g<MR, 64>(w, s, b, x, y, k, n, m, stream);
  }
}

}  // namespace

hipError_t launch_qgemv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                        const uint16_t* x, uint16_t* y, int k, int n, int m, hipStream_t stream) {
  // M is rounded up to a power of two for the register tile; rows >= M are
  // not stored.
  if (m <= 1) return launch_m<1>(w, scales, biases, x, y, k, n, m, stream);
  if (m <= 2) return launch_m<2>(w, scales, biases, x, y, k, n, m, stream);
  if (m <= 4) return launch_m<4>(w, scales, biases, x, y, k, n, m, stream);
  if (m <= 8) return launch_m<8>(w, scales, biases, x, y, k, n, m, stream);
  if (m <= 16) return launch_m<16>(w, scales, biases, x, y, k, n, m, stream);
  return hipErrorInvalidValue;
}

}  // namespace imq
