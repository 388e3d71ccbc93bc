// qgemv.hip -- skinny quantized matmul (1 <= M <= 16) for gfx950, no MFMA.
//
// y[m][n] = sum_k x[m][k] * deq(W)[n][k], fp32 accumulation, output in T:
// the M <= 16 regime of MLX quantizedMM(transpose: true, groupSize: 64,
// bits: 4) (Sources/ImarelloDiT/AttentionUtils.swift:212-221) and of the
// reference's M=1 conditioner qmm with f32 x, scales, biases and y
// (Sources/ImarelloDirect/DirectConditioner.swift:48,75-84,168-213).
// T in {bf16, f16, f32}; x, scales, biases and y share T.
//
// Bandwidth-bound on the packed weight (0.5 B/element) at small M; the fp32
// dot products (0.5 v_dot2 per element and row of x) take over towards M = 16.
// Layout:
//  * R consecutive rows of W are owned by G consecutive lanes (G in
//    {16, 32, 64}, R = 1 for M <= 4, 2 above); lane l of the group reads 16-byte
//    chunks l, l+G, l+2G, ... of each of its rows (32 codes, half a
//    quantization group each), so one wave instruction reads 64/G contiguous
//    row segments of G*16 bytes;
//  * x[M][K-tile] is staged per workgroup in LDS by direct buffer->LDS loads;
//    each x read feeds all R rows of the lane;
//  * codes are dequantized in registers to T (the dequantize kernel's
//    rounding, RNE_T(fl32(s*q + b)); for f32 the weight is fl32(s*q + b)) and
//    multiplied into fp32 accumulators with v_dot2_f32_bf16 / v_dot2_f32_f16
//    (16-bit T) or fma (f32);
//  * the G partial sums of a row are combined with DPP adds.
#include "epilogue.hpp"
#include "imq_device.hpp"
#include "imq_kernels.hpp"

#include <algorithm>
#include <cstdlib>

namespace imq {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLdsBudget = 64 * 1024;  // x tile bytes per workgroup

// Rows per lane and the most 16-byte chunks per row a lane keeps in flight.
constexpr int rows_per_lane(int mr) { return mr >= 8 ? 2 : 1; }
constexpr int max_chunks(int mr) { return mr >= 8 ? 4 : 8; }

// One K tile of x in LDS, in 16-byte pieces (EPP = 16 / sizeof(T) elements;
// P = 32 / EPP pieces per chunk of 32 elements): row m, piece p of chunk j
// sits at slot m * vpr + P j + (p ^ f(j)), vpr = tile length / EPP, with
// f(j) = (j >> 2) & 3 for 16-bit T and (j >> 1) & 7 for f32.  The lanes of a
// row group read chunks j, j+1, ... in the same instruction; the swizzle
// spreads their 16-byte reads over all bank groups while p stays a
// compile-time constant in the reader.
//
// Per tile: x goes first, by buffer->LDS loads (no registers, so the compiler
// adds no waits for them); then every weight/scale load of the tile; one
// `s_waitcnt vmcnt(3 U R)` (the x loads are the older ones) and a barrier make
// x visible while the weights are still in flight, and the dot products of
// chunk u wait only for chunk u's own loads.  Loads are never predicated: an
// index past the end is clamped (a duplicate read) and its sum dropped by a
// select, so every load is consumed in straight-line code.
template <int T>
struct XTile {
  static constexpr int kEpp = 16 / Elem<T>::kBytes;  // elements per 16-byte piece
  static constexpr int kP = 32 / kEpp;               // pieces per chunk
  static constexpr int kSh = (kP == 4) ? 2 : 1;
  static __device__ __forceinline__ int swz(int j) { return (j >> kSh) & (kP - 1); }
};

// Byte offset within the tile of row m's chunk j, already XORed with its
// swizzle: piece v of the chunk is at that offset ^ 16 v.  A chunk's P pieces
// start at a multiple of 16 P (rows are kl / 32 whole chunks long), so the
// swizzle of every piece is one XOR of this offset.
template <int T>
__device__ __forceinline__ uint32_t x_piece0(int m, int M, int vpr, int j, int swz) {
  return (uint32_t)(min(m, M - 1) * vpr + j * XTile<T>::kP + swz) * 16u;
}

__device__ __forceinline__ u32x4_t x_piece(const u32x4_t* xs, uint32_t xo, int v) {
  return *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(xs) +
                                           (xo ^ (uint32_t)(16 * v)));
}

// One scale or bias of T at byte offset voff + soff.
template <int T>
__device__ __forceinline__ typename Elem<T>::S load_param(__amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                                          uint32_t soff) {
  if constexpr (T == kF32)
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, voff, soff, 0));
  else
    return __builtin_amdgcn_raw_buffer_load_b16(rs, voff, soff, 0);
}

// 16 weight bytes, streamed (non-temporal: bit 1 of the cache policy).
__device__ __forceinline__ u32x4_t load_b128_nt(__amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                               uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 2));
}

// v plus the DPP-permuted v of the lanes in rows `rows` (16-lane rows of
// the wave); other lanes add 0.
template <int kCtrl, int kRows = 0xF>
__device__ __forceinline__ float add_dpp(float v) {
  return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                   kCtrl, kRows, 0xF, false));
}

// Sum of v over each aligned group of G lanes (G in {16, 32, 64}) by DPP
// adds, no LDS traffic: quad swaps, half-row and row mirrors give every lane
// its 16-lane row's sum; row_bcast15 adds row 0 (2) into row 1 (3), and
// row_bcast31 adds rows 0-1 into rows 2-3.  The group's total is then held by
// the lanes of its last row, among them lane G - 1 of the group.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  v = add_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v = add_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v = add_dpp<0x141>(v);  // row_half_mirror
  v = add_dpp<0x140>(v);  // row_mirror
  if constexpr (G >= 32) v = add_dpp<0x142, 0xA>(v);  // row_bcast15 into rows 1, 3
  if constexpr (G == 64) v = add_dpp<0x143, 0xC>(v);  // row_bcast31 into rows 2, 3
  return v;
}

// A gate/up pair of rows per lane group (the SwiGLU mode): output j of row m
// is y[m][j] (row pitch ldy) = T(g * sigmoid(g) * u * out_scale), g and u the
// T-rounded products of x row m with weight rows gate_row + j and up_row + j
// times in_scale -- the qmm followed by dq_silu_mul / dd_swiglu_pitched
// (Sources/ImarelloDirect/DirectGlueKernels.swift:77-88,
// DirectDiTKernels.swift:137-157), computed by EpSwiGLU.
// width 0: no pair; then a non-null resid makes the plain store
// y = T(float(resid) + float(T(acc))) (EpResidAdd's arithmetic, 16-bit T).
struct GvPair {
  int gate_row, up_row, width, ldy;
  float in_scale, out_scale;
  const void* resid = nullptr;
  // Non-null: x is RMSNorm'd in LDS before the products (x tile = whole rows).
  const float* norm_w = nullptr;
  float eps = 0.f;
};

bool is_pair(const GvPair* pr) { return pr && pr->width > 0; }

// RMSNorm of the staged x rows in place: row m becomes T(x * rsqrt(mean(x^2)
// + eps) * nw) with the arithmetic of the T-input RMSNorm kernel's 16-byte
// form (rmsnorm_tin_vec_kernel, norm.hip): thread t takes the 8-value pieces
// t and t + 256 of the row in that order, fma of each value's square, the
// same xor-shuffle tree in the wave, the four wave sums added in order from
// zero, __frsqrt_rn, and (x * inv) * w rounded to T per value -- so the
// products see bit for bit the values the separate RMSNorm launch would
// write.  The tile must hold whole rows (one K tile) of 16-bit T with at most
// 512 pieces; the norm weights of the thread's pieces (nwv, loaded beside the
// x staging) are already in registers.
template <int T, int MR>
__device__ __forceinline__ void norm_rows_in_lds(u32x4_t* xs, int M, int K, int vpr,
                                                 const float4 (&nwv)[2][2], float eps) {
  using E = Elem<T>;
  using X = XTile<T>;
  static_assert(X::kP == 4, "16-bit T: four 16-byte pieces per chunk of 32 values");
  __shared__ float npart[MR][kWaves];
  const int tid = threadIdx.x;
  const int n8 = K >> 3;
  auto slot = [&](int m, int e) { return m * vpr + (e >> 2) * 4 + ((e & 3) ^ X::swz(e >> 2)); };
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m >= M) break;
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + i * kThreads;
      if (e >= n8) break;
      const u32x4_t v = xs[slot(m, e)];
      const uint32_t q[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float lo = E::param((uint16_t)(q[j] & 0xFFFFu));
        const float hi = E::param((uint16_t)(q[j] >> 16));
        acc = __builtin_fmaf(lo, lo, acc);
        acc = __builtin_fmaf(hi, hi, acc);
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
    if ((tid & 63) == 0) npart[m][tid >> 6] = acc;
  }
  __syncthreads();
#pragma unroll
  for (int m = 0; m < MR; ++m) {
    if (m >= M) break;
    float total = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) total += npart[m][i];
    const float inv = __frsqrt_rn(total / (float)K + eps);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int e = tid + i * kThreads;
      if (e >= n8) break;
      const float ww[8] = {nwv[i][0].x, nwv[i][0].y, nwv[i][0].z, nwv[i][0].w,
                           nwv[i][1].x, nwv[i][1].y, nwv[i][1].z, nwv[i][1].w};
      u32x4_t& v = xs[slot(m, e)];
      const uint32_t q[4] = {v.x, v.y, v.z, v.w};
      uint32_t o[4];
#pragma unroll
      for (int j = 0; j < 4; ++j)
        o[j] = E::pack2(E::param((uint16_t)(q[j] & 0xFFFFu)) * inv * ww[2 * j],
                        E::param((uint16_t)(q[j] >> 16)) * inv * ww[2 * j + 1]);
      v = u32x4_t{o[0], o[1], o[2], o[3]};
    }
  }
  __syncthreads();
}

// NORM: x is RMSNorm'd in LDS (pr.norm_w) -- a template switch, so the other
// forms carry none of its set-up.
template <int T, int MR, int G, int U, int R, bool PAIR, bool NORM = false>
__global__ __launch_bounds__(kThreads) void qgemv_kernel(
    const uint32_t* __restrict__ w, const typename Elem<T>::S* __restrict__ scales,
    const typename Elem<T>::S* __restrict__ biases, const typename Elem<T>::S* __restrict__ x,
    typename Elem<T>::S* __restrict__ y, int K, int N, int M, int kt, const GvPair pr) {
  static_assert(!PAIR || R == 2, "a gate/up pair is two rows per lane group");
  static_assert(!NORM || (T != kF32 && MR <= 2), "the x norm: 16-bit T, at most two rows");
  using E = Elem<T>;
  using X = XTile<T>;
  constexpr int P = X::kP;
  extern __shared__ u32x4_t xs[];  // x tile, padded to whole 256-slot rounds
  constexpr int RPW = 64 / G * R;  // rows per wave
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gl = lane & (G - 1);
  const int row0 = (blockIdx.x * kWaves + wave) * RPW + (lane / G) * R;
  const int pj = (blockIdx.x * kWaves + wave) * (64 / G) + lane / G;  // PAIR: output column
  const int gpr = K >> 6;
  if constexpr (MR == 1) M = 1;  // lets the compiler drop the row arithmetic of x

  // Weights, scales and biases through buffer resources: one 32-bit byte
  // offset per row, the chunk offset added per load (the host keeps every
  // operand under 2 GiB).
  const __amdgpu_buffer_rsrc_t wr = make_rsrc(w, (uint32_t)((size_t)N * K / 2));
  const __amdgpu_buffer_rsrc_t sr = make_rsrc(scales, (uint32_t)((size_t)N * gpr * E::kBytes));
  const __amdgpu_buffer_rsrc_t br = make_rsrc(biases, (uint32_t)((size_t)N * gpr * E::kBytes));
  uint32_t woff[R], poff[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    uint32_t rr = (uint32_t)min(row0 + r, N - 1);
    if constexpr (PAIR)
      rr = (uint32_t)min((r == 0 ? pr.gate_row : pr.up_row) + min(pj, pr.width - 1), N - 1);
    woff[r] = rr * (uint32_t)(K / 2);
    poff[r] = rr * (uint32_t)gpr * E::kBytes;
  }
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(x, (uint32_t)((size_t)M * K * E::kBytes));

  float acc[R][MR];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = 0.f;
  [[maybe_unused]] float nz = 0.f;  // f32 dequant's -0 product addend
  if constexpr (T == kF32) nz = opaque_neg_zero();

  for (int k0 = 0; k0 < K; k0 += kt) {
    const int kl = min(kt, K - k0);  // tile length
    const int vpr = kl / X::kEpp;
    const int tch = kl >> 5;         // chunks in the tile
    const int c0 = k0 >> 5;
    const int xtotal = M * vpr;
    if (k0 > 0) __builtin_amdgcn_s_barrier();  // readers of the previous tile are done

    // 1. x tile -> LDS.  Slot s holds x piece (m, idx) = (s / vpr, s % vpr)
    //    at the swizzled position; slots past the end load a clamped
    //    duplicate into the padding.
    for (int base = 0; base < xtotal; base += kThreads) {
      // Unsigned: the slot indices are non-negative, and signed division by
      // a power of two costs three more instructions.
      const unsigned sl = (unsigned)min(base + tid, xtotal - 1);
      const unsigned m = (MR == 1) ? 0u : sl / (unsigned)vpr;
      const unsigned idx = sl - m * (unsigned)vpr;
      const int j = (int)(idx / (unsigned)P);
      const int pc = (int)(idx & (unsigned)(P - 1)) ^ X::swz(j);
      const uint32_t off = (uint32_t)(((int)m * K + k0 + j * 32 + pc * X::kEpp) * E::kBytes);
      load_lds16(xr, off, 0u, xs + base + wave * 64);
    }
    // The norm weights of this thread's pieces (clamped indices: no branch
    // around the loads), beside the x staging and ahead of the weights.
    float4 nwv[2][2];
    if constexpr (NORM) {
      const float4* nr = reinterpret_cast<const float4*>(pr.norm_w);
      const int n8 = K >> 3;
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int e = min(tid + i * kThreads, n8 - 1);
        nwv[i][0] = nr[2 * e];
        nwv[i][1] = nr[2 * e + 1];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    // 2. weight chunks and their scales/biases, chunk by chunk: loads retire
    //    in issue order, so chunk u's dot products then wait for chunk u's
    //    loads only (grouping all weight loads first made the first chunk
    //    wait for every weight load of the tile).
    u32x4_t q[R][U];
    typename E::S sv[R][U], bv[R][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t c = (uint32_t)min(gl + u * G, tch - 1);  // chunk within the tile
#pragma unroll
      for (int r = 0; r < R; ++r) {
        sv[r][u] = load_param<T>(sr, poff[r] + (c >> 1) * E::kBytes, (uint32_t)(c0 >> 1) * E::kBytes);
        bv[r][u] = load_param<T>(br, poff[r] + (c >> 1) * E::kBytes, (uint32_t)(c0 >> 1) * E::kBytes);
        q[r][u] = load_b128_nt(wr, woff[r] + c * 16u, (uint32_t)c0 * 16u);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // 3. x visible; the weight loads may still be in flight.
    IMQ_WAIT_VMCNT(3 * U * R);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (NORM) {
      // RMSNorm'd x (the host passes a norm weight only when the tile is the
      // whole row); its LDS traffic runs while the weights are in flight.
      norm_rows_in_lds<T, MR>(xs, M, K, vpr, nwv, pr.eps);
      __builtin_amdgcn_sched_barrier(0);
    }

#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = min(gl + u * G, tch - 1);
      const bool ok = gl + u * G < tch;
      const int swz = X::swz(j);
      // Rows m >= M (M rounded up to MR) repeat row M - 1 and are not stored.
      if constexpr (T == kF32) {
        float wf[R][32];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float sc = E::param(sv[r][u]);
          const float bi = E::param(bv[r][u]);
          dequant_word_f32(q[r][u].x, sc * 0x1p24f, sc * 0x1p20f, bi, nz, wf[r] + 0);
          dequant_word_f32(q[r][u].y, sc * 0x1p24f, sc * 0x1p20f, bi, nz, wf[r] + 8);
          dequant_word_f32(q[r][u].z, sc * 0x1p24f, sc * 0x1p20f, bi, nz, wf[r] + 16);
          dequant_word_f32(q[r][u].w, sc * 0x1p24f, sc * 0x1p20f, bi, nz, wf[r] + 24);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const uint32_t xo = x_piece0<T>(m, M, vpr, j, swz);
          float a[R];
#pragma unroll
          for (int r = 0; r < R; ++r) a[r] = acc[r][m];
#pragma unroll
          for (int v = 0; v < P; ++v) {
            const u32x4_t xx = x_piece(xs, xo, v);
#pragma unroll
            for (int r = 0; r < R; ++r) {
              a[r] = __builtin_fmaf(wf[r][4 * v + 0], __uint_as_float(xx.x), a[r]);
              a[r] = __builtin_fmaf(wf[r][4 * v + 1], __uint_as_float(xx.y), a[r]);
              a[r] = __builtin_fmaf(wf[r][4 * v + 2], __uint_as_float(xx.z), a[r]);
              a[r] = __builtin_fmaf(wf[r][4 * v + 3], __uint_as_float(xx.w), a[r]);
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r][m] = ok ? a[r] : acc[r][m];
        }
      } else {
        uint32_t wp[R][16];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const float sc = E::param(sv[r][u]);
          const float bi = E::param(bv[r][u]);
          const float s24 = sc * 0x1p24f;
          const float s20 = sc * 0x1p20f;
          E::dequant(q[r][u].x, s24, s20, bi, wp[r] + 0);
          E::dequant(q[r][u].y, s24, s20, bi, wp[r] + 4);
          E::dequant(q[r][u].z, s24, s20, bi, wp[r] + 8);
          E::dequant(q[r][u].w, s24, s20, bi, wp[r] + 12);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          const uint32_t xo = x_piece0<T>(m, M, vpr, j, swz);
          float a[R];
#pragma unroll
          for (int r = 0; r < R; ++r) a[r] = acc[r][m];
#pragma unroll
          for (int v = 0; v < P; ++v) {
            const u32x4_t xx = x_piece(xs, xo, v);
#pragma unroll
            for (int r = 0; r < R; ++r) {
              if constexpr (T == kBf16) {
                a[r] = dot2_bf16(wp[r][4 * v + 0], xx.x, a[r]);
                a[r] = dot2_bf16(wp[r][4 * v + 1], xx.y, a[r]);
                a[r] = dot2_bf16(wp[r][4 * v + 2], xx.z, a[r]);
                a[r] = dot2_bf16(wp[r][4 * v + 3], xx.w, a[r]);
              } else {
                a[r] = dot2_f16(wp[r][4 * v + 0], xx.x, a[r]);
                a[r] = dot2_f16(wp[r][4 * v + 1], xx.y, a[r]);
                a[r] = dot2_f16(wp[r][4 * v + 2], xx.z, a[r]);
                a[r] = dot2_f16(wp[r][4 * v + 3], xx.w, a[r]);
              }
            }
          }
#pragma unroll
          for (int r = 0; r < R; ++r) acc[r][m] = ok ? a[r] : acc[r][m];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MR; ++m) acc[r][m] = group_sum<G>(acc[r][m]);
  if constexpr (PAIR) {
    if (gl == G - 1 && pj < pr.width) {
      const EpSwiGLU<T> ep{nullptr, 0, 0, 0, 0, pr.in_scale, pr.out_scale, false};
#pragma unroll
      for (int m = 0; m < MR; ++m)
        if (m < M) y[(size_t)m * pr.ldy + pj] = E::out(ep.value2(acc[0][m], acc[1][m]));
    }
  } else if (gl == G - 1) {
    const auto* rs = static_cast<const typename E::S*>(pr.resid);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (row0 + r < N) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
          if (m < M) {
            const size_t i = (size_t)m * N + row0 + r;
            float v = acc[r][m];
            if constexpr (T != kF32) {
              if (rs) v = staged_value<T>(rs[i]) + round_to(v, T);
            }
            y[i] = E::out(v);
          }
        }
      }
    }
  }
}

// Plan for one call: lanes per row G, K tile length kt, chunks per lane U.
struct Plan {
  int g, kt, u;
};

// K tiles: as long as the LDS budget and U <= max_chunks allow, then evened
// out so the last tile is not a sliver.
int tile_len(int k, int mr, int g, int eb) {
  const int by_lds = (kLdsBudget / (eb * mr)) / 64 * 64;
  const int by_u = 32 * g * max_chunks(mr);
  const int cap = std::min(by_lds, by_u);
  const int tiles = (k + cap - 1) / cap;
  const int even = ((k + tiles - 1) / tiles + 63) / 64 * 64;
  return std::min(even, k);
}

// Each candidate G gives n * G / (64 R) waves and uses tch / (G U) of its
// lanes' chunk slots per tile; pick the one with the most useful waves,
// counting at most 4096 for M <= 4, 2048 for M <= 8 and 1024 above: beyond
// those counts more waves stopped paying for idle lanes (a sweep of every G
// on 9728 x 2560 and 2560 x 9728 at M = 1, 2, 4, 8, 16 picks the fastest G
// in all ten cases with these caps).  Candidates are tried 32, 64, 16, so a
// tie goes to 32 lanes: M = 1 [18432 x 3072] scores 16 and 32 alike and runs
// in 8.6 us at 32 against 9.0 at 16 (weights from HBM; [9728 x 2560] 5.6 /
// 6.1 / 7.2 us at 32 / 16 / 64).
// IMQ_QGEMV_LANES=16|32|64 overrides.
Plan make_plan(int k, int n, int mr, int eb, int r_override = 0) {
  static const int forced = [] {
    const char* e = getenv("IMQ_QGEMV_LANES");
    const int v = e ? atoi(e) : 0;
    return (v == 16 || v == 32 || v == 64) ? v : 0;
  }();
  const int r = r_override ? r_override : rows_per_lane(mr);
  Plan best{16, 0, 0};
  double best_score = -1.0;
  for (int g : {32, 64, 16}) {
    if (forced && g != forced) continue;
    const int kt = tile_len(k, mr, g, eb);
    const int tch = kt / 32;
    const int u = (tch + g - 1) / g;
    const double cap = mr <= 4 ? 4096.0 : mr <= 8 ? 2048.0 : 1024.0;
    const double waves = std::min((double)n * g / (64.0 * r), cap);
    const double score = waves * tch / (double)(g * u);
    if (score > best_score * 1.02) {
      best = Plan{g, kt, u};
      best_score = score;
    }
  }
  return best;
}

template <int T, int MR, int G, int U>
hipError_t launch_u(const uint32_t* w, const void* s, const void* b, const void* x, void* y, int k,
                    int n, int m, int kt, const GvPair* pr, hipStream_t stream) {
  using ST = typename Elem<T>::S;
  // x slots of the longest tile, rounded up to whole 256-slot rounds.
  const size_t pieces = (size_t)m * kt / XTile<T>::kEpp;
  const size_t slots = (pieces + kThreads - 1) / kThreads * kThreads;
  if (is_pair(pr)) {
    if constexpr (MR <= 4 && T != kF32) {
      constexpr int kOutsPerBlock = kWaves * (64 / G);
      const dim3 grid((pr->width + kOutsPerBlock - 1) / kOutsPerBlock);
      if (pr->norm_w) {
        if constexpr (MR <= 2)
          hipLaunchKernelGGL((qgemv_kernel<T, MR, G, U, 2, true, true>), grid, dim3(kThreads),
                             slots * 16, stream, w, static_cast<const ST*>(s),
                             static_cast<const ST*>(b), static_cast<const ST*>(x),
                             static_cast<ST*>(y), k, n, m, kt, *pr);
        else
          return hipErrorInvalidValue;
      } else {
        hipLaunchKernelGGL((qgemv_kernel<T, MR, G, U, 2, true>), grid, dim3(kThreads), slots * 16,
                           stream, w, static_cast<const ST*>(s), static_cast<const ST*>(b),
                           static_cast<const ST*>(x), static_cast<ST*>(y), k, n, m, kt, *pr);
      }
      return hipGetLastError();
    }
    return hipErrorInvalidValue;
  }
  constexpr int R = rows_per_lane(MR);
  constexpr int rows_per_block = kWaves * (64 / G) * R;
  const dim3 grid((n + rows_per_block - 1) / rows_per_block);
  if (pr && pr->norm_w) {
    if constexpr (T != kF32 && MR <= 2)
      hipLaunchKernelGGL((qgemv_kernel<T, MR, G, U, R, false, true>), grid, dim3(kThreads),
                         slots * 16, stream, w, static_cast<const ST*>(s),
                         static_cast<const ST*>(b), static_cast<const ST*>(x),
                         static_cast<ST*>(y), k, n, m, kt, *pr);
    else
      return hipErrorInvalidValue;
  } else {
    hipLaunchKernelGGL((qgemv_kernel<T, MR, G, U, R, false>), grid, dim3(kThreads), slots * 16,
                       stream, w, static_cast<const ST*>(s), static_cast<const ST*>(b),
                       static_cast<const ST*>(x), static_cast<ST*>(y), k, n, m, kt,
                       pr ? *pr : GvPair{});
  }
  return hipGetLastError();
}

template <int T, int MR, int G>
hipError_t launch_g(const uint32_t* w, const void* s, const void* b, const void* x, void* y, int k,
                    int n, int m, const Plan& p, const GvPair* pr, hipStream_t stream) {
  if constexpr (max_chunks(MR) == 8) {
    switch (p.u) {
      case 1: return launch_u<T, MR, G, 1>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 2: return launch_u<T, MR, G, 2>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 3: return launch_u<T, MR, G, 3>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 4: return launch_u<T, MR, G, 4>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 5: return launch_u<T, MR, G, 5>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 6: return launch_u<T, MR, G, 6>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 7: return launch_u<T, MR, G, 7>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      default: return launch_u<T, MR, G, 8>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
    }
  } else {
    switch (p.u) {
      case 1: return launch_u<T, MR, G, 1>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 2: return launch_u<T, MR, G, 2>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      case 3: return launch_u<T, MR, G, 3>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
      default: return launch_u<T, MR, G, 4>(w, s, b, x, y, k, n, m, p.kt, pr, stream);
    }
  }
}

template <int T, int MR>
hipError_t launch_m(const uint32_t* w, const void* s, const void* b, const void* x, void* y, int k,
                    int n, int m, const GvPair* pr, hipStream_t stream) {
  // A pair plans as 2 width rows read two per lane group.
  const Plan p = is_pair(pr) ? make_plan(k, 2 * pr->width, MR, Elem<T>::kBytes, 2)
                             : make_plan(k, n, MR, Elem<T>::kBytes);
  switch (p.g) {
    case 16: return launch_g<T, MR, 16>(w, s, b, x, y, k, n, m, p, pr, stream);
    case 32: return launch_g<T, MR, 32>(w, s, b, x, y, k, n, m, p, pr, stream);
    default: return launch_g<T, MR, 64>(w, s, b, x, y, k, n, m, p, pr, stream);
  }
}

template <int T>
hipError_t launch_t(const uint32_t* w, const void* s, const void* b, const void* x, void* y, int k,
                    int n, int m, const GvPair* pr, hipStream_t stream) {
  // M is rounded up to a power of two for the register tile; rows >= M are
  // not stored.
  if (m <= 1) return launch_m<T, 1>(w, s, b, x, y, k, n, m, pr, stream);
  if (m <= 2) return launch_m<T, 2>(w, s, b, x, y, k, n, m, pr, stream);
  if (m <= 4) return launch_m<T, 4>(w, s, b, x, y, k, n, m, pr, stream);
  if (pr) return hipErrorInvalidValue;  // pair and residual forms: m <= 4
  if (m <= 8) return launch_m<T, 8>(w, s, b, x, y, k, n, m, nullptr, stream);
  if (m <= 16) return launch_m<T, 16>(w, s, b, x, y, k, n, m, nullptr, stream);
  return hipErrorInvalidValue;
}

}  // namespace

hipError_t launch_qgemv(const uint32_t* w, const void* scales, const void* biases, const void* x,
                        void* y, int k, int n, int m, int dtype, hipStream_t stream) {
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(w, scales, biases, x, y, k, n, m, nullptr, stream);
    case kF16: return launch_t<kF16>(w, scales, biases, x, y, k, n, m, nullptr, stream);
    case kF32: return launch_t<kF32>(w, scales, biases, x, y, k, n, m, nullptr, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_qgemv_resid_add(const uint32_t* w, const void* scales, const void* biases,
                                  const void* x, const void* resid, void* y, int k, int n, int m,
                                  int dtype, hipStream_t stream) {
  if (m > 4 || !resid) return hipErrorInvalidValue;
  GvPair pr{0, 0, 0, 0, 1.0f, 1.0f};
  pr.resid = resid;
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(w, scales, biases, x, y, k, n, m, &pr, stream);
    case kF16: return launch_t<kF16>(w, scales, biases, x, y, k, n, m, &pr, stream);
    default: return hipErrorInvalidValue;
  }
}

bool qgemv_norm_fits(int k, int n, int m, int width, int dtype, const void* x, const float* nw) {
  if (m < 1 || m > kQgemvNormMaxM || (dtype != kBf16 && dtype != kF16)) return false;
  // The RMSNorm kernel's 16-byte form, at most two pieces per thread.
  if (k % 8 != 0 || k / 8 > 2 * kThreads) return false;
  if (((uintptr_t)x & 15u) != 0 || ((uintptr_t)nw & 15u) != 0) return false;
  // The x tile must be the whole row.
  const Plan p = width > 0 ? make_plan(k, 2 * width, m <= 1 ? 1 : 2, 2, 2)
                           : make_plan(k, n, m <= 1 ? 1 : 2, 2);
  return p.kt == k;
}

hipError_t launch_qgemv_norm(const uint32_t* w, const void* scales, const void* biases,
                             const void* x, const float* nw, float eps, void* y, int k, int n,
                             int m, int dtype, hipStream_t stream) {
  if (!qgemv_norm_fits(k, n, m, 0, dtype, x, nw)) return hipErrorInvalidValue;
  GvPair pr{0, 0, 0, 0, 1.0f, 1.0f};
  pr.norm_w = nw;
  pr.eps = eps;
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(w, scales, biases, x, y, k, n, m, &pr, stream);
    default: return launch_t<kF16>(w, scales, biases, x, y, k, n, m, &pr, stream);
  }
}

hipError_t launch_qgemv_swiglu_norm(const uint32_t* w, const void* scales, const void* biases,
                                    const void* x, const float* nw, float eps, void* y, int ldy,
                                    int k, int n, int m, int width, int gate_row, int up_row,
                                    int dtype, hipStream_t stream) {
  if (!qgemv_norm_fits(k, n, m, width, dtype, x, nw)) return hipErrorInvalidValue;
  GvPair pr{gate_row, up_row, width, ldy, 1.0f, 1.0f};
  pr.norm_w = nw;
  pr.eps = eps;
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(w, scales, biases, x, y, k, n, m, &pr, stream);
    default: return launch_t<kF16>(w, scales, biases, x, y, k, n, m, &pr, stream);
  }
}

hipError_t launch_qgemv_swiglu(const uint32_t* w, const void* scales, const void* biases,
                               const void* x, void* y, int ldy, int k, int n, int m, int width,
                               int gate_row, int up_row, float in_scale, float out_scale,
                               int dtype, hipStream_t stream) {
  if (m > kQgemvSwigluMaxM) return hipErrorInvalidValue;
  const GvPair pr{gate_row, up_row, width, ldy, in_scale, out_scale};
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(w, scales, biases, x, y, k, n, m, &pr, stream);
    case kF16: return launch_t<kF16>(w, scales, biases, x, y, k, n, m, &pr, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace imq
