// qskinny.hip -- y[m][n] = x . deq(W)^T for 1 <= m <= 16 with the products on
// the matrix cores: a weight-streaming kernel for the few-row shapes between
// the qGEMV (whose dot products and reductions grow with M) and the tiled
// qGEMM (whose split-K plans read the weights at a fraction of HBM speed).
//
// A workgroup owns 16 weight rows (output features) and all of K; its W waves
// take interleaved chunks of 128 k (64 bytes of each row, two quantization
// groups).  In a v_mfma_f32_16x16x32 lane (c, h) = (lane % 16, lane / 16)
// supplies k = 8 h .. 8 h + 7 of a 32-k slice for A row c and B column c.
// Lane (c, h) loads bytes [16 h, 16 h + 16) of weight row c's 64-byte chunk
// (one wave instruction: 16 rows x 64 contiguous bytes); word j of those 16
// bytes feeds slice j, so slice j covers k = 32 h + 8 j .. +8 of the chunk in
// lane group h.  The activations take the same mapping as B: lane (c, h)
// reads x[c][32 h .. 32 h + 32) of the chunk, 64 contiguous bytes (columns of
// B past M only feed outputs that are never stored) -- from an LDS copy of all
// of x when it fits 96 KiB (staged by direct buffer->LDS loads while the
// weights are in flight; 52 VGPRs, 8 waves per SIMD; lanes past M read row
// M - 1), else straight from memory when token c < M (about 130 VGPRs).  Each
// lane's four words lie in one quantization group (group h / 2 of the chunk),
// so one scale and one bias per lane and chunk.  Weights A are dequantized in
// registers exactly as in the other kernels (RNE_T(fl32(s q + b))); the MFMA
// accumulates the products in fp32.  The waves' partial 16 x 16 sums are added
// in wave order through LDS (deterministic) and rounded to T.
//
// For 12 <= M <= 16 with K <= 4096 a second kernel (qskinny_lds_kernel) takes
// the call: its workgroups own up to four 16-row tiles and stage x in LDS once
// for all of them (see plan_lds).
#include <algorithm>

#include "epilogue.hpp"
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kRows = 16;     // weight rows per workgroup
constexpr int kChunkK = 128;  // k per chunk

template <int T>
__device__ __forceinline__ f32x4_t mfma16x16x32(u32x4_t a, u32x4_t b, f32x4_t c) {
  if constexpr (T == kBf16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// The value of the adjacent lane (lane ^ 1), by DPP.
__device__ __forceinline__ float swap_adjacent(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF,
                                                            0xF, true));  // quad_perm 1,0,3,2
}

// x staged in LDS when the whole [M, K] tile fits kXLdsMax bytes (rounded up
// to whole wave instructions): one 16-byte DMA per lane and slot instead of
// four register loads per chunk and lane.  96 KiB against 64: [9728 x 2560]
// M = 16 14.1 -> 13.3 us, [2560 x 9728] M = 4 12.0 -> 11.3 us, the rest equal.
// The rows are 2 K bytes apart, so the 16 rows of a B-operand read share a
// bank group (about 11 conflict cycles per LDS read); rows padded by 16 bytes
// as in the multi-tile kernel remove that but measured 4-7% slower at M = 4,
// 5 and 8 (same box, identical outputs): the reads hide under the weight stream.
constexpr int kXLdsMax = 96 * 1024;

template <int T, int W, int U, bool XLDS>
__global__ __launch_bounds__(64 * W) void qskinny_kernel(const uint32_t* __restrict__ w,
                                                         const uint16_t* __restrict__ scales,
                                                         const uint16_t* __restrict__ biases,
                                                         const uint16_t* __restrict__ x,
                                                         uint16_t* __restrict__ y, int M, int N,
                                                         int K, bool vec) {
  __shared__ f32x4_t part[W][64];
  extern __shared__ uint4 xs[];  // XLDS: x[M][K] as 16-byte slots, row-major
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * kRows;
  const int row = min(n0 + c, N - 1);  // rows past N are clamped; their outputs are not stored
  const int gpr = K >> 6;
  const int chunks = K / kChunkK;
  const auto wr = make_rsrc(w, (uint32_t)((size_t)N * K / 2));
  const auto sr = make_rsrc(scales, (uint32_t)((size_t)N * gpr * 2));
  const auto br = make_rsrc(biases, (uint32_t)((size_t)N * gpr * 2));
  const auto xr = make_rsrc(x, (uint32_t)((size_t)M * K * 2));
  const uint32_t w_off = (uint32_t)row * (uint32_t)(K / 2) + (uint32_t)h * 16u;
  const uint32_t p_off = ((uint32_t)row * (uint32_t)gpr + (uint32_t)(h >> 1)) * 2u;
  const uint32_t x_off = (uint32_t)c * (uint32_t)K * 2u + (uint32_t)h * 64u;
  const bool has_x = c < M;
  // LDS B fragments: lanes of tokens past M read row M - 1 (their outputs are
  // never stored), so the reads need no exec mask and no zero fill (82 v_mov
  // and 26 exec-mask saves per wave fewer at M = 4; 1-3.5% faster).
  const uint32_t xl_off = (uint32_t)min(c, M - 1) * (uint32_t)K * 2u + (uint32_t)h * 64u;

  if constexpr (XLDS) {
    // Slot i * 64 W + 64 wave + lane; lanes past the tile read past x (zeros)
    // into the rounded-up part of the allocation.
    const int slots = M * K / 8, per = 64 * W;
    for (int i = 0; i * per < slots; ++i)
      load_lds16(xr, (uint32_t)(i * per + wave * 64 + lane) * 16u, 0u, xs + i * per + wave * 64);
    __builtin_amdgcn_sched_barrier(0);
  }

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int ch0 = wave; ch0 < chunks; ch0 += W * U) {
    u32x4_t wv[U], xv[U][4];
    uint16_t sv[U], bv[U];
    // Chunks past the end are clamped to the last one (in range) and dropped.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t ch = (uint32_t)min(ch0 + u * W, chunks - 1);
      wv[u] = load_b128(wr, w_off + ch * 64u, 0);
      sv[u] = __builtin_amdgcn_raw_buffer_load_b16(sr, p_off + ch * 4u, 0, 0);
      bv[u] = __builtin_amdgcn_raw_buffer_load_b16(br, p_off + ch * 4u, 0, 0);
    }
    if constexpr (XLDS) {
      // The x tile is in LDS once this wave's DMA loads (issued before the 3 U
      // loads above) have landed and every wave has passed the barrier; only
      // the first pass waits (U covers every chunk of a wave).
      __builtin_amdgcn_sched_barrier(0);
      if (ch0 == wave) {
        IMQ_WAIT_VMCNT(3 * U);
        __builtin_amdgcn_s_barrier();
      }
      __builtin_amdgcn_sched_barrier(0);
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint32_t ch = (uint32_t)min(ch0 + u * W, chunks - 1);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          xv[u][j] = has_x ? load_b128(xr, x_off + ch * 256u + (uint32_t)j * 16u, 0)
                           : u32x4_t{0u, 0u, 0u, 0u};
      }
    }
    // No branch per chunk (the compiler would sink each chunk's loads into its
    // branch, behind the products of the chunks before it): a chunk past the
    // end gets scale and bias 0, so its weights are +0 and add nothing.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = ch0 + u * W < chunks;  // uniform across the wave
      const float s = valid ? Elem<T>::param(sv[u]) : 0.0f;
      const float s24 = s * 0x1p24f, s20 = s * 0x1p20f;
      const float b = valid ? Elem<T>::param(bv[u]) : 0.0f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        uint32_t p[4];
        Elem<T>::dequant(wv[u][j], s24, s20, b, p);
        u32x4_t xj;
        if constexpr (XLDS) {
          // B fragment read from the staged tile right before its MFMA.
          const uint32_t ch = (uint32_t)min(ch0 + u * W, chunks - 1);
          xj = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(xs) + xl_off +
                                                  ch * 256u + j * 16u);
        } else {
          xj = xv[u][j];
        }
        acc = mfma16x16x32<T>(u32x4_t{p[0], p[1], p[2], p[3]}, xj, acc);
      }
    }
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0 || !has_x) return;
  f32x4_t sum = part[0][lane];
#pragma unroll
  for (int i = 1; i < W; ++i) sum += part[i][lane];
  // Lane (c, h) holds outputs (token c, features n0 + 4 h + v), v = 0..3.
  const int f0 = n0 + 4 * h;
  uint16_t* yr = y + (size_t)c * N;
  if (vec && f0 + 3 < N) {
    *reinterpret_cast<uint2*>(yr + f0) =
        make_uint2(Elem<T>::pack2(sum[0], sum[1]), Elem<T>::pack2(sum[2], sum[3]));
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (f0 + v < N) yr[f0 + v] = Elem<T>::out(sum[v]);
  }
}

// ---------------------------------------------------------------------------
// x in LDS.  A workgroup owns TPW tiles of 16 weight rows over all of K and
// stages x [M, K] once, by direct buffer->LDS loads (16 bytes per lane, no
// registers), issued before its weight loads; its W waves split the chunks of
// 128 k (wave w: chunks w, w + W, ...) and each wave computes all TPW tiles of
// its chunks, reading one activation fragment from LDS per chunk for all of
// them.  Activation bytes cross the memory pipeline once per workgroup
// instead of once per wave and chunk.
//
// qskinny_lds_kernel (one tile per workgroup): loads read 16 rows x 64 bytes.
// LDS x layout: row m at byte m (2 K + 16), its 16-byte pieces in order: the 16
// lanes (c, 0..15) of one B-operand read group (rows c, the same piece) hit 16
// different 16-byte bank groups.
// The x staging waits (s_waitcnt vmcnt with the weight loads' count left
// outstanding, then a raw barrier) while the weights are still in flight.
template <int T, int TPW, int W, int U>
__global__ __launch_bounds__(64 * W) void qskinny_lds_kernel(const uint32_t* __restrict__ w,
                                                             const uint16_t* __restrict__ scales,
                                                             const uint16_t* __restrict__ biases,
                                                             const uint16_t* __restrict__ x,
                                                             uint16_t* __restrict__ y, int M,
                                                             int N, int K, bool vec) {
  constexpr int kWeightLoads = 3 * U * TPW < 63 ? 3 * U * TPW : 63;
  __shared__ f32x4_t part[W][TPW][64];
  extern __shared__ uint4 xs[];  // x [M, K], rows 2 K + 16 bytes apart
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * (kRows * TPW);
  const int gpr = K >> 6;
  const int chunks = K / kChunkK;
  const auto wr = make_rsrc(w, (uint32_t)((size_t)N * K / 2));
  const auto sr = make_rsrc(scales, (uint32_t)((size_t)N * gpr * 2));
  const auto br = make_rsrc(biases, (uint32_t)((size_t)N * gpr * 2));
  const auto xr = make_rsrc(x, (uint32_t)((size_t)M * K * 2));

  // 1. x -> LDS, one wave instruction per 1 KB piece q of the [M, K] tile (K %
  //    512 == 0: a row is K / 512 pieces): row m = q / rp, part q % rp (both
  //    wave-uniform, scalar arithmetic), to LDS row m at a stride of 2 K + 16
  //    bytes; the 16-byte pad puts the 16 rows of one B-operand read into 16
  //    different bank groups.
  {
    const int rp = K >> 9, pieces = M * rp;
    for (int q = wave; q < pieces; q += W) {
      const int m = q / rp, part = q - m * rp;
      load_lds16(xr, (uint32_t)lane * 16u, (uint32_t)(m * K * 2 + part * 1024),
                 reinterpret_cast<char*>(xs) + m * (2 * K + 16) + part * 1024);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. This wave's weight, scale and bias fragments, all of them.
  uint32_t w_off[TPW], p_off[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const uint32_t row = (uint32_t)min(n0 + kRows * t + c, N - 1);
    w_off[t] = row * (uint32_t)(K / 2) + (uint32_t)h * 16u;
    p_off[t] = (row * (uint32_t)gpr + (uint32_t)(h >> 1)) * 2u;
  }
  f32x4_t acc[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  const int xrow = min(c, M - 1);
  bool first = true;
  for (int ch0 = wave; ch0 < chunks; ch0 += W * U) {
    u32x4_t wv[U][TPW];
    uint16_t sv[U][TPW], bv[U][TPW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t ch = (uint32_t)min(ch0 + u * W, chunks - 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        wv[u][t] = load_b128(wr, w_off[t], ch * 64u);
        sv[u][t] = __builtin_amdgcn_raw_buffer_load_b16(sr, p_off[t], ch * 4u, 0);
        bv[u][t] = __builtin_amdgcn_raw_buffer_load_b16(br, p_off[t], ch * 4u, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (first) {
      // The x loads (issued first) have landed once at most the 3 U TPW
      // weight-side loads are outstanding (the counter tracks at most 63: with
      // more, the oldest had retired before the last could issue); after the
      // barrier every wave's have.
      IMQ_WAIT_VMCNT(kWeightLoads);
      __builtin_amdgcn_s_barrier();
      first = false;
    }
    __builtin_amdgcn_sched_barrier(0);
    // A chunk past the end gets scale and bias 0 (weights +0): no branch, so
    // its loads stay above.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = ch0 + u * W < chunks;
      const int j = min(ch0 + u * W, chunks - 1);
      u32x4_t xf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xf[i] = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(xs) +
                                                   xrow * (2 * K + 16) + j * 256 + (4 * h + i) * 16);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float s = valid ? Elem<T>::param(sv[u][t]) : 0.0f;
        const float s24 = s * 0x1p24f, s20 = s * 0x1p20f;
        const float b = valid ? Elem<T>::param(bv[u][t]) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t p[4];
          Elem<T>::dequant(wv[u][t][i], s24, s20, b, p);
          acc[t] = mfma16x16x32<T>(u32x4_t{p[0], p[1], p[2], p[3]}, xf[i], acc[t]);
        }
      }
    }
  }
  if (first) {  // a wave with no chunk (W > chunks) still meets the others at the barrier
    IMQ_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t) part[wave][t][lane] = acc[t];
  __syncthreads();
  if (wave >= TPW || c >= M) return;
  const int t = wave;
  f32x4_t sum = part[0][t][lane];
#pragma unroll
  for (int i = 1; i < W; ++i) sum += part[i][t][lane];
  const int f0 = n0 + kRows * t + 4 * h;
  uint16_t* yr = y + (size_t)c * N;
  if (vec && f0 + 3 < N) {
    *reinterpret_cast<uint2*>(yr + f0) =
        make_uint2(Elem<T>::pack2(sum[0], sum[1]), Elem<T>::pack2(sum[2], sum[3]));
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (f0 + v < N) yr[f0 + v] = Elem<T>::out(sum[v]);
  }
}

// qskinny_lds8_kernel (two or more tiles per workgroup): loads read 8 weight
// rows x 128 bytes, as in qskinny_half_kernel (below).  Over a span of 256 k
// the B operand's columns carry (token, K half) as j = 2 t' + p, A lane (c, h)
// holds row c / 2 of an octet of a tile at k = 128 (c % 2) + 32 h + 8 s, and
// the blocks with p = p' are the halves of a row's dot product with a token.
// With 12-16 tokens there are two token groups (tokens 8 g + t'): two MFMAs
// and two B fragments per A fragment, which pay where a B fragment serves two
// or more tiles (A/B against the 16-row-load form: [9728 x 2560] M = 12 / 16
// 10.6 / 10.8 -> 10.0 / 10.3 us at three tiles, [6144 x 2560] M = 13 -5% at
// two; 4-6% slower at one tile).  W is even: wave w takes octet w % 2 of every
// tile over spans w / 2, w / 2 + W / 2, ... (as many units as it had chunks).
//
// LDS x layout: row m's 16-byte piece q at m K / 8 + (q ^ (2 (m % 8) + bit 4 of
// q) % 16): the 16 lanes of a B read (tokens 8 g + t', halves p) hit 16
// different 16-byte bank groups.
// The x staging waits (s_waitcnt vmcnt with the weight loads' count left
// outstanding, then a raw barrier) while the weights are still in flight.
template <int T, int TPW, int W, int U>
__global__ __launch_bounds__(64 * W) void qskinny_lds8_kernel(const uint32_t* __restrict__ w,
                                                             const uint16_t* __restrict__ scales,
                                                             const uint16_t* __restrict__ biases,
                                                             const uint16_t* __restrict__ x,
                                                             uint16_t* __restrict__ y, int M,
                                                             int N, int K, bool vec) {
  static_assert(W % 2 == 0, "waves pair up over the two octets of a tile");
  constexpr int kStride = W / 2;  // span stride of a wave
  constexpr int kWeightLoads = 3 * U * TPW < 63 ? 3 * U * TPW : 63;
  __shared__ float2 part[W][TPW][2][64];
  extern __shared__ uint4 xs[];  // x [M, K], pieces XOR-placed within 16-piece blocks
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int o = wave & 1;
  const int c = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * (kRows * TPW);
  const int gpr = K >> 6;
  const int spans = K >> 8;
  const int row_pieces = K >> 3;
  const auto wr = make_rsrc(w, (uint32_t)((size_t)N * K / 2));
  const auto sr = make_rsrc(scales, (uint32_t)((size_t)N * gpr * 2));
  const auto br = make_rsrc(biases, (uint32_t)((size_t)N * gpr * 2));
  const auto xr = make_rsrc(x, (uint32_t)((size_t)M * K * 2));

  // 1. x -> LDS: instruction e stages pieces [64 i, 64 i + 64) of row m (1 KB
  //    of x, read contiguously: the XOR stays inside 16-piece blocks).
  {
    const int per_row = K >> 9;
    for (int e = wave; e < M * per_row; e += W) {
      const int m = e / per_row, i = e - m * per_row;
      const int u = 64 * i + lane;
      const int q = u ^ ((2 * (m & 7) + ((u >> 4) & 1)) & 15);
      load_lds16(xr, (uint32_t)(m * K + 8 * q) * 2u, 0u, xs + m * row_pieces + 64 * i);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. This wave's weight, scale and bias fragments: octet o of tile t, tile
  //    row 4 (c / 4) + 2 o + (c / 2) % 2.
  uint32_t w_off[TPW], p_off[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const uint32_t row =
        (uint32_t)min(n0 + kRows * t + 4 * (c >> 2) + 2 * o + ((c >> 1) & 1), N - 1);
    w_off[t] = row * (uint32_t)(K / 2) + (uint32_t)(c & 1) * 64u + (uint32_t)h * 16u;
    p_off[t] = (row * (uint32_t)gpr + 2u * (uint32_t)(c & 1) + (uint32_t)(h >> 1)) * 2u;
  }
  // B operand of token group g: row min(8 g + c / 2, M - 1) (columns past M are
  // never stored), half c % 2.
  uint32_t xo[2][4];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int m = min(8 * g + (c >> 1), M - 1);
    const int sw = 2 * (m & 7) + (c & 1);
    const uint32_t xb = (uint32_t)(m * row_pieces + 16 * (c & 1)) * 16u;
#pragma unroll
    for (int s = 0; s < 4; ++s) xo[g][s] = xb + (uint32_t)(((4 * h + s) ^ sw) * 16);
  }
  f32x4_t acc[TPW][2];
#pragma unroll
  for (int t = 0; t < TPW; ++t) acc[t][0] = acc[t][1] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  bool first = true;
  for (int sp0 = wave >> 1; sp0 < spans; sp0 += kStride * U) {
    u32x4_t wv[U][TPW];
    uint16_t sv[U][TPW], bv[U][TPW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t sp = (uint32_t)min(sp0 + u * kStride, spans - 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        wv[u][t] = load_b128(wr, w_off[t], sp * 128u);
        sv[u][t] = __builtin_amdgcn_raw_buffer_load_b16(sr, p_off[t], sp * 8u, 0);
        bv[u][t] = __builtin_amdgcn_raw_buffer_load_b16(br, p_off[t], sp * 8u, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (first) {
      // The x loads (issued first) have landed once at most the 3 U TPW
      // weight-side loads are outstanding (the counter tracks at most 63: with
      // more, the oldest had retired before the last could issue); after the
      // barrier every wave's have.
      IMQ_WAIT_VMCNT(kWeightLoads);
      __builtin_amdgcn_s_barrier();
      first = false;
    }
    __builtin_amdgcn_sched_barrier(0);
    // A span past the end gets scale and bias 0 (weights +0): no branch, so
    // its loads stay above.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = sp0 + u * kStride < spans;
      const uint32_t sp = (uint32_t)min(sp0 + u * kStride, spans - 1);
      u32x4_t xf[2][4];
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int s = 0; s < 4; ++s)
          xf[g][s] = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(xs) +
                                                       xo[g][s] + sp * 512u);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float sc = valid ? Elem<T>::param(sv[u][t]) : 0.0f;
        const float s24 = sc * 0x1p24f, s20 = sc * 0x1p20f;
        const float b = valid ? Elem<T>::param(bv[u][t]) : 0.0f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          uint32_t p[4];
          Elem<T>::dequant(wv[u][t][s], s24, s20, b, p);
          const u32x4_t a = u32x4_t{p[0], p[1], p[2], p[3]};
          acc[t][0] = mfma16x16x32<T>(a, xf[0][s], acc[t][0]);
          acc[t][1] = mfma16x16x32<T>(a, xf[1][s], acc[t][1]);
        }
      }
    }
  }
  if (first) {  // a wave with no span (W / 2 > spans) still meets the others at the barrier
    IMQ_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
  }
  // Lane (j, g') holds rows 4 g' + v of column j: its half j % 2 is in v = j % 2
  // (octet row 2 g') and v = 2 + j % 2 (octet row 2 g' + 1).
  const bool odd = (c & 1) != 0;
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float v0 = odd ? acc[t][g][1] : acc[t][g][0];
      float v1 = odd ? acc[t][g][3] : acc[t][g][2];
      v0 += swap_adjacent(v0);
      v1 += swap_adjacent(v1);
      part[wave][t][g][lane] = make_float2(v0, v1);
    }
  __syncthreads();
  if (wave >= TPW || odd) return;
  const int t = wave;
  const int f0 = n0 + kRows * t + 4 * h;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const int m = 8 * g + (c >> 1);
    if (m >= M) continue;
    float sum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < W; ++i) {
      const float2 v = part[i][t][g][lane];
      sum[2 * (i & 1)] += v.x;
      sum[2 * (i & 1) + 1] += v.y;
    }
    uint16_t* yr = y + (size_t)m * N;
    if (vec && f0 + 3 < N) {
      *reinterpret_cast<uint2*>(yr + f0) =
          make_uint2(Elem<T>::pack2(sum[0], sum[1]), Elem<T>::pack2(sum[2], sum[3]));
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (f0 + v < N) yr[f0 + v] = Elem<T>::out(sum[v]);
    }
  }
}

// ---------------------------------------------------------------------------
// M <= 8, x in LDS, K % 512 == 0: eight weight rows x 128 bytes per load.
//
// Over a span of 256 k the B operand's 16 columns carry (token t, K half p)
// as j = 2 t + p: lane (c, h) of A holds weight row r = c / 2 of an octet of
// the tile, k = 128 (c % 2) + 32 h + 8 s .. +8 of the span in k-slice s; lane
// (j, h) of B holds x[t][128 p + 32 h + 8 s .. +8].  Output (2 r + p, 2 t + p')
// is half p of row r against half p' of token t; the blocks with p = p',
// added, are row r's dot product with token t over the span (the others are
// never used).  A wave instruction then reads 8 rows x 128 contiguous bytes
// (8 cache lines; the 16-row kernel's read 16 rows x 64 bytes), with the same
// number of loads and MFMAs per weight byte.  W is even: wave w takes octet
// w % 2 and the spans w / 2, w / 2 + W / 2, ... (as many as the 16-row kernel
// gives a wave chunks; its x fragment serves one octet).
//
// Octet o's row r is tile row 4 (r / 2) + 2 o + r % 2: once the p = p' pairs
// are added (a DPP swap of adjacent lanes) lane (j, g) of a wave of octet o
// holds features 4 g + 2 o, 4 g + 2 o + 1 of token j / 2; the reduction over
// the waves gives it features 4 g .. 4 g + 3, stored as 8 bytes.
//
// x in LDS: row t's 16-byte piece q (k = 8 q) at t K / 8 + (q ^ (2 t + bit 4
// of q) % 16), so the 16 lanes of a B read (tokens t, halves p, one h and s)
// hit 16 different 16-byte bank groups (rows are K / 8 pieces apart, a
// multiple of 16).  One DMA instruction stages 64 pieces of a row: the XOR
// stays inside 16-piece blocks, so it still reads 1 KB of x contiguously.
template <int T, int W, int U>
__global__ __launch_bounds__(64 * W) void qskinny_half_kernel(const uint32_t* __restrict__ w,
                                                              const uint16_t* __restrict__ scales,
                                                              const uint16_t* __restrict__ biases,
                                                              const uint16_t* __restrict__ x,
                                                              uint16_t* __restrict__ y, int M,
                                                              int N, int K, bool vec) {
  static_assert(W % 2 == 0, "waves pair up over the two octets");
  constexpr int kStride = W / 2;  // span stride of a wave
  __shared__ float2 part[W][64];
  extern __shared__ uint4 xs[];  // x [M, K], pieces XOR-placed within 16-piece blocks
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int o = wave & 1;
  const int c = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * kRows;
  const int gpr = K >> 6;
  const int spans = K >> 8;
  const int row_pieces = K >> 3;
  const auto wr = make_rsrc(w, (uint32_t)((size_t)N * K / 2));
  const auto sr = make_rsrc(scales, (uint32_t)((size_t)N * gpr * 2));
  const auto br = make_rsrc(biases, (uint32_t)((size_t)N * gpr * 2));
  const auto xr = make_rsrc(x, (uint32_t)((size_t)M * K * 2));

  // 1. x -> LDS: instruction e stages pieces [64 i, 64 i + 64) of row t.
  {
    const int per_row = K >> 9;
    for (int e = wave; e < M * per_row; e += W) {
      const int t = e / per_row, i = e - t * per_row;
      const int u = 64 * i + lane;
      const int q = u ^ ((2 * t + ((u >> 4) & 1)) & 15);
      load_lds16(xr, (uint32_t)(t * K + 8 * q) * 2u, 0u, xs + t * row_pieces + 64 * i);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // A operand: octet o, tile row 4 (c / 4) + 2 o + (c / 2) % 2, bytes 64 (c % 2) + 16 h of
  // each 128-byte span; group 2 (c % 2) + h / 2 of the span's four.
  const uint32_t row = (uint32_t)min(n0 + 4 * (c >> 2) + 2 * o + ((c >> 1) & 1), N - 1);
  const uint32_t w_off = row * (uint32_t)(K / 2) + (uint32_t)(c & 1) * 64u + (uint32_t)h * 16u;
  const uint32_t p_off = (row * (uint32_t)gpr + 2u * (uint32_t)(c & 1) + (uint32_t)(h >> 1)) * 2u;
  // B operand: token min(c / 2, M - 1) (columns past M are never stored), half c % 2.
  const int t = min(c >> 1, M - 1);
  const int sw = 2 * t + (c & 1);
  const uint32_t xb = (uint32_t)(t * row_pieces + 16 * (c & 1)) * 16u;
  uint32_t xo[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) xo[s] = xb + (uint32_t)(((4 * h + s) ^ sw) * 16);

  f32x4_t acc = {0.f, 0.f, 0.f, 0.f};
  for (int sp0 = wave >> 1; sp0 < spans; sp0 += kStride * U) {
    u32x4_t wv[U];
    uint16_t sv[U], bv[U];
    // Spans past the end are clamped to the last one and dropped.
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t sp = (uint32_t)min(sp0 + u * kStride, spans - 1);
      wv[u] = load_b128(wr, w_off + sp * 128u, 0);
      sv[u] = __builtin_amdgcn_raw_buffer_load_b16(sr, p_off + sp * 8u, 0, 0);
      bv[u] = __builtin_amdgcn_raw_buffer_load_b16(br, p_off + sp * 8u, 0, 0);
    }
    // x is in LDS once this wave's DMA loads (issued before the 3 U loads
    // above) have landed and every wave has passed the barrier; every wave
    // has a first pass (W / 2 <= spans).
    __builtin_amdgcn_sched_barrier(0);
    if (sp0 == (wave >> 1)) {
      IMQ_WAIT_VMCNT(3 * U);
      __builtin_amdgcn_s_barrier();
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = sp0 + u * kStride < spans;  // uniform across the wave
      const uint32_t sp = (uint32_t)min(sp0 + u * kStride, spans - 1);
      const float sc = valid ? Elem<T>::param(sv[u]) : 0.0f;
      const float s24 = sc * 0x1p24f, s20 = sc * 0x1p20f;
      const float bb = valid ? Elem<T>::param(bv[u]) : 0.0f;
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        uint32_t p[4];
        Elem<T>::dequant(wv[u][s], s24, s20, bb, p);
        const u32x4_t xj = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(xs) +
                                                             xo[s] + sp * 512u);
        acc = mfma16x16x32<T>(u32x4_t{p[0], p[1], p[2], p[3]}, xj, acc);
      }
    }
  }
  // Lane (j, g) holds rows 4 g + v of column j: its half j % 2 is in v = j % 2
  // (octet row 2 g) and v = 2 + j % 2 (octet row 2 g + 1).
  const bool odd = (c & 1) != 0;
  float v0 = odd ? acc[1] : acc[0];
  float v1 = odd ? acc[3] : acc[2];
  v0 += swap_adjacent(v0);
  v1 += swap_adjacent(v1);
  part[wave][lane] = make_float2(v0, v1);
  __syncthreads();
  if (wave != 0 || odd || (c >> 1) >= M) return;
  float sum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const float2 v = part[i][lane];
    sum[2 * (i & 1)] += v.x;
    sum[2 * (i & 1) + 1] += v.y;
  }
  const int f0 = n0 + 4 * h;
  uint16_t* yr = y + (size_t)(c >> 1) * N;
  if (vec && f0 + 3 < N) {
    *reinterpret_cast<uint2*>(yr + f0) =
        make_uint2(Elem<T>::pack2(sum[0], sum[1]), Elem<T>::pack2(sum[2], sum[3]));
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v)
      if (f0 + v < N) yr[f0 + v] = Elem<T>::out(sum[v]);
  }
}

// Waves per workgroup: enough that the device holds about 2048 waves and
// each wave at most 8 chunks, at most 16 waves and at most half the chunks;
// but 8 where that leaves a wave at most 4 chunks.  16 waves of 1-2 chunks
// each lost to 8 waves of 3-4 (same box, weights from HBM): [3072 x 3072] M
// = 4 / 8 5.7 / 6.0 -> 5.0 / 5.2 us (16 waves over 24 chunks leave a quarter
// of the slots idle), [2560 x 4096] M = 4 / 8 5.9 / 6.4 -> 5.8 / 6.2 us; at
// K = 9728 (76 chunks) 16 waves stay far ahead (9.9 against 12.5 us).
int skinny_waves(int n, int k) {
  const long blocks = (n + kRows - 1) / kRows;
  const int chunks = k / kChunkK;
  int wv = 1;
  while (wv < 16 && (blocks * wv < 2048 || chunks > 8 * wv) && wv * 2 <= chunks &&
         !(wv == 8 && chunks <= 4 * wv))
    wv *= 2;
  return wv;
}

template <int T, int W>
hipError_t launch_w(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                    uint16_t* y, int k, int n, int m, bool vec, hipStream_t stream) {
  // Chunks per wave, all loaded before any is computed (one memory round trip).
  const int chunks = k / kChunkK, u = (chunks + W - 1) / W;
  const dim3 grid((unsigned)((n + kRows - 1) / kRows)), block(64 * W);
  // LDS for the x tile: the slots rounded up to whole wave-instruction rounds.
  const size_t per = 64 * (size_t)W, slots = (size_t)m * k / 8;
  const size_t xbytes = (slots + per - 1) / per * per * 16;
  const bool xlds = xbytes <= (size_t)kXLdsMax;
  if constexpr (W % 2 == 0) {
    if (xlds && m <= 8 && k % 512 == 0) {
      // Units of 8 rows x 256 k, as many per wave as chunks: W / 2 <= k / 256,
      // as 2 W <= chunks.
      const size_t hbytes = (size_t)m * k * 2;
#define IMQ_HALF(UU)                                                                             \
  hipLaunchKernelGGL((qskinny_half_kernel<T, W, UU>), grid, block, hbytes, stream, w, s, b, x, y, \
                     m, n, k, vec)
      if (u <= 2) IMQ_HALF(2);
      else if (u <= 3) IMQ_HALF(3);
      else if (u <= 4) IMQ_HALF(4);
      else if (u <= 5) IMQ_HALF(5);
      else if (u <= 6) IMQ_HALF(6);
      else IMQ_HALF(8);
#undef IMQ_HALF
      return hipGetLastError();
    }
  }
#define IMQ_SKINNY(UU)                                                                            \
  do {                                                                                           \
    if (xlds)                                                                                    \
      hipLaunchKernelGGL((qskinny_kernel<T, W, UU, true>), grid, block, xbytes, stream, w, s, b, \
                         x, y, m, n, k, vec);                                                    \
    else                                                                                         \
      hipLaunchKernelGGL((qskinny_kernel<T, W, UU, false>), grid, block, 0, stream, w, s, b, x,  \
                         y, m, n, k, vec);                                                       \
  } while (0)
  if (u <= 2) IMQ_SKINNY(2);
  else if (u <= 3) IMQ_SKINNY(3);
  else if (u <= 4) IMQ_SKINNY(4);
  else if (u <= 5) IMQ_SKINNY(5);
  else if (u <= 6) IMQ_SKINNY(6);
  else IMQ_SKINNY(8);
#undef IMQ_SKINNY
  return hipGetLastError();
}

// ---- the x-in-LDS multi-tile kernel ----

// Taken for 12 <= M <= 16 with K <= 4096, K % 512 == 0: there x [M, K] is
// 48-128 KB, which leaves the 16-row kernel one workgroup (four waves) per CU
// in several rounds; here each workgroup stages x once for up to four row
// tiles and the grid fits one round.  Measured with the weights from HBM (48
// rotated copies), [9728 x 2560] M = 16: 11.2 us against 13.7 us.  At M <= 8,
// and for K = 9728, the 16-row kernel stays faster (8.2 / 8.8 us at M = 4 / 8
// against 8.7 / 9.5 us).
constexpr int kLdsMinM = 12;
constexpr int kLdsMaxK = 4096;
constexpr int kLdsWaves = 8;

// Largest U compiled for (TPW, W) of the LDS kernel (6 registers per tile and
// span, W / 4 waves per SIMD; with eight waves four tiles x 8 spans would spill,
// and K <= kLdsMaxK gives a wave at most 4 spans anyway).
constexpr int max_u_lds(int tpw, int w) {
  return w == 16 ? (tpw == 1 ? 8 : tpw == 2 ? 6 : tpw == 3 ? 4 : 3) : (tpw == 4 ? 6 : 8);
}

// Bytes of the x tile in LDS: M rows of 2 K bytes, plus a 16-byte pad each for
// the one-tile kernel.
size_t lds_x_bytes(int k, int m, int tpw) {
  return (size_t)m * (2 * (size_t)k + (tpw == 1 ? 16 : 0));
}

struct LdsPlan {
  int tpw, u;
  bool ok;
};

// Tiles per workgroup: the fewest (at most four) that keep the grid within
// one workgroup per CU.
LdsPlan plan_lds(int k, int n, int m) {
  const int chunks = k / kChunkK;
  const long tiles = (n + kRows - 1) / kRows;
  int tpw = 4;
  for (int t = 1; t <= 4; ++t)
    if ((tiles + t - 1) / t <= 256) {
      tpw = t;
      break;
    }
  const bool ok = m >= kLdsMinM && k <= kLdsMaxK && k % 512 == 0 &&
                  lds_x_bytes(k, m, tpw) + (size_t)kLdsWaves * tpw * 1024 <= 128 * 1024;
  const int u = std::max(1, std::min((chunks + kLdsWaves - 1) / kLdsWaves,
                                     max_u_lds(tpw, kLdsWaves)));
  return LdsPlan{tpw, u, ok};
}

template <int T, int TPW, int W, int U>
hipError_t launch_lds_twu(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          const uint16_t* x, uint16_t* y, int k, int n, int m, bool vec,
                          hipStream_t stream) {
  if constexpr (U > max_u_lds(TPW, W)) {
    return hipErrorInvalidValue;
  } else {
    const dim3 grid((unsigned)((n + kRows * TPW - 1) / (kRows * TPW))), block(64 * W);
    if constexpr (TPW == 1)
      hipLaunchKernelGGL((qskinny_lds_kernel<T, TPW, W, U>), grid, block, lds_x_bytes(k, m, TPW),
                         stream, w, s, b, x, y, m, n, k, vec);
    else
      hipLaunchKernelGGL((qskinny_lds8_kernel<T, TPW, W, U>), grid, block, lds_x_bytes(k, m, TPW),
                         stream, w, s, b, x, y, m, n, k, vec);
    return hipGetLastError();
  }
}

template <int T, int TPW, int W>
hipError_t launch_lds_tw(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                         const uint16_t* x, uint16_t* y, int k, int n, int m, int u, bool vec,
                         hipStream_t stream) {
  switch (u) {
    case 1: return launch_lds_twu<T, TPW, W, 1>(w, s, b, x, y, k, n, m, vec, stream);
    case 2: return launch_lds_twu<T, TPW, W, 2>(w, s, b, x, y, k, n, m, vec, stream);
    case 3: return launch_lds_twu<T, TPW, W, 3>(w, s, b, x, y, k, n, m, vec, stream);
    case 4: return launch_lds_twu<T, TPW, W, 4>(w, s, b, x, y, k, n, m, vec, stream);
    case 5:
    case 6: return launch_lds_twu<T, TPW, W, 6>(w, s, b, x, y, k, n, m, vec, stream);
    default: return launch_lds_twu<T, TPW, W, 8>(w, s, b, x, y, k, n, m, vec, stream);
  }
}

template <int T, int TPW>
hipError_t launch_lds_t(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                        const uint16_t* x, uint16_t* y, int k, int n, int m, const LdsPlan& p,
                        bool vec, hipStream_t stream) {
  return launch_lds_tw<T, TPW, kLdsWaves>(w, s, b, x, y, k, n, m, p.u, vec, stream);
}

// ---- K split, rows per wave ----
//
// For long K or more than 16 rows: workgroup (g, s) owns W x R 16-row tiles
// (wave v the R tiles from row (g W + v) 16 R) and the K range of split s:
// `per` pieces of 512 k, CH = 4 per chunks of 128 k.  Each wave runs the
// whole range for its own tiles, so no sums cross waves, and the W waves
// share one x slice [M, 512 per] in LDS (rows 1024 per + 16 bytes apart).
// Its predecessor split the K range among the waves of a workgroup of one to
// four tiles and added their sums in LDS: at 30 rows and [2560 x 9728] it
// read some 98 MB of x slices from L2 for 12.5 MB of weights, and took 17.1
// us (with the split sums) where this takes 12.5.  A wave issues every load
// of its range before its first MFMA: its x pieces, then its scale and bias
// blocks (8 groups of a row per 16-byte load), then the weights chunk by
// chunk, and waits once for its x pieces (loads return in issue order)
// before a barrier; the compiler's own waits then take the weights chunk by
// chunk.  Fp32 partial sums go to ws[s][m][n]; qskinny_reduce_kernel (or a
// fused-stage split sum) adds the splits in order (deterministic).
template <int T, int R, int W, int TG, int CH>
__global__ __launch_bounds__(64 * W) void qskinny_rows_kernel(const uint32_t* __restrict__ w,
                                                              const uint16_t* __restrict__ scales,
                                                              const uint16_t* __restrict__ biases,
                                                              const uint16_t* __restrict__ x,
                                                              float* __restrict__ ws, int M,
                                                              int N, int K, int per, bool vec) {
  static_assert(CH % 4 == 0 && CH * R + CH / 2 * R <= 63, "the loads after x fit vmcnt");
  constexpr int kBlk = CH / 4;  // 16-byte scale (bias) blocks per row: 8 groups, 512 k each
  extern __shared__ uint4 xs[];  // x [M, 512 per], rows 1024 per + 16 bytes apart
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int n0 = ((int)blockIdx.x * W + wave) * (kRows * R);
  const int gpr = K >> 6;
  const int p0 = (int)blockIdx.y * per;
  const int np = min(per, (K >> 9) - p0);  // pieces of 512 k in this range (>= 1)
  const int chunks = np * 4;
  const int c0 = p0 * 4;                   // first global chunk of 128 k
  const int xstride = 1024 * per + 16;
  const auto wr = make_rsrc(w, (uint32_t)((size_t)N * K / 2));
  const auto sr = make_rsrc(scales, (uint32_t)((size_t)N * gpr * 2));
  const auto br = make_rsrc(biases, (uint32_t)((size_t)N * gpr * 2));
  const auto xr = make_rsrc(x, (uint32_t)((size_t)M * K * 2));

  // 1. The x slice -> LDS, one wave instruction per 1 KB piece (row m = q /
  //    np, piece q % np, wave-uniform).
  {
    const int pieces = M * np;
    for (int q = wave; q < pieces; q += W) {
      const int m = q / np, pc = q - m * np;
      load_lds16(xr, (uint32_t)lane * 16u, (uint32_t)((m * K + (p0 + pc) * 512) * 2),
                 reinterpret_cast<char*>(xs) + m * xstride + pc * 1024);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. Scale and bias blocks (groups 8 b .. 8 b + 7 from the range's first
  //    group; a short last range repeats its last block, never used), then
  //    the weights: lane (c, h) holds row c of each tile, bytes [16 h, +16) of
  //    each chunk's 64 (chunks past a short range repeat its last one).
  uint32_t w_off[R], p_off[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const uint32_t row = (uint32_t)min(n0 + kRows * r + c, N - 1);
    w_off[r] = row * (uint32_t)(K / 2) + (uint32_t)h * 16u;
    p_off[r] = row * (uint32_t)gpr * 2u;
  }
  uint4 sblk[kBlk][R], bblk[kBlk][R];
#pragma unroll
  for (int b = 0; b < kBlk; ++b)
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint32_t g = (uint32_t)(2 * c0 + 8 * min(b, (chunks - 1) / 4));
      sblk[b][r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(sr, p_off[r], g * 2u, 0));
      bblk[b][r] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(br, p_off[r], g * 2u, 0));
    }
  u32x4_t wv[CH][R];
#pragma unroll
  for (int j = 0; j < CH; ++j)
#pragma unroll
    for (int r = 0; r < R; ++r)
      wv[j][r] = load_b128(wr, w_off[r], (uint32_t)(c0 + min(j, chunks - 1)) * 64u);
  __builtin_amdgcn_sched_barrier(0);

  f32x4_t acc[R][TG];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int g = 0; g < TG; ++g) acc[r][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // B operand of token group g (16 tokens): row min(16 g + c, M - 1); columns
  // past M are never stored.
  int xrow[TG];
#pragma unroll
  for (int g = 0; g < TG; ++g) xrow[g] = min(16 * g + c, M - 1);
  IMQ_WAIT_VMCNT(2 * kBlk * R + CH * R);  // this wave's x pieces have landed
  __builtin_amdgcn_s_barrier();           // and every other wave's
  __builtin_amdgcn_sched_barrier(0);
  // Every chunk runs, so that no load is sunk into a conditional block past
  // the wait above; a chunk past a short range reads the range's last x
  // chunk and dequantizes to zero (scale and bias 0), adding nothing.
#pragma unroll
  for (int j = 0; j < CH; ++j) {
    const bool valid = j < chunks;
    const int jx = min(j, chunks - 1);
    u32x4_t xf[TG][4];
#pragma unroll
    for (int g = 0; g < TG; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        xf[g][i] = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(xs) +
                                                    xrow[g] * xstride + jx * 256 + (4 * h + i) * 16);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // Group 2 j + h / 2 of the range: half h / 2 of dword j % 4 of block j / 4.
      const uint4 sb = sblk[j / 4][r], bb = bblk[j / 4][r];
      const uint32_t sw = (j % 4 == 0) ? sb.x : (j % 4 == 1) ? sb.y : (j % 4 == 2) ? sb.z : sb.w;
      const uint32_t bw = (j % 4 == 0) ? bb.x : (j % 4 == 1) ? bb.y : (j % 4 == 2) ? bb.z : bb.w;
      const int sh = 16 * (h >> 1);
      const float sc = valid ? Elem<T>::param((uint16_t)(sw >> sh)) : 0.0f;
      const float s24 = sc * 0x1p24f, s20 = sc * 0x1p20f;
      const float b = valid ? Elem<T>::param((uint16_t)(bw >> sh)) : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t pq[4];
        Elem<T>::dequant(wv[j][r][i], s24, s20, b, pq);
        const u32x4_t a = u32x4_t{pq[0], pq[1], pq[2], pq[3]};
#pragma unroll
        for (int g = 0; g < TG; ++g) acc[r][g] = mfma16x16x32<T>(a, xf[g][i], acc[r][g]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int f0 = n0 + kRows * r + 4 * h;
#pragma unroll
    for (int g = 0; g < TG; ++g) {
      const int m = 16 * g + c;
      if (m >= M) continue;
      float* dst = ws + ((size_t)blockIdx.y * M + m) * N;
      const f32x4_t sum = acc[r][g];
      if (vec && f0 + 3 < N) {
        *reinterpret_cast<float4*>(dst + f0) = make_float4(sum[0], sum[1], sum[2], sum[3]);
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v)
          if (f0 + v < N) dst[f0 + v] = sum[v];
      }
    }
  }
}

// Splits whose partial sums a thread of the split sum + RMSNorm loads before
// adding them.  The wide split sums keep one split per load: with many
// workgroups in flight, batching measured 0.2-0.4 us slower at 5-10 splits.
constexpr int kNormBatch = 8;

// y[i] = T(sum over s of ws[s][i]) for i < count (= M N), splits added in
// order; with RES, y[i] = T(float(r[i]) + float(T(sum))), the text encoder's
// dq_add after the qmm (EpResidAdd's arithmetic; y may be r).  VEC (count % 4
// == 0, y and r 8-byte aligned): four outputs per thread, 16-byte partial
// loads, an 8-byte store; otherwise one output per thread.
template <int T, bool VEC, bool RES>
__global__ __launch_bounds__(256) void qskinny_reduce_kernel(const float* __restrict__ ws,
                                                             int splits, int count,
                                                             const uint16_t* r, uint16_t* y) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  if constexpr (VEC) {
    const int i = t * 4;
    if (i >= count) return;
    float4 a = *reinterpret_cast<const float4*>(ws + i);
#pragma unroll 4
    for (int sp = 1; sp < splits; ++sp) {
      const float4 v = *reinterpret_cast<const float4*>(ws + (size_t)sp * count + i);
      a.x += v.x;
      a.y += v.y;
      a.z += v.z;
      a.w += v.w;
    }
    if constexpr (RES) {
      const uint2 rv = *reinterpret_cast<const uint2*>(r + i);
      a.x = staged_value<T>(rv.x & 0xFFFFu) + round_to(a.x, T);
      a.y = staged_value<T>(rv.x >> 16) + round_to(a.y, T);
      a.z = staged_value<T>(rv.y & 0xFFFFu) + round_to(a.z, T);
      a.w = staged_value<T>(rv.y >> 16) + round_to(a.w, T);
    }
    *reinterpret_cast<uint2*>(y + i) = make_uint2(Elem<T>::pack2(a.x, a.y), Elem<T>::pack2(a.z, a.w));
  } else {
    if (t >= count) return;
    float a = ws[t];
#pragma unroll 4
    for (int sp = 1; sp < splits; ++sp) a += ws[(size_t)sp * count + t];
    if constexpr (RES) a = staged_value<T>(r[t]) + round_to(a, T);
    y[t] = Elem<T>::out(a);
  }
}

// One row m per workgroup: r = T(float(resid) + float(T(sum over s of
// ws[s][m][:]))) as qskinny_reduce_kernel's RES form, stored to y, then the
// row's RMSNorm h = T(r * rsqrt(mean(r^2) + eps) * nw) with the arithmetic of
// the T-input RMSNorm kernel (thread i takes the 8-value pieces i, i + 256,
// ..., the same fma order, wave and workgroup sums): the text encoder's
// o projection, dq_add and the RMSNorm before the MLP in one launch instead
// of two.  N % 8 == 0, N <= 2048 V, 16-byte aligned rows; y may be resid.
template <int T, int V>
__global__ __launch_bounds__(256) void qskinny_reduce_norm_kernel(
    const float* __restrict__ ws, int splits, int count, int N, const uint16_t* r, uint16_t* y,
    const float* __restrict__ nw, uint16_t* __restrict__ h, float eps) {
  __shared__ float part[4];
  const int n8 = N >> 3;
  const size_t row = (size_t)blockIdx.x * N;
  const float4* wr = reinterpret_cast<const float4*>(nw);
  uint4 v[V];
  float4 wv[V][2];  // the norm weights load beside the sums, not after them
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * 256;
    if (idx < n8) {
      wv[i][0] = wr[2 * idx];
      wv[i][1] = wr[2 * idx + 1];
    }
  }
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * 256;
    v[i] = make_uint4(0u, 0u, 0u, 0u);
    if (idx < n8) {
      const size_t o = row + 8 * (size_t)idx;
      // The partial sums of kNormBatch splits are loaded before the first of
      // their adds (one workgroup per row has few loads in flight otherwise:
      // a memory latency per split); the adds keep split order.
      float4 a0 = *reinterpret_cast<const float4*>(ws + o);
      float4 a1 = *reinterpret_cast<const float4*>(ws + o + 4);
      for (int s0 = 1; s0 < splits; s0 += kNormBatch) {
        float4 p0[kNormBatch], p1[kNormBatch];
#pragma unroll
        for (int j = 0; j < kNormBatch; ++j) {
          const size_t so = (size_t)min(s0 + j, splits - 1) * count + o;
          p0[j] = *reinterpret_cast<const float4*>(ws + so);
          p1[j] = *reinterpret_cast<const float4*>(ws + so + 4);
        }
        // Selects, not a branch: a branch would let the compiler sink each
        // load to its add again.
#pragma unroll
        for (int j = 0; j < kNormBatch; ++j) {
          const bool take = s0 + j < splits;
          a0.x = take ? a0.x + p0[j].x : a0.x;
          a0.y = take ? a0.y + p0[j].y : a0.y;
          a0.z = take ? a0.z + p0[j].z : a0.z;
          a0.w = take ? a0.w + p0[j].w : a0.w;
          a1.x = take ? a1.x + p1[j].x : a1.x;
          a1.y = take ? a1.y + p1[j].y : a1.y;
          a1.z = take ? a1.z + p1[j].z : a1.z;
          a1.w = take ? a1.w + p1[j].w : a1.w;
        }
      }
      const uint4 rv = *reinterpret_cast<const uint4*>(r + o);
      const float f[8] = {staged_value<T>(rv.x & 0xFFFFu) + round_to(a0.x, T),
                          staged_value<T>(rv.x >> 16) + round_to(a0.y, T),
                          staged_value<T>(rv.y & 0xFFFFu) + round_to(a0.z, T),
                          staged_value<T>(rv.y >> 16) + round_to(a0.w, T),
                          staged_value<T>(rv.z & 0xFFFFu) + round_to(a1.x, T),
                          staged_value<T>(rv.z >> 16) + round_to(a1.y, T),
                          staged_value<T>(rv.w & 0xFFFFu) + round_to(a1.z, T),
                          staged_value<T>(rv.w >> 16) + round_to(a1.w, T)};
      v[i] = make_uint4(Elem<T>::pack2(f[0], f[1]), Elem<T>::pack2(f[2], f[3]),
                        Elem<T>::pack2(f[4], f[5]), Elem<T>::pack2(f[6], f[7]));
      *reinterpret_cast<uint4*>(y + o) = v[i];
    }
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
  for (int i = 0; i < 4; ++i) total += part[i];
  const float inv = __frsqrt_rn(total / (float)N + eps);
#pragma unroll
  for (int i = 0; i < V; ++i) {
    const int idx = threadIdx.x + i * 256;
    if (idx < n8) {
      const float4 w0 = wv[i][0], w1 = wv[i][1];
      const float ww[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
      const uint32_t q[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = Elem<T>::pack2(Elem<T>::param((uint16_t)(q[e] & 0xFFFFu)) * inv * ww[2 * e],
                              Elem<T>::param((uint16_t)(q[e] >> 16)) * inv * ww[2 * e + 1]);
      *reinterpret_cast<uint4*>(h + row + 8 * (size_t)idx) = make_uint4(o[0], o[1], o[2], o[3]);
    }
  }
}

// A K split of the few-row product: `per` pieces of 512 k per split, rr
// 16-row tiles per wave, rw waves per workgroup (qskinny_rows_kernel).
struct SplitPlan {
  int per, splits, rr, rw;
  bool ok;
};

// Fewest rows for the K split of a plain product: at M <= 5 all of x fits
// LDS up to K = 9728 and the unsplit kernels were as fast as the split that
// the rows kernel replaced ([2560 x 9728] M = 4: 10.2 us either way).
constexpr int kSplitMinM = 6;

// Bytes of the rows kernel's x slice in LDS.
size_t split_x_bytes(int per, int m) { return (size_t)m * (1024 * (size_t)per + 16); }

// The rows kernel's plan: 64-row workgroups (four waves of one tile), 128
// where that leaves more than 800 workgroups; two 512-k pieces per split
// from K = 8192, and from K = 4096 where that still leaves 160 workgroups of
// 64 rows, one below.  Forced plans on 12 shapes (M = 8-30, weights
// from HBM, the split-sum launch included) put it within 4% of the fastest
// rows plan on each ([19456 x 2560] M = 30: 128-row workgroups 15.8 us
// against 17.0 at 64; [2560 x 9728]: two pieces 12.4 / 10.3 / 9.6 us at M =
// 30 / 16 / 8 against 13.4 / 10.9 / 10.0 with one; [2560 x 4096] M = 30
// 8.9 against 9.0; [6144 x 2560] and [3072 x 3072] one piece, 9.2 and 8.1
// us against 10.8 and 8.5; [1000 x 4608] M = 12 / 24 one piece, 5.8 / 6.9 us
// against 6.4 / 7.9 on 80 workgroups).
SplitPlan rows_plan(int k, int n, int m) {
  const int pieces = k / 512;
  const long groups = (n + 63) / 64;
  const int per = pieces >= 16 || (pieces >= 8 && groups * ((pieces + 1) / 2) >= 160) ? 2 : 1;
  const int splits = (pieces + per - 1) / per;
  (void)m;
  return SplitPlan{per, splits, groups * splits > 800 ? 2 : 1, 4, true};
}

// Weight bytes from which the rows kernel's split runs where an unsplit
// kernel would finish in one round of the CUs: [9728 x 2560] M = 16 (12.5
// MB) 10.3 -> 9.6 us; [6144 x 2560] M = 16 (7.9 MB) ties (7.55 / 7.65).
constexpr size_t kRowsOverOneRound = (size_t)10 << 20;

// Whether (and how) the few-row product splits K: the rows kernel, from M =
// 6 (from 1 row for the residual-add form, which the unsplit kernels do not
// have) to 32, K % 512 == 0 with at least two pieces of 512.  Up to 16 rows
// the unsplit kernels stay where they finish in one round of the CUs below
// kRowsOverOneRound bytes of weights (the split's second launch costs more
// than it saves: [2560 x 2560] M = 12 4.7 us unsplit, 6.1 split), and where
// all of x fits LDS without the multi-tile kernel.  Past 16 rows it runs
// wherever it plans; the tile kernel's 32-row tiles are its alternative (M =
// 30, same box, the split-sum launch included: [9728 x 2560] 14.8 -> 11.7
// us, [19456 x 2560] 18.9 -> 15.8, [6144 x 2560] 12.7 -> 9.1 against the
// split kernel it replaced, [2560 x 9728] 17.6 -> 12.2).
SplitPlan plan_split(int k, int n, int m, bool resid = false) {
  const SplitPlan best{0, 0, 0, 0, false};
  if (k % 512 != 0 || k / 512 < 2 || m < (resid ? 1 : kSplitMinM) || m > 2 * kRows) return best;
  const long tiles = (n + kRows - 1) / kRows;
  if (m <= kRows && !resid) {
    const LdsPlan lp = plan_lds(k, n, m);
    if (lp.ok) {
      const long groups = (tiles + lp.tpw - 1) / lp.tpw;
      if (groups <= 256 && (size_t)n * k / 2 < kRowsOverOneRound) return best;
    } else if ((size_t)m * k * 2 <= (size_t)kXLdsMax) {
      return best;
    }
  }
  return rows_plan(k, n, m);
}

template <int T, int R, int W, int CH>
hipError_t launch_rows_k(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                         const uint16_t* x, float* ws, int k, int n, int m, const SplitPlan& p,
                         bool vec, hipStream_t stream) {
  const int wg_rows = kRows * R * W;
  const dim3 grid((unsigned)((n + wg_rows - 1) / wg_rows), (unsigned)p.splits);
  if (m > kRows)
    hipLaunchKernelGGL((qskinny_rows_kernel<T, R, W, 2, CH>), grid, dim3(64 * W),
                       split_x_bytes(p.per, m), stream, w, s, b, x, ws, m, n, k, p.per, vec);
  else
    hipLaunchKernelGGL((qskinny_rows_kernel<T, R, W, 1, CH>), grid, dim3(64 * W),
                       split_x_bytes(p.per, m), stream, w, s, b, x, ws, m, n, k, p.per, vec);
  return hipGetLastError();
}

template <int T, int R, int W>
hipError_t launch_rows_rw(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          const uint16_t* x, float* ws, int k, int n, int m, const SplitPlan& p,
                          bool vec, hipStream_t stream) {
  if (p.per == 1) return launch_rows_k<T, R, W, 4>(w, s, b, x, ws, k, n, m, p, vec, stream);
  if (p.per == 2) return launch_rows_k<T, R, W, 8>(w, s, b, x, ws, k, n, m, p, vec, stream);
  return hipErrorInvalidValue;
}

// The rows kernel: 1 or 2 tiles per wave, 4 or 8 waves, 1 or 2 pieces of 512 k.
template <int T>
hipError_t launch_rows(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                       float* ws, int k, int n, int m, const SplitPlan& p, bool vec,
                       hipStream_t stream) {
  if (p.rw == 4) {
    if (p.rr == 1) return launch_rows_rw<T, 1, 4>(w, s, b, x, ws, k, n, m, p, vec, stream);
    if (p.rr == 2) return launch_rows_rw<T, 2, 4>(w, s, b, x, ws, k, n, m, p, vec, stream);
  } else if (p.rw == 8) {
    if (p.rr == 1) return launch_rows_rw<T, 1, 8>(w, s, b, x, ws, k, n, m, p, vec, stream);
    if (p.rr == 2) return launch_rows_rw<T, 2, 8>(w, s, b, x, ws, k, n, m, p, vec, stream);
  }
  return hipErrorInvalidValue;
}

// Rows of the fused split sum + residual + RMSNorm: N % 8 == 0, at most 8192
// columns, 16-byte aligned rows and partial sums.
bool norm_fits(int n, const void* resid, const void* y, const float* nw, const void* h,
               const float* ws) {
  auto a16 = [](const void* p) { return ((uintptr_t)p & 15u) == 0; };
  return n % 8 == 0 && n <= 2048 * 4 && a16(resid) && a16(y) && a16(nw) && a16(h) && a16(ws);
}

// The split kernel alone: fp32 partial sums ws[split][m][n].
template <int T>
hipError_t launch_split_partials(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                                 const uint16_t* x, float* ws, int k, int n, int m,
                                 const SplitPlan& p, hipStream_t stream) {
  const bool vec = n % 4 == 0 && ((uintptr_t)ws & 15u) == 0;
  return launch_rows<T>(w, s, b, x, ws, k, n, m, p, vec, stream);
}

template <int T>
hipError_t launch_split(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                        const uint16_t* resid, uint16_t* y, float* ws, int k, int n, int m,
                        const SplitPlan& p, hipStream_t stream, const float* nw = nullptr,
                        uint16_t* h = nullptr, float eps = 0.f) {
  const hipError_t e = launch_split_partials<T>(w, s, b, x, ws, k, n, m, p, stream);
  if (e != hipSuccess) return e;
  const int count = m * n;
  if (nw) {
    const int v = (n / 8 + 255) / 256;
    if (v <= 1)
      hipLaunchKernelGGL((qskinny_reduce_norm_kernel<T, 1>), dim3(m), dim3(256), 0, stream, ws,
                         p.splits, count, n, resid, y, nw, h, eps);
    else if (v == 2)
      hipLaunchKernelGGL((qskinny_reduce_norm_kernel<T, 2>), dim3(m), dim3(256), 0, stream, ws,
                         p.splits, count, n, resid, y, nw, h, eps);
    else
      hipLaunchKernelGGL((qskinny_reduce_norm_kernel<T, 4>), dim3(m), dim3(256), 0, stream, ws,
                         p.splits, count, n, resid, y, nw, h, eps);
    return hipGetLastError();
  }
  // The vector form loads float4 partials at ws + split * count + i (i % 4 == 0)
  // and stores four T values: ws 16-byte and y / resid 8-byte aligned.
  const bool rvec = count % 4 == 0 && ((uintptr_t)ws & 15u) == 0 && ((uintptr_t)y & 7u) == 0 &&
                    ((uintptr_t)resid & 7u) == 0;
  const dim3 grid((unsigned)(((rvec ? count / 4 : count) + 255) / 256));
  if (resid) {
    if (rvec)
      hipLaunchKernelGGL((qskinny_reduce_kernel<T, true, true>), grid, dim3(256), 0, stream, ws,
                         p.splits, count, resid, y);
    else
      hipLaunchKernelGGL((qskinny_reduce_kernel<T, false, true>), grid, dim3(256), 0, stream, ws,
                         p.splits, count, resid, y);
  } else {
    if (rvec)
      hipLaunchKernelGGL((qskinny_reduce_kernel<T, true, false>), grid, dim3(256), 0, stream, ws,
                         p.splits, count, nullptr, y);
    else
      hipLaunchKernelGGL((qskinny_reduce_kernel<T, false, false>), grid, dim3(256), 0, stream, ws,
                         p.splits, count, nullptr, y);
  }
  return hipGetLastError();
}

template <int T>
hipError_t launch_t(const uint32_t* w, const uint16_t* s, const uint16_t* b, const uint16_t* x,
                    uint16_t* y, int k, int n, int m, hipStream_t stream, SplitWs ws) {
  const SplitPlan sp = plan_split(k, n, m);
  if (sp.ok && ws.p && ws.bytes >= (size_t)sp.splits * m * n * sizeof(float))
    return launch_split<T>(w, s, b, x, nullptr, y, ws.p, k, n, m, sp, stream);
  if (m > kRows) return hipErrorInvalidValue;  // past 16 rows only the K split runs
  const bool vec = n % 4 == 0 && ((uintptr_t)y & 7u) == 0;
  const LdsPlan lp = plan_lds(k, n, m);
  if (lp.ok) {
    switch (lp.tpw) {
      case 1: return launch_lds_t<T, 1>(w, s, b, x, y, k, n, m, lp, vec, stream);
      case 2: return launch_lds_t<T, 2>(w, s, b, x, y, k, n, m, lp, vec, stream);
      case 3: return launch_lds_t<T, 3>(w, s, b, x, y, k, n, m, lp, vec, stream);
      default: return launch_lds_t<T, 4>(w, s, b, x, y, k, n, m, lp, vec, stream);
    }
  }
  switch (skinny_waves(n, k)) {
    case 1: return launch_w<T, 1>(w, s, b, x, y, k, n, m, vec, stream);
    case 2: return launch_w<T, 2>(w, s, b, x, y, k, n, m, vec, stream);
    case 4: return launch_w<T, 4>(w, s, b, x, y, k, n, m, vec, stream);
    case 8: return launch_w<T, 8>(w, s, b, x, y, k, n, m, vec, stream);
    default: return launch_w<T, 16>(w, s, b, x, y, k, n, m, vec, stream);
  }
}

}  // namespace

bool qskinny_supported(int k, int n, int m, int dtype) {
  return m >= 1 && m <= kQskinnyMaxM && n >= 1 && k >= kChunkK && k % kChunkK == 0 &&
         (dtype == kBf16 || dtype == kF16) && (size_t)n * k / 2 < ((size_t)1 << 32) &&
         (size_t)m * k * 2 < ((size_t)1 << 31);
}

hipError_t launch_qskinny_resid_add(const uint32_t* w, const void* scales, const void* biases,
                                    const void* x, const void* resid, void* y, int k, int n, int m,
                                    int dtype, hipStream_t stream, SplitWs ws) {
  if (!qskinny_supported(k, n, m, dtype)) return hipErrorInvalidValue;
  const SplitPlan sp = plan_split(k, n, m, true);
  if (!sp.ok || !ws.p || ws.bytes < (size_t)sp.splits * m * n * sizeof(float))
    return hipErrorInvalidValue;
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  const auto* rr = static_cast<const uint16_t*>(resid);
  auto* yy = static_cast<uint16_t*>(y);
  if (dtype == kBf16) return launch_split<kBf16>(w, s, b, xx, rr, yy, ws.p, k, n, m, sp, stream);
  return launch_split<kF16>(w, s, b, xx, rr, yy, ws.p, k, n, m, sp, stream);
}

bool qskinny_resid_add_norm_fits(int k, int n, int m, int dtype, const void* resid,
                                 const void* y, const float* norm_w, const void* h, SplitWs ws) {
  if (!qskinny_supported(k, n, m, dtype)) return false;
  const SplitPlan sp = plan_split(k, n, m, true);
  return sp.ok && ws.p && ws.bytes >= (size_t)sp.splits * m * n * sizeof(float) &&
         norm_fits(n, resid, y, norm_w, h, ws.p);
}

hipError_t launch_qskinny_resid_add_norm(const uint32_t* w, const void* scales,
                                         const void* biases, const void* x, const void* resid,
                                         void* y, const float* norm_w, void* h, float eps, int k,
                                         int n, int m, int dtype, hipStream_t stream, SplitWs ws) {
  if (!qskinny_resid_add_norm_fits(k, n, m, dtype, resid, y, norm_w, h, ws))
    return hipErrorInvalidValue;
  const SplitPlan sp = plan_split(k, n, m, true);
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  const auto* rr = static_cast<const uint16_t*>(resid);
  auto* yy = static_cast<uint16_t*>(y);
  auto* hh = static_cast<uint16_t*>(h);
  if (dtype == kBf16)
    return launch_split<kBf16>(w, s, b, xx, rr, yy, ws.p, k, n, m, sp, stream, norm_w, hh, eps);
  return launch_split<kF16>(w, s, b, xx, rr, yy, ws.p, k, n, m, sp, stream, norm_w, hh, eps);
}

size_t qskinny_split_bytes(int k, int n, int m) {
  const SplitPlan sp = plan_split(k, n, m);
  return sp.ok ? (size_t)sp.splits * m * n * sizeof(float) : 0;
}

hipError_t launch_qskinny_swiglu(const uint32_t* w, const void* scales, const void* biases,
                                 const void* x, void* y, int ldy, int k, int n, int m, int width,
                                 float in_scale, float out_scale, int dtype, hipStream_t stream,
                                 SplitWs ws) {
  if (!qskinny_supported(k, n, m, dtype) || n != 2 * width || ldy < width)
    return hipErrorInvalidValue;
  const SplitPlan sp = plan_split(k, n, m, true);
  if (!sp.ok || !ws.p || ws.bytes < (size_t)sp.splits * m * n * sizeof(float))
    return hipErrorInvalidValue;
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  const hipError_t e =
      dtype == kBf16 ? launch_split_partials<kBf16>(w, s, b, xx, ws.p, k, n, m, sp, stream)
                     : launch_split_partials<kF16>(w, s, b, xx, ws.p, k, n, m, sp, stream);
  if (e != hipSuccess) return e;
  return launch_reduce_swiglu(ws.p, sp.splits, m, width, y, ldy, in_scale, out_scale, dtype,
                              stream);
}

size_t qskinny_resid_split_bytes(int k, int n, int m) {
  const SplitPlan sp = plan_split(k, n, m, true);
  return sp.ok ? (size_t)sp.splits * m * n * sizeof(float) : 0;
}

int qskinny_splits(int k, int n, int m) {
  const SplitPlan sp = plan_split(k, n, m);
  return sp.ok ? sp.splits : 1;
}

hipError_t launch_qskinny(const uint32_t* w, const void* scales, const void* biases, const void* x,
                          void* y, int k, int n, int m, int dtype, hipStream_t stream, SplitWs ws) {
  if (!qskinny_supported(k, n, m, dtype)) return hipErrorInvalidValue;
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  if (dtype == kBf16) return launch_t<kBf16>(w, s, b, xx, yy, k, n, m, stream, ws);
  return launch_t<kF16>(w, s, b, xx, yy, k, n, m, stream, ws);
}

}  // namespace imq
