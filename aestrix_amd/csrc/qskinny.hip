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

// ---- K split: the multi-tile kernel over a range of K, for long K ----
//
// Workgroup (g, s) owns TPW 16-row tiles and the K pieces [s per, s per + per)
// for TG groups of 16 tokens (M <= 16 TG tokens; each dequantized weight
// fragment feeds one MFMA per group)
// (512 k each, the last range shorter); it stages only its x slice [M, 512
// per] in LDS (rows 1024 per + 16 bytes apart) and writes fp32 partial sums
// to ws[s][m][n]; qskinny_reduce_kernel adds the splits in order and rounds
// to T (deterministic).  The second launch costs about 2.9 us per call
// ([2560 x 9728] M = 16: 13.7 us, 10.8 without it), but adding the splits in
// the last-arriving workgroup of each tile group (arrival counters, no
// waiting) measured slower in every form tried: device-scope fences in every
// workgroup (each writes back and invalidates its XCD's L2) 84 us,
// agent-scope atomic stores and loads of the partial sums 19 us, atomic
// stores with one acquire fence in the last workgroup 16.8 us.  For [2560 x 9728] (160 row tiles, x of 16 rows 311
// KB) the 16-row kernel re-reads all of x from L2 per tile (about 50 MB for
// 12.5 MB of weights) on 160 workgroups; here each x byte is read once per
// tile group and split and the grid fills the CUs.
template <int T, int TPW, int W, int U, int TG>
__global__ __launch_bounds__(64 * W) void qskinny_split_kernel(const uint32_t* __restrict__ w,
                                                               const uint16_t* __restrict__ scales,
                                                               const uint16_t* __restrict__ biases,
                                                               const uint16_t* __restrict__ x,
                                                               float* __restrict__ ws, int M,
                                                               int N, int K, int per, bool vec) {
  constexpr int kWeightLoads = 3 * U * TPW < 63 ? 3 * U * TPW : 63;
  __shared__ f32x4_t part[W][TPW][TG][64];
  extern __shared__ uint4 xs[];  // x [M, 512 per], rows 1024 per + 16 bytes apart
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, h = lane >> 4;
  const int n0 = blockIdx.x * (kRows * TPW);
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

  uint32_t w_off[TPW], p_off[TPW];
#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const uint32_t row = (uint32_t)min(n0 + kRows * t + c, N - 1);
    w_off[t] = row * (uint32_t)(K / 2) + (uint32_t)h * 16u;
    p_off[t] = (row * (uint32_t)gpr + (uint32_t)(h >> 1)) * 2u;
  }
  f32x4_t acc[TPW][TG];
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g) acc[t][g] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  // B operand of token group g (16 tokens): row min(16 g + c, M - 1); columns
  // past M are never stored.
  int xrow[TG];
#pragma unroll
  for (int g = 0; g < TG; ++g) xrow[g] = min(16 * g + c, M - 1);
  bool first = true;
  for (int ch0 = wave; ch0 < chunks; ch0 += W * U) {
    u32x4_t wv[U][TPW];
    uint16_t sv[U][TPW], bv[U][TPW];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t ch = (uint32_t)(c0 + min(ch0 + u * W, chunks - 1));
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        wv[u][t] = load_b128(wr, w_off[t], ch * 64u);
        sv[u][t] = __builtin_amdgcn_raw_buffer_load_b16(sr, p_off[t], ch * 4u, 0);
        bv[u][t] = __builtin_amdgcn_raw_buffer_load_b16(br, p_off[t], ch * 4u, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if (first) {
      IMQ_WAIT_VMCNT(kWeightLoads);
      __builtin_amdgcn_s_barrier();
      first = false;
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const bool valid = ch0 + u * W < chunks;
      const int j = min(ch0 + u * W, chunks - 1);
      u32x4_t xf[TG][4];
#pragma unroll
      for (int g = 0; g < TG; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          xf[g][i] = *reinterpret_cast<const u32x4_t*>(reinterpret_cast<const char*>(xs) +
                                                      xrow[g] * xstride + j * 256 + (4 * h + i) * 16);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float sc = valid ? Elem<T>::param(sv[u][t]) : 0.0f;
        const float s24 = sc * 0x1p24f, s20 = sc * 0x1p20f;
        const float b = valid ? Elem<T>::param(bv[u][t]) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          uint32_t pq[4];
          Elem<T>::dequant(wv[u][t][i], s24, s20, b, pq);
          const u32x4_t a = u32x4_t{pq[0], pq[1], pq[2], pq[3]};
#pragma unroll
          for (int g = 0; g < TG; ++g) acc[t][g] = mfma16x16x32<T>(a, xf[g][i], acc[t][g]);
        }
      }
    }
  }
  if (first) {
    IMQ_WAIT_VMCNT(0);
    __builtin_amdgcn_s_barrier();
  }
#pragma unroll
  for (int t = 0; t < TPW; ++t)
#pragma unroll
    for (int g = 0; g < TG; ++g) part[wave][t][g][lane] = acc[t][g];
  __syncthreads();
  if (wave >= TPW) return;
  const int t = wave;
  const int f0 = n0 + kRows * t + 4 * h;
#pragma unroll
  for (int g = 0; g < TG; ++g) {
    const int m = 16 * g + c;
    if (m >= M) continue;
    f32x4_t sum = part[0][t][g][lane];
#pragma unroll
    for (int i = 1; i < W; ++i) sum += part[i][t][g][lane];
    float* dst = ws + ((size_t)blockIdx.y * M + m) * N;
    if (vec && f0 + 3 < N) {
      *reinterpret_cast<float4*>(dst + f0) = make_float4(sum[0], sum[1], sum[2], sum[3]);
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (f0 + v < N) dst[f0 + v] = sum[v];
    }
  }
}

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
      float4 a0 = *reinterpret_cast<const float4*>(ws + o);
      float4 a1 = *reinterpret_cast<const float4*>(ws + o + 4);
      for (int sp = 1; sp < splits; ++sp) {
        const float4 p0 = *reinterpret_cast<const float4*>(ws + (size_t)sp * count + o);
        const float4 p1 = *reinterpret_cast<const float4*>(ws + (size_t)sp * count + o + 4);
        a0.x += p0.x;
        a0.y += p0.y;
        a0.z += p0.z;
        a0.w += p0.w;
        a1.x += p1.x;
        a1.y += p1.y;
        a1.z += p1.z;
        a1.w += p1.w;
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

struct SplitPlan {
  int tpw, per, splits, u;
  bool ok;
};

constexpr int kSplitWaves = 8;
// Fewest rows for the K split: at M <= 5 all of x fits LDS up to K = 9728
// and the unsplit kernels stay faster ([2560 x 9728] M = 4: 10.2 us unsplit,
// 10.2 us for the best split plan).
constexpr int kSplitMinM = 6;

// Bytes of the split kernel's x slice in LDS.
size_t split_x_bytes(int per, int m) { return (size_t)m * (1024 * (size_t)per + 16); }

// Taken, from M = 6, where the unsplit kernels would stream x per chunk from
// L2 (x [M, K] past the 96 KiB LDS budget and not the multi-tile kernel's
// case), and where it saves more than a quarter of the multi-tile kernel's
// wave work (the plan rule below).  Its first planner (M >= 8, at most 128
// row tiles or K >= 8192, least L2 traffic), measured with the weights from
// HBM (same box, A/B builds): [2560 x 9728] M = 8 / 12
// / 16 13.9 / 15.9 / 18.1 -> 13.2 / 13.5 / 13.8 us, [1000 x 4608] M = 12 9.5
// -> 6.3 us, [1030 x 4608] M = 13 9.6 -> 6.6 us; elsewhere slower: M = 4 and
// 5 at K = 9728 (x in LDS: 11.7 -> 12.2, 11.9 -> 12.9 us), [2560 x 4096] M =
// 16 (9.4 -> 10.0), [3072 x 3072] at M = 4 / 8 / 16 (6.3 -> 8.3-8.9 us): there
// the second launch and the partial sums cost more than the better-filled
// grid saves.  17 to 32 rows (two token groups per weight fragment) take it
// wherever the row tiles are fewer than 256 (now 512), against the tile kernel's 32-row
// tiles and their split K (same box, A/B builds, M = 30 unless stated):
// [2560 x 9728] 19.1 -> 17.0 us (M = 17 18.0 -> 15.9), [2560 x 4096] 14.7 ->
// 13.2, [2560 x 2560] 11.4 -> 8.0, [1000 x 4608] 13.6 -> 7.2, [3072 x 3072]
// 12.7 -> 12.4, M = 24 [1024 x 2560] 10.5 -> 5.8.
//
// Plan: among the (tiles per workgroup, pieces per split) whose x slice fits
// 64 KB (80 KB for two token groups), the least wave work on the busiest CU:
// ceil(workgroups / 256) x U x TPW x TG, U = the chunk rounds of a wave
// (ceil(4 per / 8): an odd number of pieces leaves half the waves a dummy
// round); ties go to more tiles per workgroup (fewer x slices), then to
// fewer splits.  Measured against every plan forced in turn on 15 shapes
// (same box, weights from HBM): within 1.4% of the fastest on average (5.8%
// at most), 12.5% faster on average than the former choice (the least L2
// traffic among grids of at least 256 workgroups): [2560 x 9728] M = 8 / 12
// / 16 13.2 / 13.5 / 13.7 -> 11.1 / 11.6 / 12.5 us, M = 30 [2560 x 4096]
// 13.3 -> 9.2, [3072 x 3072] 12.3 -> 8.5, [2560 x 2560] 7.9 -> 6.8,
// [1024 x 9728] M = 16 10.1 -> 8.2 us.
// resid: for the residual-add form, which the unsplit kernels do not have
// (the tile kernel is its alternative): from 1 row, and where the unsplit
// kernels would be preferred for a plain product.
SplitPlan plan_split(int k, int n, int m, bool resid = false) {
  SplitPlan best{0, 0, 0, 0, false};
  if (k % 512 != 0 || k / 512 < 2 || m < (resid ? 1 : kSplitMinM) || m > 2 * kRows) return best;
  const int pieces = k / 512;
  const long tiles = (n + kRows - 1) / kRows;
  // Up to 16 rows the unsplit kernels are the alternative: the multi-tile
  // kernel where it plans (in one round of the CUs it stays; in more it is
  // compared by the same wave work below), otherwise the kernels with all of
  // x in LDS; past 16 rows (two token groups, this kernel only) the tile
  // kernel is, from 512 row tiles on: M = 30 / 24 / 17 [6144 x 2560] 13.3 /
  // 13.5 / 12.7 -> 12.8 / 12.1 / 10.1 us, [4096 x 2560] M = 30 12.6 -> 9.5
  // split; [9728 x 2560] M = 30 / 20 15.0 / 13.8 on the tile kernel against
  // 15.8 / 14.8 for the planned split, [19456 x 2560] M = 30 18.3 against 23
  // or more for any split.
  long lds_work = -1;
  if (m <= kRows && !resid) {
    const LdsPlan lp = plan_lds(k, n, m);
    if (lp.ok) {
      const long groups = (tiles + lp.tpw - 1) / lp.tpw;
      if (groups <= 256) return best;
      lds_work = (groups + 255) / 256 * ((k / kChunkK + kLdsWaves - 1) / kLdsWaves) * lp.tpw;
    } else if ((size_t)m * k * 2 <= (size_t)kXLdsMax) {
      return best;
    }
  } else if (m > kRows && tiles >= 512) {
    return best;
  }
  const int tg = m > kRows ? 2 : 1;
  long best_work = -1;
  for (int tpw = 1; tpw <= 4; ++tpw) {
    const long groups = (tiles + tpw - 1) / tpw;
    for (int per = 1; per <= pieces; ++per) {
      const int splits = (pieces + per - 1) / per;
      if (splits < 2) continue;
      // x slice budget: 64 KB beside the 32 KB of per-wave sums of one token
      // group; 80 KB beside the 64 KB of two (32 rows then still take two
      // 512-k pieces per split).
      if (split_x_bytes(per, m) > (m > kRows ? 80 : 64) * 1024) continue;
      const int u = std::max(1, std::min((per * 4 + kSplitWaves - 1) / kSplitWaves,
                                         max_u_lds(tpw, kSplitWaves)));
      const long work = (groups * splits + 255) / 256 * u * tpw * tg;
      if (best_work < 0 || work < best_work ||
          (work == best_work && (tpw > best.tpw || (tpw == best.tpw && splits < best.splits)))) {
        best_work = work;
        best = SplitPlan{tpw, per, splits, u, true};
      }
    }
  }
  // Against the multi-tile kernel in two or more rounds the split (a second
  // launch, partial sums) must save more than a quarter of the wave work:
  // [19456 x 2560] M = 12 / 16 (15 against 24) 21.6 / 22.4 -> 15.3 / 16.6 us.
  // In one round the second launch costs more than the split saves:
  // [2560 x 4096] M = 13 7.2 -> 8.3 us, [2560 x 2560] M = 12 4.7 -> 6.1,
  // [1024 x 2560] M = 12 4.6 -> 5.3 us when split.
  if (lds_work >= 0 && best.ok && best_work * 4 >= lds_work * 3) best.ok = false;
  return best;
}

template <int T, int TPW, int U>
hipError_t launch_split_tu(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                           const uint16_t* x, float* ws, int k, int n, int m, const SplitPlan& p,
                           bool vec, hipStream_t stream) {
  if constexpr (U > max_u_lds(TPW, kSplitWaves)) {
    return hipErrorInvalidValue;
  } else {
    const dim3 grid((unsigned)((n + kRows * TPW - 1) / (kRows * TPW)), (unsigned)p.splits);
    if (m > kRows)
      hipLaunchKernelGGL((qskinny_split_kernel<T, TPW, kSplitWaves, U, 2>), grid,
                         dim3(64 * kSplitWaves), split_x_bytes(p.per, m), stream, w, s, b, x, ws,
                         m, n, k, p.per, vec);
    else
      hipLaunchKernelGGL((qskinny_split_kernel<T, TPW, kSplitWaves, U, 1>), grid,
                         dim3(64 * kSplitWaves), split_x_bytes(p.per, m), stream, w, s, b, x, ws,
                         m, n, k, p.per, vec);
    return hipGetLastError();
  }
}

template <int T, int TPW>
hipError_t launch_split_t(const uint32_t* w, const uint16_t* s, const uint16_t* b,
                          const uint16_t* x, float* ws, int k, int n, int m, const SplitPlan& p,
                          bool vec, hipStream_t stream) {
  switch (p.u) {
    case 1: return launch_split_tu<T, TPW, 1>(w, s, b, x, ws, k, n, m, p, vec, stream);
    case 2: return launch_split_tu<T, TPW, 2>(w, s, b, x, ws, k, n, m, p, vec, stream);
    case 3: return launch_split_tu<T, TPW, 3>(w, s, b, x, ws, k, n, m, p, vec, stream);
    case 4: return launch_split_tu<T, TPW, 4>(w, s, b, x, ws, k, n, m, p, vec, stream);
    case 5:
    case 6: return launch_split_tu<T, TPW, 6>(w, s, b, x, ws, k, n, m, p, vec, stream);
    default: return launch_split_tu<T, TPW, 8>(w, s, b, x, ws, k, n, m, p, vec, stream);
  }
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
  switch (p.tpw) {
    case 1: return launch_split_t<T, 1>(w, s, b, x, ws, k, n, m, p, vec, stream);
    case 2: return launch_split_t<T, 2>(w, s, b, x, ws, k, n, m, p, vec, stream);
    case 3: return launch_split_t<T, 3>(w, s, b, x, ws, k, n, m, p, vec, stream);
    default: return launch_split_t<T, 4>(w, s, b, x, ws, k, n, m, p, vec, stream);
  }
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
