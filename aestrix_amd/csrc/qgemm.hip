// qgemm.hip -- dense quantized matmul for gfx950 on bf16 MFMA.
//
// y[M][N] = x[M][K] . deq(W)^T, fp32 accumulation, bf16 output: the prefill /
// DiT regime of MLX quantizedMM(transpose: true, groupSize: 64, bits: 4),
// i.e. the `affine_qmm_t_*` dispatches of the reference's direct engine
// (Sources/ImarelloDirect/DirectDiTStep.swift:374-406,
//  Sources/ImarelloDirect/DirectTELayer.swift:109-128).
//
// Design (one workgroup = 4 waves = a 128 x 256 output tile):
//  * Each wave owns a 128 (M) x 64 (N) sub-tile: 4 x 2 MFMA tiles of
//    v_mfma_f32_32x32x16_bf16, 128 fp32 accumulators per lane.
//  * The weight operand never goes through LDS.  In MFMA operand layout a lane
//    owns one output column n and 8 consecutive k; that is exactly one packed
//    uint32 word.  Per K-step of 64 (one quantization group) a lane loads the
//    16 bytes (4 words = 32 codes) of its half of the group and dequantizes them
//    in registers into four bf16x8 operands -- each code is dequantized once per
//    workgroup because the four waves split N, not M.
//  * The activation tile (128 x 64 bf16 = 16 KiB) is shared by the four waves
//    through LDS, double-buffered, with the 16-byte chunk index XOR-swizzled by
//    the row so that the MFMA operand reads are free of bank conflicts.
//  * K is consumed one quantization group per step; loads of step g+1 are
//    issued before the MFMAs of step g.
//  * Workgroup ids are remapped so that each XCD (ids are dealt round-robin to
//    the 8 XCDs) walks a contiguous, M-grouped stretch of tiles, keeping the
//    shared x and W panels in that XCD's L2.
#include "imq_device.hpp"
#include "imq_kernels.hpp"

namespace imq {
namespace {

constexpr int kThreads = 256;
constexpr int BM = 128;           // workgroup tile rows (M)
constexpr int BN = 256;           // workgroup tile cols (N)
constexpr int MT = BM / 32;       // MFMA row tiles per wave
constexpr int NT = BN / 4 / 32;   // MFMA col tiles per wave
constexpr int kGroupM = 8;        // M tiles per raster group
constexpr int kXcds = 8;

__device__ __forceinline__ void tile_coords(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  int id = bid;
  if (total % kXcds == 0) {
    const int per = total / kXcds;
    id = (bid % kXcds) * per + bid / kXcds;
  }
  const int per_group = kGroupM * tiles_n;
  const int grp = id / per_group;
  const int first_m = grp * kGroupM;
  const int gsz = (tiles_m - first_m < kGroupM) ? (tiles_m - first_m) : kGroupM;
  const int in = id - grp * per_group;
  tm = first_m + in % gsz;
  tn = in / gsz;
}

__global__ __launch_bounds__(kThreads, 2) void qgemm_kernel(const uint32_t* __restrict__ w,
                                                            const uint16_t* __restrict__ scales,
                                                            const uint16_t* __restrict__ biases,
                                                            const uint16_t* __restrict__ x,
                                                            uint16_t* __restrict__ y, int M, int N,
                                                            int K, int tiles_m, int tiles_n) {
  __shared__ uint4 a_lds[2][BM * 8];  // [buffer][row * 8 + (chunk ^ (row & 7))]

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r32 = lane & 31;
  const int h = lane >> 5;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int nw0 = tn * BN + wave * (NT * 32);
  const int wpr = K >> 3;
  const int gpr = K >> 6;

  // Weight rows of this lane (one per MFMA column tile).  Rows past N are
  // clamped to row 0: their columns are computed but never stored.
  const uint4* brow[NT];
  const uint16_t* srow[NT];
  const uint16_t* bbrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = nw0 + nt * 32 + r32;
    const size_t nn = (n < N) ? (size_t)n : 0;
    brow[nt] = reinterpret_cast<const uint4*>(w + nn * wpr) + h;
    srow[nt] = scales + nn * gpr;
    bbrow[nt] = biases + nn * gpr;
  }

  // Activation rows this thread stages: idx = tid + 256 * i -> row idx/8, chunk idx%8.
  const uint4* arow[4];
  bool aok[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + kThreads * i;
    const int row = idx >> 3;
    const int ch = idx & 7;
    aok[i] = (m0 + row) < M;
    const size_t rr = aok[i] ? (size_t)(m0 + row) : 0;
    arow[i] = reinterpret_cast<const uint4*>(x + rr * K) + ch;
  }

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.f;

  // Prologue: K-step 0.
  uint4 a_reg[4];
  uint4 b_reg[NT];
  uint32_t s_reg[NT], bi_reg[NT];
#pragma unroll
  for (int i = 0; i < 4; ++i) a_reg[i] = aok[i] ? arow[i][0] : make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    b_reg[nt] = brow[nt][0];
    s_reg[nt] = srow[nt][0];
    bi_reg[nt] = bbrow[nt][0];
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int idx = tid + kThreads * i;
    const int row = idx >> 3;
    const int ch = idx & 7;
    a_lds[0][row * 8 + (ch ^ (row & 7))] = a_reg[i];
  }
  __syncthreads();

  for (int g = 0; g < gpr; ++g) {
    const int cur = g & 1;
    const bool more = (g + 1) < gpr;
    uint4 a_nxt[4];
    uint4 b_nxt[NT];
    uint32_t s_nxt[NT], bi_nxt[NT];
    if (more) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        a_nxt[i] = aok[i] ? arow[i][(g + 1) * 8] : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        b_nxt[nt] = brow[nt][(g + 1) * 2];
        s_nxt[nt] = srow[nt][g + 1];
        bi_nxt[nt] = bbrow[nt][g + 1];
      }
    }

    // Dequantize this lane's 32 codes per column tile into 4 MFMA operands.
    bf16x8_t bfrag[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float s = bf16_to_f32(s_reg[nt]);
      const float b = bf16_to_f32(bi_reg[nt]);
      const float s24 = s * 0x1p24f;
      const float s20 = s * 0x1p20f;
      const uint32_t words[4] = {b_reg[nt].x, b_reg[nt].y, b_reg[nt].z, b_reg[nt].w};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint32_t p[4];
        dequant_word_bf16(words[kk], s24, s20, b, p);
        u32x4_t v = {p[0], p[1], p[2], p[3]};
        bfrag[nt][kk] = __builtin_bit_cast(bf16x8_t, v);
      }
    }

    // MFMA: physical k of operand slot j in step kk = 64 g + 32 h + 8 kk + j,
    // for both operands.
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      bf16x8_t afrag[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int row = mt * 32 + r32;
        const int ch = 4 * h + kk;
        afrag[mt] = __builtin_bit_cast(bf16x8_t, a_lds[cur][row * 8 + (ch ^ (row & 7))]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(afrag[mt], bfrag[nt][kk],
                                                                 acc[mt][nt], 0, 0, 0);
    }

    if (more) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int idx = tid + kThreads * i;
        const int row = idx >> 3;
        const int ch = idx & 7;
        a_lds[cur ^ 1][row * 8 + (ch ^ (row & 7))] = a_nxt[i];
      }
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        b_reg[nt] = b_nxt[nt];
        s_reg[nt] = s_nxt[nt];
        bi_reg[nt] = bi_nxt[nt];
      }
    }
    __syncthreads();
  }

  // Epilogue: accumulator r of a 32x32 tile holds row 8*(r/4) + 4*h + r%4, column r32.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int col = nw0 + nt * 32 + r32;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = m0 + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < M) y[(size_t)row * N + col] = (uint16_t)f32_to_bf16_int(acc[mt][nt][r]);
      }
    }
  }
}

}  // namespace

hipError_t launch_qgemm(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                        const uint16_t* x, uint16_t* y, int k, int n, int m, hipStream_t stream) {
  const int tiles_m = (m + BM - 1) / BM;
  const int tiles_n = (n + BN - 1) / BN;
  const dim3 grid((unsigned)tiles_m * (unsigned)tiles_n);
  hipLaunchKernelGGL(qgemm_kernel, grid, dim3(kThreads), 0, stream, w, scales, biases, x, y, m,
                     n, k, tiles_m, tiles_n);
  return hipGetLastError();
}

}  // namespace imq
