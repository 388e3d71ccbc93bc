// qgemm.hip -- dense quantized matmul for gfx950 on bf16 / f16 MFMA.
//
// y[M][N] = x[M][K] . deq(W)^T, fp32 accumulation, output in T (bf16, or f16
// for the reference's DiT kernels, DirectDiTStep.swift:82-85): the prefill /
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
#include <type_traits>

#include "epilogue.hpp"
#include "imq_device.hpp"
#include "imq_kernels.hpp"



namespace imq {
namespace {

constexpr int kThreads = 256;
// M tiles per raster group: an XCD's 32 CUs work on 4 M x 8 N tiles at a time,
// which is what its L2 must hold of each K slab (4 activation and 8 weight
// panels, about 8.9 MB per tile round at the headline against 12.7 MB for 8 x
// 4); time equal or up to 1% better than 8 or 2 on the six large shapes
// (same box, interleaved runs).
constexpr int kGroupM = 4;
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

// LDS slot of 16-byte chunk c (0..7) of activation-tile row r.  Conflict-free
// for the MFMA operand reads (16 lanes = 16 consecutive rows, one chunk) with
// 64 banks, and for 8-lane groups with 32 banks.
__device__ __forceinline__ int a_slot(int r, int c) {
  return r * 8 + (c ^ ((r & 7) ^ ((r >> 3) & 1)));
}

// LDS slot of 16-byte chunk c (0 .. 8 KG - 1) of a row of a KG-group
// activation tile (rows of 8 KG slots).  KG = 1 is a_slot; with 256-byte rows
// (KG = 2) the chunk index is XORed with the row's low four bits, so the 16
// rows an MFMA operand read touches at once hit 16 different 16-byte bank
// groups.  The swizzle is an involution: a_chunk_kg, its inverse, is the same
// XOR.
template <int KG>
__device__ __forceinline__ int a_slot_kg(int r, int c) {
  if constexpr (KG == 1) return a_slot(r, c);
  else return r * 16 + (c ^ (r & 15));
}
template <int KG>
__device__ __forceinline__ int a_chunk_kg(int r, int p) {
  if constexpr (KG == 1) return p ^ ((r & 7) ^ ((r >> 3) & 1));
  else return p ^ (r & 15);
}

// One 32x32x16 MFMA on 16-bit operands held as raw dwords (8 elements per lane).
template <int T>
__device__ __forceinline__ f32x16_t mfma32(u32x4_t a, u32x4_t b, f32x16_t c) {
  if constexpr (T == kBf16)
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                  __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

// One workgroup = 4 waves along N; a wave owns MT x NT MFMA tiles of 32x32,
// i.e. a (32 MT) x (32 NT) sub-tile; the workgroup tile is (32 MT) x (128 NT).
// EP is the output stage (epilogue.hpp), applied per output straight from the
// MFMA layout (emit1).  With EP::kPair (SwiGLU, NT == 2) a wave's column tile
// 0 holds gate rows and tile 1 the up rows of the same 32 output columns.
template <int T, int MT, int NT, class EP>
__global__ __launch_bounds__(kThreads, (MT * NT * 16 > 128) ? 1 : 2) void qgemm_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x, const EP ep,
    int M, int N, int K, int tiles_m, int tiles_n) {
  static_assert(!EP::kPair || NT == 2, "a gate/up pair takes two column tiles per wave");
  static_assert(!EP::kPartial, "the register-staged kernel does not split K");
  constexpr int BM = 32 * MT;
  constexpr int BN = 128 * NT;
  constexpr int A_CHUNKS = BM * 8;                 // 16-byte chunks per activation tile
  constexpr int A_PER_THREAD = A_CHUNKS / kThreads;
  __shared__ uint4 a_lds[2][A_CHUNKS];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int r32 = lane & 31;
  const int h = lane >> 5;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * BM;
  const int nw0 = tn * BN + wave * (NT * 32);
  const int pcol0 = tn * (BN / 2) + wave * 32;  // paired stage: this wave's first output
  const int wpr = K >> 3;
  const int gpr = K >> 6;

  // Weight rows of this lane (one per MFMA column tile).  Rows past N are
  // clamped to row 0: their columns are computed but never stored.
  const uint4* brow[NT];
  const uint16_t* srow[NT];
  const uint16_t* bbrow[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    int n = nw0 + nt * 32 + r32;
    if constexpr (EP::kPair)
      n = (nt == 0 ? ep.gate_row : ep.up_row) + min(pcol0 + r32, ep.width - 1);
    const size_t nn = (n < N) ? (size_t)n : 0;
    brow[nt] = reinterpret_cast<const uint4*>(w + nn * wpr) + h;
    srow[nt] = scales + nn * gpr;
    bbrow[nt] = biases + nn * gpr;
  }

  // Activation chunks this thread stages: idx = tid + 256 i -> row idx/8, chunk idx%8.
  // Rows past M are clamped to the last row (read, never stored).
  const uint4* arow[A_PER_THREAD];
#pragma unroll
  for (int i = 0; i < A_PER_THREAD; ++i) {
    const int idx = tid + kThreads * i;
    const int row = m0 + (idx >> 3);
    const size_t rr = (row < M) ? (size_t)row : (size_t)(M - 1);
    arow[i] = reinterpret_cast<const uint4*>(x + rr * K) + (idx & 7);
  }

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.f;

  // Prologue: K-step 0.
  uint4 a_reg[A_PER_THREAD];
  uint4 b_reg[NT];
  uint32_t s_reg[NT], bi_reg[NT];
#pragma unroll
  for (int i = 0; i < A_PER_THREAD; ++i) a_reg[i] = arow[i][0];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    b_reg[nt] = brow[nt][0];
    s_reg[nt] = srow[nt][0];
    bi_reg[nt] = bbrow[nt][0];
  }
#pragma unroll
  for (int i = 0; i < A_PER_THREAD; ++i) {
    const int idx = tid + kThreads * i;
    a_lds[0][a_slot(idx >> 3, idx & 7)] = a_reg[i];
  }
  __syncthreads();

  for (int g = 0; g < gpr; ++g) {
    const int cur = g & 1;
    const bool more = (g + 1) < gpr;
    // Loads of step g+1 (clamped to the last step: a harmless re-read).
    const int gn = more ? g + 1 : g;
    uint4 a_nxt[A_PER_THREAD];
    uint4 b_nxt[NT];
    uint32_t s_nxt[NT], bi_nxt[NT];
#pragma unroll
    for (int i = 0; i < A_PER_THREAD; ++i) a_nxt[i] = arow[i][gn * 8];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      b_nxt[nt] = brow[nt][gn * 2];
      s_nxt[nt] = srow[nt][gn];
      bi_nxt[nt] = bbrow[nt][gn];
    }

    // Dequantize this lane's 32 codes per column tile into 4 MFMA operands.
    u32x4_t bfrag[NT][4];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float sc = Elem<T>::param(s_reg[nt]);
      const float bi = Elem<T>::param(bi_reg[nt]);
      const float s24 = sc * 0x1p24f;
      const float s20 = sc * 0x1p20f;
      const uint32_t words[4] = {b_reg[nt].x, b_reg[nt].y, b_reg[nt].z, b_reg[nt].w};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        uint32_t p[4];
        Elem<T>::dequant(words[kk], s24, s20, bi, p);
        bfrag[nt][kk] = u32x4_t{p[0], p[1], p[2], p[3]};
      }
    }

    // MFMA: physical k of operand slot j in step kk = 64 g + 32 h + 8 kk + j,
    // for both operands.
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      u32x4_t afrag[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        afrag[mt] = __builtin_bit_cast(u32x4_t, a_lds[cur][a_slot(mt * 32 + r32, 4 * h + kk)]);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
          acc[mt][nt] = mfma32<T>(afrag[mt], bfrag[nt][kk], acc[mt][nt]);
    }

#pragma unroll
    for (int i = 0; i < A_PER_THREAD; ++i) {
      const int idx = tid + kThreads * i;
      a_lds[cur ^ 1][a_slot(idx >> 3, idx & 7)] = a_nxt[i];
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      b_reg[nt] = b_nxt[nt];
      s_reg[nt] = s_nxt[nt];
      bi_reg[nt] = bi_nxt[nt];
    }
    __syncthreads();
  }

  // Epilogue: accumulator r of a 32x32 tile holds row 8*(r/4) + 4*h + r%4,
  // column r32.  Each output is rounded to T (Elem::out, the same RNE as the
  // staged stores of the large-M kernel) and handed to the output stage.
  if constexpr (EP::kPair) {
    const int j = pcol0 + r32;
    if (j < ep.width) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = m0 + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (row < M) ep.emit1(row, j, Elem<T>::out(ep.value2(acc[mt][0][r], acc[mt][1][r])));
        }
    }
  } else {
    // 64 rows at a time through the activation buffer (64 x BN T values, 32
    // KiB at BN = 256): each lane's values from the MFMA layout as 2-byte LDS
    // stores, 16-byte chunk c of row r at chunk c ^ (4 ((r / 4) % 2)) (the two
    // rows 4 apart that a store instruction's lane halves write hit disjoint
    // banks), then 16 bytes per lane along the rows to the output stage
    // (emit8).  Written straight from the MFMA layout, each store instruction
    // covered two 128-byte row pieces: the x_embedder's qmm with its x16 into
    // 50 MB of fp32 output took 24.7 us per launch back to back, 18.3 this way
    // (a 50 MB fill: 8.7 us).
    static_assert(MT % 2 == 0 && BN * 64 * 2 <= (int)sizeof(a_lds), "64-row halves fit the buffer");
    constexpr int kCPR = BN / 8;                // 16-byte chunks per staged row
    constexpr int kIters = 64 * kCPR / kThreads;
    uint16_t* st = reinterpret_cast<uint16_t*>(&a_lds[0][0]);
    auto at = [&](int row, int col) {
      return st + row * BN + (((col >> 3) ^ (((row >> 2) & 1) << 2)) << 3) + (col & 7);
    };
    const int col0 = tn * BN;
#pragma unroll
    for (int half = 0; half < MT / 2; ++half) {
      __syncthreads();  // the previous half's reads (or the K loop's) are done
#pragma unroll
      for (int mh = 0; mh < 2; ++mh) {
        const int mt = 2 * half + mh;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int col = wave * (NT * 32) + nt * 32 + r32;
#pragma unroll
          for (int r = 0; r < 16; r += 2) {
            const int row = mh * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            const uint32_t v =
                Elem<T>::pack2(ep.value(acc[mt][nt][r]), ep.value(acc[mt][nt][r + 1]));
            *at(row, col) = (uint16_t)v;
            *at(row + 1, col) = (uint16_t)(v >> 16);
          }
        }
      }
      __syncthreads();
      const int c = tid % kCPR;
      const int col = col0 + c * 8;
      uint4 v[kIters];
#pragma unroll
      for (int i = 0; i < kIters; ++i)
        v[i] = *reinterpret_cast<const uint4*>(at((i * kThreads + tid) / kCPR, c * 8));
      if (col >= N) continue;
#pragma unroll
      for (int i = 0; i < kIters; ++i) {
        const int row = m0 + half * 64 + (i * kThreads + tid) / kCPR;
        if (row >= M) continue;
        if (ep.vec && col + 8 <= N) {
          ep.emit8(row, col, v[i]);
        } else {
          const uint32_t w4[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
          for (int e = 0; e < 8; ++e)
            if (col + e < N) ep.emit1(row, col + e, (uint16_t)(w4[e >> 1] >> (16 * (e & 1))));
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Large-M kernel: a (32 MT) x 256 workgroup tile, one wave per SIMD, the four
// waves side by side along N (each a (32 MT) x 64 sub-tile: MT x 2 MFMA tiles,
// up to 256 fp32 accumulators per lane in AGPRs).  Each code is dequantized
// once per workgroup.  A K-step covers two quantization groups: 128 K, eight
// k-slices of 16.
//
// Activations are staged by direct buffer->LDS loads (buffer_load_dwordx4 ...
// lds: lane L writes LDS base + 16 L, no VGPRs; the per-lane byte offset is
// fixed for the whole K loop and the K-step advance is a scalar offset, so a
// load costs no vector ALU work) into a 2-stage LDS ring.  Packed weights need
// no sharing between waves (each wave owns its columns), so they are loaded
// straight into registers.  Both are loaded one step ahead.  A weight load
// reads 16 rows x the step's 64 bytes (lane L: row L % 16, bytes 16 (L / 16)),
// 16 cache lines per instruction; two of them (rows 0-15 and 16-31 of a
// column tile) are turned into the 32-row MFMA operand layout by one
// v_permlane16_swap per dword (the 16-lane rows 1, 3 of the first trade places
// with rows 0, 2 of the second): lane (r32, h) then holds row r32's bytes
// [32 h, 32 h + 16) in the first register and [32 h + 16, 32 h + 32) in the
// second, i.e. all 64 codes of group h of the step.  Loaded directly in that
// layout, one instruction touched 32 rows x 32 bytes (32 lines) and the
// weights took about as many memory-pipeline cycles as the activations.
// Scales and biases are loaded eight groups at a time (16 bytes of a row per
// load, the four steps of an unrolled iteration, one iteration ahead): a
// lane's per-group 2-byte loads touch one cache line per row each and cost
// more memory-pipeline time than the weights and activations together, and 8
// bytes per two steps still cost 2-5% against none at all.  The K loop is unrolled by four steps so that the
// ring stage, the weight registers, the scale-block slot and the group's
// position in its block are compile-time constants: the compiler can prove
// that loads in flight into the other stage do not alias this stage's reads
// and emits no waits of its own in the loop.
//
// Step g (stage g % 2):
//  * s_waitcnt vmcnt(0) lgkmcnt(0) and a raw s_barrier (no fence, which would
//    wait for every outstanding load): this wave's loads of step g have
//    landed, and once every wave has passed, all of them have; every wave's
//    LDS reads of the other stage (step g-1) have returned, so it may be
//    refilled.
//  * The LDS reads and the weight dequant of k-slice 0, then the MFMAs of step
//    g-1's last k-slice with the loads of step g+1 (and, every other step, the
//    next scale block) issued between them.
//  * k-slices 0 .. 6: the MFMAs of slice i with the LDS reads and dequant of
//    slice i+1 interleaved; the MFMAs of slice 7 wait for the top of step g+1.
// Deferring the last slice keeps the matrix core busy through the barrier,
// the issue of the next step's loads and the LDS latency of the first slice.
//
// Requires K % 256 == 0 (whole scale blocks); other K take the
// register-staged kernel.
// ---------------------------------------------------------------------------
constexpr int kBigBN = 256;
constexpr int kBigKG = 2;                // quantization groups per K-step
constexpr int kBigSlices = 4 * kBigKG;   // k-slices of 16 per K-step
constexpr int kBigUnroll = 4;            // K-steps per loop iteration (two scale blocks)

// PD: how many K-steps ahead a step's loads are issued.  Tiles of up to 128
// rows take two: a K-step of a 64 x 128 tile lasts about 0.4 us, less than a
// weight load from HBM or the last-level cache takes to return, so with one
// step of lead the wave waited on it (M = 512 [2560 x 4096] 25.8 us with the
// weights from HBM against 20.4 with them cached).  Their LDS ring then has
// four stages and the weights four register sets; taller tiles keep one step
// of lead and two stages (the headline's 224-row tile fills the LDS with two).
template <int MT>
struct BigCfg {
  static constexpr int kBM = 32 * MT;
  static constexpr int kSlots = kBM * 8 * kBigKG;     // 16-byte LDS slots per stage
  static constexpr int kA = kSlots / kThreads;        // activation slots per thread per step
  static constexpr int kPD = MT <= 4 ? 2 : 1;         // prefetch distance in K-steps
  static constexpr int kStages = 2 * kPD;             // LDS stages and weight register sets
};

struct BigRing {
  uint4* a[4];
};

template <int MT>
struct BigSrc {
  __amdgpu_buffer_rsrc_t xr, wr, sr, br;
  uint32_t a_off[BigCfg<MT>::kA];  // byte offsets of this thread's activation slots
  uint32_t w_off[2][kBigKG];  // byte offsets of this lane's 16 weight bytes, per column
                              // tile and 16-row half
  uint32_t p_off[2];  // byte offsets of this lane's scale / bias row, per column tile
};

// MFMA operands of two consecutive k-slices (buffer = slice parity).
template <int MT>
struct BigFrags {
  u32x4_t a[2][MT];
  u32x4_t b[2][2];
};

// Eight consecutive scales (or biases) of a row: groups 2 g .. 2 g + 7, the
// four K-steps from step g (a 4-byte aligned offset).  The prefetch after a
// split's last block is clamped to two steps before its end and reads 8 bytes
// past it (the next row's, or zeros past the buffer; never used).
__device__ __forceinline__ uint4 load_param_block(__amdgpu_buffer_rsrc_t rs, uint32_t voff,
                                                  uint32_t g) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, voff, g * 4u, 0);
  return __builtin_bit_cast(uint4, v);
}

// Scale or bias of group h of step S (0..3) of a block.
template <int S>
__device__ __forceinline__ uint32_t param_at(uint4 blk, int h) {
  const uint32_t w = S == 0 ? blk.x : S == 1 ? blk.y : S == 2 ? blk.z : blk.w;
  return (w >> (16 * h)) & 0xFFFFu;
}

// Dequant parameters of one group for the two column tiles: s * 2^24 and
// s * 2^20 (the fma_mix nibble trick) and the bias.
struct GroupParams {
  float s24[2], s20[2], b[2];
};

template <int T, int S, int NT>
__device__ __forceinline__ GroupParams group_params(const uint4 (&sblk)[2], const uint4 (&bblk)[2],
                                                    int h) {
  GroupParams p;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float sv = Elem<T>::param((typename Elem<T>::S)param_at<S>(sblk[nt], h));
    p.s24[nt] = sv * 0x1p24f;
    p.s20[nt] = sv * 0x1p20f;
    p.b[nt] = Elem<T>::param((typename Elem<T>::S)param_at<S>(bblk[nt], h));
  }
  return p;
}

// The loads of a step are spread over kIssuePts points of the previous step
// (its top and its first k-slices): a burst of some twenty 1 KiB loads per
// wave at one point stalls the wave's issue behind the memory pipeline.
constexpr int kIssuePts = 7;
template <int MT>
__device__ __forceinline__ constexpr int a_split(int p) {
  return p * BigCfg<MT>::kA / kIssuePts;
}

// Weight loads of step gs into register set ST: per column tile the rows
// 0-15 (i = 0) and 16-31 (i = 1), 64 bytes each.
template <int MT, int NT, int ST>
__device__ __forceinline__ void big_issue_w(uint32_t gs, const BigSrc<MT>& src,
                                            u32x4_t (&wr)[BigCfg<MT>::kStages][2][kBigKG]) {
#pragma unroll
  for (int i = 0; i < kBigKG; ++i)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      wr[ST][nt][i] = load_b128(src.wr, src.w_off[nt][i], gs * 64u);
}

// The landed weight registers of a step into MFMA operand layout (see the
// kernel's comment): afterwards wr[nt][0] holds words 0-3 and wr[nt][1]
// words 4-7 of the lane's group.
template <int NT>
__device__ __forceinline__ void big_swap_w(u32x4_t (&wr)[2][kBigKG]) {
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const auto r = __builtin_amdgcn_permlane16_swap(wr[nt][0][j], wr[nt][1][j], false, false);
      wr[nt][0][j] = r[0];
      wr[nt][1][j] = r[1];
    }
}

// Activation loads [a_split(p), a_split(p + 1)) of step gs into stage ST.
template <int MT, int ST>
__device__ __forceinline__ void big_issue_a(int p, uint32_t gs, const BigRing& ring,
                                            const BigSrc<MT>& src, int wave) {
  uint4* ab = ring.a[ST] + wave * 64;
#pragma unroll
  for (int i = 0; i < BigCfg<MT>::kA; ++i)
    if (i >= a_split<MT>(p) && i < a_split<MT>(p + 1))
      load_lds16(src.xr, src.a_off[i], gs * (128u * kBigKG), ab + i * kThreads);
}

// LDS reads and weight dequant of k-slice t of a step into buffer B: lane
// (r32, h) holds k = 64 h + 8 t .. +8 of its activation row and of its weight
// row (word t of its group h), so the two operands agree.
template <int T, int MT, int NT, int B>
__device__ __forceinline__ void big_operands(int t, const uint4* at, const u32x4_t (&wr)[2][kBigKG],
                                             const GroupParams& gp, BigFrags<MT>& f, int arow0,
                                             int r32, int h) {
  const int q = t >> 2, kk = t & 3;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
    f.a[B][mt] = __builtin_bit_cast(
        u32x4_t, at[a_slot_kg<kBigKG>(arow0 + mt * 32 + r32, 8 * h + t)]);
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const u32x4_t wv = wr[nt][q];
    const uint32_t word = (kk == 0) ? wv.x : (kk == 1) ? wv.y : (kk == 2) ? wv.z : wv.w;
    uint32_t p[4];
    Elem<T>::dequant(word, gp.s24[nt], gp.s20[nt], gp.b[nt], p);
    f.b[B][nt] = u32x4_t{p[0], p[1], p[2], p[3]};
  }
}

template <int T, int MT, int NT, int B>
__device__ __forceinline__ void big_mfmas(const BigFrags<MT>& f, f32x16_t (&acc)[MT][NT]) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = mfma32<T>(f.a[B][mt], f.b[B][nt], acc[mt][nt]);
}

// One K-step.  S = g % kBigUnroll: stage and weight registers S % 2, dword S
// of the scale / bias blocks in slot 0 (slot 1: the next four steps').
// Vector-memory loads a thread issues in a step with position S in its block:
// the activation parts, the weights and, at S = 0, the next scale block.
template <int MT, int NT, int S>
constexpr int big_step_loads() {
  return BigCfg<MT>::kA + NT * kBigKG + (S == 0 ? 2 * NT : 0);
}

// TAIL: one of the split's last two steps after the unrolled loop.  With
// two steps of lead those issue no loads (every step they would load lies
// past the split), and the second waits for everything: the count a step's
// wait leaves in flight must match what the previous step really issued, and
// loads whose registers are never read again are dropped by the compiler.
template <int T, int MT, int NT, int S, bool TAIL = false>
__device__ __forceinline__ void big_step(int g, int steps, const BigRing& ring,
                                         const BigSrc<MT>& src, uint4 (&sblk)[2][2],
                                         uint4 (&bblk)[2][2],
                                         u32x4_t (&wr)[BigCfg<MT>::kStages][2][kBigKG],
                                         BigFrags<MT>& f, f32x16_t (&acc)[MT][NT], int wave,
                                         int arow0, int r32, int h) {
  constexpr int PD = BigCfg<MT>::kPD;
  constexpr int ST = S % BigCfg<MT>::kStages;       // this step's stage and weight set
  constexpr int SN = (S + PD) % BigCfg<MT>::kStages;  // step g + PD's
  constexpr int kMfma = NT * MT;
  constexpr bool kIssue = !(TAIL && PD == 2);  // this step issues the loads of step g + PD
  // This wave's loads of step g have landed: with one step of lead, all of
  // its loads; with two, all but those the previous step issued (loads
  // return in issue order).  After the barrier every wave's have.
  if constexpr (PD == 1 || (TAIL && S == 1)) {
    IMQ_WAIT_VM_LGKM_0();
  } else {
    constexpr int n = big_step_loads<MT, NT, (S + kBigUnroll - 1) % kBigUnroll>();
    static_assert(n <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((n & 15) | ((n >> 4) << 14) | (7 << 4));  // vmcnt(n) lgkmcnt(0)
  }
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);

  const uint4* at = ring.a[ST];
  big_swap_w<NT>(wr[ST]);
  const GroupParams gp = group_params<T, S, NT>(sblk[0], bblk[0], h);
  big_operands<T, MT, NT, 0>(0, at, wr[ST], gp, f, arow0, r32, h);
  if constexpr (S == 0 && kIssue) {
    // The next block (steps g+4 .. g+7) goes to slot 1; the K loop moves it to
    // slot 0 after step g+3.
    const uint32_t nb = (uint32_t)min(g + 4, steps - 2);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      sblk[1][nt] = load_param_block(src.sr, src.p_off[nt], nb);
      bblk[1][nt] = load_param_block(src.br, src.p_off[nt], nb);
    }
  }
  const uint32_t gs1 = (uint32_t)min(g + PD, steps - 1);
  if constexpr (kIssue) {
    big_issue_w<MT, NT, SN>(gs1, src, wr);
    big_issue_a<MT, SN>(0, gs1, ring, src, wave);
  }
  big_mfmas<T, MT, NT, 1>(f, acc);  // the previous step's last k-slice
  {
    // LDS reads first, then each deferred MFMA followed by a share of the
    // loads and of slice 0's dequant.
    constexpr int kVmem =
        kIssue ? NT * kBigKG + a_split<MT>(1) + (S == 0 ? 2 * NT : 0) : 0;
    constexpr int kVmemPer = (kVmem + kMfma - 1) / kMfma;
    constexpr int kValuPer = (NT * 17 + 4 * NT + kMfma - 1) / kMfma;
#pragma unroll
    for (int i = 0; i < MT; ++i) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
#pragma unroll
    for (int i = 0; i < kMfma; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);          // MFMA
      if (kVmemPer > 0) __builtin_amdgcn_sched_group_barrier(0x020, kVmemPer, 0);  // VMEM read
      __builtin_amdgcn_sched_group_barrier(0x002, kValuPer, 0);   // VALU
    }
  }

#pragma unroll
  for (int t = 0; t + 1 < kBigSlices; ++t) {
    __builtin_amdgcn_sched_barrier(0);
    if (kIssue && t + 1 < kIssuePts) big_issue_a<MT, SN>(t + 1, gs1, ring, src, wave);
    if (t & 1) {
      big_operands<T, MT, NT, 0>(t + 1, at, wr[ST], gp, f, arow0, r32, h);
      big_mfmas<T, MT, NT, 1>(f, acc);
    } else {
      big_operands<T, MT, NT, 1>(t + 1, at, wr[ST], gp, f, arow0, r32, h);
      big_mfmas<T, MT, NT, 0>(f, acc);
    }
    // Every MFMA of this k-slice is followed by a share of the next slice's
    // dequant VALU work, for the first MT one LDS read, and for the first few
    // one of the next step's activation loads, so a single wave keeps the
    // matrix core fed while it dequantizes.
    constexpr int kValuPer = (NT * 17 + kMfma - 1) / kMfma;
    const int n_dma =
        kIssue && t + 1 < kIssuePts ? a_split<MT>(t + 2) - a_split<MT>(t + 1) : 0;
#pragma unroll
    for (int i = 0; i < kMfma; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                 // MFMA
      if (i < MT) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // DS read
      if (i < n_dma) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
      __builtin_amdgcn_sched_group_barrier(0x002, kValuPer, 0);          // VALU
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

// Output tile staging.  Row r of the tile's kCW T values (kCW = 256 outputs,
// 128 for a gate/up pair) sits in ring stage r / (kBM / 2) at row r % (kBM / 2)
// of kCW * 2 bytes, its 16-byte chunk c at slot c ^ (4 * ((r / 4) % 2)): a
// wave's 2-byte writes (rows r and r + 4 in its two lane halves) then hit
// disjoint banks.
template <class EP, int NT>
constexpr int tile_cols() {
  return EP::kPair ? kBigBN / 2 : 128 * NT;
}

template <int MT, int NT, class EP>
__device__ __forceinline__ uint16_t* staged_at(const BigRing& ring, int row, int col) {
  constexpr int kHalf = BigCfg<MT>::kBM / 2;
  constexpr int kCW = tile_cols<EP, NT>();
  const int chunk = (col >> 3) ^ (((row >> 2) & 1) << 2);
  uint16_t* base = reinterpret_cast<uint16_t*>(row < kHalf ? ring.a[0] : ring.a[1]);
  return base + (row % kHalf) * kCW + chunk * 8 + (col & 7);
}

// Accumulator r of a 32x32 tile holds row 8*(r/4) + 4*h + r%4, column r32:
// registers r and r+1 are rows one apart in the same column, rounded to T as a
// pair.
template <int T, int MT, int NT, class EP>
__device__ __forceinline__ void big_stage_tile(const EP& ep, const f32x16_t (&acc)[MT][NT],
                                               const BigRing& ring, int wave, int r32, int h) {
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
      const int row = mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
      if constexpr (EP::kPair) {
        const int col = wave * 32 + r32;
        const uint32_t v = Elem<T>::pack2(ep.value2(acc[mt][0][r], acc[mt][NT - 1][r]),
                                          ep.value2(acc[mt][0][r + 1], acc[mt][NT - 1][r + 1]));
        *staged_at<MT, NT, EP>(ring, row, col) = (uint16_t)v;
        *staged_at<MT, NT, EP>(ring, row + 1, col) = (uint16_t)(v >> 16);
      } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int col = wave * (32 * NT) + nt * 32 + r32;
          const uint32_t v =
              Elem<T>::pack2(ep.value(acc[mt][nt][r]), ep.value(acc[mt][nt][r + 1]));
          *staged_at<MT, NT, EP>(ring, row, col) = (uint16_t)v;
          *staged_at<MT, NT, EP>(ring, row + 1, col) = (uint16_t)(v >> 16);
        }
      }
    }
}

// Write the staged tile to output rows m0.., columns col0.. (< ncols): all of
// a thread's LDS reads first, so their latencies overlap, then the stores.
template <int MT, int NT, class EP>
__device__ __forceinline__ void big_write_tile(const EP& ep, const BigRing& ring, int tid, int m0,
                                               int col0, int M, int ncols) {
  constexpr int kCPR = tile_cols<EP, NT>() / 8;  // 16-byte chunks per row
  constexpr int kIters = BigCfg<MT>::kBM * kCPR / kThreads;
  uint4 v[kIters];
#pragma unroll
  for (int i = 0; i < kIters; ++i) {
    const int q = i * kThreads + tid;
    v[i] = *reinterpret_cast<const uint4*>(staged_at<MT, NT, EP>(ring, q / kCPR, (q % kCPR) * 8));
  }
  const int c = tid % kCPR;
  const int col = col0 + c * 8;
  if (col >= ncols) return;
  if (ep.vec && col + 8 <= ncols) {
#pragma unroll
    for (int i = 0; i < kIters; ++i) {
      const int grow = m0 + (i * kThreads + tid) / kCPR;
      if (grow < M) ep.emit8(grow, col, v[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < kIters; ++i) {
      const int grow = m0 + (i * kThreads + tid) / kCPR;
      if (grow >= M) continue;
      const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (col + e < ncols) ep.emit1(grow, col + e, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
    }
  }
}

// EP is the output stage (epilogue.hpp).  With EP::kPair (SwiGLU) the
// workgroup's 256 weight rows are 128 gate rows and the 128 matching up rows:
// a wave's column tile 0 holds gate rows, tile 1 the up rows of the same 32
// output columns, so each lane has both accumulators of an output.
// NT = 1: each wave owns one 32-column tile, the workgroup tile is (32 MT) x
// 128 -- twice the tiles of a shape at the same height, so a short M can keep
// a taller tile (each dequantized weight fragment feeds MT MFMAs; at one or
// two row tiles the dequant VALU work, not the matrix core, bounds a step).
template <int T, int MT, int NT, class EP>
__global__ __launch_bounds__(kThreads, 1) void qgemm_big_kernel(
    const uint32_t* __restrict__ w, const uint16_t* __restrict__ scales,
    const uint16_t* __restrict__ biases, const uint16_t* __restrict__ x, const EP ep,
    int M, int N, int K, int tiles_m, int tiles_n, int split_steps) {
  static_assert(NT == 1 || NT == 2, "one or two 32-column tiles per wave");
  static_assert(!EP::kPair || NT == 2, "a gate/up pair takes two column tiles per wave");
  using C = BigCfg<MT>;
  constexpr int kExtra = C::kStages > 2 ? C::kSlots : 1;  // stages 2, 3 (two steps of lead)
  __shared__ uint4 a_st0[C::kSlots], a_st1[C::kSlots], a_st2[kExtra], a_st3[kExtra];
  const BigRing ring = {{a_st0, a_st1, a_st2, a_st3}};

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r32 = lane & 31;
  const int h = lane >> 5;
  int tm, tn;
  tile_coords(blockIdx.x, tiles_m, tiles_n, tm, tn);
  const int m0 = tm * C::kBM;
  const int n0 = tn * (128 * NT);
  const int arow0 = 0;                      // every wave covers all rows of the tile
  const int ncol0 = n0 + wave * (32 * NT);  // this wave's first output column
  const int pcol0 = tn * (kBigBN / 2) + wave * 32;  // paired epilogue: first output column
  const int gpr = K >> 6;
  // K-steps [g0, g1) of split blockIdx.y (splits of `split_steps` steps, an
  // even number: whole scale blocks).
  const int g0 = (int)blockIdx.y * split_steps;
  const int g1 = min(g0 + split_steps, gpr / kBigKG);

  BigSrc<MT> src;
  src.xr = make_rsrc(x, (uint32_t)((size_t)M * K * 2));
  src.wr = make_rsrc(w, (uint32_t)((size_t)N * K / 2));
  src.sr = make_rsrc(scales, (uint32_t)((size_t)N * gpr * 2));
  src.br = make_rsrc(biases, (uint32_t)((size_t)N * gpr * 2));
  // Activation slot s = i*256 + tid holds tile row s / 16, physical chunk
  // s % 16, i.e. logical chunk a_slot_kg's inverse of that row.  Rows past M
  // are clamped.
#pragma unroll
  for (int i = 0; i < C::kA; ++i) {
    const int slot = i * kThreads + tid;
    const int row = slot / (8 * kBigKG);
    const int c = a_chunk_kg<kBigKG>(row, slot % (8 * kBigKG));
    const uint32_t gr = (uint32_t)min(m0 + row, M - 1);
    src.a_off[i] = (gr * (uint32_t)K + (uint32_t)c * 8u) * 2u;
  }
  // In MFMA operand layout lane (r32, h) of column tile nt owns weight row
  // ncol0 + 32 nt + r32 (its scales and biases); its loads read row
  // ncol0 + 32 nt + 16 i + lane % 16, bytes [16 (lane / 16), +16) of the step.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    int wrow = ncol0 + nt * 32 + r32;
    if constexpr (EP::kPair) wrow = (nt == 0 ? ep.gate_row : ep.up_row) + min(pcol0 + r32, ep.width - 1);
    src.p_off[nt] = (uint32_t)min(wrow, N - 1) * (uint32_t)gpr * 2u;
#pragma unroll
    for (int i = 0; i < kBigKG; ++i) {
      const int c = 16 * i + (lane & 15);
      int lrow = ncol0 + nt * 32 + c;
      if constexpr (EP::kPair) lrow = (nt == 0 ? ep.gate_row : ep.up_row) + min(pcol0 + c, ep.width - 1);
      src.w_off[nt][i] = (uint32_t)min(lrow, N - 1) * (uint32_t)(K / 2) + (uint32_t)(lane >> 4) * 16u;
    }
  }

  f32x16_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[mt][nt][r] = 0.f;

  // Prologue: the first scale block, the loads of the first PD steps (step
  // g0 + 1's last: with two steps of lead the first step's wait leaves them
  // in flight), and zero operands for the first step's deferred MFMAs (they
  // add nothing).
  uint4 sblk[2][2], bblk[2][2];
  u32x4_t wr[C::kStages][2][kBigKG];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    sblk[0][nt] = load_param_block(src.sr, src.p_off[nt], (uint32_t)g0);
    bblk[0][nt] = load_param_block(src.br, src.p_off[nt], (uint32_t)g0);
  }
  big_issue_w<MT, NT, 0>((uint32_t)g0, src, wr);
#pragma unroll
  for (int p = 0; p < kIssuePts; ++p) big_issue_a<MT, 0>(p, (uint32_t)g0, ring, src, wave);
  if constexpr (C::kPD == 2) {
    const uint32_t gn = (uint32_t)min(g0 + 1, g1 - 1);
    big_issue_w<MT, NT, 1>(gn, src, wr);
#pragma unroll
    for (int p = 0; p < kIssuePts; ++p) big_issue_a<MT, 1>(p, gn, ring, src, wave);
  }
  BigFrags<MT> f;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) f.a[1][mt] = u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) f.b[1][nt] = u32x4_t{0u, 0u, 0u, 0u};

  // g1 - g0 is even: full unrolls, then possibly two steps.  The ring stage
  // and scale blocks count from g0; loads past g1 are clamped to g1 - 1.
  int g = g0;
  for (; g + kBigUnroll <= g1; g += kBigUnroll) {
    big_step<T, MT, NT, 0>(g, g1, ring, src, sblk, bblk, wr, f, acc, wave, arow0, r32, h);
    big_step<T, MT, NT, 1>(g + 1, g1, ring, src, sblk, bblk, wr, f, acc, wave, arow0, r32, h);
    big_step<T, MT, NT, 2>(g + 2, g1, ring, src, sblk, bblk, wr, f, acc, wave, arow0, r32, h);
    big_step<T, MT, NT, 3>(g + 3, g1, ring, src, sblk, bblk, wr, f, acc, wave, arow0, r32, h);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      sblk[0][nt] = sblk[1][nt];
      bblk[0][nt] = bblk[1][nt];
    }
  }
  if (g < g1) {
    big_step<T, MT, NT, 0, true>(g, g1, ring, src, sblk, bblk, wr, f, acc, wave, arow0, r32, h);
    big_step<T, MT, NT, 1, true>(g + 1, g1, ring, src, sblk, bblk, wr, f, acc, wave, arow0, r32,
                                 h);
  }
  big_mfmas<T, MT, NT, 1>(f, acc);  // the last step's last k-slice

  if constexpr (EP::kPartial) {
    // Split-K partial sums: fp32 straight from the MFMA layout into split
    // blockIdx.y's [M][ldp] slice of the workspace.
    IMQ_WAIT_VMCNT(0);  // drain the clamped tail loads before the workgroup ends
    float* part = ep.ws + (size_t)blockIdx.y * M * ep.ldp;
    if constexpr (EP::kPair) {
      const int j = pcol0 + r32;
      if (j < ep.width) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = m0 + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (row < M) {
              part[(size_t)row * ep.ldp + j] = acc[mt][0][r];
              part[(size_t)row * ep.ldp + ep.width + j] = acc[mt][1][r];
            }
          }
      }
    } else {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int col = ncol0 + nt * 32 + r32;
          if (col >= N) continue;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int row = m0 + mt * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
            if (row < M) part[(size_t)row * ep.ldp + col] = acc[mt][nt][r];
          }
        }
    }
  } else {
  // Output: the tile's T values are staged in the LDS ring, then written out
  // row by row, 16 bytes per lane.  Written straight from the MFMA layout, a
  // lane holds one column of 16 rows per 32x32 tile: 2-byte stores, 14 of
  // them per 32 output bytes per wave, and every CU issues them at the same
  // moment of each tile round; that cost about 10% of the kernel.  The ring is
  // free once every wave is past this barrier (its LDS reads returned, the
  // clamped tail loads landed).
  IMQ_WAIT_VM_LGKM_0();
  __builtin_amdgcn_s_barrier();
  big_stage_tile<T, MT, NT>(ep, acc, ring, wave, r32, h);
  __syncthreads();
  if constexpr (EP::kPair)
    big_write_tile<MT, NT>(ep, ring, tid, m0, tn * (kBigBN / 2), M, ep.width);
  else
    big_write_tile<MT, NT>(ep, ring, tid, m0, n0, M, N);
  }
}

template <int T, int MT, int NT, class EP>
hipError_t launch_big(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                      const uint16_t* x, const EP& ep, int k, int n, int m, hipStream_t stream,
                      int splits = 1, int split_steps = 0) {
  constexpr int BM = BigCfg<MT>::kBM;
  const int tiles_m = (m + BM - 1) / BM;
  int cols = n;  // weight rows the workgroups cover
  if constexpr (EP::kPair) cols = 2 * ep.width;
  const int tiles_n = (cols + 128 * NT - 1) / (128 * NT);
  if (splits <= 1) split_steps = k / (64 * kBigKG);
  const dim3 grid((unsigned)tiles_m * (unsigned)tiles_n, (unsigned)splits);
  hipLaunchKernelGGL((qgemm_big_kernel<T, MT, NT, EP>), grid, dim3(kThreads), 0, stream, w,
                     scales, biases, x, ep, m, n, k, tiles_m, tiles_n, split_steps);
  return hipGetLastError();
}

// Adds the split-K partial sums of each output in split order and applies
// the output stage ep (its T rounding of value / value2, then emit8 or
// emit1): 8 consecutive outputs of a row per thread.  Partials of split s
// sit at ws + s * M * ldp; plain stages read column c at c, pair stages the
// gate sum at c and the up sum at width + c.  vload: ldp % 4 == 0 and
// ncols % 8 == 0 (16-byte partial loads).
template <int T, class EP>
__global__ __launch_bounds__(256) void reduce_ep_kernel(const float* __restrict__ ws, int splits,
                                                        int M, int ncols, int ldp, bool vload,
                                                        const EP ep) {
  const int cpr = (ncols + 7) / 8;
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long)M * cpr) return;
  const int row = (int)(t / cpr);
  const int c0 = (int)(t % cpr) * 8;
  const size_t stride = (size_t)M * ldp;
  float a[8], u[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = u[e] = 0.f;
  if (vload) {
    // The loads of kBatch splits go out before the first add (indices past
    // the last split repeat it and are not added): one memory round trip per
    // batch instead of one per split.
    constexpr int kBatch = EP::kPair ? 4 : 8;
    for (int s0 = 0; s0 < splits; s0 += kBatch) {
      float4 p[kBatch][2], q[kBatch][2];
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const float* pr = ws + (size_t)min(s0 + j, splits - 1) * stride + (size_t)row * ldp + c0;
        p[j][0] = reinterpret_cast<const float4*>(pr)[0];
        p[j][1] = reinterpret_cast<const float4*>(pr)[1];
        if constexpr (EP::kPair) {
          q[j][0] = reinterpret_cast<const float4*>(pr + ep.width)[0];
          q[j][1] = reinterpret_cast<const float4*>(pr + ep.width)[1];
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        if (s0 + j >= splits) break;
        a[0] += p[j][0].x; a[1] += p[j][0].y; a[2] += p[j][0].z; a[3] += p[j][0].w;
        a[4] += p[j][1].x; a[5] += p[j][1].y; a[6] += p[j][1].z; a[7] += p[j][1].w;
        if constexpr (EP::kPair) {
          u[0] += q[j][0].x; u[1] += q[j][0].y; u[2] += q[j][0].z; u[3] += q[j][0].w;
          u[4] += q[j][1].x; u[5] += q[j][1].y; u[6] += q[j][1].z; u[7] += q[j][1].w;
        }
      }
    }
  } else {
    for (int sp = 0; sp < splits; ++sp) {
      const float* pr = ws + sp * stride + (size_t)row * ldp + c0;
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (c0 + e < ncols) {
          a[e] += pr[e];
          if constexpr (EP::kPair) u[e] += pr[ep.width + e];
        }
    }
  }
  uint32_t w[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if constexpr (EP::kPair)
      w[e] = Elem<T>::pack2(ep.value2(a[2 * e], u[2 * e]), ep.value2(a[2 * e + 1], u[2 * e + 1]));
    else
      w[e] = Elem<T>::pack2(ep.value(a[2 * e]), ep.value(a[2 * e + 1]));
  }
  if (ep.vec && c0 + 8 <= ncols) {
    ep.emit8(row, c0, make_uint4(w[0], w[1], w[2], w[3]));
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (c0 + e < ncols) ep.emit1(row, c0 + e, (uint16_t)(w[e >> 1] >> (16 * (e & 1))));
  }
}

template <int T, class EP>
hipError_t launch_reduce(const SplitWs& ws, int splits, int m, int ncols, int ldp, const EP& ep,
                         hipStream_t stream) {
  const long threads = (long)m * ((ncols + 7) / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  // 16-byte partial loads: ws 16-byte aligned and every row / pair offset a
  // multiple of four floats.
  bool vload = ldp % 4 == 0 && ncols % 8 == 0 && ((uintptr_t)ws.p & 15u) == 0;
  if constexpr (EP::kPair) vload = vload && ep.width % 4 == 0;
  hipLaunchKernelGGL((reduce_ep_kernel<T, EP>), grid, dim3(256), 0, stream, ws.p, splits, m, ncols,
                     ldp, vload, ep);
  return hipGetLastError();
}

// Tile height, width and K split of the large-M kernel (small: 32- and 64-row
// and 128-column tiles allowed without a split -- the plain store and the
// residual add are built for them, the other fused stages are not, the
// split-K partial sums always are; split: K may be split).  Cost in units of about
// 0.36 us (a K-step of a 32-row slice of the tile): a round of tiles costs
// split_steps * (MT + 1.5) plus 12 for its prologue and output; a split adds
// the workspace traffic of its reduction (8 bytes per output and split, at
// about 1.4 MB per unit) plus 3 for the extra launch.  Splits are taken only
// when the tiles leave CUs idle.  160-row tiles exist for row counts that
// leave a round of 192-row tiles part empty: 1024 x 9216 at K = 3072 is 252
// tiles in one round instead of 216 (58.4 -> 57.0 us), 2048 x 9216 is 468
// tiles in two rounds instead of 396 in two (115.0 -> 105.6 us).
//
// 128-column tiles (one 32-column tile per wave, NT = 1) double the tiles of
// a shape at a given height, so a short M keeps a taller tile.  What bounds a
// K-step of a 32- or 64-row tile is its dequant VALU work, the same per wave
// and weight fragment at any height (each fragment feeds MT MFMAs), not its
// MFMAs: half the columns per wave halve it.  Cost of a NT = 1 step:
// max(kNt1Floor, kNt1Step + kNt1PerRow * MT), fitted to forced plans timed on
// the text-encoder and DiT shapes (M = 128-2048, same box: e.g. M = 512 K =
// 2560 N = 6144 at 128 x 128 tiles 18.8 us against 21.5 at 64 x 256; N = 2560
// K = 4096 unsplit at 64 x 128 20.0 against 23.4 split three ways at 64 x
// 256).  The narrower tiles read 1.5x the activation and weight bytes per
// flop of 256-column ones from L2: they are taken only where a split's
// activation panel (M rows x its K range) fits one XCD's 4 MB L2 (at M = 512
// K = 9216 unsplit 64 x 128 tiles ran at 57.6 us against 42.0 for 128 x 256
// tiles split four ways), and a split of them is costed 3 units more.  Only
// for stages other than a gate/up pair (whose wave holds gate and up
// columns), unsplit only for the plain store.
constexpr double kNt1Floor = 1.5, kNt1Step = -0.35, kNt1PerRow = 0.925;
constexpr size_t kNt1MaxPanel = (size_t)4 << 20;
struct BigPlan {
  int mt, nt, splits, split_steps;
};

BigPlan pick_big_plan(int m, int n, int k, int cus, bool small, bool split, bool pair = false) {
  const int steps = k / (64 * kBigKG);
  BigPlan best{8, 2, 1, steps};
  double best_cost = 1e30;
  for (int nt : {2, 1}) {
    if (nt == 1 && pair) continue;
    const int tiles_n = (n + 128 * nt - 1) / (128 * nt);
    for (int mt : {8, 7, 6, 5, 4, 2, 1}) {
      // 32 x 128 tiles are not planned: that instantiation spills registers
      // to scratch memory (the 32 x 256 tile or the few-row kernel take
      // those shapes).
      if (nt == 1 && mt == 1) continue;
      const long tiles = (long)((m + 32 * mt - 1) / (32 * mt)) * tiles_n;
      const int max_splits = split && tiles < cus ? std::max(1, steps / 2) : 1;
      for (int sp = 1; sp <= max_splits; ++sp) {
        const int sps = ((steps + sp - 1) / sp + 1) / 2 * 2;  // even
        const int eff = (steps + sps - 1) / sps;
        if (eff != sp || (eff == 1 && mt < 4 && !small)) continue;
        if (nt == 1 && ((eff == 1 && !small) || (size_t)m * sps * 128 * 2 > kNt1MaxPanel))
          continue;
        const long rounds = (tiles * eff + cus - 1) / cus;
        const double step =
            nt == 2 ? mt + 1.5 : std::max(kNt1Floor, kNt1Step + kNt1PerRow * mt);
        double cost = (double)rounds * (sps * step + 12.0);
        if (eff > 1) cost += (double)eff * m * n * 8.0 / 1.4e6 + (nt == 2 ? 3.0 : 6.0);
        if (cost < best_cost - 1e-9) {
          best_cost = cost;
          best = BigPlan{mt, nt, eff, sps};
        }
      }
    }
  }
  return best;
}

// The register-staged kernel (any K % 64 == 0) with output stage ep; a
// gate/up pair covers 2 * width weight rows.
template <int T, int MT, int NT, class EP>
hipError_t launch_tile(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                       const uint16_t* x, const EP& ep, int k, int n, int m, hipStream_t stream) {
  int cols = n;
  if constexpr (EP::kPair) cols = 2 * ep.width;
  const int tiles_m = (m + 32 * MT - 1) / (32 * MT);
  const int tiles_n = (cols + 128 * NT - 1) / (128 * NT);
  const dim3 grid((unsigned)tiles_m * (unsigned)tiles_n);
  hipLaunchKernelGGL((qgemm_kernel<T, MT, NT, EP>), grid, dim3(kThreads), 0, stream, w, scales,
                     biases, x, ep, m, n, k, tiles_m, tiles_n);
  return hipGetLastError();
}

// 16-byte alignment of an output or residual pointer (vector output stores).
bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int device_cus() {
  static const int cus = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0)
      return v;
    return 256;
  }();
  return cus;
}

// Stages built for every tile height and for 128-column tiles: the plain
// store, the split-K partial sums and the text encoder's residual add.
template <int T, class EP>
constexpr bool kAnyTile = EP::kPartial || (!EP::kPair && (std::is_same<EP, EpStore<T>>::value ||
                                                          std::is_same<EP, EpResidAdd<T>>::value));

template <int T, int NT, class EP>
hipError_t launch_big_mt_nt(int mt, const uint32_t* w, const uint16_t* scales,
                            const uint16_t* biases, const uint16_t* x, const EP& ep, int k, int n,
                            int m, hipStream_t stream, int splits, int split_steps) {
  // The other fused stages are built for 128 rows and more.
  constexpr bool kSmall = kAnyTile<T, EP>;
  switch (mt) {
    case 1:
      if constexpr (kSmall) return launch_big<T, 1, NT>(w, scales, biases, x, ep, k, n, m, stream, splits, split_steps);
      return hipErrorInvalidValue;
    case 2:
      if constexpr (kSmall) return launch_big<T, 2, NT>(w, scales, biases, x, ep, k, n, m, stream, splits, split_steps);
      return hipErrorInvalidValue;
    case 4: return launch_big<T, 4, NT>(w, scales, biases, x, ep, k, n, m, stream, splits, split_steps);
    case 5: return launch_big<T, 5, NT>(w, scales, biases, x, ep, k, n, m, stream, splits, split_steps);
    case 6: return launch_big<T, 6, NT>(w, scales, biases, x, ep, k, n, m, stream, splits, split_steps);
    case 7: return launch_big<T, 7, NT>(w, scales, biases, x, ep, k, n, m, stream, splits, split_steps);
    default: return launch_big<T, 8, NT>(w, scales, biases, x, ep, k, n, m, stream, splits, split_steps);
  }
}

// nt = 1 (128-column tiles) is built for the kAnyTile stages other than a
// gate/up pair's partial sums.
template <int T, class EP>
hipError_t launch_big_mt(int mt, int nt, const uint32_t* w, const uint16_t* scales,
                         const uint16_t* biases, const uint16_t* x, const EP& ep, int k, int n,
                         int m, hipStream_t stream, int splits = 1, int split_steps = 0) {
  constexpr bool kNt1 = !EP::kPair && kAnyTile<T, EP>;
  if (nt == 1) {
    if constexpr (kNt1)
      return launch_big_mt_nt<T, 1>(mt, w, scales, biases, x, ep, k, n, m, stream, splits,
                                    split_steps);
    return hipErrorInvalidValue;
  }
  return launch_big_mt_nt<T, 2>(mt, w, scales, biases, x, ep, k, n, m, stream, splits,
                                split_steps);
}

// The large-M kernel with output stage ep (two groups per K-step, 2-stage
// ring: half the barriers and waits of one group per step, measured 3.5%
// faster at M=4608 K=3072 N=18432).  When the planner splits K and ws holds
// the partial sums, the kernel writes fp32 partials and reduce_ep_kernel adds
// them and applies ep; otherwise one pass.
template <int T, class EP>
hipError_t launch_big_ep(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                         const uint16_t* x, const EP& ep, int k, int n, int m, hipStream_t stream,
                         SplitWs ws) {
  // K % 256 != 0 (e.g. the DiT's x_embedder, K = 128) or operands past 32-bit
  // offsets: the register-staged kernel, one pass.
  if (!qgemm_big_supported(k, n, m)) return launch_tile<T, 4, 2>(w, scales, biases, x, ep, k, n, m, stream);
  constexpr bool kSmall = kAnyTile<T, EP>;
  int cols = n;  // weight rows covered
  int width = n, gate_row = 0, up_row = 0;
  if constexpr (EP::kPair) {
    cols = 2 * ep.width;
    width = ep.width;
    gate_row = ep.gate_row;
    up_row = ep.up_row;
  }
  const int cus = ws.cus > 0 ? ws.cus : device_cus();
  BigPlan p = pick_big_plan(m, cols, k, cus, kSmall, ws.p != nullptr, EP::kPair);
  if (p.splits > 1 && ws.bytes < (size_t)p.splits * m * cols * sizeof(float))
    p = pick_big_plan(m, cols, k, cus, kSmall, false, EP::kPair);  // no room for the partial sums
  if (p.splits == 1) return launch_big_mt<T>(p.mt, p.nt, w, scales, biases, x, ep, k, n, m, stream);
  const EpPartial<EP::kPair> part{ws.p, cols, width, gate_row, up_row};
  const hipError_t e = launch_big_mt<T>(p.mt, p.nt, w, scales, biases, x, part, k, n, m, stream,
                                        p.splits, p.split_steps);
  if (e != hipSuccess) return e;
  return launch_reduce<T>(ws, p.splits, m, width, cols, ep, stream);
}

template <int T>
hipError_t launch_t(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                    const uint16_t* x, uint16_t* y, int k, int n, int m, hipStream_t stream,
                    SplitWs ws) {
  return launch_big_ep<T>(w, scales, biases, x, EpStore<T>{y, n, al16(y) && n % 8 == 0}, k, n, m,
                          stream, ws);
}

}  // namespace

bool qgemm_big_supported(int k, int n, int m) {
  // The buffer-load kernel addresses x and w with 32-bit byte offsets and
  // loads scales in blocks of four groups.
  return (size_t)m * k * 2 < ((size_t)1 << 31) && (size_t)n * k / 2 < ((size_t)1 << 31) &&
         k % 256 == 0;
}

hipError_t launch_qgemm(const uint32_t* w, const void* scales, const void* biases, const void* x,
                        void* y, int k, int n, int m, int dtype, hipStream_t stream, SplitWs ws) {
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  switch (dtype) {
    case kBf16: return launch_t<kBf16>(w, s, b, xx, yy, k, n, m, stream, ws);
    case kF16: return launch_t<kF16>(w, s, b, xx, yy, k, n, m, stream, ws);
    default: return hipErrorInvalidValue;
  }
}

size_t qgemm_split_bytes(int k, int n, int m, bool fused) {
  if (!qgemm_big_supported(k, n, m)) return 0;
  // The most a stage over these rows takes: a fused stage may be a gate/up
  // pair (no 128-column tiles), the residual add (every tile) or another.
  size_t bytes = 0;
  for (int v = 0; v < (fused ? 3 : 1); ++v) {
    const bool small = !fused || v == 2, pair = v == 1;
    const BigPlan p = pick_big_plan(m, n, k, device_cus(), small, true, pair);
    if (p.splits > 1) bytes = std::max(bytes, (size_t)p.splits * m * n * sizeof(float));
  }
  return bytes;
}

QgemmPlan qgemm_plan(int k, int n, int m, bool fused, bool split, int cus, bool pair) {
  if (!qgemm_big_supported(k, n, m)) return QgemmPlan{false, 128, 1, 0, 256};
  const BigPlan p = pick_big_plan(m, n, k, cus > 0 ? cus : device_cus(), !fused, split, pair);
  return QgemmPlan{true, 32 * p.mt, p.splits,
                   p.splits > 1 ? (size_t)p.splits * m * n * sizeof(float) : 0, 128 * p.nt};
}

hipError_t launch_qgemm_postscale(const uint32_t* w, const void* scales, const void* biases,
                                  const void* x, float* y, int k, int n, int m, float scale,
                                  int dtype, hipStream_t stream, SplitWs ws,
                                  const float* scale_dev) {
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  const bool vec = al16(y) && n % 4 == 0;
  switch (dtype) {
    case kBf16:
      return launch_big_ep<kBf16>(w, s, b, xx, EpPostscale<kBf16>{y, n, scale, vec, scale_dev}, k,
                                  n, m, stream, ws);
    case kF16:
      return launch_big_ep<kF16>(w, s, b, xx, EpPostscale<kF16>{y, n, scale, vec, scale_dev}, k,
                                 n, m, stream, ws);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_qgemm_postscale_f16(const uint32_t* w, const void* scales, const void* biases,
                                      const void* x, void* y, int k, int n, int m, float scale,
                                      hipStream_t stream, const float* scale_dev) {
  auto* yy = static_cast<uint16_t*>(y);
  const bool vec = al16(y) && n % 8 == 0;
  return launch_big_ep<kF16>(w, static_cast<const uint16_t*>(scales),
                             static_cast<const uint16_t*>(biases), static_cast<const uint16_t*>(x),
                             EpPostscaleF16{yy, n, scale, vec, scale_dev}, k, n, m, stream,
                             SplitWs{});
}

hipError_t launch_qgemm_resid_add(const uint32_t* w, const void* scales, const void* biases,
                                  const void* x, const void* resid, void* y, int k, int n, int m,
                                  int dtype, hipStream_t stream, SplitWs ws) {
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  const auto* rr = static_cast<const uint16_t*>(resid);
  const bool vec = al16(y) && al16(resid) && n % 8 == 0;
  switch (dtype) {
    case kBf16:
      return launch_big_ep<kBf16>(w, s, b, xx, EpResidAdd<kBf16>{yy, rr, n, vec}, k, n, m, stream,
                                  ws);
    case kF16:
      return launch_big_ep<kF16>(w, s, b, xx, EpResidAdd<kF16>{yy, rr, n, vec}, k, n, m, stream,
                                 ws);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_qgemm_gate_add(const uint32_t* w, const void* scales, const void* biases,
                                 const void* x, const float* residual, const float* gate, float* y,
                                 int k, int n, int m, float scale, int dtype, hipStream_t stream,
                                 SplitWs ws, const float* scale_dev) {
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  const bool vec = al16(y) && al16(residual) && al16(gate) && n % 4 == 0;
  switch (dtype) {
    case kBf16:
      return launch_big_ep<kBf16>(
          w, s, b, xx, EpGateAdd<kBf16>{y, residual, gate, n, scale, vec, scale_dev}, k, n, m,
          stream, ws);
    case kF16:
      return launch_big_ep<kF16>(
          w, s, b, xx, EpGateAdd<kF16>{y, residual, gate, n, scale, vec, scale_dev}, k, n, m,
          stream, ws);
    default: return hipErrorInvalidValue;
  }
}

namespace {

// y[row][j] = T(EpSwiGLU(g, u)) from a T product [rows, 2 width] (gate at
// column j, up at width + j): the fused stage's arithmetic on values already
// rounded to T (its round_to is then exact).
template <int T>
__global__ __launch_bounds__(256) void swiglu_t_kernel(const uint16_t* __restrict__ gu, int ld,
                                                       int rows, const EpSwiGLU<T> ep) {
  const long t = (long)blockIdx.x * 256 + threadIdx.x;
  if (t >= (long)rows * ep.width) return;
  const int row = (int)(t / ep.width), j = (int)(t % ep.width);
  const uint16_t* r = gu + (size_t)row * ld;
  ep.emit1(row, j, Elem<T>::out(ep.value2(Elem<T>::param(r[j]), Elem<T>::param(r[ep.width + j]))));
}

}  // namespace

hipError_t launch_swiglu_t(const void* gu, int ld, int rows, int width, void* y, int ldy,
                           float in_scale, float out_scale, int dtype, hipStream_t stream) {
  if (rows <= 0 || width <= 0) return hipSuccess;
  const auto* g = static_cast<const uint16_t*>(gu);
  auto* yy = static_cast<uint16_t*>(y);
  const dim3 grid((unsigned)(((long)rows * width + 255) / 256));
  switch (dtype) {
    case kBf16:
      hipLaunchKernelGGL((swiglu_t_kernel<kBf16>), grid, dim3(256), 0, stream, g, ld, rows,
                         EpSwiGLU<kBf16>{yy, ldy, width, 0, width, in_scale, out_scale, false});
      return hipGetLastError();
    case kF16:
      hipLaunchKernelGGL((swiglu_t_kernel<kF16>), grid, dim3(256), 0, stream, g, ld, rows,
                         EpSwiGLU<kF16>{yy, ldy, width, 0, width, in_scale, out_scale, false});
      return hipGetLastError();
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_reduce_swiglu(const float* ws, int splits, int m, int width, void* y, int ldy,
                                float in_scale, float out_scale, int dtype, hipStream_t stream) {
  auto* yy = static_cast<uint16_t*>(y);
  const bool vec = al16(y) && ldy % 8 == 0;
  const SplitWs sw{const_cast<float*>(ws), 0, 0};
  switch (dtype) {
    case kBf16:
      return launch_reduce<kBf16>(
          sw, splits, m, width, 2 * width,
          EpSwiGLU<kBf16>{yy, ldy, width, 0, width, in_scale, out_scale, vec}, stream);
    case kF16:
      return launch_reduce<kF16>(
          sw, splits, m, width, 2 * width,
          EpSwiGLU<kF16>{yy, ldy, width, 0, width, in_scale, out_scale, vec}, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_qgemm_swiglu(const uint32_t* w, const void* scales, const void* biases,
                               const void* x, void* y, int ldy, int k, int n, int m, int width,
                               int gate_row, int up_row, float in_scale, float out_scale, int dtype,
                               hipStream_t stream, SplitWs ws) {
  const auto* s = static_cast<const uint16_t*>(scales);
  const auto* b = static_cast<const uint16_t*>(biases);
  const auto* xx = static_cast<const uint16_t*>(x);
  auto* yy = static_cast<uint16_t*>(y);
  const bool vec = al16(y) && ldy % 8 == 0;
  switch (dtype) {
    case kBf16:
      return launch_big_ep<kBf16>(
          w, s, b, xx,
          EpSwiGLU<kBf16>{yy, ldy, width, gate_row, up_row, in_scale, out_scale, vec}, k, n, m,
          stream, ws);
    case kF16:
      return launch_big_ep<kF16>(
          w, s, b, xx,
          EpSwiGLU<kF16>{yy, ldy, width, gate_row, up_row, in_scale, out_scale, vec}, k, n, m,
          stream, ws);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace imq
