// epilogue.hpp -- output stages of the quantized matmul kernels.
//
// Each functor turns the fp32 accumulator of output (row, col) into its T
// value and writes outputs out.  The fused ones replace the reference's glue
// kernels that run right after a qmm on its f16 output
// (Sources/ImarelloDirect/DirectDiTKernels.swift): they first round the
// accumulator to T, as the qmm's store would, and then apply the glue
// arithmetic in fp32, so the result equals qmm + glue kernel.
#pragma once

#include "imq_device.hpp"

namespace imq {

// Interface.  The large-M kernel stages each output in LDS as the T rounding
// (Elem<T>::pack2, two rows at a time) of value(acc) -- value2(acc_g, acc_u)
// for a gate/up pair -- then writes the staged tile out row by row: emit8 for
// 8 consecutive outputs starting at a multiple of 8 when `vec` (set by the
// host: every pointer and row pitch the functor touches allows 16-byte
// accesses there), emit1 for single outputs otherwise.

// y[row][col] = T(acc): the plain qmm output (row pitch ldy).
template <int T>
struct EpStore {
  static constexpr bool kPair = false;
  static constexpr bool kPartial = false;
  typename Elem<T>::S* y;
  int ldy;
  bool vec;
  __device__ __forceinline__ float value(float acc) const { return acc; }
  __device__ __forceinline__ void emit1(int row, int col, uint16_t v) const {
    y[(size_t)row * ldy + col] = v;
  }
  // Streamed (non-temporal): the output is not read back by this kernel and
  // should not push the activation and weight panels other tiles still read
  // out of the L2 (+0.3-0.7% on the large shapes).
  __device__ __forceinline__ void emit8(int row, int col, uint4 v) const {
    __builtin_nontemporal_store(__builtin_bit_cast(u32x4_t, v),
                                reinterpret_cast<u32x4_t*>(y + (size_t)row * ldy + col));
  }
};

__device__ __forceinline__ float round_to(float v, int t) {
  if (t == kBf16) return bf16_to_f32(f32_to_bf16_int(v));
  if (t == kF16) return (float)(_Float16)v;
  return v;
}

// The float value of a staged T.
template <int T>
__device__ __forceinline__ float staged_value(uint32_t bits) {
  if constexpr (T == kBf16) return __builtin_bit_cast(float, bits << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)bits);
}

// y[row][col] = float(T(acc)) * scale, fp32 out: dd_cast_postscale
// (DirectDiTKernels.swift:199-209), the x16 that undoes the qmm input's /16.
// With scale_dev set the scale is read from device memory when the kernel
// runs (the per-tensor dynamic scale).
template <int T>
struct EpPostscale {
  static constexpr bool kPair = false;
  static constexpr bool kPartial = false;
  float* y;
  int ldy;
  float scale;
  bool vec;
  const float* scale_dev;
  __device__ __forceinline__ float value(float acc) const { return acc; }
  __device__ __forceinline__ float the_scale() const { return scale_dev ? *scale_dev : scale; }
  __device__ __forceinline__ void emit1(int row, int col, uint16_t v) const {
    y[(size_t)row * ldy + col] = staged_value<T>(v) * the_scale();
  }
  __device__ __forceinline__ void emit8(int row, int col, uint4 v) const {
    const float scale = the_scale();
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float o[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[2 * e] = staged_value<T>(w[e] & 0xFFFFu) * scale;
      o[2 * e + 1] = staged_value<T>(w[e] >> 16) * scale;
    }
    float4* d = reinterpret_cast<float4*>(y + (size_t)row * ldy + col);
    d[0] = make_float4(o[0], o[1], o[2], o[3]);
    d[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
};

// y[row][col] (f16) = f16(float(f16(acc)) * float(f16(scale))): the
// post-scale without the f32 upcast (compiledPostScaleF16,
// Sources/ImarelloDiT/AttentionUtils.swift:166-171, `y * s.asType(.float16)`).
// The product of two f16 values is exact in f32, so rounding it once to f16
// is the f16 multiply.  T = f16.
struct EpPostscaleF16 {
  static constexpr bool kPair = false;
  static constexpr bool kPartial = false;
  uint16_t* y;
  int ldy;
  float scale;
  bool vec;
  const float* scale_dev;
  __device__ __forceinline__ float value(float acc) const { return acc; }
  __device__ __forceinline__ float s16() const {
    return (float)(_Float16)(scale_dev ? *scale_dev : scale);
  }
  __device__ __forceinline__ void emit1(int row, int col, uint16_t v) const {
    y[(size_t)row * ldy + col] =
        __builtin_bit_cast(uint16_t, (_Float16)(staged_value<kF16>(v) * s16()));
  }
  __device__ __forceinline__ void emit8(int row, int col, uint4 v) const {
    const float s = s16();
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = pack_f16x2(staged_value<kF16>(w[e] & 0xFFFFu) * s, staged_value<kF16>(w[e] >> 16) * s);
    *reinterpret_cast<uint4*>(y + (size_t)row * ldy + col) = make_uint4(o[0], o[1], o[2], o[3]);
  }
};

// y[row][col] = T(float(r[row][col]) + float(T(acc))), T residual stream: the
// text encoder's dq_add after a qmm (DirectGlueKernels.swift:88-96,
// DirectTEEncoder.swift:392,411).  y may alias r.
template <int T>
struct EpResidAdd {
  static constexpr bool kPair = false;
  static constexpr bool kPartial = false;
  uint16_t* y;
  const uint16_t* r;
  int ld;
  bool vec;
  __device__ __forceinline__ float value(float acc) const { return acc; }
  __device__ __forceinline__ void emit1(int row, int col, uint16_t v) const {
    const size_t i = (size_t)row * ld + col;
    y[i] = Elem<T>::out(staged_value<T>(r[i]) + staged_value<T>(v));
  }
  __device__ __forceinline__ void emit8(int row, int col, uint4 v) const {
    const size_t i = (size_t)row * ld + col;
    const uint4 rv = *reinterpret_cast<const uint4*>(r + i);
    const uint32_t a[4] = {v.x, v.y, v.z, v.w}, b[4] = {rv.x, rv.y, rv.z, rv.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = Elem<T>::pack2(staged_value<T>(b[e] & 0xFFFFu) + staged_value<T>(a[e] & 0xFFFFu),
                            staged_value<T>(b[e] >> 16) + staged_value<T>(a[e] >> 16));
    *reinterpret_cast<uint4*>(y + i) = make_uint4(o[0], o[1], o[2], o[3]);
  }
};

// y[row][col] = fma(gate[col], float(T(acc)) * scale, x[row][col]), fp32
// residual stream: dd_gate_add (DirectDiTKernels.swift:211-224).  y may alias x.
// With scale_dev set, the scale is read from device memory when the kernel runs
// (a graph replay with the Euler step's 16 dt of the current step).
template <int T>
struct EpGateAdd {
  static constexpr bool kPair = false;
  static constexpr bool kPartial = false;
  float* y;
  const float* x;
  const float* gate;
  int ld;
  float scale;
  bool vec;
  const float* scale_dev;
  __device__ __forceinline__ float value(float acc) const { return acc; }
  __device__ __forceinline__ float the_scale() const { return scale_dev ? *scale_dev : scale; }
  __device__ __forceinline__ void emit1(int row, int col, uint16_t v) const {
    const size_t i = (size_t)row * ld + col;
    y[i] = __builtin_fmaf(gate[col], staged_value<T>(v) * the_scale(), x[i]);
  }
  __device__ __forceinline__ void emit8(int row, int col, uint4 v) const {
    const float scale = the_scale();
    const size_t i = (size_t)row * ld + col;
    const float4* xs = reinterpret_cast<const float4*>(x + i);
    const float4* gs = reinterpret_cast<const float4*>(gate + col);
    const float4 x0 = xs[0], x1 = xs[1], g0 = gs[0], g1 = gs[1];
    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
    const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t bits = (e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xFFFFu);
      o[e] = __builtin_fmaf(gv[e], staged_value<T>(bits) * scale, xv[e]);
    }
    float4* d = reinterpret_cast<float4*>(y + i);
    d[0] = make_float4(o[0], o[1], o[2], o[3]);
    d[1] = make_float4(o[4], o[5], o[6], o[7]);
  }
};

// SwiGLU over a gate/up pair of projection rows: dd_swiglu_pitched
// (DirectDiTKernels.swift:137-157).  Output column j pairs weight rows
// gate_row + j and up_row + j; y[row][j] = T(g * sigmoid(g) * u * out_scale)
// with g, u the T-rounded products times in_scale.
template <int T>
struct EpSwiGLU {
  static constexpr bool kPair = true;
  static constexpr bool kPartial = false;
  typename Elem<T>::S* y;
  int ldy;
  int width;
  int gate_row;
  int up_row;
  float in_scale;
  float out_scale;
  bool vec;
  // The sigmoid's reciprocal is v_rcp_f32 (1 ulp) rather than a correctly
  // rounded division: the stage runs after the K loop with nothing to hide
  // it, and the division's ten-instruction sequence per output was most of
  // its cost.  exp(-g) = inf for very negative g gives rcp = 0, g * 0 = -0.
  __device__ __forceinline__ float value2(float acc_g, float acc_u) const {
    const float g = round_to(acc_g, T) * in_scale;
    const float u = round_to(acc_u, T) * in_scale;
    const float sig = __builtin_amdgcn_rcpf(1.0f + __expf(-g));
    return g * sig * u * out_scale;
  }
  __device__ __forceinline__ void emit1(int row, int j, uint16_t v) const {
    y[(size_t)row * ldy + j] = v;
  }
  __device__ __forceinline__ void emit8(int row, int j, uint4 v) const {
    *reinterpret_cast<uint4*>(y + (size_t)row * ldy + j) = v;
  }
};

// Split-K partial sums: the fp32 accumulators themselves, unrounded, into
// ws[split][row][...] (row pitch ldp); a second kernel adds the splits and
// applies the real output stage.  Plain: column col at col (ldp = N).  PAIR
// (a SwiGLU projection): output j's gate sum at j and its up sum at width + j
// (ldp = 2 width), with gate_row, up_row and width as in EpSwiGLU.
template <bool PAIR>
struct EpPartial {
  static constexpr bool kPair = PAIR;
  static constexpr bool kPartial = true;
  float* ws;
  int ldp;
  int width;
  int gate_row;
  int up_row;
};

}  // namespace imq
