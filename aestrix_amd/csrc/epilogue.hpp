// epilogue.hpp -- output stages of the quantized matmul kernels.
//
// Each functor receives the fp32 accumulator of output (row, col) and writes
// it out.  The fused ones replace the reference's glue kernels that run right
// after a qmm on its f16 output (Sources/ImarelloDirect/DirectDiTKernels.swift):
// they first round the accumulator to T, as the qmm's store would, and then
// apply the glue arithmetic in fp32, so the result equals qmm + glue kernel.
#pragma once

#include "imq_device.hpp"

namespace imq {

// y[row][col] = T(acc): the plain qmm output (row pitch ldy).
template <int T>
struct EpStore {
  static constexpr bool kPair = false;
  typename Elem<T>::S* y;
  int ldy;
  __device__ __forceinline__ void store(int row, int col, float acc) const {
    y[(size_t)row * ldy + col] = Elem<T>::out(acc);
  }
};

__device__ __forceinline__ float round_to(float v, int t) {
  if (t == kBf16) return bf16_to_f32(f32_to_bf16_int(v));
  if (t == kF16) return (float)(_Float16)v;
  return v;
}

// y[row][col] = float(T(acc)) * scale, fp32 out: dd_cast_postscale
// (DirectDiTKernels.swift:199-209), the x16 that undoes the qmm input's /16.
template <int T>
struct EpPostscale {
  static constexpr bool kPair = false;
  float* y;
  int ldy;
  float scale;
  __device__ __forceinline__ void store(int row, int col, float acc) const {
    y[(size_t)row * ldy + col] = round_to(acc, T) * scale;
  }
};

// y[row][col] = fma(gate[col], float(T(acc)) * scale, x[row][col]), fp32
// residual stream: dd_gate_add (DirectDiTKernels.swift:211-224).  y may alias x.
template <int T>
struct EpGateAdd {
  static constexpr bool kPair = false;
  float* y;
  const float* x;
  const float* gate;
  int ld;
  float scale;
  __device__ __forceinline__ void store(int row, int col, float acc) const {
    const size_t i = (size_t)row * ld + col;
    y[i] = __builtin_fmaf(gate[col], round_to(acc, T) * scale, x[i]);
  }
};

// SwiGLU over a gate/up pair of projection rows: dd_swiglu_pitched
// (DirectDiTKernels.swift:137-157).  Output column j pairs weight rows
// gate_row + j and up_row + j; y[row][j] = T(g * sigmoid(g) * u * out_scale)
// with g, u the T-rounded products times in_scale.
template <int T>
struct EpSwiGLU {
  static constexpr bool kPair = true;
  typename Elem<T>::S* y;
  int ldy;
  int width;
  int gate_row;
  int up_row;
  float in_scale;
  float out_scale;
  __device__ __forceinline__ void store2(int row, int j, float acc_g, float acc_u) const {
    const float g = round_to(acc_g, T) * in_scale;
    const float u = round_to(acc_u, T) * in_scale;
    const float sig = 1.0f / (1.0f + __expf(-g));
    y[(size_t)row * ldy + j] = Elem<T>::out(g * sig * u * out_scale);
  }
};

}  // namespace imq
