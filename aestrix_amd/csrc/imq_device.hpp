// imq_device.hpp -- device helpers shared by the gfx950 kernels.
//
// Format: uint32 words of eight 4-bit codes, low nibble first; one bf16
// (scale, bias) pair per 64 consecutive K elements of a row;
// w = RNE_bf16(fl32(scale * q + bias))
// (Sources/ImarelloDirect/DirectTEEncoder.swift:39-46,106-123).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace imq {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kGroup = 64;  // quantization group along K
constexpr int kPack = 8;    // codes per uint32 word

__device__ __forceinline__ float bf16_to_f32(uint32_t h) { return __uint_as_float(h << 16); }

// RNE f32 -> bf16 by the integer formula of DirectTEEncoder.swift:39-43
// (wrapping add, no NaN special case).  Used where results must be
// bit-identical to that formula for every input pattern (the dequantize kernel).
__device__ __forceinline__ uint32_t f32_to_bf16_int(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

// Hardware RNE pack of two floats into a bf16 pair (v_cvt_pk_bf16_f32):
// identical to f32_to_bf16_int for every non-NaN input (finite, +-inf and
// overflow-to-inf alike); NaN inputs become a quiet NaN instead of the
// integer formula's wrapped pattern.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t p;
  p[0] = (__bf16)lo;
  p[1] = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, p);
}

// A 16-bit lane of a dword holding a 4-bit code c at bit position 0 (or 4) is
// the f16 subnormal c * 2^-24 (or c * 2^-20), exactly.  Decoding with a scale
// pre-multiplied by 2^24 (or 2^20) gives fma(s', c * 2^-24, b) == fl32(s*c + b):
// the power-of-two rescale is exact and the fma rounds once, like the
// reference's `scale * q + bias` (for bf16 and f16 scales s*q is exact in f32,
// so one rounding and two agree).  hipcc turns the
// f16 -> f32 conversion + fma into one v_fma_mix_f32.
__device__ __forceinline__ float f16_lo(uint32_t d) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(d & 0xFFFFu));
}
__device__ __forceinline__ float f16_hi(uint32_t d) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(d >> 16));
}

// Dequantize one packed word (codes k..k+7) to four bf16 pairs
// out[p] = (w[2p], w[2p+1]) in k order.  s24 = scale * 2^24, s20 = scale * 2^20.
__device__ __forceinline__ void dequant_word_bf16(uint32_t word, float s24, float s20, float b,
                                                  uint32_t out[4]) {
  const uint32_t d0 = word & 0x000F000Fu;   // codes 0 (lo) and 4 (hi), at bit 0
  const uint32_t d1 = word & 0x00F000F0u;   // codes 1 and 5, at bit 4
  const uint32_t w8 = word >> 8;
  const uint32_t d2 = w8 & 0x000F000Fu;     // codes 2 and 6
  const uint32_t d3 = w8 & 0x00F000F0u;     // codes 3 and 7
  out[0] = pack_bf16x2(__builtin_fmaf(s24, f16_lo(d0), b), __builtin_fmaf(s20, f16_lo(d1), b));
  out[1] = pack_bf16x2(__builtin_fmaf(s24, f16_lo(d2), b), __builtin_fmaf(s20, f16_lo(d3), b));
  out[2] = pack_bf16x2(__builtin_fmaf(s24, f16_hi(d0), b), __builtin_fmaf(s20, f16_hi(d1), b));
  out[3] = pack_bf16x2(__builtin_fmaf(s24, f16_hi(d2), b), __builtin_fmaf(s20, f16_hi(d3), b));
}

typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// Pack two floats into an f16 pair, each rounded to nearest even: one
// v_cvt_pk_f16_f32 on gfx950 (two v_cvt_f16_f32 and a pack when written as
// two scalar conversions).
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  f16x2_t p;
  p[0] = (_Float16)lo;
  p[1] = (_Float16)hi;
  return __builtin_bit_cast(uint32_t, p);
}

// dequant_word_bf16 with f16 results: out[p] = (w[2p], w[2p+1]) as RNE_f16(fl32(s*q + b)).
__device__ __forceinline__ void dequant_word_f16(uint32_t word, float s24, float s20, float b,
                                                 uint32_t out[4]) {
  const uint32_t d0 = word & 0x000F000Fu;
  const uint32_t d1 = word & 0x00F000F0u;
  const uint32_t w8 = word >> 8;
  const uint32_t d2 = w8 & 0x000F000Fu;
  const uint32_t d3 = w8 & 0x00F000F0u;
  out[0] = pack_f16x2(__builtin_fmaf(s24, f16_lo(d0), b), __builtin_fmaf(s20, f16_lo(d1), b));
  out[1] = pack_f16x2(__builtin_fmaf(s24, f16_lo(d2), b), __builtin_fmaf(s20, f16_lo(d3), b));
  out[2] = pack_f16x2(__builtin_fmaf(s24, f16_hi(d0), b), __builtin_fmaf(s20, f16_hi(d1), b));
  out[3] = pack_f16x2(__builtin_fmaf(s24, f16_hi(d2), b), __builtin_fmaf(s20, f16_hi(d3), b));
}

// -0.0f the compiler cannot see: fma(a, b, -0.0f) is a * b exactly (one
// rounding, the product's own zero sign), and a literal -0.0f addend is
// simplified into a multiply, which then needs the f16 -> f32 conversion of
// the code as an instruction of its own; with this addend the fma stays a
// v_fma_mix_f32 that reads the code's 16-bit half directly.
__device__ __forceinline__ float opaque_neg_zero() {
  float z;
  asm volatile("v_mov_b32 %0, 0x80000000" : "=v"(z));
  return z;
}

// The eight codes of a word as f32 weights fl32(fl32(s*q) + b), in k order:
// two rounded operations, like the reference's `scale * q + bias` on Float.
// With f32 scales (24-bit significands) s*q is not exact in f32, so one fma
// of all three would round differently: the product is rounded by an fma with
// a -0 addend (nz, from opaque_neg_zero), the sum by an add.  s24 = s * 2^24
// and s20 = s * 2^20 are exact.
__device__ __forceinline__ void dequant_word_f32(uint32_t word, float s24, float s20, float b,
                                                 float nz, float out[8]) {
#pragma clang fp contract(off)
  const uint32_t d0 = word & 0x000F000Fu;
  const uint32_t d1 = word & 0x00F000F0u;
  const uint32_t w8 = word >> 8;
  const uint32_t d2 = w8 & 0x000F000Fu;
  const uint32_t d3 = w8 & 0x00F000F0u;
  out[0] = __builtin_fmaf(s24, f16_lo(d0), nz) + b;
  out[1] = __builtin_fmaf(s20, f16_lo(d1), nz) + b;
  out[2] = __builtin_fmaf(s24, f16_lo(d2), nz) + b;
  out[3] = __builtin_fmaf(s20, f16_lo(d3), nz) + b;
  out[4] = __builtin_fmaf(s24, f16_hi(d0), nz) + b;
  out[5] = __builtin_fmaf(s20, f16_hi(d1), nz) + b;
  out[6] = __builtin_fmaf(s24, f16_hi(d2), nz) + b;
  out[7] = __builtin_fmaf(s20, f16_hi(d3), nz) + b;
}

// Element type T of x, scales, biases and y (the values of imq_dtype).
enum Dtype : int { kBf16 = 0, kF16 = 1, kF32 = 2 };

template <int T>
struct Elem;

template <>
struct Elem<kBf16> {
  using S = uint16_t;
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float param(S v) { return bf16_to_f32(v); }
  static __device__ __forceinline__ S out(float v) { return (S)f32_to_bf16_int(v); }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_bf16x2(lo, hi); }
  static __device__ __forceinline__ void dequant(uint32_t word, float s24, float s20, float b,
                                                 uint32_t o[4]) {
    dequant_word_bf16(word, s24, s20, b, o);
  }
};

template <>
struct Elem<kF16> {
  using S = uint16_t;
  static constexpr int kBytes = 2;
  static __device__ __forceinline__ float param(S v) {
    return (float)__builtin_bit_cast(_Float16, v);
  }
  static __device__ __forceinline__ S out(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) { return pack_f16x2(lo, hi); }
  static __device__ __forceinline__ void dequant(uint32_t word, float s24, float s20, float b,
                                                 uint32_t o[4]) {
    dequant_word_f16(word, s24, s20, b, o);
  }
};

template <>
struct Elem<kF32> {
  using S = float;
  static constexpr int kBytes = 4;
  static __device__ __forceinline__ float param(S v) { return v; }
  static __device__ __forceinline__ S out(float v) { return v; }
};

typedef __attribute__((address_space(3))) void lds_void_t;

// Raw buffer resource over [base, base + bytes) (gfx9 word 3: 32-bit data
// format).  Buffer loads take a per-lane 32-bit byte offset plus a scalar one.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// Direct buffer -> LDS load of 16 bytes per lane: lane L writes
// lds_wave_base + 16 L (lds_wave_base must be uniform across the wave).
__device__ __forceinline__ void load_lds16(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff,
                                           void* lds_wave_base) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)lds_wave_base, 16, voff, soff, 0, 0);
}

// 16 bytes straight into registers (buffer_load_dwordx4).
__device__ __forceinline__ u32x4_t load_b128(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
  return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, voff, soff, 0));
}

// s_waitcnt vmcnt(n) leaving expcnt and lgkmcnt unconstrained (gfx9 encoding).
#define IMQ_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))
// s_waitcnt vmcnt(0) lgkmcnt(0): every load of this wave, to registers or LDS,
// and every LDS read has completed.
#define IMQ_WAIT_VM_LGKM_0() __builtin_amdgcn_s_waitcnt(7 << 4)

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), acc, false);
}

__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float acc) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b),
                                acc, false);
}

}  // namespace imq
