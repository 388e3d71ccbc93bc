// imq_kernels.hpp -- host-side launchers of the gfx950 kernels.
// Inputs are validated by the caller (the C ABI); launchers only launch.
// dtype is the element type T of x, scales, biases and y/out: 0 bf16, 1 f16,
// 2 f32 (the values of imq_dtype).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace imq {

// out[n][k] = deq(W) in T (bf16, f16 or f32).
hipError_t launch_dequant(const uint32_t* w, const void* scales, const void* biases, void* out,
                          int k, int n, int dtype, hipStream_t stream);

// y[m][n] = x . deq(W)^T for 1 <= m <= 16, T in {bf16, f16, f32}; no MFMA.
hipError_t launch_qgemv(const uint32_t* w, const void* scales, const void* biases, const void* x,
                        void* y, int k, int n, int m, int dtype, hipStream_t stream);

// y[m][n] = x . deq(W)^T, any m >= 1, T in {bf16, f16}; MFMA.
hipError_t launch_qgemm(const uint32_t* w, const void* scales, const void* biases, const void* x,
                        void* y, int k, int n, int m, int dtype, hipStream_t stream);

// Largest M routed to the qGEMV kernel by the regime dispatcher.
constexpr int kQgemvMaxM = 16;

}  // namespace imq
