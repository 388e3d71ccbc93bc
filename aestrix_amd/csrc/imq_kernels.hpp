// imq_kernels.hpp -- host-side launchers of the gfx950 kernels.
// Inputs are validated by the caller (the C ABI); launchers only launch.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace imq {

// out[n][k] = deq(W), bf16 (f16 = false) or f16 (f16 = true) bit patterns.
hipError_t launch_dequant(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                          uint16_t* out, int k, int n, bool f16, hipStream_t stream);

// y[m][n] = x . deq(W)^T for 1 <= m <= 16 (bf16).
hipError_t launch_qgemv(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                        const uint16_t* x, uint16_t* y, int k, int n, int m, hipStream_t stream);

// y[m][n] = x . deq(W)^T, any m >= 1 (bf16, MFMA).
hipError_t launch_qgemm(const uint32_t* w, const uint16_t* scales, const uint16_t* biases,
                        const uint16_t* x, uint16_t* y, int k, int n, int m, hipStream_t stream);

// Largest M routed to the qGEMV kernel by the regime dispatcher.
constexpr int kQgemvMaxM = 16;

}  // namespace imq
