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

// out[r][k] = deq(W)[clamp(rows[r], 0, n - 1)][k] for r < count (rows on the
// device): the embedding rows of a batch of token ids.  count * k / 8 < 2^32.
hipError_t launch_dequant_rows(const uint32_t* w, const void* scales, const void* biases,
                               const int32_t* rows, int count, void* out, int k, int n, int dtype,
                               hipStream_t stream);

// y[m][n] = x . deq(W)^T for 1 <= m <= 16, T in {bf16, f16, f32}; no MFMA.
hipError_t launch_qgemv(const uint32_t* w, const void* scales, const void* biases, const void* x,
                        void* y, int k, int n, int m, int dtype, hipStream_t stream);

// The qGEMV with a gate/up pair of weight rows per output (the SwiGLU stage
// of launch_qgemm_swiglu, same arguments and result) for 1 <= m <=
// kQgemvSwigluMaxM, T in {bf16, f16}: the gate and up rows of an output are
// read by one lane group and combined after the reduction.
constexpr int kQgemvSwigluMaxM = 4;
hipError_t launch_qgemv_swiglu(const uint32_t* w, const void* scales, const void* biases,
                               const void* x, void* y, int ldy, int k, int n, int m, int width,
                               int gate_row, int up_row, float in_scale, float out_scale,
                               int dtype, hipStream_t stream);

// The qGEMV on RMSNorm'd x: y = x' . deq(W)^T (launch_qgemv_norm) or the
// SwiGLU pair of launch_qgemv_swiglu at in / out scale 1
// (launch_qgemv_swiglu_norm), x' = T(x * rsqrt(mean(x^2) + eps) * nw) row by
// row, bit for bit what launch_rmsnorm_t writes -- the text encoder's
// RMSNorm before q/k/v or gate/up folded into the projection's x staging.
// Only where qgemv_norm_fits (1 <= m <= kQgemvNormMaxM, 16-bit T, k % 8 == 0
// and k <= 4096, x and nw 16-byte aligned, whole rows in one x tile; width 0
// for the plain form); otherwise hipErrorInvalidValue.
constexpr int kQgemvNormMaxM = 2;
bool qgemv_norm_fits(int k, int n, int m, int width, int dtype, const void* x, const float* nw);
hipError_t launch_qgemv_norm(const uint32_t* w, const void* scales, const void* biases,
                             const void* x, const float* nw, float eps, void* y, int k, int n,
                             int m, int dtype, hipStream_t stream);
hipError_t launch_qgemv_swiglu_norm(const uint32_t* w, const void* scales, const void* biases,
                                    const void* x, const float* nw, float eps, void* y, int ldy,
                                    int k, int n, int m, int width, int gate_row, int up_row,
                                    int dtype, hipStream_t stream);

// fp32 scratch for split-K partial sums.  With too few output tiles to fill
// the chip, the MFMA kernel splits K, writes each split's partial sums here
// and a second kernel adds them; a null or short workspace runs unsplit.
// cus: the compute units the tile planner counts on (0: the device's); a
// launch that shares the GPU with another stream's plans for its share.
struct SplitWs {
  float* p = nullptr;
  size_t bytes = 0;
  int cus = 0;
};

// y[m][n] = x . deq(W)^T, any m >= 1, T in {bf16, f16}; MFMA.
hipError_t launch_qgemm(const uint32_t* w, const void* scales, const void* biases, const void* x,
                        void* y, int k, int n, int m, int dtype, hipStream_t stream,
                        SplitWs ws = {});

// Workspace bytes launch_qgemm (fused: a fused stage over n weight rows, 2 *
// width for swiglu) uses for this shape (0: it does not split K).
size_t qgemm_split_bytes(int k, int n, int m, bool fused = false);

// The plan launch_qgemm / the fused launchers choose: big = the buffer-load
// MFMA kernel (else the register-staged 128 x 256 tile kernel), its tile
// height in rows, its K splits and their fp32 workspace bytes.  fused: an
// output stage other than the plain store over n weight rows (2 * width for a
// SwiGLU pair); split: a workspace is available; cus: the compute units the
// planner counts on (0: the device's); pair: the stage is a gate/up pair.
struct QgemmPlan {
  bool big;
  int tile_rows;
  int splits;
  size_t workspace_bytes;
  int tile_cols;
};
QgemmPlan qgemm_plan(int k, int n, int m, bool fused, bool split, int cus, bool pair = false);

// Whether the buffer-load MFMA kernel (and so the fused epilogues) takes
// these shapes: K % 256 == 0 and x, w addressable with 32-bit byte offsets.
bool qgemm_big_supported(int k, int n, int m);

// Fused output stages on the MFMA kernels (T in {bf16, f16}; any K % 64 == 0:
// shapes outside qgemm_big_supported run the register-staged tile kernel,
// never split).  Without a workspace they equal the qmm
// followed by the reference's glue kernel on its T output bit for bit; with
// one (ws.bytes >= qgemm_split_bytes(k, n, m, true)) K may be split, the
// glue applied after the splits are added, which reorders the K sum:
//
//   postscale: y[m][n] (f32) = float(T(acc)) * scale
//   gate_add:  y[m][n] (f32) = residual[m][n] + gate[n] * float(T(acc)) * scale
//              (scale read from scale_dev when the kernel runs, if given)
//   swiglu:    y[m][j] (T, row pitch ldy) = T(g * sigmoid(g) * u * out_scale), j < width,
//              g = float(T(x . W[gate_row + j])) * in_scale, u likewise with up_row.
hipError_t launch_qgemm_postscale(const uint32_t* w, const void* scales, const void* biases,
                                  const void* x, float* y, int k, int n, int m, float scale,
                                  int dtype, hipStream_t stream, SplitWs ws = {},
                                  const float* scale_dev = nullptr);
// postscale with an f16 result (T = f16 only): y[m][n] (f16) =
// f16(float(f16(acc)) * float(f16(scale))), the product of two f16 values
// rounded once (the reference's y * s.asType(.float16)).
hipError_t launch_qgemm_postscale_f16(const uint32_t* w, const void* scales, const void* biases,
                                      const void* x, void* y, int k, int n, int m, float scale,
                                      hipStream_t stream, const float* scale_dev = nullptr);
hipError_t launch_qgemm_gate_add(const uint32_t* w, const void* scales, const void* biases,
                                 const void* x, const float* residual, const float* gate, float* y,
                                 int k, int n, int m, float scale, int dtype, hipStream_t stream,
                                 SplitWs ws = {}, const float* scale_dev = nullptr);
// resid_add: y[m][n] (T) = T(float(resid[m][n]) + float(T(acc))), resid T
//            (the text encoder's dq_add after its o_proj / down_proj); y may be resid.
hipError_t launch_qgemm_resid_add(const uint32_t* w, const void* scales, const void* biases,
                                  const void* x, const void* resid, void* y, int k, int n, int m,
                                  int dtype, hipStream_t stream, SplitWs ws = {});
// The qGEMV with the residual add in its store, m <= 4, 16-bit T:
// y = T(float(resid) + float(T(x . deq(W)^T))) (EpResidAdd's arithmetic).
hipError_t launch_qgemv_resid_add(const uint32_t* w, const void* scales, const void* biases,
                                  const void* x, const void* resid, void* y, int k, int n, int m,
                                  int dtype, hipStream_t stream);
hipError_t launch_qgemm_swiglu(const uint32_t* w, const void* scales, const void* biases,
                               const void* x, void* y, int ldy, int k, int n, int m, int width,
                               int gate_row, int up_row, float in_scale, float out_scale, int dtype,
                               hipStream_t stream, SplitWs ws = {});

// y[i] (T) = T(x[i] / scale) for i < count, x fp32; T in {bf16, f16}; with
// scale_dev the scale is read from device memory when the kernel runs.
hipError_t launch_prescale(const float* x, void* y, size_t count, float scale, int dtype,
                           hipStream_t stream, const float* scale_dev = nullptr);

// *out (device) = max(max_i |x[i]| / target, 1): the per-tensor dynamic scale
// of the f16 qmm sandwich (three small launches; order independent, so the
// result is deterministic).
hipError_t launch_dynamic_scale(const float* x, size_t count, float target, float* out,
                                hipStream_t stream);

// y[r][c] (T) = x[r][c] * rsqrt(mean(x[r]^2) + eps) * w[c] * out_scale, x fp32
// [rows, cols]; out_scale a power of two.
hipError_t launch_rmsnorm(const float* x, const float* w, void* y, int rows, int cols, float eps,
                          int dtype, hipStream_t stream, float out_scale = 1.0f);

// p[i] = v for i < n (a kernel, so that it can precede a graph launch on a
// stream without a host buffer that must outlive the call).
hipError_t launch_fill_f32(float* p, float v, int n, hipStream_t stream);

// y[r][c] (T) = T(x[r][c] * rsqrt(mean(x[r]^2) + eps) * w[c]), x T [rows, cols]
// (the text encoder's RMSNorm on its T residual stream); T in {bf16, f16}.
hipError_t launch_rmsnorm_t(const void* x, const float* w, void* y, int rows, int cols, float eps,
                            int dtype, hipStream_t stream);

// y[i] = x[i] / (1 + exp(-x[i])) for i < n, fp32 (y may be x).
hipError_t launch_silu_f32(const float* x, float* y, int n, hipStream_t stream);

// Largest M the qGEMV kernel takes.
constexpr int kQgemvMaxM = 16;
// Largest bf16 / f16 M the regime dispatcher routes to the qGEMV kernel when
// the few-row kernel below does not take the call: from M = 5 the tiled
// matrix-core kernel is faster, the qGEMV's VALU dot products and reductions
// growing with M.
constexpr int kDispatchGemvMaxM = 4;

// Largest M the weight-streaming MFMA kernel (qskinny.hip) takes: up to 16
// rows every form of it, 17 to 32 rows its K split (two token groups per
// weight fragment) where it plans one.
constexpr int kQskinnyMaxM = 32;
// The M range the regime dispatcher routes to it (bf16 / f16, K % 128 == 0),
// ahead of the qGEMV.  With the weights coming from HBM (text-encoder MLP
// shapes, 48 rotated copies), [9728 x 2560] M = 1 / 2 / 3 / 4: 7.7 / 7.7 /
// 7.7 / 7.9 us against 5.8 / 6.9 / 8.5 / 8.9 us for the qGEMV; [2560 x 9728]:
// 11.2 / 11.1 / 11.2 / 11.6 against 6.2 / 8.5 / 12.1 / 13.1 us.  From M = 3
// this kernel is faster on both.
constexpr int kDispatchSkinnyMinM = 3;
constexpr int kDispatchSkinnyMaxM = 16;

// Whether a SwiGLU qmm runs the qGEMV's pair mode: few rows, 16-bit T, and the
// qGEMV's 32-bit offsets (weights under 4 GiB, one x tile under 2 GiB).
inline bool qgemv_swiglu_fits(int k, int n, int m, int dtype) {
  return m <= kQgemvSwigluMaxM && dtype != 2 /* f32 */ &&
         (size_t)n * (size_t)k / 2 < ((size_t)1 << 32) &&
         (size_t)m * k * 2 < ((size_t)1 << 31);
}

// Bytes of the statically allocated split-K scratch of the allocation-free
// dispatcher (one copy per GPU, scratch.hip).  64 MiB covers the split plans
// of the text-encoder, conditioner and DiT shapes up to M = 2048 (the largest:
// M = 2048 [2560 x 9728], three splits, 60 MiB).
constexpr size_t kStaticScratchBytes = (size_t)64 << 20;
// Device address of that scratch on `device`, which must be current; looked
// up with hipGetSymbolAddress on the first call for a device.
hipError_t static_scratch(int device, void** out);
// Orders the calls that use that scratch on one device: scratch_acquire
// locks the device's order and makes `stream` wait for the previous such
// call (an event recorded on whatever stream it ran on); scratch_release
// records this call's event on `stream` and unlocks.  Outside stream capture
// only (a capturing caller orders its graph replays itself).  The event is
// created by static_scratch, at set-up, so these allocate nothing.
hipError_t scratch_acquire(int device, hipStream_t stream);
hipError_t scratch_release(int device, hipStream_t stream);

// Whether the weight-streaming kernel takes this call: 1 <= m <= 32,
// k % 128 == 0, T in {bf16, f16}, 32-bit byte offsets (past 16 rows only with
// its K split, below).
bool qskinny_supported(int k, int n, int m, int dtype);
// y[m][n] = x . deq(W)^T on the matrix cores, 16 weight rows per workgroup.
// With a workspace of at least qskinny_split_bytes(k, n, m) (nonzero when
// K % 512 == 0 and 6 <= m <= 32: up to 16 rows where x does not fit LDS or
// the multi-tile kernel would take two rounds of the CUs, past 16 rows where
// the row tiles are fewer than 512), K is split over
// qskinny_splits(k, n, m) workgroup ranges whose fp32 partial sums a second
// kernel adds in order; without one the unsplit kernels run (m <= 16, else
// hipErrorInvalidValue).
size_t qskinny_split_bytes(int k, int n, int m);
int qskinny_splits(int k, int n, int m);
hipError_t launch_qskinny(const uint32_t* w, const void* scales, const void* biases, const void* x,
                          void* y, int k, int n, int m, int dtype, hipStream_t stream,
                          SplitWs ws = {});
// The K split with the residual add of launch_qgemm_resid_add in its second
// kernel: y = T(float(resid) + float(T(x . deq(W)^T))), y may be resid.  Only
// where qskinny_resid_split_bytes(k, n, m) > 0 and ws holds that many bytes
// (hipErrorInvalidValue otherwise).  Its plan is the K split's own from 1
// row, also where a plain product would run unsplit (no unsplit kernel has
// the residual add; the tile kernel's form is the alternative).
size_t qskinny_resid_split_bytes(int k, int n, int m);
// y[m][j] = EpSwiGLU(gate sum j, up sum j) for j < width over a pair weight of
// n = 2 width rows (gate rows [0, width), up rows [width, n)): the few-row
// kernel's K split, its fp32 partial sums summed by the tile kernel's
// split-sum kernel with the SwiGLU stage (launch_reduce_swiglu).  Its plan is
// the residual form's (qskinny_resid_split_bytes(k, n, m) > 0, and ws holds
// that many bytes); hipErrorInvalidValue otherwise, before any launch.
hipError_t launch_qskinny_swiglu(const uint32_t* w, const void* scales, const void* biases,
                                 const void* x, void* y, int ldy, int k, int n, int m, int width,
                                 float in_scale, float out_scale, int dtype, hipStream_t stream,
                                 SplitWs ws);
// The SwiGLU output stage over fp32 partial sums ws[split][row][2 width]
// (gate sums at [0, width), up sums at [width, 2 width)): the tile kernel's
// split-sum kernel with EpSwiGLU, in split order.
hipError_t launch_reduce_swiglu(const float* ws, int splits, int m, int width, void* y, int ldy,
                                float in_scale, float out_scale, int dtype, hipStream_t stream);
// y[row][j] = T(silu(g) * u) (EpSwiGLU's arithmetic) from a T product gu
// [rows, ld] with g at column j and u at width + j.
hipError_t launch_swiglu_t(const void* gu, int ld, int rows, int width, void* y, int ldy,
                           float in_scale, float out_scale, int dtype, hipStream_t stream);
hipError_t launch_qskinny_resid_add(const uint32_t* w, const void* scales, const void* biases,
                                    const void* x, const void* resid, void* y, int k, int n, int m,
                                    int dtype, hipStream_t stream, SplitWs ws);
// The same, followed in the split sum's own launch by the row RMSNorm of its
// result: y as above, then h = T(y * rsqrt(mean_n(y^2) + eps) * norm_w)
// (launch_rmsnorm_t's arithmetic) -- the text encoder's o projection, dq_add
// and post-attention RMSNorm in two launches.  Where the _fits predicate holds
// (the split as above, N % 8 == 0, N <= 8192, 16-byte aligned operands);
// hipErrorInvalidValue otherwise, before any launch.
bool qskinny_resid_add_norm_fits(int k, int n, int m, int dtype, const void* resid,
                                 const void* y, const float* norm_w, const void* h, SplitWs ws);
hipError_t launch_qskinny_resid_add_norm(const uint32_t* w, const void* scales,
                                         const void* biases, const void* x, const void* resid,
                                         void* y, const float* norm_w, void* h, float eps, int k,
                                         int n, int m, int dtype, hipStream_t stream, SplitWs ws);

}  // namespace imq
