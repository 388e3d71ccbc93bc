// cond.cpp -- the per-step conditioning chain (include/imq_cond.h): timestep
// sinusoid on the host, then the f32 quantized projections and SiLU stages of
// DirectConditioner.stepConditioning (Sources/ImarelloDirect/DirectConditioner.swift:168-213)
// for a batch of timesteps at once.
//
// The reference runs six M = 1 dispatches per timestep, each followed by a
// blocking wait.  Each op of the chain is row-local, so the timesteps of one
// call are the rows of one pass: the qGEMV streams every weight once per 16
// timesteps, and the four modulation heads, which read the same input, are
// one launch over their concatenation.
#include <hip/hip_runtime.h>

#include <cmath>
#include <new>

#include "ctx.hpp"
#include "imq.h"
#include "imq_cond.h"
#include "imq_kernels.hpp"

using namespace imq::detail;

namespace {

constexpr int kRows = imq::kQgemvMaxM;  // timesteps per pass

void sinusoid_row(float t, int sin_dim, float* out) {
  // DirectConditioner.sinusoid (:152-166): the same float operations in the
  // same order (flipSinToCos: the cosine half first).
  const int half = sin_dim / 2;
  const float ln_base = logf(10000.0f);
  for (int i = 0; i < half; ++i) {
    const float freq = expf(-ln_base * (float)i / (float)half);
    const float arg = t * freq;
    out[i] = cosf(arg);
    out[half + i] = sinf(arg);
  }
}

// A projection the f32 qGEMV takes: f32 parameters, K % 64 == 0, the packed
// weights 16-byte aligned and under the kernel's 4 GiB of 32-bit offsets.
bool is_f32_weight(const imq_qweight* q) {
  return q && q->w && q->scales && q->biases && q->n > 0 && q->k > 0 && q->k % 64 == 0 &&
         q->dtype == IMQ_F32 && aligned(q->w, 16) && aligned(q->scales, 4) &&
         aligned(q->biases, 4) && (size_t)q->n * (size_t)q->k / 2 < ((size_t)1 << 32);
}

}  // namespace

struct imq_cond {
  imq_ctx* ctx = nullptr;
  imq_qweight l1{}, l2{}, heads{};
  int dim = 0, sin_dim = 0, n_heads = 0;
  void* arena = nullptr;      // device: sin [kRows][sin_dim], t1 / temb_s [kRows][dim]
  float* sin_dev = nullptr;
  float* t1 = nullptr;
  float* temb_s = nullptr;
  float* staging = nullptr;   // pinned host [2][kRows][sin_dim]
  hipEvent_t copied[2] = {};  // the last copy out of each staging half
  int next = 0;
};

namespace {

void release(imq_cond* c) {
  for (hipEvent_t& e : c->copied)
    if (e) (void)hipEventDestroy(e), e = nullptr;
  if (c->staging) (void)hipHostFree(c->staging), c->staging = nullptr;
  if (c->arena) (void)hipFree(c->arena), c->arena = nullptr;
}

}  // namespace

extern "C" {

int imq_cond_sinusoid(const float* timesteps, int count, int sin_dim, float* out) {
  const char* fn = "imq_cond_sinusoid";
  if (count < 0 || sin_dim <= 0 || sin_dim % 2 != 0)
    return fail(nullptr, IMQ_EINVAL, "%s: count %d, sin_dim %d (even, positive)", fn, count,
                sin_dim);
  if (count > 0 && (!timesteps || !out)) return fail(nullptr, IMQ_EINVAL, "%s: null pointer", fn);
  for (int r = 0; r < count; ++r) sinusoid_row(timesteps[r], sin_dim, out + (size_t)r * sin_dim);
  return IMQ_OK;
}

int imq_cond_create(imq_ctx* ctx, const imq_qweight* time_l1, const imq_qweight* time_l2,
                    const imq_qweight* heads, imq_cond** out) {
  const char* fn = "imq_cond_create";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!out) return fail(ctx, IMQ_EINVAL, "%s: null output handle", fn);
  *out = nullptr;
  if (!is_f32_weight(time_l1) || !is_f32_weight(time_l2) || !is_f32_weight(heads))
    return fail(ctx, IMQ_EINVAL,
                "%s: every projection needs 16-byte aligned weights under 4 GiB, f32 scales and "
                "biases, K %% 64 == 0",
                fn);
  const int dim = time_l1->n;
  if (time_l1->k % 2 != 0 || time_l2->n != dim || time_l2->k != dim || heads->k != dim)
    return fail(ctx, IMQ_EINVAL,
                "%s: shapes linear_1 [%d, %d], linear_2 [%d, %d], heads [%d, %d] do not chain "
                "(want [dim, sin_dim], [dim, dim], [n, dim])",
                fn, time_l1->n, time_l1->k, time_l2->n, time_l2->k, heads->n, heads->k);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  auto* c = new (std::nothrow) imq_cond;
  if (!c) return fail(ctx, IMQ_ENOMEM, "%s: out of host memory", fn);
  c->ctx = ctx;
  c->l1 = *time_l1;
  c->l2 = *time_l2;
  c->heads = *heads;
  c->dim = dim;
  c->sin_dim = time_l1->k;
  c->n_heads = heads->n;
  const size_t sin_bytes = (size_t)kRows * c->sin_dim * sizeof(float);
  const size_t row_bytes = (size_t)kRows * dim * sizeof(float);
  hipError_t e = hipMalloc(&c->arena, sin_bytes + 2 * row_bytes);
  if (e == hipSuccess) e = hipHostMalloc((void**)&c->staging, 2 * sin_bytes, hipHostMallocDefault);
  for (int i = 0; i < 2 && e == hipSuccess; ++i)
    e = hipEventCreateWithFlags(&c->copied[i], hipEventDisableTiming);
  if (e != hipSuccess) {
    release(c);
    delete c;
    return hip_fail(ctx, e, fn);
  }
  c->sin_dev = static_cast<float*>(c->arena);
  c->t1 = reinterpret_cast<float*>(static_cast<char*>(c->arena) + sin_bytes);
  c->temb_s = reinterpret_cast<float*>(static_cast<char*>(c->arena) + sin_bytes + row_bytes);
  *out = c;
  return IMQ_OK;
}

int imq_cond_step_conditioning(imq_cond* c, const float* timesteps, int count, float* temb,
                               float* heads, imq_stream stream) {
  const char* fn = "imq_cond_step_conditioning";
  if (!c) return fail(nullptr, IMQ_EINVAL, "%s: null chain", fn);
  imq_ctx* ctx = c->ctx;
  if (count <= 0) return fail(ctx, IMQ_EINVAL, "%s: count %d must be positive", fn, count);
  if (!timesteps || !temb || !heads) return fail(ctx, IMQ_EINVAL, "%s: null pointer", fn);
  if (!aligned(temb, 4) || !aligned(heads, 4))
    return fail(ctx, IMQ_EINVAL, "%s: temb and heads must be 4-byte aligned", fn);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const auto st = static_cast<hipStream_t>(stream);
  const int d = c->dim;
  for (int r0 = 0; r0 < count; r0 += kRows) {
    const int m = count - r0 < kRows ? count - r0 : kRows;
    // The staging half written here was last read by the copy two passes
    // ago; wait for that copy before overwriting it.
    const int half = c->next;
    c->next ^= 1;
    hipError_t e = hipEventSynchronize(c->copied[half]);
    float* stage = c->staging + (size_t)half * kRows * c->sin_dim;
    if (e == hipSuccess) {
      for (int r = 0; r < m; ++r) sinusoid_row(timesteps[r0 + r], c->sin_dim, stage + (size_t)r * c->sin_dim);
      e = hipMemcpyAsync(c->sin_dev, stage, (size_t)m * c->sin_dim * sizeof(float),
                         hipMemcpyHostToDevice, st);
    }
    if (e == hipSuccess) e = hipEventRecord(c->copied[half], st);
    float* temb_r = temb + (size_t)r0 * d;
    if (e == hipSuccess)
      e = imq::launch_qgemv(c->l1.w, c->l1.scales, c->l1.biases, c->sin_dev, c->t1, c->sin_dim, d,
                            m, IMQ_F32, st);
    if (e == hipSuccess) e = imq::launch_silu_f32(c->t1, c->t1, m * d, st);
    if (e == hipSuccess)
      e = imq::launch_qgemv(c->l2.w, c->l2.scales, c->l2.biases, c->t1, temb_r, d, d, m, IMQ_F32,
                            st);
    if (e == hipSuccess) e = imq::launch_silu_f32(temb_r, c->temb_s, m * d, st);
    if (e == hipSuccess)
      e = imq::launch_qgemv(c->heads.w, c->heads.scales, c->heads.biases, c->temb_s,
                            heads + (size_t)r0 * c->n_heads, d, c->n_heads, m, IMQ_F32, st);
    if (e != hipSuccess) return hip_fail(ctx, e, fn);
  }
  return IMQ_OK;
}

int imq_cond_destroy(imq_cond* c) {
  if (!c) return IMQ_OK;
  (void)hipSetDevice(c->ctx->device);
  (void)hipDeviceSynchronize();
  release(c);
  delete c;
  return IMQ_OK;
}

}  // extern "C"
