// capi.cpp -- the C ABI of include/imq.h over the gfx950 kernels.
//
// Error conventions follow the reference's engine: misuse is reported, never
// crashes (the reference throws SpikeError.missingTensor / .metal,
// Sources/ImarelloDirect/DirectQmmSpike.swift:17-19, and checks the command
// buffer error after the wait, Sources/ImarelloDirect/DirectDiTStep.swift:968-970).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <new>
#include <string>

#include "ctx.hpp"
#include "imq.h"
#include "imq_kernels.hpp"

imq_ctx::~imq_ctx() {
  for (int i = 0; i < kStagingBuffers; ++i) {
    if (staging_done[i]) (void)hipEventDestroy(staging_done[i]);
    if (staging[i]) (void)hipHostFree(staging[i]);
  }
  for (auto& kv : split_ws)
    if (kv.second.first) (void)hipFree(kv.second.first);
  for (void* p : retired_ws) (void)hipFree(p);
}

namespace imq {

CopyPool::CopyPool(int workers) {
  for (int i = 0; i < workers; ++i) {
    try {
      threads_.emplace_back([this] { work(); });
    } catch (...) {
      break;  // fewer workers: the calling thread does the rest
    }
  }
}

CopyPool::~CopyPool() {
  {
    std::lock_guard<std::mutex> lk(mu_);
    stop_ = true;
  }
  start_cv_.notify_all();
  for (auto& t : threads_) t.join();
}

void CopyPool::run(int parts, const std::function<void(int)>& fn) {
  std::unique_lock<std::mutex> lk(mu_);
  fn_ = &fn;
  parts_ = parts;
  next_ = 0;
  remaining_ = parts;
  ++gen_;
  start_cv_.notify_all();
  while (next_ < parts_) {
    const int i = next_++;
    lk.unlock();
    fn(i);
    lk.lock();
    --remaining_;
  }
  done_cv_.wait(lk, [this] { return remaining_ == 0; });
  fn_ = nullptr;
}

void CopyPool::work() {
  unsigned long seen = 0;
  std::unique_lock<std::mutex> lk(mu_);
  for (;;) {
    start_cv_.wait(lk, [&] { return stop_ || gen_ != seen; });
    if (stop_) return;
    seen = gen_;
    while (fn_ && next_ < parts_) {
      const int i = next_++;
      const std::function<void(int)>* fn = fn_;
      lk.unlock();
      (*fn)(i);
      lk.lock();
      if (--remaining_ == 0) done_cv_.notify_all();
    }
  }
}

namespace detail {

thread_local std::string g_create_error;  // failures before a context exists

int fail(imq_ctx* ctx, int status, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) {
    std::lock_guard<std::mutex> lk(ctx->mu);
    ctx->err = buf;
  } else {
    g_create_error = buf;
  }
  return status;
}

int hip_fail(imq_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, IMQ_EHIP, "%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
}

bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

size_t elem_size(imq_dtype dtype) { return dtype == IMQ_F32 ? 4 : 2; }

int bind_device(imq_ctx* ctx) {
  const hipError_t e = hipSetDevice(ctx->device);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, "hipSetDevice");
}

}  // namespace detail
}  // namespace imq

using namespace imq::detail;

namespace {

// Shared validation of the quantized-matmul entry points.
int check_qmm(imq_ctx* ctx, const char* fn, const uint32_t* w, const void* s, const void* b,
              const void* x, void* y, int k, int n, int m, int group_size, int bits,
              imq_dtype dtype) {
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!w || !s || !b || !x || !y)
    return fail(ctx, IMQ_EINVAL, "%s: null device pointer (w=%p scales=%p biases=%p x=%p y=%p)",
                fn, (const void*)w, s, b, x, y);
  if (group_size != 64)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: group_size %d (only 64 is provided)", fn, group_size);
  if (bits != 4) return fail(ctx, IMQ_EUNSUPPORTED, "%s: bits %d (only 4 is provided)", fn, bits);
  if (dtype != IMQ_BF16 && dtype != IMQ_F16 && dtype != IMQ_F32)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d (bf16, f16 and f32 are provided)", fn,
                (int)dtype);
  if (k <= 0 || n <= 0 || m <= 0)
    return fail(ctx, IMQ_EINVAL, "%s: non-positive shape K=%d N=%d M=%d", fn, k, n, m);
  if (k % 64 != 0)
    return fail(ctx, IMQ_EINVAL, "%s: K=%d is not a multiple of the group size 64", fn, k);
  if (!aligned(w, 16) || !aligned(x, 16))
    return fail(ctx, IMQ_EINVAL, "%s: w and x must be 16-byte aligned", fn);
  const size_t es = elem_size(dtype);
  if (!aligned(s, es) || !aligned(b, es) || !aligned(y, es))
    return fail(ctx, IMQ_EINVAL, "%s: scales, biases and y must be %zu-byte aligned", fn, es);
  return IMQ_OK;
}

// kAuto: the regime dispatcher (imq_qmm_t); kAutoNoAlloc: the same plan with
// the split-K partial sums in the library's static scratch
// (imq_qmm_t_noalloc); kGemv / kGemm: one kernel family alone.
enum class Regime { kAuto, kAutoNoAlloc, kGemv, kGemm };

// The split-K workspace of stream st, at least `need` bytes; empty (run
// unsplit) when it would have to grow during stream capture or the
// allocation fails.  A workspace that is outgrown is retired, not freed: a
// graph captured earlier on this stream still addresses it, and so may the
// stream's queued work; retired buffers are freed with the context.
imq::SplitWs split_ws(imq_ctx* ctx, hipStream_t st, size_t need) {
  if (need == 0) return {};
  std::lock_guard<std::mutex> lk(ctx->ws_mu);
  auto& e = ctx->split_ws[st];
  if (e.second >= need) return {static_cast<float*>(e.first), e.second};
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
    (void)hipGetLastError();
    return {};
  }
  void* p = nullptr;
  if (hipMalloc(&p, need) != hipSuccess) {
    (void)hipGetLastError();
    return {};
  }
  if (e.first) ctx->retired_ws.push_back(e.first);
  e = {p, need};
  return {static_cast<float*>(p), need};
}

// Orders an allocation-free call that uses the static scratch after the
// previous such call on the same GPU, whatever stream or thread made it, so
// that eager calls never share the scratch in flight.  Not under stream
// capture: a captured call's graph replays are ordered by their caller.
class ScratchOrder {
 public:
  ~ScratchOrder() { (void)release(); }
  hipError_t acquire(int device, hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess || cs != hipStreamCaptureStatusNone) return e;
    e = imq::scratch_acquire(device, st);
    if (e == hipSuccess) {
      device_ = device;
      st_ = st;
      held_ = true;
    }
    return e;
  }
  hipError_t release() {
    if (!held_) return hipSuccess;
    held_ = false;
    return imq::scratch_release(device_, st_);
  }

 private:
  int device_ = -1;
  hipStream_t st_ = nullptr;
  bool held_ = false;
};

int run_qmm(imq_ctx* ctx, const char* fn, Regime regime, const uint32_t* w, const void* s,
            const void* b, const void* x, void* y, int k, int n, int m, int group_size, int bits,
            imq_dtype dtype, imq_stream stream) {
  int rc = check_qmm(ctx, fn, w, s, b, x, y, k, n, m, group_size, bits, dtype);
  if (rc != IMQ_OK) return rc;
  if (regime == Regime::kGemv && m > imq::kQgemvMaxM)
    return fail(ctx, IMQ_EINVAL, "%s: M=%d exceeds the qGEMV limit %d", fn, m, imq::kQgemvMaxM);
  if (regime == Regime::kGemm && dtype == IMQ_F32)
    return fail(ctx, IMQ_EUNSUPPORTED,
                "%s: f32 has no MFMA kernel (imq_qmm_t runs f32 at any M on the qGEMV kernel)", fn);
  const size_t es = elem_size(dtype);
  // The qGEMV kernel addresses one 16-row block of x with 32-bit byte offsets.
  if (regime != Regime::kGemm && (size_t)std::min(m, imq::kQgemvMaxM) * k * es >= ((size_t)1 << 31))
    return fail(ctx, IMQ_EINVAL, "%s: K=%d too long for the qGEMV kernel", fn, k);
  // The qGEMV kernel addresses the packed weights with 32-bit byte offsets.
  const bool w_fits_gemv = (size_t)n * (size_t)k / 2 < ((size_t)1 << 32);
  if (!w_fits_gemv && (regime == Regime::kGemv || dtype == IMQ_F32))
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: %zu bytes of packed weights: the qGEMV kernel takes "
                "under 4 GiB", fn, (size_t)n * (size_t)k / 2);
  if ((rc = bind_device(ctx)) != IMQ_OK) return rc;
  const bool automatic = regime == Regime::kAuto || regime == Regime::kAutoNoAlloc;
  const bool gemv = regime == Regime::kGemv ||
                    (automatic && w_fits_gemv && (m <= imq::kDispatchGemvMaxM || dtype == IMQ_F32));
  const bool few = automatic && m >= imq::kDispatchSkinnyMinM && m <= imq::kQskinnyMaxM &&
                   imq::qskinny_supported(k, n, m, (int)dtype);
  auto st = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  // The few-row kernel may split K over a workspace (long K, few row tiles);
  // past kDispatchSkinnyMaxM rows it runs only that way, and only with the
  // workspace in hand (otherwise the tile kernel takes the call).
  imq::SplitWs sws{};
  bool skinny = false;
  if (few) {
    const size_t need = imq::qskinny_split_bytes(k, n, m);
    if (regime == Regime::kAuto) {
      sws = split_ws(ctx, st, need);
    } else if (regime == Regime::kAutoNoAlloc && need > 0) {
      // imq_qmm_t would split here; running unsplit (or on the tile kernel)
      // would change the bits, so a plan the static scratch cannot hold is
      // refused, as on the tile path below.
      if (need > imq::kStaticScratchBytes)
        return fail(ctx, IMQ_EINVAL,
                    "%s: M=%d N=%d K=%d needs %zu bytes of split-K scratch; the static scratch "
                    "holds %zu (imq_qmm_t takes this shape)",
                    fn, m, n, k, need, imq::kStaticScratchBytes);
      sws = imq::SplitWs{static_cast<float*>(ctx->static_scratch), need};
    }
    skinny = m <= imq::kDispatchSkinnyMaxM || (need > 0 && sws.p && sws.bytes >= need);
  }
  ScratchOrder order;
  if (skinny) {
    if (regime == Regime::kAutoNoAlloc && sws.p && (e = order.acquire(ctx->device, st)) != hipSuccess)
      return hip_fail(ctx, e, fn);
    e = imq::launch_qskinny(w, s, b, x, y, k, n, m, (int)dtype, st, sws);
  } else if (!gemv) {
    // The dispatcher may split K over a workspace; imq_qgemm is the plain
    // tile kernel (the fused output stages equal it bit for bit).
    imq::SplitWs ws{};
    if (regime == Regime::kAuto) {
      ws = split_ws(ctx, st, imq::qgemm_split_bytes(k, n, m));
    } else if (regime == Regime::kAutoNoAlloc) {
      const size_t need = imq::qgemm_split_bytes(k, n, m);
      if (need > imq::kStaticScratchBytes)
        return fail(ctx, IMQ_EINVAL,
                    "%s: M=%d N=%d K=%d needs %zu bytes of split-K scratch; the static scratch "
                    "holds %zu (imq_qmm_t takes this shape)",
                    fn, m, n, k, need, imq::kStaticScratchBytes);
      if (need > 0) ws = imq::SplitWs{static_cast<float*>(ctx->static_scratch), need};
      if (ws.p && (e = order.acquire(ctx->device, st)) != hipSuccess) return hip_fail(ctx, e, fn);
    }
    e = imq::launch_qgemm(w, s, b, x, y, k, n, m, (int)dtype, st, ws);
  } else {
    // f32 beyond 16 rows (the conditioner's multi-row calls): blocks of 16 rows.
    const auto* xb = static_cast<const char*>(x);
    auto* yb = static_cast<char*>(y);
    for (int m0 = 0; m0 < m && e == hipSuccess; m0 += imq::kQgemvMaxM) {
      const int mb = std::min(imq::kQgemvMaxM, m - m0);
      e = imq::launch_qgemv(w, s, b, xb + (size_t)m0 * k * es, yb + (size_t)m0 * n * es, k, n, mb,
                            (int)dtype, st);
    }
  }
  const hipError_t eo = order.release();
  if (e == hipSuccess) e = eo;
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

}  // namespace

namespace {

// Shared checks of the fused-epilogue entry points: the qmm checks, then T in
// {bf16, f16} (any K % 64 == 0: K % 256 != 0 runs the register-staged tile
// kernel with the same output stage).
int check_epilogue(imq_ctx* ctx, const char* fn, const uint32_t* w, const void* s, const void* b,
                   const void* x, const void* y, int k, int n, int m, int group_size, int bits,
                   imq_dtype dtype) {
  int rc = check_qmm(ctx, fn, w, s, b, x, const_cast<void*>(y), k, n, m, group_size, bits, dtype);
  if (rc != IMQ_OK) return rc;
  if (dtype == IMQ_F32)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: f32 has no MFMA kernel (bf16 and f16 are provided)",
                fn);
  return bind_device(ctx);
}

bool swiglu_on_qgemv(int k, int n, int m, imq_dtype dtype) {
  return imq::qgemv_swiglu_fits(k, n, m, (int)dtype);
}

}  // namespace

extern "C" {

int imq_abi_version(void) { return IMQ_ABI_VERSION; }

const char* imq_status_string(int status) {
  switch (status) {
    case IMQ_OK: return "IMQ_OK";
    case IMQ_EINVAL: return "IMQ_EINVAL";
    case IMQ_EUNSUPPORTED: return "IMQ_EUNSUPPORTED";
    case IMQ_EHIP: return "IMQ_EHIP";
    case IMQ_ENOMEM: return "IMQ_ENOMEM";
    default: return "IMQ_UNKNOWN";
  }
}

int imq_create(int device, imq_ctx** out) {
  if (!out) return fail(nullptr, IMQ_EINVAL, "imq_create: null output pointer");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return hip_fail(nullptr, e, "imq_create: hipGetDeviceCount");
  if (device < 0 || device >= count)
    return fail(nullptr, IMQ_EINVAL, "imq_create: device %d out of range [0, %d)", device, count);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(nullptr, e, "imq_create: hipSetDevice");
  // The device address of this GPU's copy of the static split-K scratch
  // (imq_qmm_t_noalloc), looked up once per device with the device current.
  void* scratch = nullptr;
  e = imq::static_scratch(device, &scratch);
  if (e != hipSuccess) return hip_fail(nullptr, e, "imq_create: static scratch address");
  auto* c = new (std::nothrow) imq_ctx;
  if (!c) return fail(nullptr, IMQ_ENOMEM, "imq_create: out of host memory");
  c->device = device;
  c->static_scratch = scratch;
  *out = c;
  return IMQ_OK;
}

int imq_destroy(imq_ctx* ctx) {
  delete ctx;
  return IMQ_OK;
}

const char* imq_last_error(const imq_ctx* ctx) {
  if (!ctx) return g_create_error.c_str();
  std::lock_guard<std::mutex> lk(ctx->mu);
  return ctx->err.c_str();
}

int imq_stream_create(imq_ctx* ctx, imq_stream* out) {
  if (!ctx || !out) return fail(ctx, IMQ_EINVAL, "imq_stream_create: null argument");
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  hipStream_t s = nullptr;
  const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(ctx, e, "imq_stream_create");
  *out = static_cast<imq_stream>(s);
  return IMQ_OK;
}

int imq_stream_destroy(imq_ctx* ctx, imq_stream stream) {
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "imq_stream_destroy: null context");
  if (!stream) return IMQ_OK;
  const hipError_t e = hipStreamDestroy(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, "imq_stream_destroy");
}

int imq_stream_sync(imq_ctx* ctx, imq_stream stream) {
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "imq_stream_sync: null context");
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = hipStreamSynchronize(static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, "imq_stream_sync");
}

int imq_malloc(imq_ctx* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return fail(ctx, IMQ_EINVAL, "imq_malloc: null argument");
  *out = nullptr;
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = hipMalloc(out, bytes ? bytes : 1);
  if (e == hipErrorOutOfMemory)
    return fail(ctx, IMQ_ENOMEM, "imq_malloc: %zu bytes: out of device memory", bytes);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, "imq_malloc");
}

int imq_free(imq_ctx* ctx, void* ptr) {
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "imq_free: null context");
  if (!ptr) return IMQ_OK;
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = hipFree(ptr);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, "imq_free");
}

static int copy(imq_ctx* ctx, const char* fn, void* dst, const void* src, size_t bytes,
                hipMemcpyKind kind, imq_stream stream) {
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (bytes == 0) return IMQ_OK;
  if (!dst || !src) return fail(ctx, IMQ_EINVAL, "%s: null pointer", fn);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_memcpy_h2d(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream) {
  return copy(ctx, "imq_memcpy_h2d", dst, src, bytes, hipMemcpyHostToDevice, stream);
}

int imq_memcpy_d2h(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream) {
  return copy(ctx, "imq_memcpy_d2h", dst, src, bytes, hipMemcpyDeviceToHost, stream);
}

int imq_memcpy_d2d(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream) {
  return copy(ctx, "imq_memcpy_d2d", dst, src, bytes, hipMemcpyDeviceToDevice, stream);
}

int imq_dequantize_rows(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                        const int32_t* rows, int count, void* out, int k, int n, int group_size,
                        int bits, imq_dtype dtype, imq_stream stream) {
  const char* fn = "imq_dequantize_rows";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (group_size != 64)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: group_size %d (only 64 is provided)", fn, group_size);
  if (bits != 4) return fail(ctx, IMQ_EUNSUPPORTED, "%s: bits %d (only 4 is provided)", fn, bits);
  if (dtype != IMQ_BF16 && dtype != IMQ_F16 && dtype != IMQ_F32)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d (bf16, f16 and f32 are provided)", fn,
                (int)dtype);
  if (k <= 0 || n <= 0 || count < 0)
    return fail(ctx, IMQ_EINVAL, "%s: shape K=%d N=%d count=%d", fn, k, n, count);
  if (k % 64 != 0)
    return fail(ctx, IMQ_EINVAL, "%s: K=%d is not a multiple of the group size 64", fn, k);
  if ((size_t)count * (size_t)(k / 8) >= ((size_t)1 << 32))
    return fail(ctx, IMQ_EINVAL, "%s: count %d x K %d past the kernel's 32-bit word index", fn,
                count, k);
  if (count == 0) return IMQ_OK;
  if (!w || !scales || !biases || !rows || !out)
    return fail(ctx, IMQ_EINVAL, "%s: null device pointer", fn);
  const size_t es = elem_size(dtype);
  if (!aligned(w, 4) || !aligned(rows, 4) || !aligned(out, 16) || !aligned(scales, es) ||
      !aligned(biases, es))
    return fail(ctx, IMQ_EINVAL, "%s: misaligned pointer (w, rows 4; out 16; scales, biases %zu)",
                fn, es);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = imq::launch_dequant_rows(w, scales, biases, rows, count, out, k, n,
                                                (int)dtype, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_dequantize(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                   void* out, int k, int n, int group_size, int bits, imq_dtype dtype,
                   imq_stream stream) {
  const char* fn = "imq_dequantize";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!w || !scales || !biases || !out)
    return fail(ctx, IMQ_EINVAL, "%s: null device pointer", fn);
  if (group_size != 64)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: group_size %d (only 64 is provided)", fn, group_size);
  if (bits != 4) return fail(ctx, IMQ_EUNSUPPORTED, "%s: bits %d (only 4 is provided)", fn, bits);
  if (dtype != IMQ_BF16 && dtype != IMQ_F16 && dtype != IMQ_F32)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d (bf16, f16 and f32 are provided)", fn,
                (int)dtype);
  if (k <= 0 || n <= 0)
    return fail(ctx, IMQ_EINVAL, "%s: non-positive shape K=%d N=%d", fn, k, n);
  if (k % 64 != 0)
    return fail(ctx, IMQ_EINVAL, "%s: K=%d is not a multiple of the group size 64", fn, k);
  if (!aligned(w, 16) || !aligned(out, 16))
    return fail(ctx, IMQ_EINVAL, "%s: w and out must be 16-byte aligned", fn);
  const size_t es = elem_size(dtype);
  if (!aligned(scales, es) || !aligned(biases, es))
    return fail(ctx, IMQ_EINVAL, "%s: scales and biases must be %zu-byte aligned", fn, es);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = imq::launch_dequant(w, scales, biases, out, k, n, (int)dtype,
                                           static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_qmm_t(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
              const void* x, void* y, int k, int n, int m, int group_size, int bits,
              imq_dtype dtype, imq_stream stream) {
  return run_qmm(ctx, "imq_qmm_t", Regime::kAuto, w, scales, biases, x, y, k, n, m, group_size,
                 bits, dtype, stream);
}

int imq_qmm_t_noalloc(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                      const void* x, void* y, int k, int n, int m, int group_size, int bits,
                      imq_dtype dtype, imq_stream stream) {
  return run_qmm(ctx, "imq_qmm_t_noalloc", Regime::kAutoNoAlloc, w, scales, biases, x, y, k, n, m,
                 group_size, bits, dtype, stream);
}

int imq_qmm_plan(imq_ctx* ctx, int entry, int k, int n, int m, imq_dtype dtype, imq_plan* out) {
  const char* fn = "imq_qmm_plan";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!out) return fail(ctx, IMQ_EINVAL, "%s: null output", fn);
  *out = imq_plan{};
  if (dtype != IMQ_BF16 && dtype != IMQ_F16 && dtype != IMQ_F32)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d", fn, (int)dtype);
  if (k <= 0 || n <= 0 || m <= 0 || k % 64 != 0)
    return fail(ctx, IMQ_EINVAL, "%s: shape K=%d N=%d M=%d (K a multiple of 64, all > 0)", fn, k,
                n, m);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const bool w_fits_gemv = (size_t)n * (size_t)k / 2 < ((size_t)1 << 32);
  auto tile = [&](bool fused, bool split, bool pair = false) {
    const imq::QgemmPlan p = imq::qgemm_plan(k, n, m, fused, split, 0, pair);
    *out = imq_plan{p.big ? IMQ_KERNEL_TILE : IMQ_KERNEL_TILE_REG, p.tile_rows, p.splits,
                    p.workspace_bytes, p.tile_cols};
    return IMQ_OK;
  };
  switch (entry) {
    case IMQ_ENTRY_QGEMV:
      if (m > imq::kQgemvMaxM)
        return fail(ctx, IMQ_EINVAL, "%s: M=%d exceeds the qGEMV limit %d", fn, m,
                    imq::kQgemvMaxM);
      if (!w_fits_gemv)
        return fail(ctx, IMQ_EUNSUPPORTED, "%s: packed weights of 4 GiB or more", fn);
      *out = imq_plan{IMQ_KERNEL_QGEMV, 0, 1, 0};
      return IMQ_OK;
    case IMQ_ENTRY_SWIGLU:
      if (dtype == IMQ_F32) return fail(ctx, IMQ_EUNSUPPORTED, "%s: f32 has no MFMA kernel", fn);
      if (swiglu_on_qgemv(k, n, m, dtype)) {
        *out = imq_plan{IMQ_KERNEL_QGEMV, 0, 1, 0};
        return IMQ_OK;
      }
      return tile(true, false, true);
    case IMQ_ENTRY_QGEMM:
    case IMQ_ENTRY_FUSED:
      if (dtype == IMQ_F32) return fail(ctx, IMQ_EUNSUPPORTED, "%s: f32 has no MFMA kernel", fn);
      return tile(entry == IMQ_ENTRY_FUSED, false);
    case IMQ_ENTRY_QMM_T: {
      const bool gemv = w_fits_gemv && (m <= imq::kDispatchGemvMaxM || dtype == IMQ_F32);
      const size_t few_need = imq::qskinny_supported(k, n, m, (int)dtype)
                                  ? imq::qskinny_split_bytes(k, n, m) : 0;
      if (m >= imq::kDispatchSkinnyMinM && imq::qskinny_supported(k, n, m, (int)dtype) &&
          (m <= imq::kDispatchSkinnyMaxM || few_need > 0)) {
        const size_t need = few_need;
        *out = imq_plan{IMQ_KERNEL_FEW_ROW, 0, need ? imq::qskinny_splits(k, n, m) : 1, need};
        return IMQ_OK;
      }
      if (gemv) {
        *out = imq_plan{IMQ_KERNEL_QGEMV, 0, 1, 0};
        return IMQ_OK;
      }
      if (dtype == IMQ_F32) return fail(ctx, IMQ_EUNSUPPORTED, "%s: f32 weights of 4 GiB", fn);
      return tile(false, true);
    }
    default:
      return fail(ctx, IMQ_EINVAL, "%s: unknown entry %d", fn, entry);
  }
}

int imq_qgemv(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
              const void* x, void* y, int k, int n, int m, int group_size, int bits,
              imq_dtype dtype, imq_stream stream) {
  return run_qmm(ctx, "imq_qgemv", Regime::kGemv, w, scales, biases, x, y, k, n, m, group_size,
                 bits, dtype, stream);
}

int imq_qgemm(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
              const void* x, void* y, int k, int n, int m, int group_size, int bits,
              imq_dtype dtype, imq_stream stream) {
  return run_qmm(ctx, "imq_qgemm", Regime::kGemm, w, scales, biases, x, y, k, n, m, group_size,
                 bits, dtype, stream);
}


int imq_cast_prescale(imq_ctx* ctx, const float* x, void* y, size_t count, float scale,
                      imq_dtype dtype, imq_stream stream) {
  const char* fn = "imq_cast_prescale";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (dtype != IMQ_BF16 && dtype != IMQ_F16)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d (bf16 and f16 are provided)", fn, (int)dtype);
  if (!std::isfinite(scale) || scale == 0.0f)
    return fail(ctx, IMQ_EINVAL, "%s: scale %g must be finite and nonzero", fn, (double)scale);
  if (count == 0) return IMQ_OK;
  if (!x || !y) return fail(ctx, IMQ_EINVAL, "%s: null device pointer", fn);
  if (!aligned(x, 4) || !aligned(y, 2))
    return fail(ctx, IMQ_EINVAL, "%s: x must be 4-byte and y 2-byte aligned", fn);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e =
      imq::launch_prescale(x, y, count, scale, (int)dtype, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_dynamic_scale(imq_ctx* ctx, const float* x, size_t count, float target, float* scale,
                      imq_stream stream) {
  const char* fn = "imq_dynamic_scale";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!scale || (count > 0 && !x)) return fail(ctx, IMQ_EINVAL, "%s: null device pointer", fn);
  if (!std::isfinite(target) || target <= 0.0f)
    return fail(ctx, IMQ_EINVAL, "%s: target %g must be finite and positive", fn, (double)target);
  if (!aligned(x, 4) || !aligned(scale, 4))
    return fail(ctx, IMQ_EINVAL, "%s: x and scale must be 4-byte aligned", fn);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e =
      imq::launch_dynamic_scale(x, count, target, scale, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_cast_prescale_ex(imq_ctx* ctx, const float* x, void* y, size_t count, float scale,
                         const float* scale_dev, imq_dtype dtype, imq_stream stream) {
  const char* fn = "imq_cast_prescale_ex";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (dtype != IMQ_BF16 && dtype != IMQ_F16)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d (bf16 and f16 are provided)", fn, (int)dtype);
  if (!scale_dev && (!std::isfinite(scale) || scale == 0.0f))
    return fail(ctx, IMQ_EINVAL, "%s: scale %g must be finite and nonzero", fn, (double)scale);
  if (count == 0) return IMQ_OK;
  if (!x || !y) return fail(ctx, IMQ_EINVAL, "%s: null device pointer", fn);
  if (!aligned(x, 4) || !aligned(y, 2) || !aligned(scale_dev, 4))
    return fail(ctx, IMQ_EINVAL, "%s: x and scale_dev must be 4-byte and y 2-byte aligned", fn);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const hipError_t e = imq::launch_prescale(x, y, count, scale, (int)dtype,
                                            static_cast<hipStream_t>(stream), scale_dev);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_qmm_postscale_ex(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                         const void* x, void* y, imq_dtype y_dtype, int k, int n, int m,
                         float scale, const float* scale_dev, int group_size, int bits,
                         imq_dtype dtype, imq_stream stream) {
  const char* fn = "imq_qmm_postscale_ex";
  int rc = check_epilogue(ctx, fn, w, scales, biases, x, y, k, n, m, group_size, bits, dtype);
  if (rc != IMQ_OK) return rc;
  if (y_dtype != IMQ_F32 && y_dtype != IMQ_F16)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: y dtype %d (f32 or f16)", fn, (int)y_dtype);
  if (y_dtype == IMQ_F16 && dtype != IMQ_F16)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: an f16 result needs the f16 qmm (dtype f16)", fn);
  if (!aligned(y, y_dtype == IMQ_F32 ? 4 : 2) || !aligned(scale_dev, 4))
    return fail(ctx, IMQ_EINVAL, "%s: y or scale_dev misaligned", fn);
  const auto st = static_cast<hipStream_t>(stream);
  const hipError_t e =
      y_dtype == IMQ_F32
          ? imq::launch_qgemm_postscale(w, scales, biases, x, static_cast<float*>(y), k, n, m,
                                        scale, (int)dtype, st, imq::SplitWs{}, scale_dev)
          : imq::launch_qgemm_postscale_f16(w, scales, biases, x, y, k, n, m, scale, st,
                                            scale_dev);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_qmm_postscale(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                      const void* x, float* y, int k, int n, int m, float scale, int group_size,
                      int bits, imq_dtype dtype, imq_stream stream) {
  const char* fn = "imq_qmm_postscale";
  int rc = check_epilogue(ctx, fn, w, scales, biases, x, y, k, n, m, group_size, bits, dtype);
  if (rc != IMQ_OK) return rc;
  if (!aligned(y, 4)) return fail(ctx, IMQ_EINVAL, "%s: y must be 4-byte aligned", fn);
  const hipError_t e = imq::launch_qgemm_postscale(w, scales, biases, x, y, k, n, m, scale,
                                                   (int)dtype, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_rmsnorm(imq_ctx* ctx, const void* x, imq_dtype x_dtype, const float* w, void* y,
                imq_dtype y_dtype, int rows, int cols, float eps, imq_stream stream) {
  const char* fn = "imq_rmsnorm";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (y_dtype != IMQ_BF16 && y_dtype != IMQ_F16)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: y dtype %d (bf16 or f16)", fn, (int)y_dtype);
  if (x_dtype != IMQ_F32 && x_dtype != y_dtype)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: x dtype %d (f32, or y's dtype)", fn, (int)x_dtype);
  if (rows < 0 || cols <= 0) return fail(ctx, IMQ_EINVAL, "%s: rows %d, cols %d", fn, rows, cols);
  if (!std::isfinite(eps) || eps < 0.f)
    return fail(ctx, IMQ_EINVAL, "%s: eps %g must be finite and non-negative", fn, (double)eps);
  if (rows == 0) return IMQ_OK;
  if (!x || !w || !y) return fail(ctx, IMQ_EINVAL, "%s: null device pointer", fn);
  if (!aligned(x, elem_size(x_dtype)) || !aligned(w, 4) || !aligned(y, 2))
    return fail(ctx, IMQ_EINVAL, "%s: x, w or y misaligned for its element type", fn);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  const auto st = static_cast<hipStream_t>(stream);
  const hipError_t e =
      x_dtype == IMQ_F32
          ? imq::launch_rmsnorm(static_cast<const float*>(x), w, y, rows, cols, eps, (int)y_dtype, st)
          : imq::launch_rmsnorm_t(x, w, y, rows, cols, eps, (int)y_dtype, st);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_qmm_add(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                const void* x, const void* residual, void* y, int k, int n, int m, int group_size,
                int bits, imq_dtype dtype, imq_stream stream) {
  const char* fn = "imq_qmm_add";
  int rc = check_epilogue(ctx, fn, w, scales, biases, x, y, k, n, m, group_size, bits, dtype);
  if (rc != IMQ_OK) return rc;
  if (!residual) return fail(ctx, IMQ_EINVAL, "%s: null residual", fn);
  if (!aligned(residual, 2)) return fail(ctx, IMQ_EINVAL, "%s: residual must be 2-byte aligned", fn);
  const hipError_t e = imq::launch_qgemm_resid_add(w, scales, biases, x, residual, y, k, n, m,
                                                   (int)dtype, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_qmm_gate_add(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                     const void* x, const float* residual, const float* gate, float* y, int k,
                     int n, int m, float scale, int group_size, int bits, imq_dtype dtype,
                     imq_stream stream) {
  const char* fn = "imq_qmm_gate_add";
  int rc = check_epilogue(ctx, fn, w, scales, biases, x, y, k, n, m, group_size, bits, dtype);
  if (rc != IMQ_OK) return rc;
  if (!residual || !gate) return fail(ctx, IMQ_EINVAL, "%s: null residual or gate", fn);
  if (!aligned(y, 4) || !aligned(residual, 4) || !aligned(gate, 4))
    return fail(ctx, IMQ_EINVAL, "%s: y, residual and gate must be 4-byte aligned", fn);
  const hipError_t e = imq::launch_qgemm_gate_add(w, scales, biases, x, residual, gate, y, k, n,
                                                  m, scale, (int)dtype,
                                                  static_cast<hipStream_t>(stream));
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

int imq_qmm_swiglu(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                   const void* x, void* y, int ldy, int k, int n, int m, int width, int gate_row,
                   int up_row, float in_scale, float out_scale, int group_size, int bits,
                   imq_dtype dtype, imq_stream stream) {
  const char* fn = "imq_qmm_swiglu";
  int rc = check_epilogue(ctx, fn, w, scales, biases, x, y, k, n, m, group_size, bits, dtype);
  if (rc != IMQ_OK) return rc;
  if (width <= 0 || gate_row < 0 || up_row < 0 || (int64_t)gate_row + width > n ||
      (int64_t)up_row + width > n || ldy < width)
    return fail(ctx, IMQ_EINVAL,
                "%s: sections gate [%d, +%d) / up [%d, +%d) must lie in the %d weight rows and "
                "ldy (%d) >= width",
                fn, gate_row, width, up_row, width, n, ldy);
  const auto st = static_cast<hipStream_t>(stream);
  // Few rows: the qGEMV with the gate and up rows of an output in one lane
  // group (one launch streams both weight sections).
  const hipError_t e =
      swiglu_on_qgemv(k, n, m, dtype)
          ? imq::launch_qgemv_swiglu(w, scales, biases, x, y, ldy, k, n, m, width, gate_row,
                                     up_row, in_scale, out_scale, (int)dtype, st)
          : imq::launch_qgemm_swiglu(w, scales, biases, x, y, ldy, k, n, m, width, gate_row,
                                     up_row, in_scale, out_scale, (int)dtype, st);
  return e == hipSuccess ? IMQ_OK : hip_fail(ctx, e, fn);
}

}  // extern "C"
