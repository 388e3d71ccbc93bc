// step.cpp -- whole-step replay of a DiT step's quantized linear layers as a
// HIP graph: the C ABI of include/imq_step.h.
//
// Mirrors DirectDiTStep (Sources/ImarelloDirect/DirectDiTStep.swift): scratch
// allocated once in one arena (allocateScratch, :155-274), the blocks encoded
// in the reference's order (encodeBlocks / encodeDouble / encodeSingle,
// :545-685), inputs copied into the internal residual so the step re-runs on
// pristine inputs (:644-654).  Where the reference encodes ~25 command
// encoders per step, the step here is one graph launch.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <vector>

#include "ctx.hpp"
#include "imq.h"
#include "imq_kernels.hpp"
#include "imq_step.h"

using namespace imq::detail;

struct imq_dit_step {
  imq_ctx* ctx = nullptr;
  imq_dit_dims d{};
  imq_dtype dtype = IMQ_BF16;
  std::vector<imq_qweight> w;
  void* arena = nullptr;
  float* X = nullptr;       // fp32 [J, dim] residual, text rows first
  char* nX = nullptr;       // T [J, dim]
  char* Q = nullptr;        // T [J, dim]
  char* K = nullptr;
  char* V = nullptr;
  char* SW = nullptr;       // T [J, ff_inner]
  char* QKV = nullptr;      // T [J, 3 dim]
  char* C = nullptr;        // T [J, dim + ff_inner]
  float* norm_w = nullptr;  // fp32 [dim]
  float* gates = nullptr;   // fp32 [4 n_double + n_single][dim]
  imq::SplitWs split;       // partial sums of the projections that split K
  imq::SplitWs split_txt;   // the same for the double blocks' text rows (side stream)
  // CUs the double blocks' image / text chains plan for where they run side by
  // side (rows in proportion, the text share rounded up).
  int cus_img = 0, cus_txt = 0;
  hipStream_t cap = nullptr;
  // The double blocks' text-row projections run on `side`, beside the image
  // rows on the main stream, forked and joined by these events.
  hipStream_t side = nullptr;
  hipEvent_t ev_fork = nullptr;
  hipEvent_t ev_join = nullptr;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int launches = 0;
  // The head (loadHead, DirectDiTStep.swift:844-884), once set: x_embedder
  // [dim, C] and proj_out [C, dim] over C latent channels, with buffers of
  // their own (a second arena) and the denoise step's own graph.
  bool has_head = false;
  imq_qweight x_emb{}, proj_out{};
  int lat_ch = 0;
  void* head_arena = nullptr;
  float* lat_in = nullptr;    // fp32 [l_img, C], the caller's latents copied in
  float* lat_out = nullptr;   // fp32 [l_img, C]
  char* lat16 = nullptr;      // T [l_img, C]: lat_in / 16
  char* nH = nullptr;         // T [l_img, dim]: the head norm's output / 16
  float* ones = nullptr;      // fp32 [C]: the Euler gate-add's gate
  float* euler = nullptr;     // fp32 [1]: 16 dt of the current step
  imq::SplitWs split_head;    // proj_out's split-K partial sums
  hipGraph_t dgraph = nullptr;
  hipGraphExec_t dexec = nullptr;
};

namespace {

constexpr float kEps = 1e-5f;  // DirectDiTStep.swift:416

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// Launch every kernel of the blocks on stream s (st->launches counts them).
hipError_t encode(imq_dit_step* st, hipStream_t s) {
  const imq_dit_dims& d = st->d;
  const int J = d.l_txt + d.l_img;
  const int dim = d.dim, ffi = d.ff_inner;
  const int T = (int)st->dtype;
  const size_t es = 2;
  hipError_t e = hipSuccess;
  auto ok = [&](hipError_t r) {
    ++st->launches;
    if (e == hipSuccess) e = r;
  };
  auto sync = [&](hipError_t r) {
    if (e == hipSuccess) e = r;
  };
  // The text rows' chain (on st->side) depends on the main stream up to here.
  auto fork = [&]() {
    sync(hipEventRecord(st->ev_fork, s));
    sync(hipStreamWaitEvent(st->side, st->ev_fork, 0));
  };
  auto join = [&]() {
    sync(hipEventRecord(st->ev_join, st->side));
    sync(hipStreamWaitEvent(s, st->ev_join, 0));
  };
  auto rows = [&](char* base, int row0, int width) { return base + (size_t)row0 * width * es; };
  hipStream_t t = st->side;
  // The image and text chains each plan their tiles for their share of the
  // CUs, so that both fit side by side in one tile round: at 4096 + 512 rows
  // and dim 3072, 192 + 24 tiles of 256 rows on 256 CUs instead of the 228
  // tiles of 224 rows the image rows take alone.  The SwiGLU projections keep
  // the whole device (1152 tiles, 4.5 rounds): the text rows fill the last.
  imq::SplitWs wi = st->split, wt = st->split_txt;
  wi.cus = st->cus_img;
  wt.cus = st->cus_txt;
  float* Xt = st->X;
  float* Xi = st->X + (size_t)d.l_txt * dim;
  for (int b = 0; b < d.n_double; ++b) {
    const imq_qweight* W = &st->w[(size_t)12 * b];
    const float* g = st->gates + (size_t)4 * b * dim;
    ok(imq::launch_rmsnorm(st->X, st->norm_w, st->nX, J, dim, kEps, T, s));
    char* nXt = rows(st->nX, 0, dim);
    char* nXi = rows(st->nX, d.l_txt, dim);
    char* outs[3] = {st->Q, st->K, st->V};
    // Image rows (4096 at 1024^2) on s and text rows (512) on t at the same
    // time: an image-row projection leaves CUs idle in its last tile round
    // and a text-row one never fills the GPU.  The two chains touch disjoint
    // rows of every buffer and have their own split-K workspaces.
    fork();
    for (int q = 0; q < 3; ++q)
      ok(imq::launch_qgemm(W[q].w, W[q].scales, W[q].biases, nXi, rows(outs[q], d.l_txt, dim), dim,
                           dim, d.l_img, T, s, wi));
    // to_out / to_add_out on the V rows (the attention output's stand-in).
    ok(imq::launch_qgemm_gate_add(W[6].w, W[6].scales, W[6].biases, rows(st->V, d.l_txt, dim), Xi,
                                  g, Xi, dim, dim, d.l_img, 1.0f, T, s, wi));
    for (int q = 0; q < 3; ++q)
      ok(imq::launch_qgemm(W[3 + q].w, W[3 + q].scales, W[3 + q].biases, nXt, rows(outs[q], 0, dim),
                           dim, dim, d.l_txt, T, t, wt));
    ok(imq::launch_qgemm_gate_add(W[7].w, W[7].scales, W[7].biases, rows(st->V, 0, dim), Xt,
                                  g + dim, Xt, dim, dim, d.l_txt, 1.0f, T, t, wt));
    join();
    ok(imq::launch_rmsnorm(st->X, st->norm_w, st->nX, J, dim, kEps, T, s));
    fork();
    ok(imq::launch_qgemm_swiglu(W[8].w, W[8].scales, W[8].biases, nXi, rows(st->SW, d.l_txt, ffi),
                                ffi, dim, 2 * ffi, d.l_img, ffi, 0, ffi, 1.0f, 1.0f, T, s,
                                st->split));
    ok(imq::launch_qgemm_gate_add(W[9].w, W[9].scales, W[9].biases, rows(st->SW, d.l_txt, ffi), Xi,
                                  g + 2 * dim, Xi, ffi, dim, d.l_img, 1.0f, T, s, wi));
    ok(imq::launch_qgemm_swiglu(W[10].w, W[10].scales, W[10].biases, nXt, rows(st->SW, 0, ffi), ffi,
                                dim, 2 * ffi, d.l_txt, ffi, 0, ffi, 1.0f, 1.0f, T, t,
                                st->split_txt));
    ok(imq::launch_qgemm_gate_add(W[11].w, W[11].scales, W[11].biases, rows(st->SW, 0, ffi), Xt,
                                  g + 3 * dim, Xt, ffi, dim, d.l_txt, 1.0f, T, t, wt));
    join();
  }
  const int cw = dim + ffi;
  for (int b = 0; b < d.n_single; ++b) {
    const imq_qweight* W = &st->w[(size_t)12 * d.n_double + 2 * b];
    const float* g = st->gates + ((size_t)4 * d.n_double + b) * dim;
    ok(imq::launch_rmsnorm(st->X, st->norm_w, st->nX, J, dim, kEps, T, s));
    // The Q/K/V rows (side stream) and the SwiGLU rows (main stream) of
    // to_qkv_mlp_proj read the same input and write different buffers: run
    // side by side, each one's part-empty last tile round fills with the
    // other's tiles.
    fork();
    ok(imq::launch_qgemm(W[0].w, W[0].scales, W[0].biases, st->nX, st->QKV, dim, 3 * dim, J, T, t,
                         st->split_txt));
    ok(imq::launch_qgemm_swiglu(W[0].w, W[0].scales, W[0].biases, st->nX, st->C + (size_t)dim * es,
                                cw, dim, 3 * dim + 2 * ffi, J, ffi, 3 * dim, 3 * dim + ffi, 1.0f,
                                1.0f, T, s, st->split));
    join();
    ok(imq::launch_qgemm_gate_add(W[1].w, W[1].scales, W[1].biases, st->C, st->X, g, st->X, cw, dim,
                                  J, 1.0f, T, s, st->split));
  }
  return e;
}

// One denoise step (encodeDenoiseStep, DirectDiTStep.swift:908-971) on stream
// s, the inputs already in the plan's buffers: lat16 = T(lat_in / 16), the
// image rows of X = float(T(lat16 . x_embedder^T)) * 16 (cast ÷16, qmm,
// cast ×16: :917-941), the blocks, then the head: nH = T(RMSNorm(image rows) /
// 16) (the stand-in for lnMod "out", whose AdaLN modulation is outside the
// quantized-linear path), and lat_out = lat_in + float(T(nH . proj_out^T)) *
// 16 dt (proj_out and the Euler gate-add with gate ones, :947-965), the scale
// read from st->euler when the kernel runs.
hipError_t encode_denoise(imq_dit_step* st, hipStream_t s) {
  const imq_dit_dims& d = st->d;
  const int T = (int)st->dtype;
  const int C = st->lat_ch;
  float* Xi = st->X + (size_t)d.l_txt * d.dim;
  hipError_t e = hipSuccess;
  auto ok = [&](hipError_t r) {
    ++st->launches;
    if (e == hipSuccess) e = r;
  };
  ok(imq::launch_prescale(st->lat_in, st->lat16, (size_t)d.l_img * C, 16.0f, T, s));
  ok(imq::launch_qgemm_postscale(st->x_emb.w, st->x_emb.scales, st->x_emb.biases, st->lat16, Xi,
                                 C, d.dim, d.l_img, 16.0f, T, s));
  const hipError_t eb = encode(st, s);
  if (e == hipSuccess) e = eb;
  ok(imq::launch_rmsnorm(Xi, st->norm_w, st->nH, d.l_img, d.dim, kEps, T, s, 1.0f / 16.0f));
  ok(imq::launch_qgemm_gate_add(st->proj_out.w, st->proj_out.scales, st->proj_out.biases, st->nH,
                                st->lat_in, st->ones, st->lat_out, d.dim, C, d.l_img, 0.0f, T, s,
                                st->split_head, st->euler));
  return e;
}

void release_head(imq_dit_step* st) {
  if (st->dexec) (void)hipGraphExecDestroy(st->dexec);
  if (st->dgraph) (void)hipGraphDestroy(st->dgraph);
  if (st->head_arena) (void)hipFree(st->head_arena);
  st->dexec = nullptr;
  st->dgraph = nullptr;
  st->head_arena = nullptr;
  st->has_head = false;
}

void release(imq_dit_step* st) {
  release_head(st);
  if (st->exec) (void)hipGraphExecDestroy(st->exec);
  if (st->graph) (void)hipGraphDestroy(st->graph);
  if (st->cap) (void)hipStreamDestroy(st->cap);
  if (st->side) (void)hipStreamDestroy(st->side);
  if (st->ev_fork) (void)hipEventDestroy(st->ev_fork);
  if (st->ev_join) (void)hipEventDestroy(st->ev_join);
  if (st->arena) (void)hipFree(st->arena);
}

// Split-K workspace of the plan: the largest any of its projections takes
// (fused ones over their weight rows, 2 * ff_inner for a SwiGLU pair).
size_t split_bytes(const imq_dit_dims& d) {
  const int J = d.l_txt + d.l_img, ffi = d.ff_inner, cw = d.dim + d.ff_inner;
  size_t b = 0;
  for (int m : {d.l_img, d.l_txt}) {
    b = std::max({b, imq::qgemm_split_bytes(d.dim, d.dim, m),
                  imq::qgemm_split_bytes(d.dim, d.dim, m, true),
                  imq::qgemm_split_bytes(d.dim, 2 * ffi, m, true),
                  imq::qgemm_split_bytes(ffi, d.dim, m, true)});
  }
  return std::max({b, imq::qgemm_split_bytes(d.dim, 3 * d.dim, J),
                   imq::qgemm_split_bytes(d.dim, 2 * ffi, J, true),
                   imq::qgemm_split_bytes(cw, d.dim, J, true)});
}

// Expected [N, K] of projection i of the plan.
void expected_shape(const imq_dit_dims& d, int i, int& n, int& k) {
  const int dim = d.dim, ffi = d.ff_inner;
  if (i < 12 * d.n_double) {
    switch (i % 12) {
      case 8: case 10: n = 2 * ffi; k = dim; return;
      case 9: case 11: n = dim; k = ffi; return;
      default: n = dim; k = dim; return;
    }
  }
  const int j = (i - 12 * d.n_double) % 2;
  if (j == 0) {
    n = 3 * dim + 2 * ffi;
    k = dim;
  } else {
    n = dim;
    k = dim + ffi;
  }
}

// First graph run of an encoder: one eager pass on the plan's own stream does
// the launches' first-use set-up (device queries) outside the capture, then
// the pass is captured there once.  The eager pass only writes scratch that
// every run rewrites.
hipError_t capture(imq_dit_step* st, hipError_t (*enc)(imq_dit_step*, hipStream_t),
                   hipGraph_t* graph, hipGraphExec_t* exec) {
  hipError_t e = hipDeviceSynchronize();
  st->launches = 0;
  if (e == hipSuccess) e = enc(st, st->cap);
  if (e == hipSuccess) e = hipStreamSynchronize(st->cap);
  if (e == hipSuccess) e = hipStreamBeginCapture(st->cap, hipStreamCaptureModeRelaxed);
  if (e == hipSuccess) {
    st->launches = 0;
    const hipError_t r = enc(st, st->cap);
    e = hipStreamEndCapture(st->cap, graph);
    if (e == hipSuccess) e = r;
  }
  if (e == hipSuccess) e = hipGraphInstantiate(exec, *graph, nullptr, nullptr, 0);
  return e;
}

}  // namespace

extern "C" {

int imq_dit_step_create(imq_ctx* ctx, const imq_dit_dims* dims, const imq_qweight* weights,
                        int n_weights, imq_dtype dtype, imq_dit_step** out) {
  const char* fn = "imq_dit_step_create";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!dims || !out || (n_weights > 0 && !weights)) return fail(ctx, IMQ_EINVAL, "%s: null argument", fn);
  *out = nullptr;
  const imq_dit_dims d = *dims;
  if (d.l_img <= 0 || d.l_txt <= 0 || d.dim <= 0 || d.ff_inner <= 0 || d.n_double < 0 ||
      d.n_single < 0)
    return fail(ctx, IMQ_EINVAL, "%s: non-positive dimension", fn);
  if (d.dim % 256 != 0 || d.ff_inner % 256 != 0)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dim and ff_inner must be multiples of 256", fn);
  if (dtype != IMQ_BF16 && dtype != IMQ_F16)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d (bf16 and f16 are provided)", fn, (int)dtype);
  const int need = 12 * d.n_double + 2 * d.n_single;
  if (n_weights != need)
    return fail(ctx, IMQ_EINVAL, "%s: %d projections given, the plan needs %d", fn, n_weights, need);
  for (int i = 0; i < n_weights; ++i) {
    int n = 0, k = 0;
    expected_shape(d, i, n, k);
    const imq_qweight& q = weights[i];
    if (!q.w || !q.scales || !q.biases || q.n != n || q.k != k || q.dtype != dtype)
      return fail(ctx, IMQ_EINVAL, "%s: projection %d is [%d, %d] dtype %d, expected [%d, %d] dtype %d",
                  fn, i, q.n, q.k, (int)q.dtype, n, k, (int)dtype);
  }
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  auto* st = new (std::nothrow) imq_dit_step;
  if (!st) return fail(ctx, IMQ_ENOMEM, "%s: out of host memory", fn);
  st->ctx = ctx;
  st->d = d;
  st->dtype = dtype;
  st->w.assign(weights, weights + n_weights);
  const size_t J = (size_t)d.l_txt + d.l_img;
  const size_t es = 2;
  const size_t sizes[] = {J * d.dim * 4,
                          J * d.dim * es,
                          J * d.dim * es,
                          J * d.dim * es,
                          J * d.dim * es,
                          J * d.ff_inner * es,
                          J * 3 * d.dim * es,
                          J * (d.dim + d.ff_inner) * es,
                          (size_t)d.dim * 4,
                          ((size_t)4 * d.n_double + d.n_single) * d.dim * 4,
                          split_bytes(d),
                          split_bytes(d)};
  size_t off[12], total = 0;
  for (int i = 0; i < 12; ++i) {
    off[i] = total;
    total += align256(sizes[i]);
  }
  hipError_t e = hipMalloc(&st->arena, total);
  if (e != hipSuccess) {
    st->arena = nullptr;
    release(st);
    delete st;
    return e == hipErrorOutOfMemory
               ? fail(ctx, IMQ_ENOMEM, "%s: %zu bytes of scratch: out of device memory", fn, total)
               : hip_fail(ctx, e, fn);
  }
  char* a = static_cast<char*>(st->arena);
  st->X = reinterpret_cast<float*>(a + off[0]);
  st->nX = a + off[1];
  st->Q = a + off[2];
  st->K = a + off[3];
  st->V = a + off[4];
  st->SW = a + off[5];
  st->QKV = a + off[6];
  st->C = a + off[7];
  st->norm_w = reinterpret_cast<float*>(a + off[8]);
  st->gates = reinterpret_cast<float*>(a + off[9]);
  st->split = imq::SplitWs{reinterpret_cast<float*>(a + off[10]), sizes[10]};
  st->split_txt = imq::SplitWs{reinterpret_cast<float*>(a + off[11]), sizes[11]};
  {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    st->cus_txt = std::max(1, (int)(((size_t)cus * d.l_txt + J - 1) / J));
    st->cus_img = std::max(1, cus - st->cus_txt);
  }
  // Zero everything (the attention half of C stays zero), ones for the
  // conditioning vectors.  Plain (uncaptured) memsets at set-up.
  e = hipMemset(st->arena, 0, total);
  if (e == hipSuccess) e = hipMemsetD32(st->norm_w, 0x3F800000u, (size_t)d.dim);
  if (e == hipSuccess)
    e = hipMemsetD32(st->gates, 0x3F800000u, ((size_t)4 * d.n_double + d.n_single) * d.dim);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&st->cap, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&st->side, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&st->ev_fork, hipEventDisableTiming);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&st->ev_join, hipEventDisableTiming);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    release(st);
    delete st;
    return hip_fail(ctx, e, fn);
  }
  *out = st;
  return IMQ_OK;
}

int imq_dit_step_set_conditioning(imq_dit_step* st, const float* norm_weight, const float* gates,
                                  imq_stream stream) {
  if (!st) return fail(nullptr, IMQ_EINVAL, "imq_dit_step_set_conditioning: null step");
  int rc = bind_device(st->ctx);
  if (rc != IMQ_OK) return rc;
  auto s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (norm_weight)
    e = hipMemcpyAsync(st->norm_w, norm_weight, (size_t)st->d.dim * 4, hipMemcpyDefault, s);
  if (e == hipSuccess && gates)
    e = hipMemcpyAsync(st->gates, gates,
                       ((size_t)4 * st->d.n_double + st->d.n_single) * st->d.dim * 4,
                       hipMemcpyDefault, s);
  return e == hipSuccess ? IMQ_OK : hip_fail(st->ctx, e, "imq_dit_step_set_conditioning");
}

int imq_dit_step_run(imq_dit_step* st, const float* h_in, const float* e_in, float* x_out,
                     int use_graph, imq_stream stream) {
  const char* fn = "imq_dit_step_run";
  if (!st) return fail(nullptr, IMQ_EINVAL, "%s: null step", fn);
  if (!h_in || !e_in || !x_out) return fail(st->ctx, IMQ_EINVAL, "%s: null buffer", fn);
  int rc = bind_device(st->ctx);
  if (rc != IMQ_OK) return rc;
  const imq_dit_dims& d = st->d;
  auto s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (use_graph && !st->exec) {
    // First graph run: one eager step on the plan's own stream does the
    // launches' first-use set-up (device queries) outside the capture, then
    // the step is captured there once.  The eager step only writes scratch
    // that every run rewrites, and runs before the inputs are copied in.
    e = capture(st, encode, &st->graph, &st->exec);
    if (e != hipSuccess) return hip_fail(st->ctx, e, "imq_dit_step_run: graph capture");
  }
  const size_t row = (size_t)d.dim * 4;
  e = hipMemcpyAsync(st->X, e_in, (size_t)d.l_txt * row, hipMemcpyDefault, s);
  if (e == hipSuccess)
    e = hipMemcpyAsync(st->X + (size_t)d.l_txt * d.dim, h_in, (size_t)d.l_img * row,
                       hipMemcpyDefault, s);
  if (e == hipSuccess) {
    if (use_graph) {
      e = hipGraphLaunch(st->exec, s);
    } else {
      st->launches = 0;
      e = encode(st, s);
    }
  }
  if (e == hipSuccess)
    e = hipMemcpyAsync(x_out, st->X, (size_t)(d.l_txt + d.l_img) * row, hipMemcpyDefault, s);
  return e == hipSuccess ? IMQ_OK : hip_fail(st->ctx, e, fn);
}

int imq_dit_step_set_head(imq_dit_step* st, const imq_qweight* x_embedder,
                          const imq_qweight* proj_out) {
  const char* fn = "imq_dit_step_set_head";
  if (!st) return fail(nullptr, IMQ_EINVAL, "%s: null step", fn);
  if (!x_embedder || !proj_out) return fail(st->ctx, IMQ_EINVAL, "%s: null projection", fn);
  const imq_dit_dims& d = st->d;
  const imq_qweight& xe = *x_embedder;
  const imq_qweight& po = *proj_out;
  const int C = xe.k;
  if (!xe.w || !xe.scales || !xe.biases || !po.w || !po.scales || !po.biases)
    return fail(st->ctx, IMQ_EINVAL, "%s: null tensor in a projection", fn);
  if (xe.n != d.dim || C <= 0 || C % 64 != 0 || po.k != d.dim || po.n != C)
    return fail(st->ctx, IMQ_EINVAL,
                "%s: x_embedder is [%d, %d] and proj_out [%d, %d]; expected [%d, C] and [C, %d] "
                "with C a positive multiple of 64",
                fn, xe.n, xe.k, po.n, po.k, d.dim, d.dim);
  if (xe.dtype != st->dtype || po.dtype != st->dtype)
    return fail(st->ctx, IMQ_EINVAL, "%s: projection dtypes %d / %d, the plan's is %d", fn,
                (int)xe.dtype, (int)po.dtype, (int)st->dtype);
  int rc = bind_device(st->ctx);
  if (rc != IMQ_OK) return rc;
  hipError_t e = hipDeviceSynchronize();  // a previous head's graph may still run
  if (e != hipSuccess) return hip_fail(st->ctx, e, fn);
  release_head(st);
  const size_t li = (size_t)d.l_img;
  const size_t ws = imq::qgemm_split_bytes(d.dim, C, d.l_img, true);
  const size_t sizes[] = {li * C * 4, li * C * 4, li * C * 2, li * d.dim * 2, (size_t)C * 4, 4, ws};
  size_t off[7], total = 0;
  for (int i = 0; i < 7; ++i) {
    off[i] = total;
    total += align256(sizes[i]);
  }
  e = hipMalloc(&st->head_arena, total);
  if (e != hipSuccess) {
    st->head_arena = nullptr;
    return e == hipErrorOutOfMemory
               ? fail(st->ctx, IMQ_ENOMEM, "%s: %zu bytes: out of device memory", fn, total)
               : hip_fail(st->ctx, e, fn);
  }
  char* a = static_cast<char*>(st->head_arena);
  st->lat_in = reinterpret_cast<float*>(a + off[0]);
  st->lat_out = reinterpret_cast<float*>(a + off[1]);
  st->lat16 = a + off[2];
  st->nH = a + off[3];
  st->ones = reinterpret_cast<float*>(a + off[4]);
  st->euler = reinterpret_cast<float*>(a + off[5]);
  st->split_head = imq::SplitWs{ws ? reinterpret_cast<float*>(a + off[6]) : nullptr, ws};
  e = hipMemset(st->head_arena, 0, total);
  if (e == hipSuccess) e = hipMemsetD32(st->ones, 0x3F800000u, (size_t)C);
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    release_head(st);
    return hip_fail(st->ctx, e, fn);
  }
  st->x_emb = xe;
  st->proj_out = po;
  st->lat_ch = C;
  st->has_head = true;
  return IMQ_OK;
}

int imq_dit_step_denoise(imq_dit_step* st, const float* lat_in, const float* e_in, float* lat_out,
                         float dt, int use_graph, imq_stream stream) {
  const char* fn = "imq_dit_step_denoise";
  if (!st) return fail(nullptr, IMQ_EINVAL, "%s: null step", fn);
  if (!st->has_head) return fail(st->ctx, IMQ_EINVAL, "%s: no head set (imq_dit_step_set_head)", fn);
  if (!lat_in || !e_in || !lat_out) return fail(st->ctx, IMQ_EINVAL, "%s: null buffer", fn);
  int rc = bind_device(st->ctx);
  if (rc != IMQ_OK) return rc;
  const imq_dit_dims& d = st->d;
  auto s = static_cast<hipStream_t>(stream);
  hipError_t e = hipSuccess;
  if (use_graph && !st->dexec) {
    e = capture(st, encode_denoise, &st->dgraph, &st->dexec);
    if (e != hipSuccess) return hip_fail(st->ctx, e, "imq_dit_step_denoise: graph capture");
  }
  const size_t lat_bytes = (size_t)d.l_img * st->lat_ch * 4;
  e = hipMemcpyAsync(st->lat_in, lat_in, lat_bytes, hipMemcpyDefault, s);
  if (e == hipSuccess)
    e = hipMemcpyAsync(st->X, e_in, (size_t)d.l_txt * d.dim * 4, hipMemcpyDefault, s);
  if (e == hipSuccess) e = imq::launch_fill_f32(st->euler, 16.0f * dt, 1, s);
  if (e == hipSuccess) {
    if (use_graph) {
      e = hipGraphLaunch(st->dexec, s);
    } else {
      st->launches = 0;
      e = encode_denoise(st, s);
    }
  }
  if (e == hipSuccess) e = hipMemcpyAsync(lat_out, st->lat_out, lat_bytes, hipMemcpyDefault, s);
  return e == hipSuccess ? IMQ_OK : hip_fail(st->ctx, e, fn);
}

int imq_dit_step_launches(const imq_dit_step* st) { return st ? st->launches : 0; }

int imq_dit_step_destroy(imq_dit_step* st) {
  if (!st) return IMQ_OK;
  (void)hipSetDevice(st->ctx->device);
  (void)hipDeviceSynchronize();
  release(st);
  delete st;
  return IMQ_OK;
}

}  // extern "C"
