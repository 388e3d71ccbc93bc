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
#include <initializer_list>
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

// The block halves share this launch bookkeeping: every kernel launched
// counts in st->launches, the first failing call's error is kept, and the
// text rows' chain (on st->side) forks from and joins back into stream s.
struct Enc {
  imq_dit_step* st;
  hipStream_t s;
  hipError_t e = hipSuccess;
  void ok(hipError_t r) {
    ++st->launches;
    if (e == hipSuccess) e = r;
  }
  void sync(hipError_t r) {
    if (e == hipSuccess) e = r;
  }
  void fork() {
    sync(hipEventRecord(st->ev_fork, s));
    sync(hipStreamWaitEvent(st->side, st->ev_fork, 0));
  }
  void join() {
    sync(hipEventRecord(st->ev_join, st->side));
    sync(hipStreamWaitEvent(s, st->ev_join, 0));
  }
  // The image and text chains each plan their tiles for their share of the
  // CUs, so that both fit side by side in one tile round: at 4096 + 512 rows
  // and dim 3072, 192 + 24 tiles of 256 rows on 256 CUs instead of the 228
  // tiles of 224 rows the image rows take alone.  The SwiGLU projections keep
  // the whole device (1152 tiles, 4.5 rounds): the text rows fill the last.
  imq::SplitWs wi() const {
    imq::SplitWs w = st->split;
    w.cus = st->cus_img;
    return w;
  }
  imq::SplitWs wt() const {
    imq::SplitWs w = st->split_txt;
    w.cus = st->cus_txt;
    return w;
  }
  static const char* rows(const void* base, int row0, int width) {
    return static_cast<const char*>(base) + (size_t)row0 * width * 2;
  }
  static char* rows(void* base, int row0, int width) {
    return static_cast<char*>(base) + (size_t)row0 * width * 2;
  }
  // The normalized block input: nx when the caller gives one, else the
  // plan's stand-in for the reference's lnMod, RMSNorm(x) into st->nX.
  const void* norm(const float* x, const void* nx) {
    if (nx) return nx;
    const imq_dit_dims& d = st->d;
    ok(imq::launch_rmsnorm(x, st->norm_w, st->nX, d.l_txt + d.l_img, d.dim, kEps, (int)st->dtype,
                           s));
    return st->nX;
  }
};

// Double block b before attention (encodeDouble's projections up to the
// attention, DirectDiTStep.swift:549-563): q, k, v of the text rows (add_q,
// add_k, add_v) and of the image rows (to_q, to_k, to_v) from the normalized
// input.  Image rows (4096 at 1024^2) on s and text rows (512) on the side
// stream at the same time: an image-row projection leaves CUs idle in its
// last tile round and a text-row one never fills the GPU.  The two chains
// touch disjoint rows of every buffer and have their own split-K workspaces.
void double_attn_in(Enc& c, int b, const float* x, const void* nx, void* q, void* k, void* v) {
  imq_dit_step* st = c.st;
  const imq_dit_dims& d = st->d;
  const int dim = d.dim, T = (int)st->dtype;
  const imq_qweight* W = &st->w[(size_t)12 * b];
  const void* n = c.norm(x, nx);
  void* outs[3] = {q, k, v};
  c.fork();
  for (int i = 0; i < 3; ++i)
    c.ok(imq::launch_qgemm(W[i].w, W[i].scales, W[i].biases, Enc::rows(n, d.l_txt, dim),
                           Enc::rows(outs[i], d.l_txt, dim), dim, dim, d.l_img, T, c.s, c.wi()));
  for (int i = 0; i < 3; ++i)
    c.ok(imq::launch_qgemm(W[3 + i].w, W[3 + i].scales, W[3 + i].biases, n, outs[i], dim, dim,
                           d.l_txt, T, st->side, c.wt()));
  c.join();
}

// Double block b after attention (:568-571): the image rows' to_out and the
// text rows' to_add_out on the attention output, each with its gated
// residual add into x.
void double_attn_out(Enc& c, int b, const void* attn, float* x) {
  imq_dit_step* st = c.st;
  const imq_dit_dims& d = st->d;
  const int dim = d.dim, T = (int)st->dtype;
  const imq_qweight* W = &st->w[(size_t)12 * b];
  const float* g = st->gates + (size_t)4 * b * dim;
  float* Xt = x;
  float* Xi = x + (size_t)d.l_txt * dim;
  c.fork();
  c.ok(imq::launch_qgemm_gate_add(W[6].w, W[6].scales, W[6].biases, Enc::rows(attn, d.l_txt, dim),
                                  Xi, g, Xi, dim, dim, d.l_img, 1.0f, T, c.s, c.wi()));
  c.ok(imq::launch_qgemm_gate_add(W[7].w, W[7].scales, W[7].biases, attn, Xt, g + dim, Xt, dim,
                                  dim, d.l_txt, 1.0f, T, st->side, c.wt()));
  c.join();
}

// Double block b's MLPs (:572-587): SwiGLU(nx . linear_in^T) then
// linear_out with the gated residual add, image rows (ff) and text rows
// (ff_context) side by side.
void double_mlp(Enc& c, int b, const void* nx, float* x) {
  imq_dit_step* st = c.st;
  const imq_dit_dims& d = st->d;
  const int dim = d.dim, ffi = d.ff_inner, T = (int)st->dtype;
  const imq_qweight* W = &st->w[(size_t)12 * b];
  const float* g = st->gates + (size_t)4 * b * dim;
  float* Xt = x;
  float* Xi = x + (size_t)d.l_txt * dim;
  const void* n = c.norm(x, nx);
  c.fork();
  c.ok(imq::launch_qgemm_swiglu(W[8].w, W[8].scales, W[8].biases, Enc::rows(n, d.l_txt, dim),
                                Enc::rows(st->SW, d.l_txt, ffi), ffi, dim, 2 * ffi, d.l_img, ffi, 0,
                                ffi, 1.0f, 1.0f, T, c.s, st->split));
  c.ok(imq::launch_qgemm_gate_add(W[9].w, W[9].scales, W[9].biases,
                                  Enc::rows(st->SW, d.l_txt, ffi), Xi, g + 2 * dim, Xi, ffi, dim,
                                  d.l_img, 1.0f, T, c.s, c.wi()));
  c.ok(imq::launch_qgemm_swiglu(W[10].w, W[10].scales, W[10].biases, n, st->SW, ffi, dim, 2 * ffi,
                                d.l_txt, ffi, 0, ffi, 1.0f, 1.0f, T, st->side, st->split_txt));
  c.ok(imq::launch_qgemm_gate_add(W[11].w, W[11].scales, W[11].biases, st->SW, Xt, g + 3 * dim, Xt,
                                  ffi, dim, d.l_txt, 1.0f, T, st->side, c.wt()));
  c.join();
}

// Single block b before attention (encodeSingle up to the attention,
// :593-611): the Q/K/V rows of to_qkv_mlp_proj into qkv and its SwiGLU rows
// into columns [dim, dim + ff_inner) of concat.  Both read the same input and
// write different buffers, so they run side by side (Q/K/V on the side
// stream): each one's part-empty last tile round fills with the other's tiles.
void single_attn_in(Enc& c, int b, const float* x, const void* nx, void* qkv, void* concat) {
  imq_dit_step* st = c.st;
  const imq_dit_dims& d = st->d;
  const int J = d.l_txt + d.l_img, dim = d.dim, ffi = d.ff_inner, T = (int)st->dtype;
  const int cw = dim + ffi;
  const imq_qweight* W = &st->w[(size_t)12 * d.n_double + 2 * b];
  const void* n = c.norm(x, nx);
  c.fork();
  c.ok(imq::launch_qgemm(W[0].w, W[0].scales, W[0].biases, n, qkv, dim, 3 * dim, J, T, st->side,
                         st->split_txt));
  c.ok(imq::launch_qgemm_swiglu(W[0].w, W[0].scales, W[0].biases, n,
                                static_cast<char*>(concat) + (size_t)dim * 2, cw, dim,
                                3 * dim + 2 * ffi, J, ffi, 3 * dim, 3 * dim + ffi, 1.0f, 1.0f, T,
                                c.s, st->split));
  c.join();
}

// Single block b after attention (:616-617): to_out over [attention | MLP]
// with the gated residual add into x.
void single_attn_out(Enc& c, int b, const void* concat, float* x) {
  imq_dit_step* st = c.st;
  const imq_dit_dims& d = st->d;
  const int J = d.l_txt + d.l_img, dim = d.dim, ffi = d.ff_inner, T = (int)st->dtype;
  const imq_qweight* W = &st->w[(size_t)12 * d.n_double + 2 * b];
  const float* g = st->gates + ((size_t)4 * d.n_double + b) * dim;
  c.ok(imq::launch_qgemm_gate_add(W[1].w, W[1].scales, W[1].biases, concat, x, g, x, dim + ffi,
                                  dim, J, 1.0f, T, c.s, st->split));
}

// Launch every kernel of the blocks on stream s over the plan's residual X,
// with the plan's stand-ins around the projections: RMSNorm for lnMod and,
// for attention, the V projection in double blocks and the attention half of
// C as it was created (zeros) in single blocks.
hipError_t encode(imq_dit_step* st, hipStream_t s) {
  Enc c{st, s};
  for (int b = 0; b < st->d.n_double; ++b) {
    double_attn_in(c, b, st->X, nullptr, st->Q, st->K, st->V);
    double_attn_out(c, b, st->V, st->X);
    double_mlp(c, b, nullptr, st->X);
  }
  for (int b = 0; b < st->d.n_single; ++b) {
    single_attn_in(c, b, st->X, nullptr, st->QKV, st->C);
    single_attn_out(c, b, st->C, st->X);
  }
  return c.e;
}

// The head's input half (encodeDenoiseStep, DirectDiTStep.swift:917-941):
// lat16 = T(lat / 16), then the image rows of x = float(T(lat16 .
// x_embedder^T)) * 16 (cast ÷16, qmm, cast ×16).
void head_embed(Enc& c, const float* lat, float* x) {
  imq_dit_step* st = c.st;
  const imq_dit_dims& d = st->d;
  const int T = (int)st->dtype, C = st->lat_ch;
  c.ok(imq::launch_prescale(lat, st->lat16, (size_t)d.l_img * C, 16.0f, T, c.s));
  c.ok(imq::launch_qgemm_postscale(st->x_emb.w, st->x_emb.scales, st->x_emb.biases, st->lat16,
                                   x + (size_t)d.l_txt * d.dim, C, d.dim, d.l_img, 16.0f, T, c.s));
}

// The head's output half (:947-965): proj_out on nh (the caller's norm_out
// output / 16; without one, the stand-in T(RMSNorm(image rows of x) / 16),
// the AdaLN modulation being outside the quantized-linear path) and the
// Euler gate-add lat_out = lat_in + float(T(nh . proj_out^T)) * 16 dt, the
// factor read from st->euler when the kernel runs.
void head_out(Enc& c, const float* x, const void* nh, const float* lat_in, float* lat_out) {
  imq_dit_step* st = c.st;
  const imq_dit_dims& d = st->d;
  const int T = (int)st->dtype, C = st->lat_ch;
  if (!nh) {
    c.ok(imq::launch_rmsnorm(x + (size_t)d.l_txt * d.dim, st->norm_w, st->nH, d.l_img, d.dim, kEps,
                             T, c.s, 1.0f / 16.0f));
    nh = st->nH;
  }
  c.ok(imq::launch_qgemm_gate_add(st->proj_out.w, st->proj_out.scales, st->proj_out.biases, nh,
                                  lat_in, st->ones, lat_out, d.dim, C, d.l_img, 0.0f, T, c.s,
                                  st->split_head, st->euler));
}

// One denoise step (encodeDenoiseStep, :908-971) on stream s, the inputs
// already in the plan's buffers: the head's input half, the blocks, the
// head's output half.
hipError_t encode_denoise(imq_dit_step* st, hipStream_t s) {
  Enc c{st, s};
  head_embed(c, st->lat_in, st->X);
  c.sync(encode(st, s));
  head_out(c, st->X, nullptr, st->lat_in, st->lat_out);
  return c.e;
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

}  // extern "C"

namespace {

// Shared checks of the block-half entry points: a plan, a block of the kind
// in range, every buffer given and 16-byte aligned (nullable ones may be
// null), then the plan's device current.
int check_half(imq_dit_step* st, const char* fn, int block, int count, const char* kind,
               std::initializer_list<const void*> need, std::initializer_list<const void*> opt) {
  if (!st) return fail(nullptr, IMQ_EINVAL, "%s: null step", fn);
  if (block < 0 || block >= count)
    return fail(st->ctx, IMQ_EINVAL, "%s: %s block %d out of range [0, %d)", fn, kind, block,
                count);
  for (const void* p : need)
    if (!p) return fail(st->ctx, IMQ_EINVAL, "%s: null buffer", fn);
  for (const void* p : need)
    if (!aligned(p, 16)) return fail(st->ctx, IMQ_EINVAL, "%s: buffers must be 16-byte aligned", fn);
  for (const void* p : opt)
    if (p && !aligned(p, 16))
      return fail(st->ctx, IMQ_EINVAL, "%s: buffers must be 16-byte aligned", fn);
  return bind_device(st->ctx);
}

int finish(imq_dit_step* st, const Enc& c, const char* fn) {
  return c.e == hipSuccess ? IMQ_OK : hip_fail(st->ctx, c.e, fn);
}

}  // namespace

extern "C" {

int imq_dit_double_attn_in(imq_dit_step* st, int block, const float* x, const void* nx, void* q,
                           void* k, void* v, imq_stream stream) {
  const char* fn = "imq_dit_double_attn_in";
  int rc = check_half(st, fn, block, st ? st->d.n_double : 0, "double", {q, k, v}, {x, nx});
  if (rc != IMQ_OK) return rc;
  if (!x && !nx) return fail(st->ctx, IMQ_EINVAL, "%s: neither x nor nx given", fn);
  Enc c{st, static_cast<hipStream_t>(stream)};
  st->launches = 0;
  double_attn_in(c, block, x, nx, q, k, v);
  return finish(st, c, fn);
}

int imq_dit_double_attn_out(imq_dit_step* st, int block, const void* attn, float* x,
                            imq_stream stream) {
  const char* fn = "imq_dit_double_attn_out";
  int rc = check_half(st, fn, block, st ? st->d.n_double : 0, "double", {attn, x}, {});
  if (rc != IMQ_OK) return rc;
  Enc c{st, static_cast<hipStream_t>(stream)};
  st->launches = 0;
  double_attn_out(c, block, attn, x);
  return finish(st, c, fn);
}

int imq_dit_double_mlp(imq_dit_step* st, int block, const void* nx, float* x, imq_stream stream) {
  const char* fn = "imq_dit_double_mlp";
  int rc = check_half(st, fn, block, st ? st->d.n_double : 0, "double", {x}, {nx});
  if (rc != IMQ_OK) return rc;
  Enc c{st, static_cast<hipStream_t>(stream)};
  st->launches = 0;
  double_mlp(c, block, nx, x);
  return finish(st, c, fn);
}

int imq_dit_single_attn_in(imq_dit_step* st, int block, const float* x, const void* nx, void* qkv,
                           void* concat, imq_stream stream) {
  const char* fn = "imq_dit_single_attn_in";
  int rc = check_half(st, fn, block, st ? st->d.n_single : 0, "single", {qkv, concat}, {x, nx});
  if (rc != IMQ_OK) return rc;
  if (!x && !nx) return fail(st->ctx, IMQ_EINVAL, "%s: neither x nor nx given", fn);
  Enc c{st, static_cast<hipStream_t>(stream)};
  st->launches = 0;
  single_attn_in(c, block, x, nx, qkv, concat);
  return finish(st, c, fn);
}

int imq_dit_single_attn_out(imq_dit_step* st, int block, const void* concat, float* x,
                            imq_stream stream) {
  const char* fn = "imq_dit_single_attn_out";
  int rc = check_half(st, fn, block, st ? st->d.n_single : 0, "single", {concat, x}, {});
  if (rc != IMQ_OK) return rc;
  Enc c{st, static_cast<hipStream_t>(stream)};
  st->launches = 0;
  single_attn_out(c, block, concat, x);
  return finish(st, c, fn);
}

int imq_dit_head_embed(imq_dit_step* st, const float* lat, float* x, imq_stream stream) {
  const char* fn = "imq_dit_head_embed";
  if (!st) return fail(nullptr, IMQ_EINVAL, "%s: null step", fn);
  if (!st->has_head) return fail(st->ctx, IMQ_EINVAL, "%s: no head set (imq_dit_step_set_head)", fn);
  int rc = check_half(st, fn, 0, 1, "head", {lat, x}, {});
  if (rc != IMQ_OK) return rc;
  Enc c{st, static_cast<hipStream_t>(stream)};
  st->launches = 0;
  head_embed(c, lat, x);
  return finish(st, c, fn);
}

int imq_dit_head_out(imq_dit_step* st, const float* x, const void* nh, const float* lat_in,
                     float* lat_out, float dt, imq_stream stream) {
  const char* fn = "imq_dit_head_out";
  if (!st) return fail(nullptr, IMQ_EINVAL, "%s: null step", fn);
  if (!st->has_head) return fail(st->ctx, IMQ_EINVAL, "%s: no head set (imq_dit_step_set_head)", fn);
  int rc = check_half(st, fn, 0, 1, "head", {lat_in, lat_out}, {x, nh});
  if (rc != IMQ_OK) return rc;
  if (!x && !nh) return fail(st->ctx, IMQ_EINVAL, "%s: neither x nor nh given", fn);
  Enc c{st, static_cast<hipStream_t>(stream)};
  st->launches = 0;
  c.sync(imq::launch_fill_f32(st->euler, 16.0f * dt, 1, c.s));
  head_out(c, x, nh, lat_in, lat_out);
  return finish(st, c, fn);
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
