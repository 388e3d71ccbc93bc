// te.cpp -- the text encoder's quantized-linear layer halves (include/imq_te.h).
//
// Mirrors DirectTEEncoder.encodeLayer (Sources/ImarelloDirect/DirectTEEncoder.swift:364-412)
// over DirectTEForward's layers and static scratch (DirectTEForward.swift:66-138).  The
// glue the reference dispatches after a qmm is folded into the qmm's output
// stage: dq_add into o_proj and down_proj (EpResidAdd), dq_silu_mul into the
// gate/up launch (the SwiGLU stage at in / out scale 1 over the concatenated
// gate and up rows), and q/k/v are one launch over their concatenation.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <new>
#include <vector>

#include "ctx.hpp"
#include "imq.h"
#include "imq_kernels.hpp"
#include "imq_te.h"

using namespace imq::detail;

struct imq_te {
  imq_ctx* ctx = nullptr;
  std::vector<imq_te_layer_weights> layers;
  int hidden = 0, nq = 0, nkv = 0, inter = 0, max_rows = 0;
  float eps = 0.f;
  imq_dtype dtype = IMQ_BF16;
  void* arena = nullptr;
  char* h1 = nullptr;  // T [max_rows, hidden]: RMSNorm output (both halves)
  char* r = nullptr;   // T [max_rows, hidden]: x + o_proj (the reference's resid1)
  char* m = nullptr;   // T [max_rows, inter]: silu(g) * u
  imq::SplitWs split;  // split-K partial sums of every projection of the plan
};

namespace {

bool weight_ok(const imq_qweight& q, imq_dtype dtype) {
  return q.w && q.scales && q.biases && q.n > 0 && q.k > 0 && q.k % 64 == 0 && q.dtype == dtype &&
         aligned(q.w, 16) && aligned(q.scales, 2) && aligned(q.biases, 2) &&
         (size_t)q.n * (size_t)q.k / 2 < ((size_t)1 << 32);
}

// Whether the few-row kernel's K split takes this plain projection (its plan
// exists, from 6 rows, and the plan's workspace holds its partial sums); past
// 16 rows in place of the tile kernel.
bool few_row_split(const imq_te* te, const imq_qweight& q, int rows) {
  const int dt = (int)te->dtype;
  if (rows < imq::kDispatchSkinnyMinM || !imq::qskinny_supported(q.k, q.n, rows, dt)) return false;
  const size_t need = imq::qskinny_split_bytes(q.k, q.n, rows);
  return need > 0 && te->split.p && te->split.bytes >= need;
}

// Rows up to which the o / down projections run the qGEMV with the residual
// add in its store (layer at L = 1 / 2 29.3 / 36.1 us against 38.3 / 41.1 on
// the K split); from 3 rows the split is ahead (the qGEMV's dot products
// grow with the rows: down at L = 4 14.1 us on it).
constexpr int kGemvResidMaxRows = 2;

// The same for the residual-add form of the o / down projections and the
// SwiGLU form of gate/up, whose alternative is the tile kernel's at any row
// count (their plan exists from 1 row).
bool resid_split(const imq_te* te, const imq_qweight& q, int rows) {
  const int dt = (int)te->dtype;
  if (!imq::qskinny_supported(q.k, q.n, rows, dt)) return false;
  const size_t need = imq::qskinny_resid_split_bytes(q.k, q.n, rows);
  return need > 0 && te->split.p && te->split.bytes >= need;
}

// The regime dispatcher's choice for a plain projection (imq_qmm_t's, with
// the plan's workspace).
hipError_t plain_qmm(const imq_te* te, const imq_qweight& q, const void* x, void* y, int rows,
                     hipStream_t st) {
  const int dt = (int)te->dtype;
  if ((rows >= imq::kDispatchSkinnyMinM && rows <= imq::kDispatchSkinnyMaxM &&
       imq::qskinny_supported(q.k, q.n, rows, dt)) ||
      few_row_split(te, q, rows))
    return imq::launch_qskinny(q.w, q.scales, q.biases, x, y, q.k, q.n, rows, dt, st, te->split);
  if (rows <= imq::kDispatchGemvMaxM)
    return imq::launch_qgemv(q.w, q.scales, q.biases, x, y, q.k, q.n, rows, dt, st);
  return imq::launch_qgemm(q.w, q.scales, q.biases, x, y, q.k, q.n, rows, dt, st, te->split);
}

}  // namespace

extern "C" {

int imq_te_create(imq_ctx* ctx, const imq_te_layer_weights* layers, int n_layers, int max_rows,
                  float eps, imq_te** out) {
  const char* fn = "imq_te_create";
  if (!ctx) return fail(nullptr, IMQ_EINVAL, "%s: null context", fn);
  if (!out) return fail(ctx, IMQ_EINVAL, "%s: null output handle", fn);
  *out = nullptr;
  if (!layers || n_layers <= 0 || max_rows <= 0)
    return fail(ctx, IMQ_EINVAL, "%s: %d layers, max_rows %d", fn, n_layers, max_rows);
  if (!std::isfinite(eps) || eps < 0.f)
    return fail(ctx, IMQ_EINVAL, "%s: eps %g must be finite and non-negative", fn, (double)eps);
  const imq_te_layer_weights& l0 = layers[0];
  const imq_dtype dtype = l0.qkv.dtype;
  if (dtype != IMQ_BF16 && dtype != IMQ_F16)
    return fail(ctx, IMQ_EUNSUPPORTED, "%s: dtype %d (bf16 and f16 are provided)", fn, (int)dtype);
  const int hidden = l0.qkv.k, nq = l0.o.k, inter = l0.down.k;
  const int nkv2 = l0.qkv.n - nq;
  if (nkv2 <= 0 || nkv2 % 2 != 0 || l0.o.n != hidden || l0.gate_up.k != hidden ||
      l0.gate_up.n != 2 * inter || l0.down.n != hidden)
    return fail(ctx, IMQ_EINVAL,
                "%s: layer 0 shapes qkv [%d, %d], o [%d, %d], gate_up [%d, %d], down [%d, %d] "
                "do not form a layer",
                fn, l0.qkv.n, l0.qkv.k, l0.o.n, l0.o.k, l0.gate_up.n, l0.gate_up.k, l0.down.n,
                l0.down.k);
  for (int i = 0; i < n_layers; ++i) {
    const imq_te_layer_weights& l = layers[i];
    const imq_qweight* ws[4] = {&l.qkv, &l.o, &l.gate_up, &l.down};
    const imq_qweight* w0[4] = {&l0.qkv, &l0.o, &l0.gate_up, &l0.down};
    for (int j = 0; j < 4; ++j)
      if (!weight_ok(*ws[j], dtype) || ws[j]->n != w0[j]->n || ws[j]->k != w0[j]->k)
        return fail(ctx, IMQ_EINVAL,
                    "%s: layer %d projection %d: missing, misaligned, of another dtype or shape "
                    "than layer 0's",
                    fn, i, j);
    if (!l.norm_in || !l.norm_post || !aligned(l.norm_in, 4) || !aligned(l.norm_post, 4))
      return fail(ctx, IMQ_EINVAL, "%s: layer %d: null or misaligned norm weights", fn, i);
  }
  if ((size_t)max_rows * std::max(hidden, std::max(nq, inter)) * 2 >= ((size_t)1 << 31))
    return fail(ctx, IMQ_EINVAL, "%s: max_rows %d too large for 32-bit activation offsets", fn,
                max_rows);
  int rc = bind_device(ctx);
  if (rc != IMQ_OK) return rc;
  auto* te = new (std::nothrow) imq_te;
  if (!te) return fail(ctx, IMQ_ENOMEM, "%s: out of host memory", fn);
  te->ctx = ctx;
  te->layers.assign(layers, layers + n_layers);
  te->hidden = hidden;
  te->nq = nq;
  te->nkv = nkv2 / 2;
  te->inter = inter;
  te->max_rows = max_rows;
  te->eps = eps;
  te->dtype = dtype;
  // The split-K workspace every projection's plan needs at any row count up
  // to max_rows (plans the workspace cannot hold run unsplit).
  size_t ws = 0;
  for (int rows = 1; rows <= max_rows; ++rows) {
    ws = std::max(ws, imq::qgemm_split_bytes(hidden, l0.qkv.n, rows, false));
    if (rows <= imq::kQskinnyMaxM) {
      ws = std::max(ws, imq::qskinny_split_bytes(hidden, l0.qkv.n, rows));
      ws = std::max(ws, imq::qskinny_resid_split_bytes(nq, hidden, rows));
      ws = std::max(ws, imq::qskinny_resid_split_bytes(inter, hidden, rows));
      ws = std::max(ws, imq::qskinny_resid_split_bytes(hidden, 2 * inter, rows));
    }
    ws = std::max(ws, imq::qgemm_split_bytes(nq, hidden, rows, true));
    ws = std::max(ws, imq::qgemm_split_bytes(hidden, 2 * inter, rows, true));
    ws = std::max(ws, imq::qgemm_split_bytes(inter, hidden, rows, true));
  }
  auto round = [](size_t b) { return (b + 255) & ~(size_t)255; };
  const size_t b_h = round((size_t)max_rows * hidden * 2);
  const size_t b_m = round((size_t)max_rows * inter * 2);
  const hipError_t e = hipMalloc(&te->arena, 2 * b_h + b_m + ws);
  if (e != hipSuccess) {
    delete te;
    return hip_fail(ctx, e, fn);
  }
  char* p = static_cast<char*>(te->arena);
  te->h1 = p;
  te->r = p + b_h;
  te->m = p + 2 * b_h;
  te->split = ws ? imq::SplitWs{reinterpret_cast<float*>(p + 2 * b_h + b_m), ws} : imq::SplitWs{};
  *out = te;
  return IMQ_OK;
}

static int te_check(imq_te* te, const char* fn, int layer, int rows) {
  if (!te) return fail(nullptr, IMQ_EINVAL, "%s: null plan", fn);
  if (layer < 0 || layer >= (int)te->layers.size())
    return fail(te->ctx, IMQ_EINVAL, "%s: layer %d of %zu", fn, layer, te->layers.size());
  if (rows <= 0 || rows > te->max_rows)
    return fail(te->ctx, IMQ_EINVAL, "%s: rows %d outside [1, %d]", fn, rows, te->max_rows);
  return bind_device(te->ctx);
}

int imq_te_attn_in(imq_te* te, int layer, const void* x, void* qkv, int rows, imq_stream stream) {
  const char* fn = "imq_te_attn_in";
  int rc = te_check(te, fn, layer, rows);
  if (rc != IMQ_OK) return rc;
  if (!x || !qkv) return fail(te->ctx, IMQ_EINVAL, "%s: null pointer", fn);
  if (!aligned(x, 2) || !aligned(qkv, 2))
    return fail(te->ctx, IMQ_EINVAL, "%s: x and qkv must be 2-byte aligned", fn);
  const imq_te_layer_weights& l = te->layers[layer];
  const auto st = static_cast<hipStream_t>(stream);
  const int dt = (int)te->dtype;
  hipError_t e;
  if (rows <= imq::kDispatchGemvMaxM &&
      imq::qgemv_norm_fits(l.qkv.k, l.qkv.n, rows, 0, dt, x, l.norm_in)) {
    // 1-2 rows: the qGEMV normalizes x in its staging (one launch, the same
    // bits as RMSNorm then q/k/v).
    e = imq::launch_qgemv_norm(l.qkv.w, l.qkv.scales, l.qkv.biases, x, l.norm_in, te->eps, qkv,
                               l.qkv.k, l.qkv.n, rows, dt, st);
  } else {
    e = imq::launch_rmsnorm_t(x, l.norm_in, te->h1, rows, te->hidden, te->eps, dt, st);
    if (e == hipSuccess) e = plain_qmm(te, l.qkv, te->h1, qkv, rows, st);
  }
  return e == hipSuccess ? IMQ_OK : hip_fail(te->ctx, e, fn);
}

int imq_te_attn_out_mlp(imq_te* te, int layer, const void* x, const void* attn_o, void* y,
                        int rows, imq_stream stream) {
  const char* fn = "imq_te_attn_out_mlp";
  int rc = te_check(te, fn, layer, rows);
  if (rc != IMQ_OK) return rc;
  if (!x || !attn_o || !y) return fail(te->ctx, IMQ_EINVAL, "%s: null pointer", fn);
  if (!aligned(x, 2) || !aligned(attn_o, 16) || !aligned(y, 2))
    return fail(te->ctx, IMQ_EINVAL, "%s: attn_o must be 16-byte, x and y 2-byte aligned", fn);
  const imq_te_layer_weights& l = te->layers[layer];
  const auto st = static_cast<hipStream_t>(stream);
  const int dt = (int)te->dtype;
  const int h = te->hidden, in = te->inter;
  // o_proj and down_proj with dq_add: the few-row kernel's K split where it
  // takes the shape (for o_proj with the RMSNorm after it in its split-sum
  // kernel, one launch fewer), else the tile kernel.
  hipError_t e;
  // 1-2 rows: gate/up's qGEMV normalizes r itself (the RMSNorm below is
  // then not launched).
  const imq_qweight& gu = l.gate_up;
  const bool norm_in_gate_up = rows <= kGemvResidMaxRows && gu.n == 2 * in &&
                               imq::qgemv_swiglu_fits(gu.k, gu.n, rows, dt) &&
                               imq::qgemv_norm_fits(gu.k, gu.n, rows, in, dt, te->r, l.norm_post);
  if (rows <= kGemvResidMaxRows) {
    // 1-2 rows: the qGEMV with the residual add in its store, then RMSNorm.
    e = imq::launch_qgemv_resid_add(l.o.w, l.o.scales, l.o.biases, attn_o, x, te->r, te->nq, h,
                                    rows, dt, st);
    if (e == hipSuccess && !norm_in_gate_up)
      e = imq::launch_rmsnorm_t(te->r, l.norm_post, te->h1, rows, h, te->eps, dt, st);
  } else if (resid_split(te, l.o, rows) &&
      imq::qskinny_resid_add_norm_fits(te->nq, h, rows, dt, x, te->r, l.norm_post, te->h1,
                                       te->split)) {
    e = imq::launch_qskinny_resid_add_norm(l.o.w, l.o.scales, l.o.biases, attn_o, x, te->r,
                                           l.norm_post, te->h1, te->eps, te->nq, h, rows, dt, st,
                                           te->split);
  } else {
    e = resid_split(te, l.o, rows)
            ? imq::launch_qskinny_resid_add(l.o.w, l.o.scales, l.o.biases, attn_o, x, te->r,
                                            te->nq, h, rows, dt, st, te->split)
            : imq::launch_qgemm_resid_add(l.o.w, l.o.scales, l.o.biases, attn_o, x, te->r, te->nq,
                                          h, rows, dt, st, te->split);
    if (e == hipSuccess)
      e = imq::launch_rmsnorm_t(te->r, l.norm_post, te->h1, rows, h, te->eps, dt, st);
  }
  if (e == hipSuccess) {
    const imq_qweight& g = l.gate_up;
    // gate/up with dq_silu_mul: the qGEMV's pair mode at few rows, then the
    // few-row kernel's K split with the SwiGLU stage in its split sum where
    // it plans, else the tile kernel.
    if (rows >= imq::kDispatchSkinnyMinM && imq::qgemv_swiglu_fits(g.k, g.n, rows, dt) &&
        g.n == 2 * in && imq::qskinny_supported(g.k, g.n, rows, dt) &&
        imq::qskinny_split_bytes(g.k, g.n, rows) == 0 && te->split.p &&
        te->split.bytes >= (size_t)rows * g.n * 2) {
      // 3-4 rows: the few-row kernel's T product [rows, 2 inter] into the
      // split workspace (free until down_proj), then the SwiGLU stage.
      e = imq::launch_qskinny(g.w, g.scales, g.biases, te->h1, te->split.p, g.k, g.n, rows, dt, st,
                              imq::SplitWs{});
      if (e == hipSuccess)
        e = imq::launch_swiglu_t(te->split.p, g.n, rows, in, te->m, in, 1.0f, 1.0f, dt, st);
    } else if (norm_in_gate_up)
      e = imq::launch_qgemv_swiglu_norm(g.w, g.scales, g.biases, te->r, l.norm_post, te->eps,
                                        te->m, in, g.k, g.n, rows, in, 0, in, dt, st);
    else if (imq::qgemv_swiglu_fits(g.k, g.n, rows, dt))
      e = imq::launch_qgemv_swiglu(g.w, g.scales, g.biases, te->h1, te->m, in, g.k, g.n, rows, in,
                                   0, in, 1.0f, 1.0f, dt, st);
    else if (g.n == 2 * in && resid_split(te, g, rows))
      e = imq::launch_qskinny_swiglu(g.w, g.scales, g.biases, te->h1, te->m, in, g.k, g.n, rows,
                                     in, 1.0f, 1.0f, dt, st, te->split);
    else
      e = imq::launch_qgemm_swiglu(g.w, g.scales, g.biases, te->h1, te->m, in, g.k, g.n, rows, in,
                                   0, in, 1.0f, 1.0f, dt, st, te->split);
  }
  if (e == hipSuccess)
    e = rows <= kGemvResidMaxRows
            ? imq::launch_qgemv_resid_add(l.down.w, l.down.scales, l.down.biases, te->m, te->r, y,
                                          in, h, rows, dt, st)
        : resid_split(te, l.down, rows)
            ? imq::launch_qskinny_resid_add(l.down.w, l.down.scales, l.down.biases, te->m, te->r, y,
                                            in, h, rows, dt, st, te->split)
            : imq::launch_qgemm_resid_add(l.down.w, l.down.scales, l.down.biases, te->m, te->r, y,
                                          in, h, rows, dt, st, te->split);
  return e == hipSuccess ? IMQ_OK : hip_fail(te->ctx, e, fn);
}

int imq_te_dims(const imq_te* te, int* hidden, int* nq, int* nkv, int* inter) {
  if (!te) return fail(nullptr, IMQ_EINVAL, "imq_te_dims: null plan");
  if (hidden) *hidden = te->hidden;
  if (nq) *nq = te->nq;
  if (nkv) *nkv = te->nkv;
  if (inter) *inter = te->inter;
  return IMQ_OK;
}

int imq_te_destroy(imq_te* te) {
  if (!te) return IMQ_OK;
  (void)hipSetDevice(te->ctx->device);
  (void)hipDeviceSynchronize();
  if (te->arena) (void)hipFree(te->arena);
  delete te;
  return IMQ_OK;
}

}  // extern "C"
