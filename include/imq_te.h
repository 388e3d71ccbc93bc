/*
 * imq_te.h -- the quantized-linear part of the Qwen3 text encoder's layers.
 *
 * Mirrors DirectTEEncoder.encodeLayer (Sources/ImarelloDirect/DirectTEEncoder.swift:364-412)
 * over the layers DirectTEForward.loadLayers uploads (DirectTEForward.swift:97-138)
 * and its static scratch plan (Scratch, :66-95).  Per layer the reference
 * encodes RMSNorm, q/k/v qmm, the per-head norms, RoPE and masked attention,
 * o_proj qmm, dq_add, RMSNorm, gate and up qmm, dq_silu_mul, down qmm and
 * dq_add: 7 qmm and 5 glue dispatches.  Here a layer is two calls around the
 * attention core (per-head norms, RoPE, attention: not quantized-linear work,
 * left to the caller):
 *
 *   imq_te_attn_in:       h1 = RMSNorm(x); qkv = h1 . [Wq; Wk; Wv]^T      (2 launches)
 *   imq_te_attn_out_mlp:  r = T(x + T(attn_o . Wo^T))                     (fused dq_add)
 *                         h2 = RMSNorm(r)
 *                         m = T(silu(g) * u), [g | u] = h2 . [Wgate; Wup]^T (one launch, fused)
 *                         y = T(r + T(m . Wdown^T))                       (fused dq_add)
 *
 * 5 launches instead of the reference's 12 for the same quantized work; the
 * q/k/v and gate/up weights stream in one launch each.  At few rows a
 * projection may take a K split, whose second (summing) launch carries the
 * fused stage (dq_add, dq_silu_mul) and, for o_proj, the RMSNorm after it.
 * T is the layers'
 * dtype (bf16, the reference's raw TE pack, or f16); x, y, qkv, attn_o are T
 * row-major, rows = tokens.  Calls are asynchronous on the given stream; the
 * plan's scratch makes calls on one plan one at a time.
 */
#ifndef IMQ_TE_H
#define IMQ_TE_H

#include "imq.h"
#include "imq_weights.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct imq_te imq_te; /* opaque */

typedef struct imq_te_layer_weights {
    imq_qweight qkv;         /* q_proj, k_proj, v_proj concatenated along N: [nq + 2 nkv, hidden] */
    imq_qweight o;           /* o_proj [hidden, nq] */
    imq_qweight gate_up;     /* gate_proj, up_proj concatenated along N: [2 inter, hidden] */
    imq_qweight down;        /* down_proj [hidden, inter] */
    const float* norm_in;    /* input_layernorm.weight, fp32 [hidden] (device) */
    const float* norm_post;  /* post_attention_layernorm.weight, fp32 [hidden] (device) */
} imq_te_layer_weights;

/* A plan over n_layers resident layers of equal shapes and dtype (bf16 or f16),
 * for up to max_rows tokens per call; eps is the RMSNorm epsilon (1e-6,
 * DirectTEForward.swift:22).  Allocates the shared scratch (h1, r, h2, m and
 * the split-K workspace) once; the weights must outlive the plan. */
int imq_te_create(imq_ctx* ctx, const imq_te_layer_weights* layers, int n_layers, int max_rows,
                  float eps, imq_te** out);

/* Layer `layer`'s input half: qkv [rows, nq + 2 nkv] (q columns first, then k,
 * then v) from x [rows, hidden]. */
int imq_te_attn_in(imq_te* te, int layer, const void* x, void* qkv, int rows, imq_stream stream);

/* Layer `layer`'s output half: y [rows, hidden] from the layer input x and
 * the attention output attn_o [rows, nq].  y may equal x. */
int imq_te_attn_out_mlp(imq_te* te, int layer, const void* x, const void* attn_o, void* y,
                        int rows, imq_stream stream);

/* Shapes of the plan: hidden, nq, nkv, inter. */
int imq_te_dims(const imq_te* te, int* hidden, int* nq, int* nkv, int* inter);

int imq_te_destroy(imq_te* te);

#ifdef __cplusplus
}
#endif
#endif /* IMQ_TE_H */
