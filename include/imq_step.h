/*
 * imq_step.h -- whole-step replay of the quantized linear layers of a FLUX.2
 * klein DiT step as one HIP graph.
 *
 * Mirrors the reference's DirectDiTStep: a static scratch plan allocated once
 * (DirectDiTStep.allocateScratch, Sources/ImarelloDirect/DirectDiTStep.swift:155-274),
 * the 5 double + 20 single blocks encoded in order (encodeBlocks / encodeDouble /
 * encodeSingle, :545-685) and run per denoise step with one blocking wait
 * (encodeStep, :636-649).  The graph holds every quantized projection of the
 * step at its real shape, with the glue the reference runs right after them
 * folded into the projection's epilogue (SwiGLU, gated residual add), and an
 * RMSNorm of the fp32 residual stream before each block's projections.
 *
 * Not in the graph (outside the quantized-linear path): attention, RoPE, the
 * per-head Q/K norms and the LayerNorm modulation.  imq_dit_step_run and
 * imq_dit_step_denoise run stand-ins for them: RMSNorm with the plan's norm
 * weight for every lnMod; where the reference feeds the attention output
 * into to_out / to_add_out, the V projection of the same rows; in single
 * blocks the attention half of the concat buffer keeps the values it was
 * created with (zeros).  Their output is therefore NOT the model's: they
 * time and check the quantized-linear work of a step at its real shapes.
 * A caller that runs the real model drives the block halves further down
 * (imq_dit_double_attn_in ... imq_dit_head_out) with its own attention core
 * and LayerNorm modulation between them; run and denoise are exactly those
 * halves with the stand-ins (same kernels, same bits).
 *
 * Data flow per double block (img rows = the l_img rows after the l_txt text
 * rows of the joint residual X, fp32 [l_txt + l_img, dim]):
 *   nX = RMSNorm(X)
 *   Q, K, V [rows] = nX[rows] . {to_q, to_k, to_v}^T (img) / {add_q, add_k, add_v}^T (txt)
 *   X[img] += gate[0] * (V[img] . to_out^T);   X[txt] += gate[1] * (V[txt] . to_add_out^T)
 *   nX = RMSNorm(X)
 *   SW[img] = SwiGLU(nX[img] . ff.linear_in^T);  X[img] += gate[2] * (SW[img] . ff.linear_out^T)
 *   SW[txt] = SwiGLU(nX[txt] . ff_context.linear_in^T);  X[txt] += gate[3] * (...linear_out^T)
 * and per single block (all J = l_txt + l_img rows):
 *   nX = RMSNorm(X)
 *   QKV = nX . to_qkv_mlp_proj[0 : 3 dim]^T
 *   C[:, dim : dim + ff_inner] = SwiGLU over to_qkv_mlp_proj rows [3 dim, 3 dim + 2 ff_inner)
 *   X += gate * (C . to_out^T)             (C = [attention | mlp], dim + ff_inner wide)
 * SwiGLU pairs gate row j with up row ff_inner + j of its section.
 */
#ifndef IMQ_STEP_H
#define IMQ_STEP_H

#include "imq.h"
#include "imq_weights.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct imq_dit_dims {
    int l_img;     /* image tokens (4096 at 1024x1024) */
    int l_txt;     /* text tokens (512) */
    int dim;       /* model width (3072) */
    int ff_inner;  /* MLP hidden width (9216) */
    int n_double;  /* double-stream blocks (5) */
    int n_single;  /* single-stream blocks (20) */
} imq_dit_dims;

typedef struct imq_dit_step imq_dit_step; /* opaque */

/* weights: n_double * 12 + n_single * 2 resident projections, per double
 * block in the reference's DoubleWeights order (DirectDiTStep.swift:310-323):
 * to_q, to_k, to_v, add_q, add_k, add_v, to_out, to_add_out, ff.linear_in,
 * ff.linear_out, ff_context.linear_in, ff_context.linear_out; per single block
 * (:328-333): to_qkv_mlp_proj, to_out.  Shapes [N, K] must be the model's
 * (ff.linear_in is [2 ff_inner, dim], to_qkv_mlp_proj [3 dim + 2 ff_inner,
 * dim], single to_out [dim, dim + ff_inner]), K % 256 == 0, and every
 * projection's dtype (its scales' element type) must be dtype, bf16 or f16.
 * The plan allocates its scratch once; the weights must outlive it. */
int imq_dit_step_create(imq_ctx* ctx, const imq_dit_dims* dims, const imq_qweight* weights,
                        int n_weights, imq_dtype dtype, imq_dit_step** out);

/* Per-step conditioning, fp32, each may be NULL to keep the current values
 * (initially all ones): the RMSNorm weight [dim], and the gate vectors
 * [n_double * 4 + n_single][dim] (double: img attention, txt attention, img
 * MLP, txt MLP; single: one).  Asynchronous on stream. */
int imq_dit_step_set_conditioning(imq_dit_step* step, const float* norm_weight,
                                  const float* gates, imq_stream stream);

/* One step: X = [e_in; h_in] (h_in fp32 [l_img, dim], e_in fp32 [l_txt, dim],
 * copied in, never written), the blocks, and x_out (fp32 [l_txt + l_img, dim],
 * text rows first) = the final X.  use_graph != 0 replays the captured graph
 * (captured on the first such call), 0 launches the same kernels one by one.
 * Asynchronous on stream: the double blocks' text-row projections run on a
 * stream of the plan forked from and joined back into `stream` by events, so
 * work queued on `stream` after this call still sees the whole step. */
int imq_dit_step_run(imq_dit_step* step, const float* h_in, const float* e_in, float* x_out,
                     int use_graph, imq_stream stream);

/* The head of encodeDenoiseStep (loadHead, DirectDiTStep.swift:844-884):
 * x_embedder [dim, C] and proj_out [C, dim] over C latent channels (128 for
 * FLUX.2 klein), C a multiple of 64, dtype the plan's.  Allocates the head's
 * buffers (replacing a head set before); the weights must outlive the plan. */
int imq_dit_step_set_head(imq_dit_step* step, const imq_qweight* x_embedder,
                          const imq_qweight* proj_out);

/* One denoise step, encodeDenoiseStep (DirectDiTStep.swift:908-971) with every
 * quantized projection of it:
 *   lat16 = T(lat_in / 16); image rows of X = float(T(lat16 . x_embedder^T)) * 16
 *   X = [e_in; image rows], the blocks as in imq_dit_step_run
 *   nH = T(RMSNorm(X image rows) / 16)   (the stand-in for norm_out's lnMod)
 *   lat_out = lat_in + float(T(nH . proj_out^T)) * (16 dt)   (the Euler gate-add)
 * lat_in, lat_out fp32 [l_img, C], e_in fp32 [l_txt, dim]; inputs copied in,
 * never written.  use_graph != 0 replays a graph of the whole step (captured
 * on the first such call; dt is read when it runs, so one graph serves every
 * step).  Needs imq_dit_step_set_head.  Asynchronous on stream. */
int imq_dit_step_denoise(imq_dit_step* step, const float* lat_in, const float* e_in,
                         float* lat_out, float dt, int use_graph, imq_stream stream);

/* ---- block halves around the caller's attention ---------------------------
 * encodeDouble / encodeSingle (DirectDiTStep.swift:546-618) and the head of
 * encodeDenoiseStep (:908-971) split where the reference runs work that is
 * not quantized-linear (lnMod, per-head RMSNorm, RoPE, attention): a caller
 * runs those itself between the calls below, in this order per step:
 *
 *   imq_dit_head_embed(lat) -> image rows of x
 *   per double block b: [lnMod "img.msa" / "txt.msa" -> nx]
 *                       imq_dit_double_attn_in(b, x, nx) -> q, k, v
 *                       [per-head norms, RoPE, attention -> attn]
 *                       imq_dit_double_attn_out(b, attn, x)
 *                       [lnMod "img.mlp" / "txt.mlp" -> nx]
 *                       imq_dit_double_mlp(b, nx, x)
 *   per single block b: [lnMod "single" -> nx]
 *                       imq_dit_single_attn_in(b, x, nx) -> qkv, concat[:, dim:]
 *                       [per-head norms, RoPE, attention -> concat[:, :dim]]
 *                       imq_dit_single_attn_out(b, concat, x)
 *   [lnMod "out" -> nh = T(norm_out(x image rows) / 16)]
 *   imq_dit_head_out(x, nh, lat_in, dt) -> lat_out
 *
 * Buffers are the caller's, device memory, 16-byte aligned, rows = tokens
 * with the l_txt text rows first (J = l_txt + l_img rows in all):
 *   x       fp32 [J, dim], the residual stream, updated in place;
 *   nx      T [J, dim], the normalized block input; NULL runs the plan's
 *           stand-in, nx = T(RMSNorm(x) * norm weight) (then x is read);
 *   q, k, v T [J, dim] (text rows from add_q / add_k / add_v, image rows
 *           from to_q / to_k / to_v);
 *   attn    T [J, dim], the double block's attention output;
 *   qkv     T [J, 3 dim], the single block's Q | K | V columns;
 *   concat  T [J, dim + ff_inner], the single block's to_out input:
 *           columns [0, dim) the attention output (the caller's, written
 *           between the two single-block calls), [dim, dim + ff_inner) the
 *           SwiGLU of the MLP rows (written by imq_dit_single_attn_in);
 *   lat     fp32 [l_img, C] latents; nh T [l_img, dim] (NULL: the stand-in
 *           T(RMSNorm(x image rows) / 16)).
 * Gates are the plan's (imq_dit_step_set_conditioning).  Calls share the
 * plan's scratch (the MLP's SwiGLU buffer, the stand-in norm output, the
 * split-K workspaces): on one plan, one call at a time, on one stream.
 * Asynchronous on stream; they may be captured into a graph. */
int imq_dit_double_attn_in(imq_dit_step* step, int block, const float* x, const void* nx, void* q,
                           void* k, void* v, imq_stream stream);
int imq_dit_double_attn_out(imq_dit_step* step, int block, const void* attn, float* x,
                            imq_stream stream);
int imq_dit_double_mlp(imq_dit_step* step, int block, const void* nx, float* x, imq_stream stream);
int imq_dit_single_attn_in(imq_dit_step* step, int block, const float* x, const void* nx, void* qkv,
                           void* concat, imq_stream stream);
int imq_dit_single_attn_out(imq_dit_step* step, int block, const void* concat, float* x,
                            imq_stream stream);
/* Need imq_dit_step_set_head. */
int imq_dit_head_embed(imq_dit_step* step, const float* lat, float* x, imq_stream stream);
int imq_dit_head_out(imq_dit_step* step, const float* x, const void* nh, const float* lat_in,
                     float* lat_out, float dt, imq_stream stream);

/* Kernel launches of the last pass encoded (eager run, graph capture, or the
 * last block-half call). */
int imq_dit_step_launches(const imq_dit_step* step);

int imq_dit_step_destroy(imq_dit_step* step);

#ifdef __cplusplus
}
#endif
#endif /* IMQ_STEP_H */
