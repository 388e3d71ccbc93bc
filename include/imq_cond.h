/*
 * imq_cond.h -- the per-step conditioning chain of the DiT: timestep
 * embedding and modulation heads on the f32 quantized matmul.
 *
 * Mirrors DirectConditioner (Sources/ImarelloDirect/DirectConditioner.swift):
 * the f32-parameter projections it loads (:75-95) and stepConditioning
 * (:168-213), which per timestep runs
 *   sin  = [cos(t f_i) | sin(t f_i)],  f_i = expf(-logf(10000) * i / half)   (:152-166)
 *   t1   = sin . time_guidance_embed.linear_1^T          (K = 256)
 *   temb = silu(t1) . time_guidance_embed.linear_2^T     (K = dim)
 *   mImg, mTxt, mSingle, outC = silu(temb) . {modulation heads}^T
 * with silu(v) = v / (1 + exp(-v)) (dd_silu_f32, DirectDiTKernels.swift:176-184),
 * six dependent M = 1 dispatches and a blocking wait each.  Here all
 * timesteps of a call are rows of one pass (every op is row-local), the four
 * heads share one launch over their concatenation along N, and nothing
 * blocks: three matmuls and two SiLU launches per 16 timesteps.
 */
#ifndef IMQ_COND_H
#define IMQ_COND_H

#include "imq.h"
#include "imq_weights.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct imq_cond imq_cond; /* opaque */

/* time_l1 [dim, sin_dim] (time_guidance_embed.linear_1), time_l2 [dim, dim]
 * (linear_2) and heads [n_heads, dim]: the modulation heads concatenated
 * along N, for FLUX.2 klein double_stream_modulation_img (6 dim rows),
 * double_stream_modulation_txt (6 dim), single_stream_modulation (3 dim) and
 * norm_out.linear (2 dim) -- imq_load_qlinear_cat with IMQ_F32 loads them so
 * (the reference's scalesF32 upload, DirectConditioner.swift:79-84).  Every
 * projection must carry f32 scales and biases; sin_dim even, K % 64 == 0.
 * The weights must outlive the chain. */
int imq_cond_create(imq_ctx* ctx, const imq_qweight* time_l1, const imq_qweight* time_l2,
                    const imq_qweight* heads, imq_cond** out);

/* stepConditioning(timesteps:) for count >= 1 timesteps (host array, read
 * before the call returns): temb (device fp32 [count][dim], the pre-SiLU
 * time embedding the reference returns) and heads (device fp32
 * [count][n_heads], the heads' outputs in their concatenation order).
 * Asynchronous on stream; the chain's own buffers make calls on one chain
 * one at a time (as the reference's class), and not under stream capture
 * (the sinusoid is computed on the host per call). */
int imq_cond_step_conditioning(imq_cond* cond, const float* timesteps, int count, float* temb,
                               float* heads, imq_stream stream);

/* The host sinusoid of the chain (DirectConditioner.sinusoid,
 * DirectConditioner.swift:152-166): out [count][sin_dim], [cos | sin] halves,
 * float arithmetic in the reference's order with the C library's expf,
 * logf, cosf and sinf. */
int imq_cond_sinusoid(const float* timesteps, int count, int sin_dim, float* out);

int imq_cond_destroy(imq_cond* cond);

#ifdef __cplusplus
}
#endif
#endif /* IMQ_COND_H */
