/*
 * imq.h -- C ABI of the MI355X (gfx950) affine 4-bit quantized linear library.
 *
 * Drop-in boundary for the quantized-linear hot path of the reference's
 * direct-dispatch engine (Sources/ImarelloDirect).  The reference binds MLX's
 * compiled Metal kernel `affine_qmm_t_{T}_gs_64_b_4_alN_true_batch_0` with
 * buffers w, scales, biases, x, y at indices 0-4 and int32 K, N, M at 5-7
 * (Sources/ImarelloDirect/DirectQmmSpike.swift:113-128,
 *  Sources/ImarelloDirect/DirectDiTStep.swift:393-405,
 *  Sources/ImarelloDirect/DirectTELayer.swift:109-128,
 *  Sources/ImarelloDirect/DirectConditioner.swift:96-117).
 * The kernel entry points below keep that argument order and meaning.
 *
 * Data format (MLX affine quantization, bits = 4, group_size = 64):
 *   w       uint32 [N, K/8]  eight 4-bit codes per word, low nibble first
 *   scales  T      [N, K/64]
 *   biases  T      [N, K/64]
 *   deq(W)[n][k] = RNE_T( fl32( fl32(scales[n][k/64] * q[n][k]) + biases[n][k/64] ) )
 *                  (for bf16 and f16 scales the product is exact)
 *   y[M, N]      = x[M, K] . deq(W)^T, accumulated in fp32, rounded to T.
 * All tensors are row-major and contiguous; sub-tensors (row halves, the
 * reference's setBuffer byte offsets, DirectDiTStep.swift:576-579) are passed
 * as offset device pointers.  w, x and the dequantize output must be 16-byte
 * aligned (any whole number of rows of a K % 64 == 0 matrix keeps that);
 * scales, biases and y must be aligned to sizeof(T).
 *
 * Conventions:
 *   - Every call returns an imq_status (0 = IMQ_OK).  No C++ exception crosses
 *     the ABI.  The text of the last failure on a context is imq_last_error().
 *   - Kernel calls are asynchronous on the given stream (NULL = the device's
 *     null stream).  imq_stream_sync is the blocking wait, the counterpart of
 *     waitUntilCompleted (DirectDiTStep.swift:968-970).
 *   - Caller inputs are never written.  The kernel entry points allocate
 *     nothing, except that imq_qmm_t grows the context's split-K workspace of
 *     a stream (hipMalloc) the first time a call on that stream needs it.
 *   - A context belongs to one device.  Calls on one context from several
 *     threads are safe; the last-error text is per context (with several
 *     threads, that of whichever call failed last).
 */
#ifndef IMQ_H
#define IMQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IMQ_ABI_VERSION 2

typedef enum imq_status {
    IMQ_OK = 0,
    IMQ_EINVAL = 1,       /* null/misaligned pointer, bad shape (K % 64 != 0, M/N/K <= 0) */
    IMQ_EUNSUPPORTED = 2, /* well-formed but not provided: bits != 4, group_size != 64, dtype */
    IMQ_EHIP = 3,         /* HIP runtime failure; hipGetErrorString text in imq_last_error */
    IMQ_ENOMEM = 4        /* device or host allocation failed */
} imq_status;

/* Element type T of x, scales, biases and y ("s and b share T",
 * DirectQmmSpike.swift:84, DirectConditioner.swift:48-49).  All three are
 * provided by imq_dequantize, imq_qmm_t and imq_qgemv; imq_qgemm (MFMA) takes
 * bf16 and f16, and imq_qmm_t runs f32 at any M on the qGEMV kernel. */
typedef enum imq_dtype {
    IMQ_BF16 = 0, /* the text encoder / context-embedder kernels (DirectTEEncoder.swift:69-72) */
    IMQ_F16 = 1,  /* the DiT kernels (DirectDiTStep.swift:82-85) */
    IMQ_F32 = 2   /* the M=1 conditioner kernels (DirectConditioner.swift:48) */
} imq_dtype;

typedef struct imq_ctx imq_ctx; /* opaque; owns the device binding and error text */
typedef void* imq_stream;       /* a hipStream_t; NULL = null stream of the context's device */

/* ---- library / context ------------------------------------------------ */

int imq_abi_version(void);
const char* imq_status_string(int status);

/* Replaces the device/queue setup of DirectDiTStep.init (DirectDiTStep.swift:74-80). */
int imq_create(int device, imq_ctx** out);
int imq_destroy(imq_ctx* ctx);
/* Text of the last failure on ctx ("" if none); valid until the next failing call. */
const char* imq_last_error(const imq_ctx* ctx);

/* ---- streams (MTLCommandQueue / command buffer counterpart) ------------ */

int imq_stream_create(imq_ctx* ctx, imq_stream* out);
int imq_stream_destroy(imq_ctx* ctx, imq_stream stream);
int imq_stream_sync(imq_ctx* ctx, imq_stream stream);

/* ---- memory (the reference's MTLBuffer upload/scratch,
 *      DirectDiTStep.swift:135-153) ------------------------------------- */

int imq_malloc(imq_ctx* ctx, size_t bytes, void** out);
int imq_free(imq_ctx* ctx, void* ptr);
int imq_memcpy_h2d(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream);
int imq_memcpy_d2h(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream);
/* Device to device (the reference's blit copies, DirectDiTStep.swift:639-648,667-670). */
int imq_memcpy_d2d(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream);

/* ---- kernels ------------------------------------------------------------ */

/* out[N, K] (T) = deq(W).  Replaces MLX `dequantized(w, scales:, biases:,
 * groupSize: 64, bits: 4)` (DirectTEEncoder.swift:129-134) and the CPU
 * embedding dequant DirectTEEncoder.embedRow (DirectTEEncoder.swift:106-123).
 * Bit-exact: RNE_T(fl32(fl32(s*q) + b)), the rounding of
 * DirectTEEncoder.swift:39-43 for every non-NaN value (a NaN result, possible
 * only when a scale or bias is inf or NaN, stays a quiet NaN). */
int imq_dequantize(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                   void* out, int k, int n, int group_size, int bits, imq_dtype dtype,
                   imq_stream stream);

/* out[i, K] (T) = deq(W)[rows[i]] for i < count: DirectTEEncoder.embedRow
 * (DirectTEEncoder.swift:106-123) for a batch of token ids in one launch, the
 * same bits as imq_dequantize's rows.  rows: int32 [count] in device memory;
 * an id outside [0, N) reads row clamp(id, 0, N - 1) (the ids are the
 * caller's to validate; no read leaves W). */
int imq_dequantize_rows(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                        const int32_t* rows, int count, void* out, int k, int n, int group_size,
                        int bits, imq_dtype dtype, imq_stream stream);

/* y[M, N] = x[M, K] . deq(W)^T -- the regime dispatcher.  Replaces the
 * dispatch of `affine_qmm_t_{T}_gs_64_b_4_alN_true_batch_0` in
 * DirectDiTStep.qmm (DirectDiTStep.swift:374-406), DirectTELayerSpike.encodeQmm
 * (DirectTELayer.swift:109-128), DirectConditioner.qmm
 * (DirectConditioner.swift:96-117) and MLX quantizedMM(transpose: true)
 * (Sources/ImarelloDiT/AttentionUtils.swift:212-221).  3 <= M <= 16 with
 * K % 128 == 0 runs a weight-streaming matrix-core kernel (16 weight rows per
 * workgroup, K over its waves; from M = 6, where x does not fit LDS or the
 * row tiles are many, K split over the workspace below; 17 <= M <= 32 that
 * split only, where the row tiles are fewer than 512); other M <= 4 the
 * qGEMV kernel;
 * larger M the MFMA qGEMM kernel (f32: the qGEMV kernel, 16 rows at a time).  When the
 * output tiles are too few to fill the GPU, the qGEMM splits
 * K: fp32 partial sums go to a workspace the context keeps per stream (grown
 * on first use, outside stream capture; under capture a call that would need
 * a larger one runs unsplit; an outgrown workspace stays allocated until
 * imq_destroy, so graphs captured earlier stay valid) and a second kernel
 * adds them in order, so the result is deterministic but its fp32 summation
 * order differs from imq_qgemm's.  A graph replay of a captured call and
 * other calls on the stream it was captured on share that stream's
 * workspace: do not run them concurrently. */
int imq_qmm_t(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
              const void* x, void* y, int k, int n, int m, int group_size, int bits,
              imq_dtype dtype, imq_stream stream);

/* imq_qmm_t that allocates nothing.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels, plan and results (bit for bit) as imq_qmm_t, except
 * that a split-K plan keeps its fp32 partial sums in the library's static
 * scratch: 64 MiB of device memory per GPU, part of the library's code object,
 * held from the first imq_create on that GPU until the process ends.  Every
 * partial sum a call reads it has written first, so nothing needs clearing.
 * A shape whose plan needs more scratch than that returns IMQ_EINVAL (the
 * largest plans of the text-encoder, conditioner and DiT shapes up to
 * M = 2048 fit), also where imq_qmm_t would run the few-row kernel's K split.
 * All calls on one GPU share the one scratch.  Eager calls that use it are
 * ordered on the device by the library (each waits, by an event and without
 * blocking the host, for the previous one on that GPU, whatever its stream,
 * context or thread).  Calls made under stream capture are not: a graph
 * replay that overlaps another call using the scratch on that GPU races and
 * may return wrong results; order such replays on one stream. */
int imq_qmm_t_noalloc(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                      const void* x, void* y, int k, int n, int m, int group_size, int bits,
                      imq_dtype dtype, imq_stream stream);

/* The skinny regime alone (1 <= M <= 16): register dequant, fp32 dot products,
 * cross-lane reductions; no matrix cores.  Same contract as imq_qmm_t, for
 * packed weights under 4 GiB (IMQ_EUNSUPPORTED above; imq_qmm_t then runs
 * bf16 / f16 at any M on the MFMA kernel). */
int imq_qgemv(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
              const void* x, void* y, int k, int n, int m, int group_size, int bits,
              imq_dtype dtype, imq_stream stream);

/* The dense regime alone (any M >= 1): dequant fused into bf16 / f16 MFMA
 * tiles, fp32 accumulators, K never split (the fused output stages below
 * equal it plus the glue bit for bit).  Same contract as imq_qmm_t; f32
 * returns IMQ_EUNSUPPORTED. */
int imq_qgemm(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
              const void* x, void* y, int k, int n, int m, int group_size, int bits,
              imq_dtype dtype, imq_stream stream);

/* ---- plan introspection --------------------------------------------------
 * No counterpart in the reference (MLX picks its kernels internally): the
 * kernel, tile height and K split a call of the given entry point would run,
 * for callers that size workspaces or pin a kernel choice in tests. */

typedef enum imq_entry {
    IMQ_ENTRY_QMM_T = 0,   /* imq_qmm_t and imq_qmm_t_noalloc */
    IMQ_ENTRY_QGEMM = 1,   /* imq_qgemm */
    IMQ_ENTRY_QGEMV = 2,   /* imq_qgemv */
    IMQ_ENTRY_FUSED = 3,   /* imq_qmm_postscale / _gate_add (n = weight rows) */
    IMQ_ENTRY_SWIGLU = 4   /* imq_qmm_swiglu (n = 2 * width: the gate and up rows it reads) */
} imq_entry;

typedef enum imq_kernel {
    IMQ_KERNEL_QGEMV = 0,    /* register dequant, fp32 dot products, no matrix cores */
    IMQ_KERNEL_FEW_ROW = 1,  /* weight-streaming matrix-core kernel, 16 weight rows per workgroup */
    IMQ_KERNEL_TILE = 2,     /* MFMA tiles, activations staged by direct buffer->LDS loads
                                (K % 256 == 0) */
    IMQ_KERNEL_TILE_REG = 3  /* MFMA tiles, activations staged through registers (other K) */
} imq_kernel;

typedef struct imq_plan {
    int kernel;             /* an imq_kernel */
    int tile_rows;          /* output rows per workgroup tile (tile kernels; 0 otherwise) */
    int splits;             /* K ranges summed by a second kernel (1: K not split) */
    size_t workspace_bytes; /* fp32 partial sums of a split plan (0 when not split) */
    int tile_cols;          /* output columns per workgroup tile (tile kernels: 256, or 128 for
                               short M; 0 otherwise) */
} imq_plan;

/* The plan of a call of `entry` with these sizes and dtype on ctx's device,
 * without launching anything; the same argument checks as the entry point on
 * the sizes (IMQ_EINVAL / IMQ_EUNSUPPORTED).  For IMQ_ENTRY_QMM_T it is the
 * plan with its split-K workspace in hand: imq_qmm_t_noalloc runs it or
 * returns IMQ_EINVAL, and imq_qmm_t runs it except under stream capture on a
 * stream whose workspace is still smaller than workspace_bytes, where it runs
 * the same kernel family unsplit (or, at 17-32 rows, the tile kernel). */
int imq_qmm_plan(imq_ctx* ctx, int entry, int k, int n, int m, imq_dtype dtype, imq_plan* out);

/* ---- fused output stages ------------------------------------------------
 * The MFMA kernel with the reference's post-qmm glue kernel folded into its
 * epilogue (Sources/ImarelloDirect/DirectDiTKernels.swift).  Each equals the
 * qmm (T output) followed by that glue kernel: the accumulator is rounded to T
 * first, then the glue arithmetic runs in fp32.  T is bf16 or f16 (f32:
 * IMQ_EUNSUPPORTED); any K % 64 == 0 (K % 256 != 0, e.g. the x_embedder's
 * K = 128, runs the register-staged tile kernel); any M >= 1.  Other
 * arguments as imq_qmm_t; fp32 arrays must be 4-byte aligned. */

/* y[i] (T) = T(x[i] / scale) for i < count, x fp32: the pre-scale half of the
 * f16 qmm sandwich, AttentionUtils.compiledPreScale (`(x / s).asType(.float16)`,
 * AttentionUtils.swift:155-160, run by applyLinearCore :198-230 with s = 16).
 * Bit-exact: the correctly rounded fp32 quotient, rounded to nearest even in
 * T.  T is f16 or bf16 (f32: IMQ_EUNSUPPORTED); scale finite and nonzero;
 * x 4-byte and y 2-byte aligned (16-byte alignment of both takes the vector
 * kernel); count 0 is a no-op. */
int imq_cast_prescale(imq_ctx* ctx, const float* x, void* y, size_t count, float scale,
                      imq_dtype dtype, imq_stream stream);

/* y[M, N] (fp32) = float(T(x . deq(W)^T)) * scale: dd_cast_postscale
 * (DirectDiTKernels.swift:199-209), the x16 after a /16 pre-scaled qmm. */
int imq_qmm_postscale(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                      const void* x, float* y, int k, int n, int m, float scale, int group_size,
                      int bits, imq_dtype dtype, imq_stream stream);

/* The other modes of applyLinearCore's f16 sandwich (AttentionUtils.swift:
 * 173-178,198-230, AttentionTuning.swift:55-61):
 *  - the per-tensor dynamic scale (linearDynamicScale): *scale (device fp32)
 *    = max(max_i |x[i]| / target, 1) over count fp32 elements (compiledDynamicScale;
 *    target 64 by default there), computed on the device, no host sync; a NaN
 *    in x gives a NaN scale;
 *  - the pre-scale cast and the post-scale reading that device scale
 *    (scale_dev, which overrides scale when not NULL);
 *  - the post-scale without the f32 upcast (linearF16FullEpilogue,
 *    compiledPostScaleF16, :166-171): y (f16) = f16(float(f16(acc)) *
 *    float(f16(scale))), only with the f16 qmm (dtype f16).
 * imq_qmm_postscale_ex's y_dtype is IMQ_F32 (imq_qmm_postscale) or IMQ_F16. */
int imq_dynamic_scale(imq_ctx* ctx, const float* x, size_t count, float target, float* scale,
                      imq_stream stream);
int imq_cast_prescale_ex(imq_ctx* ctx, const float* x, void* y, size_t count, float scale,
                         const float* scale_dev, imq_dtype dtype, imq_stream stream);
int imq_qmm_postscale_ex(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                         const void* x, void* y, imq_dtype y_dtype, int k, int n, int m,
                         float scale, const float* scale_dev, int group_size, int bits,
                         imq_dtype dtype, imq_stream stream);

/* Row RMSNorm y[r][c] = T(x[r][c] * rsqrt(mean_c(x[r]^2) + eps) * w[c]) (fp32
 * sum of squares, fp32 weight w [cols]): the DiT's dd_rmsnorm_pitched on its
 * fp32 residual (x_dtype IMQ_F32, DirectDiTKernels.swift:61-99) and the text
 * encoder's dq_rmsnorm on its T stream (x_dtype == y_dtype,
 * DirectGlueKernels.swift:14-49); y_dtype bf16 or f16. */
int imq_rmsnorm(imq_ctx* ctx, const void* x, imq_dtype x_dtype, const float* w, void* y,
                imq_dtype y_dtype, int rows, int cols, float eps, imq_stream stream);

/* y[M, N] (T) = T(float(residual) + float(T(x . deq(W)^T))), residual T [M, N]:
 * the text encoder's qmm followed by dq_add (DirectTEEncoder.swift:390-392,
 * 409-411; DirectGlueKernels.swift:88-96).  y may equal residual. */
int imq_qmm_add(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                const void* x, const void* residual, void* y, int k, int n, int m, int group_size,
                int bits, imq_dtype dtype, imq_stream stream);

/* y[M, N] (fp32) = residual + gate[n] * float(T(x . deq(W)^T)) * scale: the
 * gated residual dd_gate_add (DirectDiTKernels.swift:211-224).  y may equal
 * residual (in place). */
int imq_qmm_gate_add(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                     const void* x, const float* residual, const float* gate, float* y, int k,
                     int n, int m, float scale, int group_size, int bits, imq_dtype dtype,
                     imq_stream stream);

/* SwiGLU over the gate and up sections of one projection W [n, K/8]
 * (M <= 4: the qGEMV, the gate and up rows of an output read by one lane
 * group and combined after the reduction, one launch over both sections;
 * larger M: the MFMA kernel with the stage in its epilogue):
 * y[i][j] (T, row pitch ldy elements) = T(g * sigmoid(g) * u * out_scale) for
 * j < width, g = float(T(x_i . deq(W)[gate_row + j])) * in_scale, u the same
 * with up_row: dd_swiglu_pitched (DirectDiTKernels.swift:137-157) fused into
 * the projection that feeds it (the single block's to_qkv_mlp_proj,
 * DirectDiTStep.swift:328-333).  Requires gate_row + width <= n,
 * up_row + width <= n, ldy >= width. */
int imq_qmm_swiglu(imq_ctx* ctx, const uint32_t* w, const void* scales, const void* biases,
                   const void* x, void* y, int ldy, int k, int n, int m, int width, int gate_row,
                   int up_row, float in_scale, float out_scale, int group_size, int bits,
                   imq_dtype dtype, imq_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* IMQ_H */
