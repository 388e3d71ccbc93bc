/*
 * imq_weights.h -- packed-tensor loader of the affine 4-bit quantized linear
 * library: safetensors shards, memory-mapped, and their upload to the device.
 *
 * Replaces the reference's weight path for the quantized layers:
 *   - shard discovery, SafetensorsLoader.shardFileNames
 *     (Sources/ImarelloWeights/SafetensorsLoader.swift:6-25): the sorted set
 *     of weight_map files of model.safetensors.index.json when it exists, else
 *     the sorted *.safetensors files of the directory;
 *   - merged loading, SafetensorsLoader.loadMergedArrays
 *     (Sources/ImarelloWeights/SafetensorsLoader+MLX.swift:7-17): one name ->
 *     tensor map over all shards, a later shard's tensor replacing an earlier
 *     one of the same name;
 *   - the per-layer upload of (weight, scales, biases) with the scale dtype
 *     cast, DirectDiTStep.quant / loadBlocks / loadHead
 *     (Sources/ImarelloDirect/DirectDiTStep.swift:278-336,844-884),
 *     DirectTEForward.loadLayers (Sources/ImarelloDirect/DirectTEForward.swift:97-138),
 *     DirectConditioner.quant (Sources/ImarelloDirect/DirectConditioner.swift:75-84)
 *     and DirectDiTStep.upload (:135-145).
 *
 * The safetensors layout: an 8-byte little-endian header length H, H bytes of
 * JSON mapping each tensor name to {"dtype", "shape", "data_offsets": [begin,
 * end]} (offsets relative to the byte buffer that follows the header) plus an
 * optional "__metadata__" string map, then the byte buffer.  Opening checks
 * every entry: known dtype, offsets inside the buffer, end - begin equal to
 * the element count times the dtype size, no two tensors overlapping.
 *
 * Conventions as in imq.h: every call returns an imq_status; an imq_st is
 * read-only after opening and may be shared between threads.
 */
#ifndef IMQ_WEIGHTS_H
#define IMQ_WEIGHTS_H

#include "imq.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct imq_st imq_st; /* opaque: an opened, memory-mapped set of shards */

/* safetensors dtype strings, in this order: BOOL U8 I8 U16 I16 F16 BF16 U32
 * I32 F32 U64 I64 F64 F8_E4M3 F8_E5M2. */
typedef enum imq_st_dtype {
    IMQ_ST_BOOL = 0, IMQ_ST_U8, IMQ_ST_I8, IMQ_ST_U16, IMQ_ST_I16, IMQ_ST_F16, IMQ_ST_BF16,
    IMQ_ST_U32, IMQ_ST_I32, IMQ_ST_F32, IMQ_ST_U64, IMQ_ST_I64, IMQ_ST_F64, IMQ_ST_F8_E4M3,
    IMQ_ST_F8_E5M2
} imq_st_dtype;

#define IMQ_ST_MAX_DIMS 8

typedef struct imq_st_info {
    const char* name;                 /* valid until imq_st_close */
    int dtype;                        /* imq_st_dtype */
    int ndim;
    int64_t shape[IMQ_ST_MAX_DIMS];
    const void* data;                 /* host address inside the mapping */
    size_t bytes;
    int shard;                        /* index into the opened shard list */
} imq_st_info;

/* Open the given shard files, in order (a later shard's tensor of the same
 * name replaces an earlier one). */
int imq_st_open(const char* const* paths, int n_paths, imq_st** out);
/* Open a directory with SafetensorsLoader.shardFileNames' rule (above);
 * IMQ_EINVAL "weights not found" when it holds no shard. */
int imq_st_open_dir(const char* directory, imq_st** out);
int imq_st_close(imq_st* st);
/* Last failure on st; with st == NULL, the calling thread's last failed open. */
const char* imq_st_last_error(const imq_st* st);

int imq_st_shard_count(const imq_st* st);
const char* imq_st_shard_path(const imq_st* st, int shard);
/* The "__metadata__" value of key in a shard, or NULL. */
const char* imq_st_metadata(const imq_st* st, int shard, const char* key);

/* Tensors are indexed 0..count-1 in name order. */
int imq_st_count(const imq_st* st);
int imq_st_info_at(const imq_st* st, int index, imq_st_info* out);
/* IMQ_EINVAL with "missing tensor <name>" when absent (SpikeError.missingTensor,
 * DirectQmmSpike.swift:17-19). */
int imq_st_find(const imq_st* st, const char* name, imq_st_info* out);

/* Host -> device copy of any host memory (pageable, or a mapping) through the
 * context's pinned bounce buffers, asynchronous on stream; src may be reused
 * or unmapped as soon as the call returns. */
int imq_upload(imq_ctx* ctx, void* dst, const void* src, size_t bytes, imq_stream stream);

/* Copy one tensor of st into caller-provided device memory dst (dst_bytes
 * bytes), converting its elements to dst_dtype (an imq_st_dtype): the stored
 * dtype itself, or BF16 -> F16 (round to nearest even), BF16 -> F32, F16 -> F32.
 * Staged like imq_upload.  IMQ_EINVAL when dst_bytes is not the converted size. */
int imq_st_upload(imq_ctx* ctx, const imq_st* st, const char* name, int dst_dtype, void* dst,
                  size_t dst_bytes, imq_stream stream);

/* A resident packed projection: the reference's Q(w:s:b:n:k:)
 * (DirectDiTStep.swift:278-284).  One device allocation holds w, scales and
 * biases (base). */
typedef struct imq_qweight {
    uint32_t* w;      /* [n, k/8] */
    void* scales;     /* [n, k/64] of dtype */
    void* biases;     /* [n, k/64] of dtype */
    int n;
    int k;
    imq_dtype dtype;  /* element type of scales and biases */
    void* base;
} imq_qweight;

/* Upload <prefix>.weight (U32 [N, K/8]), <prefix>.scales and <prefix>.biases
 * (BF16, F16 or F32 [N, K/64]) with the scales and biases converted to
 * param_dtype: kept as stored, cast bf16 -> f16 (round to nearest even: the DiT
 * precast, TransformerWeights.swift:40-54, DirectDiTStep.swift:303-306) or
 * widened to f32 (the conditioner, DirectConditioner.swift:75-84).  Every
 * other conversion (f32 -> f16 or bf16, f16 -> bf16) is IMQ_EUNSUPPORTED. */
int imq_load_qlinear(imq_ctx* ctx, const imq_st* st, const char* prefix, imq_dtype param_dtype,
                     imq_qweight* out, imq_stream stream);

/* Several projections that share K (and the stored scale type) as one
 * resident projection whose rows are theirs in the given order: N = the sum
 * of their N.  One call then covers projections the reference dispatches one
 * by one on the same input -- q/k/v, gate/up (DirectTEEncoder.swift:384-410,
 * DirectTEForward.swift:98-106) -- and streams all their weights in one
 * launch.  Same conversions and errors as imq_load_qlinear. */
int imq_load_qlinear_cat(imq_ctx* ctx, const imq_st* st, const char* const* prefixes, int count,
                         imq_dtype param_dtype, imq_qweight* out, imq_stream stream);
int imq_qweight_free(imq_ctx* ctx, imq_qweight* q);

#ifdef __cplusplus
}
#endif
#endif /* IMQ_WEIGHTS_H */
