/*
 * enargeia_hip.h — C ABI of the MI355X-native quantized projection path.
 *
 * This is the drop-in boundary for the reference's kernel-op interface: the TypeScript
 * `KernelSpec` / `ComputeKernel` pair (src/kernels/kernel.ts:20-112) and the per-op binding
 * lists and uniform structs of the ops on the path. A host binding (the Node N-API addon in
 * enargeia_amd/js, the Python mirror in enargeia_amd/kernels.py) maps `ComputeKernel.encode`
 * for these op names onto the entry points below:
 *
 *   reference op (KernelSpec.name)       binding order (kernel.ts / op .ts)          entry point
 *   matmul_q4_decode                     x, packed, scales, zeros, bias, out, dims  eg_matmul_q4_decode
 *   matmul_q4_prefill                    x, packed, scales, zeros, bias, out, dims  eg_matmul_q4_prefill
 *   lm_head_q8 / lm_head_q4              x, packed, scales, zeros, out, dims        eg_lm_head
 *   argmax                               logits, out, dims                          eg_argmax
 *   sample                               logits(rw), history, out(rw), dims         eg_sample
 *
 * Conventions
 *   - Every pointer is a device pointer (from eg_buf_alloc or any HIP allocation on the
 *     context's device) unless named host_*. Sizes are in bytes unless named otherwise.
 *   - Every entry point returns an eg_status; 0 is success. On failure, eg_last_error(ctx)
 *     holds a message in the reference's style ("<op>: ..."). Nothing throws across the ABI.
 *   - Work is enqueued on the context's stream (its own, or one set with eg_set_stream) in
 *     call order, like the reference's single GPUQueue. Only eg_buf_read and eg_sync block.
 *   - A context is used from one host thread at a time (the reference is single-threaded JS).
 *   - Quantized weights are the reference's three streams, verbatim (weights.ts:56-67):
 *     packed codes, f32 scales per block, and (for EG_ENC_OFFSET_ZEROS) packed zero-points.
 *     No repacking: the kernels read the layout the reference uploads.
 */
#ifndef ENARGEIA_HIP_H
#define ENARGEIA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EG_ABI_VERSION 1

#if defined(__GNUC__)
#define EG_API __attribute__((visibility("default")))
#else
#define EG_API
#endif

typedef struct eg_context eg_context;
typedef struct eg_graph eg_graph;

typedef enum eg_status {
  EG_OK = 0,
  EG_ERR_INVALID = -1, /* caller mistake: null pointer, bad shape or format (JS Error)   */
  EG_ERR_RANGE = -2,   /* a size or grid over a limit (JS RangeError, kernel.ts:97-107) */
  EG_ERR_DEVICE = -3,  /* HIP runtime failure (device lost, launch failure)             */
  EG_ERR_NOMEM = -4,   /* device allocation failed                                      */
  EG_ERR_STATE = -5,   /* call out of order (graph capture not begun, ...)              */
} eg_status;

/* Encodings of the quantized code streams. */
typedef enum eg_encoding {
  /* Reference format: unsigned codes, value = (code - zero) * scale, zero-points packed at
   * the code width (8 per u32 for int4, 4 per u32 for int8). quant.ts:24-84,
   * quantize.py:74-103, embedding_variants.ts:56-63. */
  EG_ENC_OFFSET_ZEROS = 0,
  /* Symmetric format of the BASELINE configs: two's-complement codes, value = code * scale,
   * no zero-point stream (zeros must be NULL). Equivalent to offset-binary with zero
   * 2^(bits-1) after XOR with 0x88888888 / 0x80808080. */
  EG_ENC_SIGNED = 1,
} eg_encoding;

/* The 48-byte `Dims` uniform of matmul_q4_{decode,prefill} (matmul_q4_decode.wgsl:24-44,
 * written by matmulQ4Dims, matmul_q4.ts:50-64), field for field. grid_width is accepted and
 * ignored: the launch geometry is this library's own. */
typedef struct eg_matmul_q4_dims {
  uint32_t m, n, k, use_bias;
  uint32_t block_size, blocks_per_row, out_stride, out_offset;
  uint32_t grid_width, pad0, pad1, pad2;
} eg_matmul_q4_dims;

/* The 48-byte `Dims` of the generated embedding kernels (embedding_variants.ts:76-91, written
 * by embeddingDims :207-221). For the LM head: rows [0, row_count) of this part are
 * multiplied and written at out[row + out_offset]; seq, row_begin and out_stride are the
 * gather's and are ignored here, as the reference's head kernel ignores them. */
typedef struct eg_embedding_dims {
  uint32_t seq, hidden, row_begin, row_count;
  uint32_t block_size, blocks_per_row, out_stride, out_offset;
  uint32_t grid_width, pad0, pad1, pad2;
} eg_embedding_dims;

/* argmax's 16-byte `Dims` (argmax.wgsl:11-17, argmaxDims argmax.ts:16-18). */
typedef struct eg_argmax_dims {
  uint32_t count, offset, pad0, pad1;
} eg_argmax_dims;

/* sample's 32-byte `Dims` (sample.wgsl:30-44, sampleDims sample.ts:35-50). */
typedef struct eg_sample_dims {
  uint32_t vocab, history_length;
  float temperature, top_p, repetition_penalty, random;
  uint32_t pad0, pad1;
} eg_sample_dims;

/* ---- context ---------------------------------------------------------------------------- */

/* Replaces initGPU (src/gpu/device.ts:116): binds HIP device `device`, creates a stream at the
 * default priority and a small workspace for cross-workgroup reductions. */
EG_API int eg_create(int device, eg_context** out_ctx);
EG_API int eg_destroy(eg_context* ctx);
/* Last error message of this context, or of the calling thread when ctx is NULL. */
EG_API const char* eg_last_error(const eg_context* ctx);
EG_API int eg_abi_version(void);
/* The context's stream (hipStream_t) and a way to enqueue on a caller's stream instead.
 * Passing NULL to eg_set_stream restores the context's own stream. */
EG_API int eg_get_stream(eg_context* ctx, void** out_stream);
EG_API int eg_set_stream(eg_context* ctx, void* stream);
/* Blocks until all work on the context's stream finished (queue.onSubmittedWorkDone). */
EG_API int eg_sync(eg_context* ctx);

/* ---- buffers (src/gpu/pool.ts:55 acquire/release; queue.writeBuffer; readback.ts:18) ----- */
EG_API int eg_buf_alloc(eg_context* ctx, size_t bytes, void** out_ptr);
EG_API int eg_buf_free(eg_context* ctx, void* ptr);
/* Stream-ordered host->device copy (GPUQueue.writeBuffer). The host memory must stay valid
 * until the copy completed (eg_sync), as pageable copies may be deferred. */
EG_API int eg_buf_write(eg_context* ctx, void* dst, size_t offset, const void* host_src, size_t bytes);
/* Synchronous device->host copy after all prior work (readBuffer, readback.ts:18-38). */
EG_API int eg_buf_read(eg_context* ctx, const void* src, size_t offset, void* host_dst, size_t bytes);
/* Stream-ordered zero fill by a kernel (pool.clear), safe inside graph capture. */
EG_API int eg_buf_zero(eg_context* ctx, void* dst, size_t offset, size_t bytes);

/* ---- ops on the path --------------------------------------------------------------------- */

/* matmul_q4_decode (matmul_q4_decode.wgsl:56-101): for col < n,
 *   out[col + out_offset] = sum_k x[k] * (code - zero) * scale[block] (+ bias[col] if use_bias)
 * Matrix-by-vector; like the reference kernel it reads row 0 of x whatever dims.m says.
 * bits = 4 (the reference) or 8 (same contract at int8). zeros is NULL for EG_ENC_SIGNED and
 * bias may be NULL when use_bias is 0. Requires k % block_size == 0 and
 * blocks_per_row == k / block_size. */
EG_API int eg_matmul_q4_decode(eg_context* ctx, const float* x, const uint32_t* packed,
                        const float* scales, const uint32_t* zeros, const float* bias, float* out,
                        const eg_matmul_q4_dims* dims, int encoding, int bits);

/* matmul_q4_prefill (matmul_q4_prefill.wgsl:77-162): for m rows of x,
 *   out[r*out_stride + col + out_offset] = sum_k x[r,k] * W[col,k] (+ bias[col])
 * on the matrix cores: x and the dequantized weights are rounded to bf16, products are
 * accumulated in f32 (gfx950 v_mfma_f32_16x16x32_bf16). Same weight streams as decode. */
EG_API int eg_matmul_q4_prefill(eg_context* ctx, const float* x, const uint32_t* packed,
                         const float* scales, const uint32_t* zeros, const float* bias,
                         float* out, const eg_matmul_q4_dims* dims, int encoding, int bits);

/* lm_head_<dtype> (embedding_variants.ts:135-180, q8 body :56-63): for row < row_count,
 *   out[row + out_offset] = sum_k x[k] * (code - zero) * scale[block]
 * bits = 8 (lm_head_q8, the shipped tied head) or 4 (lm_head_q4). */
EG_API int eg_lm_head(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
               const uint32_t* zeros, float* out, const eg_embedding_dims* dims, int encoding,
               int bits);

/* The LM head with the greedy argmax fused into it: no counterpart op in the reference, which
 * runs lm_head_q8 then argmax/sample (graph.ts:543-567, graph_decode.ts:363-385). out may be
 * NULL (logits not stored). result[0] = out_offset + index of the largest logit (lowest index
 * on ties, argmax.wgsl:53-57), result[1] = its f32 bit pattern. */
EG_API int eg_lm_head_argmax(eg_context* ctx, const float* x, const uint32_t* packed,
                      const float* scales, const uint32_t* zeros, float* out, uint32_t* result,
                      const eg_embedding_dims* dims, int encoding, int bits);

/* Several decode GEMVs that share one input vector and one K, in ONE launch: no counterpart
 * op in the reference, which dispatches matmul_q4_decode once per projection
 * (graph_decode.ts:214-236). For q|k|v of a layer (same normed input), gate|up, or one shape
 * across layers. Each segment is a whole matrix of `rows` rows with the same semantics as
 * eg_matmul_q4_decode: out[row + out_offset] = sum_k x[k] * W[row, k] (+ bias[row] if bias).
 * The plan validates the table once and keeps it in device memory, so a launch is
 * capture-safe. rows must be a multiple of 8 for every segment; at most 256 segments per plan
 * (EG_ERR_RANGE beyond). */
typedef struct eg_gemv_segment {
  const uint32_t* packed;
  const float* scales;
  const uint32_t* zeros; /* NULL for EG_ENC_SIGNED */
  const float* bias;     /* nullable */
  float* out;
  uint32_t rows, out_offset;
} eg_gemv_segment;
typedef struct eg_gemv_plan eg_gemv_plan;
EG_API int eg_gemv_plan_create(eg_context* ctx, uint32_t k, uint32_t block_size, int encoding, int bits,
                               const eg_gemv_segment* segments, uint32_t count, eg_gemv_plan** out_plan);
EG_API int eg_gemv_plan_launch(eg_context* ctx, const eg_gemv_plan* plan, const float* x);
EG_API int eg_gemv_plan_destroy(eg_context* ctx, eg_gemv_plan* plan);

/* argmax (argmax.wgsl:28-66): out[0] = index of the largest of logits[offset..offset+count)
 * (lowest index on ties; -1e30 sentinel as in the reference), out[1] = its f32 bits. */
EG_API int eg_argmax(eg_context* ctx, const float* logits, uint32_t* out, const eg_argmax_dims* dims);

/* sample (sample.wgsl:143-332): repetition penalty applied to `logits` IN PLACE for the first
 * occurrence of each id in history[0..history_length), then greedy argmax (temperature <= 0)
 * or temperature / top-p (threshold bisection, 32 steps) / draw at `random` in ascending id
 * order, with the argmax fallback. out[0] = the token id. */
EG_API int eg_sample(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out,
              const eg_sample_dims* dims);

/* ---- capture (one hipGraph replaces one encoded command buffer, graph_decode.ts:442) ---- */
EG_API int eg_graph_begin(eg_context* ctx);
EG_API int eg_graph_end(eg_context* ctx, eg_graph** out_graph);
EG_API int eg_graph_launch(eg_context* ctx, eg_graph* graph);
EG_API int eg_graph_destroy(eg_graph* graph);

#ifdef __cplusplus
}
#endif
#endif /* ENARGEIA_HIP_H */
