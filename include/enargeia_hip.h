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
 *   lm_head_q8 / _q4 / _f16 / _f32        x, packed, scales, zeros, out, dims        eg_lm_head
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
  EG_ERR_FORMAT = -6,  /* a malformed .enargeia container (EnargeiaError, enargeia.ts:84) */
  EG_ERR_IO = -7,      /* a file could not be opened or read                            */
  EG_ERR_NOT_FOUND = -8, /* a named tensor is absent ("<name> is missing", weights.ts:397) */
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
/* Blocks until all work on the context's stream finished (queue.onSubmittedWorkDone). Errors
 * raised on the device since the last blocking call surface here, as WebGPU's error scopes
 * surface them asynchronously (helpers/gpu.ts:41-50): an eg_sample launch that gave up is
 * EG_ERR_DEVICE ("... sample launch(es) gave up ..."), reported once. */
EG_API int eg_sync(eg_context* ctx);

/* ---- buffers (src/gpu/pool.ts:55 acquire/release; queue.writeBuffer; readback.ts:18) ----- */
EG_API int eg_buf_alloc(eg_context* ctx, size_t bytes, void** out_ptr);
EG_API int eg_buf_free(eg_context* ctx, void* ptr);
/* Stream-ordered host->device copy (GPUQueue.writeBuffer). The host memory must stay valid
 * until the copy completed (eg_sync), as pageable copies may be deferred. */
EG_API int eg_buf_write(eg_context* ctx, void* dst, size_t offset, const void* host_src, size_t bytes);
/* Synchronous device->host copy after all prior work (readBuffer, readback.ts:18-38). Reports
 * device-side errors as eg_sync does (the data is copied either way). */
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

/* The prompt MLP's gate and up projections and silu_mul in one operator (graph.ts:484-497:
 * mlp_gate and mlp_up through matmul_q4_prefill, then SILU_MUL, silu_mul.wgsl): for m rows of x,
 *   out[r*n + j] = silu(x[r] . gate_j) * (x[r] . up_j),  silu(g) = g / (1 + e^-g),  j < n
 * with the prefill GEMM's arithmetic (bf16 operands, f32 accumulation). gate and up share the
 * dims (n rows of k each; use_bias must be 0, out_stride n, out_offset 0), the encoding and
 * the bits. One launch where the chunked staging takes both matrices and K is at most 1984;
 * otherwise gate | up side by side into scratch ([m][2n] floats, required) and silu_mul. */
EG_API int eg_matmul_q4_prefill_swiglu(eg_context* ctx, const float* x, const uint32_t* gate_packed,
                                       const float* gate_scales, const uint32_t* gate_zeros,
                                       const uint32_t* up_packed, const float* up_scales,
                                       const uint32_t* up_zeros, float* out, float* scratch,
                                       const eg_matmul_q4_dims* dims, int encoding, int bits);

/* lm_head_<dtype> (embedding_variants.ts:135-180, q8 body :56-63): for row < row_count,
 *   out[row + out_offset] = sum_k x[k] * (code - zero) * scale[block]
 * bits = 8 (lm_head_q8, the shipped tied head) or 4 (lm_head_q4); bits = 16 (lm_head_f16: packed
 * holds the table as halves, two per word, element 2j in the low half, :66-70) or 32
 * (lm_head_f32: plain floats, :71-73) reads the table itself - scales, zeros, the encoding and
 * the block fields are not used. The argmax forms below take the same four. */
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

/* eg_lm_head_argmax for callers that cannot allocate device memory (code under graph capture,
 * tight serving loops, harnesses that forbid hipMalloc): no counterpart in the reference. Same
 * arguments, kernels and results; the per-workgroup argmax partials go to a fixed 64 KiB device
 * array of the library (one per GPU, held until the process ends) instead of the context's
 * workspace, and the call allocates and frees nothing. A launch needing more than 8192 partials
 * fails with EG_ERR_RANGE (the largest grid it makes is 2048). Every call on one GPU shares that
 * array: calls that overlap on one GPU (two streams, two contexts) race. */
EG_API int eg_lm_head_argmax_noalloc(eg_context* ctx, const float* x, const uint32_t* packed,
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
 * order, with the argmax fallback. out[0] = the token id. One launch whose workgroups (one per
 * 2048 ids, vocab <= 524,288) must all be resident at once: a device that cannot hold them is
 * EG_ERR_RANGE here; should one still never start (the device shared with other work), the
 * launch's bounded waits give up, out[0] = 0xFFFFFFFF and the next eg_sync or eg_buf_read on the
 * context fails with EG_ERR_DEVICE. Calls that overlap on one context race (they share its
 * workspace). */
EG_API int eg_sample(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out,
              const eg_sample_dims* dims);

/* The int8 LM head and the sampler as one sampled token: no counterpart op in the reference,
 * which runs lm_head_q8 then sample (graph_decode.ts:363-385). Arguments as eg_lm_head (bits 8;
 * out = the logits, dims->out_offset 0) and eg_sample (history, token = its out, sample->vocab =
 * dims->row_count). The head applies the repetition penalty to each logit it computes and stores
 * it as eg_sample leaves it, and hands the sampler per-workgroup partials (max of l/T, its lowest
 * index, the float64 sum of exp(l/T - that max)) in place of the sampler's own penalty pass,
 * slice maxima, normaliser and first grid barrier; the draw, its semantics, limits and give-up
 * behaviour are eg_sample's. The normaliser's float64 sum is grouped by the head's workgroups
 * rather than the sampler's slices, so it can differ from eg_sample's in the last bits. */
EG_API int eg_lm_head_sample(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                             const uint32_t* zeros, float* out, const uint32_t* history, uint32_t* token,
                             const eg_embedding_dims* dims, int encoding, int bits, const eg_sample_dims* sample);

/* Test hook, no counterpart in the reference: with override != 0 every later sampler launch on
 * this context (eg_sample and the decoder's sampled steps, replays of captured graphs included:
 * the limit lives in device memory) gives a barrier wait up after `polls` polls instead of about
 * a second, and so does every phase wait of the decoder's persistent layers (with polls 0 such a
 * wait gives up without polling: the step fails and moves nothing), so the give-up path (out[0] = 0xFFFFFFFF and an error at the
 * next blocking call, every workgroup leaving, the barrier words restored for the next launch)
 * can be forced from the host; override 0 restores the default. Not for production use. */
EG_API int eg_test_sample_spin(eg_context* ctx, int override, uint32_t polls);

/* Profiling hook, no counterpart in the reference (its decode loop is profiled by timestamp
 * queries, graph_decode.ts:416-433): with `buffer` non-NULL (device memory of at least
 * launches * 131072 bytes, zeroed by the caller), each of the next `launches` launches of a
 * decode-step kernel on this context - GEMVs and GEMV plans (the LM head included), the decode
 * attention, the sampler, the step tail; eager, or captured into a graph whose every replay then
 * writes the same slots - stores per-wave wall-clock stamps (s_memrealtime, 100 MHz): wave w of
 * launch i at buffer[2 * (8192 * i + w)] (entry) and [... + 1] (exit), for w < 8192. *recorded
 * (nullable) receives the number of launches that took a slot since the previous call; NULL
 * turns the stamps off. Only the profiling build of the library (libenargeia_hip_prof.so,
 * compiled with EG_LAUNCH_STAMPS) records stamps; the production build returns EG_ERR_STATE for
 * a non-NULL buffer, its kernels carrying no stamp code. Not for production use. */
EG_API int eg_test_launch_stamps(eg_context* ctx, uint64_t* buffer, uint32_t launches, uint32_t* recorded);

/* ---- decode step: embedding, attention, fused GEMV inputs ----------------------------------- */

/* embed_gather_<dtype> (embedding_variants.ts:93-133, :56-63 for q8): for each of the seq token
 * ids read from DEVICE memory token[s] (a decode step's one id is the previous step's
 * argmax/sample result, so a captured step needs no host round trip): if row_begin <= id <
 * row_begin + row_count,
 *   out[out_offset + s * hidden + i] = (code[id - row_begin, i] - zero) * scale[block]   for i < hidden
 * else that row of out is left untouched (another part of a split table owns the id).
 * bits 4 / 8 as eg_lm_head; 16 / 32 gather an f16 / f32 table's row as it is (scales unused). */
EG_API int eg_embed_gather(eg_context* ctx, const uint32_t* token, const uint32_t* packed, const float* scales,
                           const uint32_t* zeros, float* out, const eg_embedding_dims* dims, int encoding,
                           int bits);

/* Decode attention over an f16 KV cache, fused: RoPE on q and on the new key (ops.ts:87-114,
 * half-rotation pairing, angle in double precision), the new key and value appended to the
 * cache at the position read from DEVICE memory position[0] (graph_decode.ts:276-320: the key
 * is cached after rotation), then scores / softmax / weighted values (ops.ts:130-205,
 * scale 1/sqrt(head_dim), grouped heads: query head h reads kv head h / (heads / kv_heads))
 * over positions 0..position. The positions are split into chunks of `chunk`; each workgroup
 * handles one kv head and one chunk for all the query heads of its group and writes a partial
 * (o[head_dim], running max m, sum l) to `partials`, chunk index fastest so that a consumer
 * reads each output's chunks as contiguous vectors (h = kv * group + g, chunks =
 * max_context / chunk, chunks past the position write m = -inf, l = 0, o = 0):
 *   o: partials[(h * head_dim + e) * chunks + c]
 *   m: partials[heads * head_dim * chunks + h * chunks + c]
 *   l: partials[(heads * head_dim + heads) * chunks + h * chunks + c]
 * Caches are [max_context][kv_heads][head_dim] f16. q is [heads][head_dim], k and v are
 * [kv_heads][head_dim] (the projection outputs, bias included).
 * With `out` (and `counter`, a device u32 that is 0 before the first launch and that every
 * launch leaves at 0), the last workgroup to finish also combines the partials into
 * out[heads * head_dim], the reference's attn_out (as eg_attention_combine would, same bits).
 * Launches that share a counter must not overlap. */
typedef struct eg_attention_dims {
  uint32_t heads, kv_heads, head_dim, max_context;
  uint32_t chunk; /* positions per workgroup: 128 */
  float theta;    /* RoPE base */
  uint32_t pad0, pad1;
} eg_attention_dims;
EG_API int eg_attention_decode(eg_context* ctx, const uint32_t* position, const float* q, const float* k,
                               const float* v, uint16_t* k_cache, uint16_t* v_cache, float* partials,
                               uint32_t* counter, float* out, const eg_attention_dims* dims);
/* eg_attention_decode over caches of f32 rows (the reference's f32 cache variant: the same four
 * attention kernels generated per cache dtype, cache_variants.ts:21-40, SessionOptions.cacheDType
 * session.ts:44, 134): the new rows are appended exactly, every cached value is read as it is.
 * Same arguments, partials and combine. */
EG_API int eg_attention_decode_f32(eg_context* ctx, const uint32_t* position, const float* q, const float* k,
                                   const float* v, float* k_cache, float* v_cache, float* partials,
                                   uint32_t* counter, float* out, const eg_attention_dims* dims);
/* The attention output from the partials: out[h * head_dim + d] = sum_c o_c[d] e^(m_c - M) /
 * sum_c l_c e^(m_c - M), M = max_c m_c (the reference's attn_out, [heads * head_dim]). The
 * decoder does this inside the o projection's input stage instead (EG_INPUT_ATTENTION). */
EG_API int eg_attention_combine(eg_context* ctx, const float* partials, float* out, const eg_attention_dims* dims);

/* How a decode GEMV's input vector is produced: each workgroup computes it into LDS in its
 * prologue, so the normalisation, the SwiGLU gate or the attention combine that precedes a
 * projection costs no launch and no round trip through memory. */
typedef enum eg_input_kind {
  EG_INPUT_VECTOR = 0,    /* x as given                                                       */
  EG_INPUT_RMSNORM = 1,   /* x * 1/sqrt(mean(x^2) + eps) * x2   (rmsnorm.wgsl, ops.ts:30-51)   */
  EG_INPUT_SILU_MUL = 2,  /* silu(x) * x2, silu(g) = g / (1 + e^-g)   (ops.ts:207-216)       */
  EG_INPUT_ATTENTION = 3, /* the combine of eg_attention_decode's partials in x (layout in dims) */
} eg_input_kind;
typedef struct eg_gemv_input {
  int kind;
  const float* x;  /* the vector / norm input / gate / attention partials */
  const float* x2; /* norm weight / up; NULL otherwise */
  float eps;       /* RMSNORM */
  eg_attention_dims attention; /* ATTENTION: the producer's dims (heads * head_dim must equal k) */
} eg_gemv_input;
EG_API int eg_gemv_plan_launch_input(eg_context* ctx, const eg_gemv_plan* plan, const eg_gemv_input* input);
EG_API int eg_lm_head_argmax_input(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed,
                                   const float* scales, const uint32_t* zeros, float* out, uint32_t* result,
                                   const eg_embedding_dims* dims, int encoding, int bits);

/* A gate|up pair in ONE launch that stores the SwiGLU product instead of both projections: no
 * counterpart op in the reference, which dispatches gate, up and silu_mul separately
 * (graph_decode.ts:330-345, ops.ts:207-216). pair[0] is the gate matrix, pair[1] the up matrix
 * (same rows, no biases; int4 only); out = pair[0].out: out[r + pair[0].out_offset] =
 * silu(g_r) * u_r with g_r, u_r the two GEMV rows on the launch's input and silu(g) =
 * g / (1 + e^-g). Launched with eg_gemv_plan_launch_input and EG_INPUT_RMSNORM (the
 * post-attention norm), so the down projection reads a plain vector (EG_INPUT_VECTOR). */
EG_API int eg_gemv_swiglu_plan_create(eg_context* ctx, uint32_t k, uint32_t block_size, int encoding, int bits,
                                      const eg_gemv_segment* pair, eg_gemv_plan** out_plan);

/* The end of a decode step (Session.decodeStep bookkeeping, session.ts:347-375, kept on the
 * device so a captured step replays without the host): position[0] += 1 and
 * history[history_length[0]++] = token[0]. */
EG_API int eg_decode_advance(eg_context* ctx, uint32_t* position, uint32_t* history, uint32_t* history_length,
                             const uint32_t* token, uint32_t history_capacity);

/* ---- the decode step driver (DecodeGraph + Session.decodeStep, graph_decode.ts:185-448,
 *      session.ts:347-375) ----------------------------------------------------------------- */

/* One quantized matrix: the three streams of the weight layout (zeros NULL when signed). */
typedef struct eg_quant_matrix {
  const uint32_t* packed;
  const float* scales;
  const uint32_t* zeros;
} eg_quant_matrix;

typedef struct eg_layer_desc {
  eg_quant_matrix q, k, v, o, gate, up, down;  /* [out][in] row-major, as the checkpoint */
  const float *q_bias, *k_bias, *v_bias;      /* nullable */
  const float *input_norm, *post_attention_norm;
} eg_layer_desc;

typedef struct eg_model_desc {
  uint32_t layers, hidden, heads, kv_heads, head_dim, intermediate, vocab, max_context;
  float rms_eps, rope_theta;
  int encoding, bits;          /* projections */
  uint32_t block_size;
  eg_quant_matrix embedding;   /* the tied table: gathered, and the LM head */
  int embed_encoding, embed_bits; /* 4 / 8 codes, or 16 / 32: an f16 / f32 table (no scales) */
  uint32_t embed_block_size;
  const float* final_norm;
  const eg_layer_desc* layer;  /* `layers` entries */
} eg_model_desc;

typedef struct eg_decoder eg_decoder;

/* Device buffers a decoder owns, for callers that fill or inspect them (the KV caches are
 * [layers][max_context][kv_heads][head_dim] of f16, or of f32 for a decoder created with
 * EG_CACHE_F32; logits f32[vocab] (penalized in place by a
 * sampled step, as the reference's sample kernel does); token u32[3] = the next input id
 * (written by each step), its logit bits (greedy steps) and the status word: the count of
 * sampled steps whose sampler gave up, which changed nothing else (cleared by the readback that
 * reports it and by eg_decoder_reset); position u32; history u32[max_context] = the sampler's history (DecodeGraph's
 * `history` buffer); sample_params = the sample step's 32-byte uniform, live on the device:
 * history_length is advanced by every step and `random` holds the last step's draw; rng = the
 * mulberry32 state). */
typedef struct eg_decoder_buffers {
  void *k_cache, *v_cache;
  float* logits;
  float* hidden;
  uint32_t* token;
  uint32_t* position;
  uint32_t* history;
  eg_sample_dims* sample_params;
  uint32_t* rng;
} eg_decoder_buffers;

/* SamplingParams (sample.ts:24-31): temperature <= 0 is greedy (GREEDY = {0, 1, 1}, sample.ts:33),
 * top_p >= 1 keeps every id, top_p <= 0 leaves the argmax fallback, repetition_penalty 1 disables
 * the penalty. Any finite values, as the reference's setSampling takes them. */
typedef struct eg_sampling_params {
  float temperature, top_p, repetition_penalty;
} eg_sampling_params;

/* Plans every launch of a step once: per layer one GEMV plan for q|k|v (RMSNorm input stage,
 * biases), one fused attention launch, the o projection (attention-combine input stage, the
 * residual as its bias), gate|up (RMSNorm input stage) and down (SiLU*up input stage, residual
 * bias); then the LM head with the final norm fused and its argmax partials, and one tail launch
 * (the token, the position advance, the next token's embedding row and RoPE table). 5 launches
 * per layer + 2, against the reference's ~19 dispatches per layer. Allocates the caches and
 * scratch. The weights stay owned by the caller and must outlive the decoder. */
EG_API int eg_decoder_create(eg_context* ctx, const eg_model_desc* desc, eg_decoder** out_decoder);
/* KV cache element types (SessionOptions.cacheDType, session.ts:44, 134; cacheElementBytes,
 * cache_variants.ts:21-26). */
#define EG_CACHE_F16 0
#define EG_CACHE_F32 1
/* eg_decoder_create with the cache dtype chosen (eg_decoder_create is EG_CACHE_F16): an f32 cache
 * doubles the cache's memory and read traffic and keeps every cached key and value exact. Its
 * steps run the attention once per layer as its own launch (the persistent layers option reads
 * an f16 cache) and its prompt chunks append the cache rows in their own launch. */
EG_API int eg_decoder_create_cache(eg_context* ctx, const eg_model_desc* desc, int cache_dtype,
                                   eg_decoder** out_decoder);
EG_API int eg_decoder_destroy(eg_decoder* decoder);
EG_API int eg_decoder_buffers_get(eg_decoder* decoder, eg_decoder_buffers* out);
/* Position and next input token (rows [0, position) of the caches are the history). */
EG_API int eg_decoder_reset(eg_decoder* decoder, uint32_t position, uint32_t token);
/* One step at the current position on the current token (Session.decodeStep, session.ts:347-375):
 * with GREEDY parameters the LM head's fused argmax gives the next token; with any other the
 * logits go through the sample step (repetition penalty over the history, temperature, top-p,
 * the draw; sample.wgsl:143-332) with one mulberry32 draw taken on the device. Either way the
 * token is appended to the history, the draw state advances once (Session draws once per step
 * whatever the parameters) and the position advances, all on the device. token_out (host,
 * nullable) receives the new token: the one readback per step (12 bytes: the token with the
 * status word). Replays the captured graph if there is one. A sampled step whose sampler gave up
 * (its grid barrier timed out) moves nothing - position, history, draw state and the next
 * step's input stay as they were, so the next step redoes it - and is reported as EG_ERR_DEVICE
 * by the readback that sees it (the one of this step or, device-chained without token_out, the
 * next one that reads). */
EG_API int eg_decoder_step(eg_decoder* decoder, uint32_t* token_out);
/* Captures one step as a hipGraph; later eg_decoder_step calls replay it (no host work per
 * launch; every per-token value already lives in device memory). A change of sampling
 * parameters between greedy and sampled captures it again. */
EG_API int eg_decoder_capture(eg_decoder* decoder);
/* The sampling parameters of the following steps (DecodeGraph.setSampling, graph_decode.ts:387;
 * a new decoder is GREEDY). */
EG_API int eg_decoder_set_sampling(eg_decoder* decoder, const eg_sampling_params* params);
/* Launches one step of the current mode enqueues (DecodeGraph.dispatchCount's counterpart): the
 * 24 layers as one persistent launch where the shapes and the device allow it (else 5 per layer),
 * the LM head, the sampler unless the parameters are GREEDY, the tail, and the input preparation
 * of a host-driven step. */
EG_API int eg_decoder_launches(eg_decoder* decoder, uint32_t* per_step);
/* Restarts the draw source: mulberry32(seed) (session.ts:75-83; a new decoder has the session's
 * default seed 0x5eed, :125), and returns the decoder to device-chained steps. */
EG_API int eg_decoder_seed(eg_decoder* decoder, uint32_t seed);
/* DecodeGraph.setPosition(position, historyLength, random) (graph_decode.ts:398-406), for a host
 * that drives the decoder as the reference's Session.decodeStep does (session.ts:347-375): it
 * writes the input token into the `token` buffer and the history into `history`, calls this,
 * then steps. The decoder is then host-driven: each step first prepares the input from token[0]
 * and the given position, and the sample step uses `random` as given instead of drawing on the
 * device. eg_decoder_seed or eg_decoder_prefill return it to device-chained steps. */
EG_API int eg_decoder_set_position(eg_decoder* decoder, uint32_t position, uint32_t history_length, float random);
/* The repetition-penalty history (Session.tokens, written before each step, session.ts:349-350):
 * every step then appends the token it produces. count <= max_context. */
EG_API int eg_decoder_set_history(eg_decoder* decoder, const uint32_t* host_ids, uint32_t count);
/* The prompt and its first token (Session.runPrefill + sampleFromPrefill, session.ts:326-344,
 * 472-495): the history becomes the prompt, positions [position, position + count) receive the
 * prompt's cache rows, and the last one's logits are sampled (one draw) into the next token,
 * which is appended to the history. A prompt past the context is EG_ERR_RANGE
 * ("prompt of N exceeds the remaining context of M"). token_out as for eg_decoder_step; should
 * the sampler give up, the decoder is left at the prompt's last position with that id as its
 * input, and the next eg_decoder_step recomputes that position and samples. */
EG_API int eg_decoder_prefill(eg_decoder* decoder, uint32_t position, const uint32_t* host_ids, uint32_t count,
                              uint32_t* token_out);
/* Rows per prompt chunk (Session's prefillChunk, session.ts:146): a longer prompt runs as several
 * chunks, each attending to the cache rows before it. The decoder holds buffers for
 * min(2048, max_context) rows, its default; the reference's default is 256. */
EG_API int eg_decoder_set_prefill_chunk(eg_decoder* decoder, uint32_t rows);

/* ---- chunked-prefill attention (cache_variants.ts:81-145 attn_scores / attn_apply with the
 * softmax between; graph.ts:411-459 for the RoPE and cache writes before them) --------------
 * The first six fields are the reference's 32-byte prefill Dims {queries, keys, queryBegin,
 * heads, kvHeads, headDim} (keys = query_begin + queries, the causal extent of the chunk); the
 * last two say what its pad words leave to other uniforms: the cache length and RoPE theta. */
typedef struct eg_attention_prefill_dims {
  uint32_t queries, keys, query_begin, heads, kv_heads, head_dim, max_context;
  float theta;
} eg_attention_prefill_dims;

/* A chunk of `queries` rows at absolute positions [query_begin, query_begin + queries): q
 * [queries][heads][64], k and v [queries][kv_heads][64] (the projections, f32, before RoPE).
 * RoPE rotates q and k; k and v are appended to the f16 caches [max_context][kv_heads][64] at
 * those positions; q_rope (f32, same shape as q) receives the rotated q scaled by 1/sqrt(64).
 * Then out [queries][heads][64] = softmax(q k^T / sqrt(64), causal: key j <= query_begin + i)
 * v over the cache. Matrix-core products in f16 with f32 accumulation; head_dim 64. */
EG_API int eg_attention_prefill(eg_context* ctx, const float* q, const float* k, const float* v, uint16_t* k_cache,
                                uint16_t* v_cache, float* q_rope, float* out,
                                const eg_attention_prefill_dims* dims);
/* eg_attention_prefill over caches of f32 rows (cache_variants.ts:21-40 and 81-145 for the f32
 * dtype): the rotated k and v rows are appended exactly and the attention runs on f32 FMAs
 * with f32 operands throughout; at most 8 query heads per kv head. */
EG_API int eg_attention_prefill_f32(eg_context* ctx, const float* q, const float* k, const float* v, float* k_cache,
                                    float* v_cache, float* q_rope, float* out,
                                    const eg_attention_prefill_dims* dims);

/* ---- the .enargeia container (enargeia.ts:1-50, 112-240; WeightStore.loadQuantized,
 * weights.ts:299-471) ------------------------------------------------------------------------
 * eg_container_open parses the prefix and JSON header on the host and applies the reference's
 * checks with its messages (parseEnargeiaHeader / parseTensor, enargeia.ts:112-242), plus one of
 * its own: the ranges must lie inside the file. It needs no device; pass ctx NULL to get the
 * message from eg_last_error(NULL). eg_container_upload reads the blob into ONE device
 * allocation (free it with eg_buf_free): a tensor's device address is that allocation plus its
 * range's begin, 256-byte aligned like the file. eg_container_model_desc points a decoder
 * description at the uploaded blob for a Qwen2 checkpoint (model.embed_tokens.weight tied,
 * model.layers.N.{self_attn.{q,k,v,o}_proj, mlp.{gate,up,down}_proj}.weight, q/k/v biases,
 * input/post_attention layernorms, model.norm.weight); layers, hidden, heads, kv_heads,
 * intermediate and vocab come from the tensor shapes, the rest from the config. */

typedef struct eg_container eg_container;

typedef enum eg_dtype { EG_DTYPE_Q4 = 0, EG_DTYPE_Q8 = 1, EG_DTYPE_F32 = 2, EG_DTYPE_F16 = 3 } eg_dtype;

#define EG_MAX_DIMS 8

/* One header entry (QuantTensorInfo / F32TensorInfo / F16TensorInfo, enargeia.ts:37-71).
 * Ranges are [begin, end) byte offsets within the blob; the unused ones are zero. */
typedef struct eg_tensor_info {
  const char* name; /* owned by the container */
  int dtype;        /* eg_dtype */
  int bits;         /* 4, 8, 32 or 16 */
  uint32_t ndim;
  uint32_t block_size, blocks_per_row; /* quantized only */
  uint64_t shape[EG_MAX_DIMS];
  uint64_t total_blocks;
  uint64_t packed[2], scales[2], zeros[2]; /* quantized */
  uint64_t data[2];                        /* F32 / F16 */
} eg_tensor_info;

/* EnargeiaHeader (enargeia.ts:73-82). */
typedef struct eg_container_header {
  uint32_t version, block_size, tensor_count, pad0;
  uint64_t header_length, data_offset, blob_bytes, file_size;
  const char* quantization; /* owned by the container; "unknown" when absent */
} eg_container_header;

/* What the container does not say about the model (ModelConfig, graph.ts:57-67). */
typedef struct eg_model_config {
  uint32_t head_dim, max_context;
  float rms_eps, rope_theta;
} eg_model_config;

EG_API int eg_container_open(eg_context* ctx, const char* host_path, eg_container** out_container);
EG_API int eg_container_close(eg_container* container);
EG_API int eg_container_header_get(const eg_container* container, eg_container_header* out);
EG_API int eg_container_tensor(const eg_container* container, uint32_t index, eg_tensor_info* out);
EG_API int eg_container_find(const eg_container* container, const char* name, eg_tensor_info* out);
EG_API int eg_container_upload(eg_context* ctx, const eg_container* container, void** out_blob);
/* Fills `desc` and `layers[0 .. model layers)`; desc->layer points at `layers`. */
EG_API int eg_container_model_desc(eg_context* ctx, const eg_container* container, const void* blob,
                                   const eg_model_config* config, eg_model_desc* desc, eg_layer_desc* layers,
                                   uint32_t layers_capacity);

/* ---- capture (one hipGraph replaces one encoded command buffer, graph_decode.ts:442) ---- */
EG_API int eg_graph_begin(eg_context* ctx);
EG_API int eg_graph_end(eg_context* ctx, eg_graph** out_graph);
EG_API int eg_graph_launch(eg_context* ctx, eg_graph* graph);
EG_API int eg_graph_destroy(eg_graph* graph);

#ifdef __cplusplus
}
#endif
#endif /* ENARGEIA_HIP_H */
