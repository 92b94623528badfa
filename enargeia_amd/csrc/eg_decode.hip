// The decode step's non-GEMV ops: the embedding gather, fused decode attention over the f16
// KV cache, the attention combine, and the device-side step bookkeeping.
//
// Reference pieces: embed_gather (embedding_variants.ts:93-133), rope.wgsl + the f16 cache
// pack (cache_variants.ts:147-305, graph_decode.ts:276-320), attn_scores / softmax /
// attn_apply decode (graph_decode.ts:322-345; CPU semantics ops.ts:87-205), and the per-token
// bookkeeping of Session.decodeStep (session.ts:347-375).
//
// MI355X design: the reference runs RoPE, the cache appends, the scores, the softmax and the
// weighted sum as six dispatches with the scores and weights round-tripping through memory.
// Here one launch does it all: each workgroup owns one kv head and one chunk of positions for
// every query head of that kv group (GQA: the K and V rows are staged once in LDS and reused
// by the group's query heads), and writes a flash-decoding partial (o, max, sum). The
// partials are combined by whoever consumes the attention output (the o projection's input
// stage), so no launch exists just to merge them.
#include <cmath>

#include "eg_attention.hpp"
#include "eg_internal.hpp"

namespace {

constexpr int kThreads = 256;

// IEEE binary16 through the compiler's native _Float16 (round to nearest even on the way in).
using egd::float_to_half;
using egd::half_to_float;
using egd::rope_apply;
using egd::rope_table;

// ---- embedding gather ------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void embed_gather_kernel(const uint32_t* token, const uint32_t* packed,
                                                                const float* scales, const uint32_t* zeros,
                                                                float* out, eg_embedding_dims d, int encoding,
                                                                int bits) {
  const uint32_t s = blockIdx.x;  // one id of the `seq` per workgroup
  const uint32_t id = token[s];
  if (id < d.row_begin || id - d.row_begin >= d.row_count) return;
  const uint32_t row = id - d.row_begin;
  float* dst = out + d.out_offset + (size_t)s * d.hidden;
  for (uint32_t i = threadIdx.x; i < d.hidden; i += blockDim.x) {
    const uint64_t blk = bits >= 16 ? 0 : (uint64_t)row * d.blocks_per_row + i / d.block_size;
    dst[i] = egd::table_value(packed, scales, zeros, (uint64_t)row * d.hidden + i, blk, encoding, bits);
  }
}

// ---- fused decode attention: eg_attention.hpp -------------------------------------------------

using eg_attn::attention_decode_kernel;
using eg_attn::combine_all;
using eg_attn::kMaxCombine;

// ---- combine ---------------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void attention_combine_kernel(const float* partials, float* out,
                                                                     eg_attention_dims d) {
  const uint32_t chunks = d.max_context / d.chunk;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < d.heads * d.head_dim; i += gridDim.x * blockDim.x)
    out[i] = egd::attention_combine_at(partials, i, d.heads, d.head_dim, chunks);
}

__global__ void advance_kernel(uint32_t* position, uint32_t* history, uint32_t* history_length,
                               const uint32_t* token, uint32_t capacity) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    position[0] += 1;
    if (history && history_length) {
      const uint32_t n = history_length[0];
      if (n < capacity) {
        history[n] = token[0];
        history_length[0] = n + 1;
      }
    }
  }
}

int check_attention(eg_context* ctx, const char* op, const eg_attention_dims* d) {
  if (!d) return eg::fail(ctx, EG_ERR_INVALID, "%s: dims is NULL", op);
  if (d->head_dim != 64) return eg::fail(ctx, EG_ERR_INVALID, "%s: head_dim %u (64 is supported)", op, d->head_dim);
  if (d->kv_heads == 0 || d->heads == 0 || d->heads % d->kv_heads != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: %u heads do not group over %u kv heads", op, d->heads, d->kv_heads);
  if (d->heads / d->kv_heads > 8)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: %u query heads per kv head (at most 8)", op, d->heads / d->kv_heads);
  if ((uint64_t)d->kv_heads * 4 > 65535)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u kv heads exceed the grid", op, d->kv_heads);
  if ((uint64_t)d->heads * (d->max_context / d->chunk) > kMaxCombine)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u heads x %u chunks exceed the combine's %u", op, d->heads,
                    d->max_context / d->chunk, kMaxCombine);
  if (d->max_context / d->chunk > egd::kMaxChunks)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u chunks per head exceed %u", op, d->max_context / d->chunk,
                    egd::kMaxChunks);
  if (d->chunk != 64 && d->chunk != 128)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: chunk %u (64 or 128 are supported)", op, d->chunk);
  if (d->max_context == 0 || d->max_context % d->chunk != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: max_context %u is not a positive multiple of %u", op, d->max_context,
                    d->chunk);
  if ((uint64_t)d->max_context / d->chunk * d->kv_heads > 65535)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u chunks exceed the grid", op, d->max_context / d->chunk);
  return EG_OK;
}

// CT: the cache element, uint16_t (f16 bits) or float
template <class CT>
int launch_attention(eg_context* ctx, const char* op, const uint32_t* position, const float* q, const float* k,
                     const float* v, CT* k_cache, CT* v_cache, float* partials, uint32_t* counter, float* out,
                     const eg_attention_dims* dims, const double* rope) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!position || !q || !k || !v || !k_cache || !v_cache || !partials)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  if ((counter == nullptr) != (out == nullptr))
    return eg::fail(ctx, EG_ERR_INVALID, "%s: counter and out go together", op);
  if ((reinterpret_cast<uintptr_t>(k_cache) & 15u) || (reinterpret_cast<uintptr_t>(v_cache) & 15u))
    return eg::fail(ctx, EG_ERR_INVALID, "%s: caches must be 16-byte aligned", op);
  int st = check_attention(ctx, op, dims);
  if (st != EG_OK) return st;
  const double2* cs = reinterpret_cast<const double2*>(rope);
  // chunk 64: two workgroups share a kv group's query heads; chunk 128: four do
  if (dims->chunk == 64) {
    const dim3 grid(dims->max_context / 64, dims->kv_heads * 2);
    hipLaunchKernelGGL((attention_decode_kernel<64, 64, 4, 2, CT>), grid, dim3(kThreads), 0, ctx->stream, position, q,
                       k, v, k_cache, v_cache, partials, counter, out, *dims, cs, eg::stamp_slot(ctx));
  } else {
    const dim3 grid(dims->max_context / 128, dims->kv_heads * 4);
    hipLaunchKernelGGL((attention_decode_kernel<64, 128, 2, 4, CT>), grid, dim3(kThreads), 0, ctx->stream, position,
                       q, k, v, k_cache, v_cache, partials, counter, out, *dims, cs, eg::stamp_slot(ctx));
  }
  return eg::check_launch(ctx, op);
}


// The end of a decode step and the start of the next, in one launch: the step's token settled
// (a greedy step reduces the LM head's argmax partials - the same (value, index) order as the
// argmax finalize: larger value, then lower index; a prompt-fill step takes the next prompt id;
// a sampled step's sampler has already written it), the position advanced, the token appended
// to the sampler's history (Session pushes every produced token, session.ts:437-445) and the
// draw state advanced (Session draws once per decodeStep whatever the temperature,
// session.ts:351; a sampled step's sampler took the draw without advancing the state); then the
// next step's input - the new token's embedding row, dequantized - and the RoPE cos/sin of the
// next position, which every attention launch of that step reads instead of computing. Without
// `advance` (a reset) the token and position already in device memory are used as they are. A
// sampled step whose sampler gave up is counted in t.status and changes nothing else.
//
// The launch is a chain of two memory round trips, each issued all at once: (1) every partial
// (up to kTailPartials per thread), the position and the small state; (2) once the token is known,
// its embedding row (one 32-bit word of codes and its scale per thread) and the next position's
// row of the precomputed RoPE table.
constexpr uint32_t kTailPartials = 8;  // per thread: 2048 partials, the LM head's largest grid

__global__ __launch_bounds__(kThreads) void step_tail_kernel(eg::StepTail t, uint32_t* token, uint32_t* position,
                                                             const uint32_t* packed, const float* scales,
                                                             const uint32_t* zeros, eg_embedding_dims d, int encoding,
                                                             int bits, float* emb, double2* rope, float theta,
                                                             uint64_t* stamp_slot) {
  const egd::WaveStamp stamp(stamp_slot);
  constexpr int D = 64;
  const uint32_t tid = threadIdx.x;
  __shared__ uint32_t next_token, next_pos;
  // (1) everything the token and the position depend on, at once
  const bool greedy = t.advance && t.partials;
  uint64_t pv[kTailPartials];
  if (greedy) {
    const auto pb = egd::buffer(t.partials, t.groups * 8u);  // past the partials: zeros, masked below
#pragma unroll
    for (uint32_t r = 0; r < kTailPartials; r++) pv[r] = egd::load_b64(pb, (tid + r * kThreads) * 8u);
  }
  const uint32_t pos0 = position[0];
  const uint32_t tok0 = token[0];
  const bool aborted = t.sync_abort && *t.sync_abort != 0u;
  const uint32_t src = t.token_src ? *t.token_src : 0u;
  const uint32_t hlen = t.history_length ? *t.history_length : 0u;
  uint32_t greedy_id = 0;  // thread 0: the reduced token of a greedy step
  if (greedy) {
    float bv = -1.0e30f;
    uint32_t bi = 0;
#pragma unroll
    for (uint32_t r = 0; r < kTailPartials; r++) {
      const float v = __uint_as_float((uint32_t)pv[r]);
      const uint32_t i = (uint32_t)(pv[r] >> 32);
      if (tid + r * kThreads < t.groups && egd::better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
    __shared__ float wv[kThreads / 64];
    __shared__ uint32_t wi[kThreads / 64];
    egd::team_argmax<64>(bv, bi);
    if ((tid & 63u) == 0) {
      wv[tid >> 6] = bv;
      wi[tid >> 6] = bi;
    }
    __syncthreads();
    if (tid == 0) {
      for (int w = 1; w < kThreads / 64; w++)
        if (egd::better(wv[w], wi[w], bv, bi)) {
          bv = wv[w];
          bi = wi[w];
        }
      if (!aborted) {  // a failed step leaves the token as it was
        token[0] = bi;
        token[1] = __float_as_uint(bv);
      }
      greedy_id = bi;
    }
  }
  // the persistent layers' counters and abort flag, zeroed for the next launch (read above)
  if (t.sync_counters) {
    for (uint32_t i = tid; i < t.sync_count; i += blockDim.x) t.sync_counters[(size_t)i * t.sync_stride] = 0u;
  }
  if (tid == 0) {
    if (t.sync_abort) *t.sync_abort = 0u;
    // a step whose layers gave up (a persistent wait timed out), or a sampled step whose sampler
    // did (no token: 0xFFFFFFFF), is counted, and nothing moves
    const bool failed =
        t.advance && !t.token_src && (aborted || (!t.partials && tok0 - d.row_begin >= d.row_count));
    if (failed) {
      if (t.status) *t.status += 1u;
      next_token = tok0;  // outside the table: the embedding row below is left as it is
      next_pos = pos0;
    } else if (t.advance) {
      const uint32_t id = t.partials ? greedy_id : t.token_src ? src : tok0;
      if (t.token_src) token[0] = id;
      next_pos = pos0 + 1;
      position[0] = next_pos;
      if (t.history && !t.token_src && hlen < t.history_capacity) {
        t.history[hlen] = id;
        *t.history_length = hlen + 1;
      }
      if (t.rng) (void)egd::mulberry32_next(t.rng);
      next_token = id;
    } else {
      // a reset; with token_src its id becomes the input
      next_token = t.token_src ? src : tok0;
      if (t.token_src) token[0] = next_token;
      next_pos = pos0;
    }
  }
  __syncthreads();
  // (2) the next step's RoPE row and the token's embedding row
  const uint32_t id = next_token, pos = next_pos;
  if (tid < D / 2) {
    if (t.rope_table && pos < t.rope_positions) rope[tid] = t.rope_table[(size_t)pos * (D / 2) + tid];
    else rope_table<D>(rope, tid, pos, theta);
  }
  if (id < d.row_begin || id - d.row_begin >= d.row_count) return;
  const uint32_t row = id - d.row_begin;
  if (bits >= 16) {  // an f16 or f32 table
    for (uint32_t i = tid; i < d.hidden; i += blockDim.x)
      emb[d.out_offset + i] = egd::table_value(packed, scales, zeros, (uint64_t)row * d.hidden + i, 0, encoding, bits);
    return;
  }
  const uint32_t per_word = 32u / (uint32_t)bits;
  const uint32_t mask = (1u << bits) - 1u;
  if (d.block_size % per_word == 0 && (uint64_t)d.hidden * bits % 32 == 0) {
    // one word of codes per thread; its per_word elements share a quant block (and zero-point)
    const uint32_t words = d.hidden / per_word;
    for (uint32_t wd = tid; wd < words; wd += blockDim.x) {
      const uint64_t e0 = (uint64_t)row * d.hidden + (uint64_t)wd * per_word;
      const uint32_t code_word = packed[e0 / per_word];
      const uint32_t blk = row * d.blocks_per_row + wd * per_word / d.block_size;
      const float sc = scales[blk];
      float zero = (float)(1u << (bits - 1));
      uint32_t flip = 0;
      if (encoding == EG_ENC_OFFSET_ZEROS) zero = (float)((zeros[blk / per_word] >> (bits * (blk % per_word))) & mask);
      else flip = 1u << (bits - 1);
      float* out = emb + d.out_offset + wd * per_word;
      for (uint32_t k = 0; k < per_word; k++)
        out[k] = ((float)(((code_word >> (bits * k)) & mask) ^ flip) - zero) * sc;
    }
    return;
  }
  for (uint32_t i = tid; i < d.hidden; i += blockDim.x) {
    const uint64_t e = (uint64_t)row * d.hidden + i;
    uint32_t code = (packed[e / per_word] >> (bits * (uint32_t)(e % per_word))) & mask;
    const uint32_t blk = row * d.blocks_per_row + i / d.block_size;
    float zero;
    if (encoding == EG_ENC_OFFSET_ZEROS) {
      zero = (float)((zeros[blk / per_word] >> (bits * (blk % per_word))) & mask);
    } else {
      code ^= 1u << (bits - 1);
      zero = (float)(1u << (bits - 1));
    }
    emb[d.out_offset + i] = ((float)code - zero) * scales[blk];
  }
}

// The RoPE cos/sin table of positions [0, positions): row p = what rope_table computes at p
// (the same function, so a step reads exactly the values it would compute).
__global__ __launch_bounds__(kThreads) void rope_table_kernel(double2* table, uint32_t positions, float theta) {
  constexpr int D = 64;
  const uint32_t i = blockIdx.x * kThreads + threadIdx.x;
  const uint32_t pos = i / (D / 2);
  if (pos < positions) rope_table<D>(table + (size_t)pos * (D / 2), i % (D / 2), pos, theta);
}

}  // namespace

int eg::attention_decode_rope(eg_context* ctx, const uint32_t* position, const float* q, const float* k,
                              const float* v, uint16_t* k_cache, uint16_t* v_cache, float* partials,
                              const eg_attention_dims* dims, const double* rope) {
  if (!rope) return eg::fail(ctx, EG_ERR_INVALID, "attention_decode: rope table is NULL");
  return launch_attention(ctx, "attention_decode", position, q, k, v, k_cache, v_cache, partials, nullptr, nullptr,
                          dims, rope);
}

int eg::attention_decode_rope(eg_context* ctx, const uint32_t* position, const float* q, const float* k,
                              const float* v, float* k_cache, float* v_cache, float* partials,
                              const eg_attention_dims* dims, const double* rope) {
  if (!rope) return eg::fail(ctx, EG_ERR_INVALID, "attention_decode_f32: rope table is NULL");
  return launch_attention(ctx, "attention_decode_f32", position, q, k, v, k_cache, v_cache, partials, nullptr,
                          nullptr, dims, rope);
}

int eg::launch_rope_table(eg_context* ctx, double* table, uint32_t positions, uint32_t head_dim, float theta) {
  if (head_dim != 64) return eg::fail(ctx, EG_ERR_INVALID, "rope_table: head_dim %u (64 is supported)", head_dim);
  if (positions == 0) return EG_OK;
  const uint64_t n = (uint64_t)positions * (head_dim / 2);
  hipLaunchKernelGGL(rope_table_kernel, dim3((unsigned)((n + kThreads - 1) / kThreads)), dim3(kThreads), 0,
                     ctx->stream, reinterpret_cast<double2*>(table), positions, theta);
  return eg::check_launch(ctx, "rope_table");
}

int eg::launch_step_tail(eg_context* ctx, const StepTail& t, uint32_t* token, uint32_t* position,
                         const uint32_t* packed, const float* scales, const uint32_t* zeros,
                         const eg_embedding_dims* ed, int encoding, int bits, float* emb, double* rope,
                         uint32_t head_dim, float theta) {
  if (head_dim != 64) return eg::fail(ctx, EG_ERR_INVALID, "step_tail: head_dim %u (64 is supported)", head_dim);
  if ((t.history == nullptr) != (t.history_length == nullptr))
    return eg::fail(ctx, EG_ERR_INVALID, "step_tail: history and history_length go together");
  if (t.partials && t.groups > kTailPartials * kThreads)
    return eg::fail(ctx, EG_ERR_RANGE, "step_tail: %u argmax partials, at most %u", t.groups, kTailPartials * kThreads);
  hipLaunchKernelGGL(step_tail_kernel, dim3(1), dim3(kThreads), 0, ctx->stream, t, token, position, packed, scales,
                     encoding == EG_ENC_SIGNED ? nullptr : zeros, *ed, encoding, bits, emb,
                     reinterpret_cast<double2*>(rope), theta, eg::stamp_slot(ctx));
  return eg::check_launch(ctx, "step_tail");
}

extern "C" {

int eg_embed_gather(eg_context* ctx, const uint32_t* token, const uint32_t* packed, const float* scales,
                    const uint32_t* zeros, float* out, const eg_embedding_dims* dims, int encoding, int bits) {
  const char* op = "embed_gather";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  const bool dense = bits == 16 || bits == 32;  // an f16 / f32 table: no scales, zeros or blocks
  if (!token || !packed || !out || !dims || (!dense && !scales))
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  if (bits != 4 && bits != 8 && !dense)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: bits must be 4, 8, 16 (f16 table) or 32 (f32 table), got %d", op, bits);
  if (dims->seq > 0x7FFFFFFFu) return eg::fail(ctx, EG_ERR_RANGE, "%s: seq %u over the grid", op, dims->seq);
  if (!dense) {
    if (encoding != EG_ENC_OFFSET_ZEROS && encoding != EG_ENC_SIGNED)
      return eg::fail(ctx, EG_ERR_INVALID, "%s: unknown encoding %d", op, encoding);
    if (encoding == EG_ENC_OFFSET_ZEROS && !zeros) return eg::fail(ctx, EG_ERR_INVALID, "%s: zeros is NULL", op);
    if (dims->block_size == 0 || dims->hidden % dims->block_size != 0 ||
        dims->blocks_per_row != dims->hidden / dims->block_size)
      return eg::fail(ctx, EG_ERR_INVALID, "%s: hidden %u / block %u / blocksPerRow %u disagree", op, dims->hidden,
                      dims->block_size, dims->blocks_per_row);
  }
  if (dims->seq == 0) return EG_OK;
  hipLaunchKernelGGL(embed_gather_kernel, dim3(dims->seq), dim3(kThreads), 0, ctx->stream, token, packed, scales,
                     dense || encoding == EG_ENC_SIGNED ? nullptr : zeros, out, *dims, encoding, bits);
  return eg::check_launch(ctx, op);
}

int eg_attention_decode(eg_context* ctx, const uint32_t* position, const float* q, const float* k, const float* v,
                        uint16_t* k_cache, uint16_t* v_cache, float* partials, uint32_t* counter, float* out,
                        const eg_attention_dims* dims) {
  return launch_attention(ctx, "attention_decode", position, q, k, v, k_cache, v_cache, partials, counter, out, dims,
                          nullptr);
}

int eg_attention_decode_f32(eg_context* ctx, const uint32_t* position, const float* q, const float* k, const float* v,
                            float* k_cache, float* v_cache, float* partials, uint32_t* counter, float* out,
                            const eg_attention_dims* dims) {
  return launch_attention(ctx, "attention_decode_f32", position, q, k, v, k_cache, v_cache, partials, counter, out,
                          dims, nullptr);
}

int eg_attention_combine(eg_context* ctx, const float* partials, float* out, const eg_attention_dims* dims) {
  const char* op = "attention_combine";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!partials || !out) return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  int st = check_attention(ctx, op, dims);
  if (st != EG_OK) return st;
  const uint32_t n = dims->heads * dims->head_dim;
  hipLaunchKernelGGL(attention_combine_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, ctx->stream,
                     partials, out, *dims);
  return eg::check_launch(ctx, op);
}

int eg_decode_advance(eg_context* ctx, uint32_t* position, uint32_t* history, uint32_t* history_length,
                      const uint32_t* token, uint32_t history_capacity) {
  const char* op = "decode_advance";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!position || !token) return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  if ((history == nullptr) != (history_length == nullptr))
    return eg::fail(ctx, EG_ERR_INVALID, "%s: history and history_length go together", op);
  hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(64), 0, ctx->stream, position, history, history_length, token,
                     history_capacity);
  return eg::check_launch(ctx, op);
}

}  // extern "C"
