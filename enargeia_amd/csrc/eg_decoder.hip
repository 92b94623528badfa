// The decode-step driver: the native counterpart of the reference's DecodeGraph (launch
// order, graph_decode.ts:185-448) and Session.decodeStep (per-token bookkeeping,
// session.ts:347-375), over the ops of this library.
//
// Per token, per layer
//   q|k|v   one batched GEMV, RMSNorm(input_layernorm) fused into its input stage, biases
//   attn    one fused launch: RoPE, f16 cache append, split-K attention partials
//   o       GEMV whose input stage combines the partials; bias = the residual stream
//   gate|up one batched GEMV, RMSNorm(post_attention_layernorm) fused into its input stage
//   down    GEMV whose input stage is SiLU(gate) * up; bias = the residual stream
// then the LM head with the final norm fused and its argmax partials, and one tail launch that
// reduces them to the token, advances the position and prepares the next step: the new token's
// embedding row (layer 0's input) and the RoPE cos/sin of the next position (read by every
// attention launch instead of computed there). Every per-token value (token id, position) lives
// in device memory, so one captured hipGraph replays every step with no host work per launch.
#include <algorithm>
#include <type_traits>
#include <vector>

#include "eg_internal.hpp"

struct eg_decoder {
  eg_context* ctx = nullptr;
  eg_model_desc desc{};
  std::vector<eg_layer_desc> layers;
  eg_attention_dims att{};
  // device buffers
  float* h[2] = {nullptr, nullptr};  // residual stream, ping-pong
  float* q = nullptr;                // [heads * head_dim]
  float* kv = nullptr;               // new k then new v: [2 * kv_heads * head_dim]
  float* gu = nullptr;               // gate then up: [2 * intermediate]
  float* partials = nullptr;         // attention partials
  float* logits = nullptr;           // [vocab]
  float* emb = nullptr;              // [hidden]: the current token's embedding, layer 0's input
  double* rope = nullptr;            // [head_dim / 2] (cos, sin) at the current position
  uint32_t* token = nullptr;         // [2]: next input id, its logit bits
  uint32_t* position = nullptr;      // [1]
  uint16_t* k_cache = nullptr;
  uint16_t* v_cache = nullptr;
  size_t layer_stride = 0;  // cache elements per layer
  std::vector<eg_gemv_plan*> plans;  // per layer: qkv, o, gateup, down
  eg_graph* graph = nullptr;
  std::vector<void*> allocations;
  uint32_t host_position = 0;  // mirrors position[0]: steps are refused once the cache is full
  uint32_t* host_token = nullptr;  // pinned: the per-token readback lands here (no staging copy)
};

namespace {

int alloc(eg_decoder* d, size_t bytes, void** out) {
  int st = eg_buf_alloc(d->ctx, bytes, out);
  if (st == EG_OK) d->allocations.push_back(*out);
  return st;
}

void release(eg_decoder* d) {
  if (d->host_token) (void)hipHostFree(d->host_token);
  if (d->graph) eg_graph_destroy(d->graph);
  for (eg_gemv_plan* p : d->plans) eg_gemv_plan_destroy(d->ctx, p);
  for (void* p : d->allocations) eg_buf_free(d->ctx, p);
  delete d;
}

bool matrix_ok(const eg_quant_matrix& m, int encoding) {
  return m.packed && m.scales && (encoding == EG_ENC_SIGNED || m.zeros);
}

// The step tail (see eg::launch_step_tail): with partials, the end of a step; without, the
// preparation of the state a reset wrote.
int tail(eg_decoder* d, const uint32_t* partials, uint32_t groups) {
  const eg_model_desc& m = d->desc;
  eg_embedding_dims ed{};
  ed.seq = 1;
  ed.hidden = m.hidden;
  ed.row_begin = 0;
  ed.row_count = m.vocab;
  ed.block_size = m.embed_block_size;
  ed.blocks_per_row = m.hidden / m.embed_block_size;
  ed.grid_width = 1;
  return eg::launch_step_tail(d->ctx, partials, groups, d->token, d->position, m.embedding.packed, m.embedding.scales,
                              m.embedding.zeros, &ed, m.embed_encoding, m.embed_bits, d->emb, d->rope, m.head_dim,
                              m.rope_theta);
}

int run_step(eg_decoder* d) {
  eg_context* ctx = d->ctx;
  const eg_model_desc& m = d->desc;
  const eg_quant_matrix& e = m.embedding;
  eg_embedding_dims ed{};
  ed.seq = 1;
  ed.hidden = m.hidden;
  ed.row_begin = 0;
  ed.row_count = m.vocab;
  ed.block_size = m.embed_block_size;
  ed.blocks_per_row = m.hidden / m.embed_block_size;
  ed.grid_width = 1;
  int st = EG_OK;
  for (uint32_t l = 0; l < m.layers; l++) {
    const eg_layer_desc& L = d->layers[l];
    eg_gemv_plan* const* P = &d->plans[4 * (size_t)l];
    eg_gemv_input in{};
    in.kind = EG_INPUT_RMSNORM;
    in.x = l == 0 ? d->emb : d->h[0];
    in.x2 = L.input_norm;
    in.eps = m.rms_eps;
    if ((st = eg_gemv_plan_launch_input(ctx, P[0], &in)) != EG_OK) return st;
    const size_t kvn = (size_t)m.kv_heads * m.head_dim;
    // The combine runs in the o projection's input stage: measured faster here than the
    // attention launch's last-workgroup combine, whose device-scope fences cost more than the
    // per-workgroup recomputation.
    if ((st = eg::attention_decode_rope(ctx, d->position, d->q, d->kv, d->kv + kvn, d->k_cache + l * d->layer_stride,
                                        d->v_cache + l * d->layer_stride, d->partials, &d->att, d->rope)) != EG_OK)
      return st;
    in = eg_gemv_input{};
    in.kind = EG_INPUT_ATTENTION;
    in.x = d->partials;
    in.attention = d->att;
    if ((st = eg_gemv_plan_launch_input(ctx, P[1], &in)) != EG_OK) return st;  // h[1] = h[0] + o(attn)
    in = eg_gemv_input{};
    in.kind = EG_INPUT_RMSNORM;
    in.x = d->h[1];
    in.x2 = L.post_attention_norm;
    in.eps = m.rms_eps;
    if ((st = eg_gemv_plan_launch_input(ctx, P[2], &in)) != EG_OK) return st;
    in = eg_gemv_input{};
    in.kind = EG_INPUT_SILU_MUL;
    in.x = d->gu;
    in.x2 = d->gu + m.intermediate;
    if ((st = eg_gemv_plan_launch_input(ctx, P[3], &in)) != EG_OK) return st;  // h[0] = h[1] + down(...)
  }
  eg_gemv_input in{};
  in.kind = EG_INPUT_RMSNORM;
  in.x = d->h[0];
  in.x2 = m.final_norm;
  in.eps = m.rms_eps;
  eg_embedding_dims hd = ed;
  hd.row_count = m.vocab;
  hd.grid_width = 65535;
  uint32_t groups = 0;
  if ((st = eg::lm_head_argmax_partials(ctx, &in, e.packed, e.scales, e.zeros, d->logits, &hd, m.embed_encoding,
                                        m.embed_bits, &groups)) != EG_OK)
    return st;
  return tail(d, reinterpret_cast<const uint32_t*>(eg::partials(ctx)), groups);
}

}  // namespace

extern "C" {

int eg_decoder_create(eg_context* ctx, const eg_model_desc* desc, eg_decoder** out_decoder) {
  const char* op = "decoder_create";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!desc || !out_decoder || !desc->layer || !desc->final_norm)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  *out_decoder = nullptr;
  const eg_model_desc& m = *desc;
  if (m.layers == 0 || m.hidden == 0 || m.heads == 0 || m.kv_heads == 0 || m.head_dim == 0 || m.intermediate == 0 ||
      m.vocab == 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: a model dimension is zero", op);
  if (m.max_context == 0 || m.max_context % 128 != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: max_context %u is not a positive multiple of 128", op, m.max_context);
  if (m.heads * m.head_dim != m.hidden)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: heads %u x head_dim %u != hidden %u", op, m.heads, m.head_dim, m.hidden);
  if (!matrix_ok(m.embedding, m.embed_encoding) || m.embed_block_size == 0 || m.hidden % m.embed_block_size != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: bad embedding table", op);
  for (uint32_t l = 0; l < m.layers; l++) {
    const eg_layer_desc& L = m.layer[l];
    if (!matrix_ok(L.q, m.encoding) || !matrix_ok(L.k, m.encoding) || !matrix_ok(L.v, m.encoding) ||
        !matrix_ok(L.o, m.encoding) || !matrix_ok(L.gate, m.encoding) || !matrix_ok(L.up, m.encoding) ||
        !matrix_ok(L.down, m.encoding) || !L.input_norm || !L.post_attention_norm)
      return eg::fail(ctx, EG_ERR_INVALID, "%s: layer %u is missing a tensor", op, l);
  }
  eg_decoder* d = new eg_decoder();
  d->ctx = ctx;
  d->desc = m;
  d->layers.assign(m.layer, m.layer + m.layers);
  d->desc.layer = d->layers.data();
  d->att.heads = m.heads;
  d->att.kv_heads = m.kv_heads;
  d->att.head_dim = m.head_dim;
  d->att.max_context = m.max_context;
  d->att.chunk = 128;  // 16 chunks at 2048 x 4 head shares x 2 kv heads: measured best of 64 / 128
  d->att.theta = m.rope_theta;

  const size_t kvn = (size_t)m.kv_heads * m.head_dim;
  const size_t chunks = m.max_context / d->att.chunk;
  d->layer_stride = (size_t)m.max_context * kvn;
  int st = EG_OK;
  void* p = nullptr;
  auto take = [&](size_t bytes, auto** field) {
    if (st != EG_OK) return;
    st = alloc(d, bytes, &p);
    if (st == EG_OK) *field = static_cast<std::remove_reference_t<decltype(**field)>*>(p);
  };
  take(m.hidden * 4, &d->h[0]);
  take(m.hidden * 4, &d->h[1]);
  take(m.hidden * 4, &d->emb);
  take((size_t)m.head_dim / 2 * 2 * sizeof(double), &d->rope);
  take((size_t)m.heads * m.head_dim * 4, &d->q);
  take(2 * kvn * 4, &d->kv);
  take((size_t)2 * m.intermediate * 4, &d->gu);
  take((size_t)m.kv_heads * chunks * (m.heads / std::max(1u, m.kv_heads)) * (m.head_dim + 2) * 4 + 4, &d->partials);
  take((size_t)m.vocab * 4, &d->logits);
  take(8, &d->token);
  take(4, &d->position);
  take(d->layer_stride * m.layers * 2, &d->k_cache);
  take(d->layer_stride * m.layers * 2, &d->v_cache);
  if (st != EG_OK) {
    release(d);
    return st;
  }

  // plans: qkv, o, gate|up, down per layer
  for (uint32_t l = 0; l < m.layers && st == EG_OK; l++) {
    const eg_layer_desc& L = d->layers[l];
    eg_gemv_plan* plan = nullptr;
    eg_gemv_segment qkv[3] = {
        {L.q.packed, L.q.scales, L.q.zeros, L.q_bias, d->q, m.heads * m.head_dim, 0},
        {L.k.packed, L.k.scales, L.k.zeros, L.k_bias, d->kv, (uint32_t)kvn, 0},
        {L.v.packed, L.v.scales, L.v.zeros, L.v_bias, d->kv, (uint32_t)kvn, (uint32_t)kvn},
    };
    st = eg_gemv_plan_create(ctx, m.hidden, m.block_size, m.encoding, m.bits, qkv, 3, &plan);
    if (st != EG_OK) break;
    d->plans.push_back(plan);
    // the residual stream enters layer 0 as the embedding
    eg_gemv_segment o[1] = {{L.o.packed, L.o.scales, L.o.zeros, l == 0 ? d->emb : d->h[0], d->h[1], m.hidden, 0}};
    st = eg_gemv_plan_create(ctx, m.hidden, m.block_size, m.encoding, m.bits, o, 1, &plan);
    if (st != EG_OK) break;
    d->plans.push_back(plan);
    eg_gemv_segment gu[2] = {
        {L.gate.packed, L.gate.scales, L.gate.zeros, nullptr, d->gu, m.intermediate, 0},
        {L.up.packed, L.up.scales, L.up.zeros, nullptr, d->gu, m.intermediate, m.intermediate},
    };
    st = eg_gemv_plan_create(ctx, m.hidden, m.block_size, m.encoding, m.bits, gu, 2, &plan);
    if (st != EG_OK) break;
    d->plans.push_back(plan);
    eg_gemv_segment dn[1] = {{L.down.packed, L.down.scales, L.down.zeros, d->h[1], d->h[0], m.hidden, 0}};
    st = eg_gemv_plan_create(ctx, m.intermediate, m.block_size, m.encoding, m.bits, dn, 1, &plan);
    if (st != EG_OK) break;
    d->plans.push_back(plan);
  }
  if (st == EG_OK) {
    const hipError_t err = hipHostMalloc(reinterpret_cast<void**>(&d->host_token), sizeof(uint32_t), hipHostMallocDefault);
    if (err != hipSuccess) {
      d->host_token = nullptr;
      st = eg::hip_fail(ctx, err, op);
    }
  }
  if (st != EG_OK) {
    // keep the plan error message; release() only frees
    release(d);
    return st;
  }
  *out_decoder = d;
  return eg_decoder_reset(d, 0, 0);
}

int eg_decoder_destroy(eg_decoder* decoder) {
  if (!decoder) return EG_OK;
  eg_sync(decoder->ctx);
  release(decoder);
  return EG_OK;
}

int eg_decoder_buffers_get(eg_decoder* d, eg_decoder_buffers* out) {
  if (!d || !out) return eg::fail(d ? d->ctx : nullptr, EG_ERR_INVALID, "decoder_buffers: NULL argument");
  out->k_cache = d->k_cache;
  out->v_cache = d->v_cache;
  out->logits = d->logits;
  out->hidden = d->h[0];
  out->token = d->token;
  out->position = d->position;
  return EG_OK;
}

int eg_decoder_reset(eg_decoder* d, uint32_t position, uint32_t token) {
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "decoder_reset: decoder is NULL");
  // a reset writes and synchronises: nothing of it may land in a caller's capture
  if (d->ctx->capturing) return eg::fail(d->ctx, EG_ERR_STATE, "decoder_reset: a graph capture is in progress");
  if (position >= d->desc.max_context)
    return eg::fail(d->ctx, EG_ERR_RANGE, "decoder_reset: position %u past the context of %u", position,
                    d->desc.max_context);
  if (token >= d->desc.vocab)
    return eg::fail(d->ctx, EG_ERR_INVALID, "decoder_reset: token %u outside the vocabulary", token);
  const uint32_t tok[2] = {token, 0};
  int st = eg_buf_write(d->ctx, d->token, 0, tok, sizeof(tok));
  if (st == EG_OK) st = eg_buf_write(d->ctx, d->position, 0, &position, 4);
  if (st == EG_OK) st = tail(d, nullptr, 0);  // this token's embedding, this position's RoPE table
  if (st == EG_OK) st = eg_sync(d->ctx);      // the host values are stack locals
  if (st == EG_OK) d->host_position = position;
  return st;
}

int eg_decoder_step(eg_decoder* d, uint32_t* token_out) {
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "decoder_step: decoder is NULL");
  // Refused before anything is enqueued: launches recorded into a caller's capture would not
  // run now, yet the host's position would advance and no longer match the device's.
  if (d->ctx->capturing) return eg::fail(d->ctx, EG_ERR_STATE, "decoder_step: a graph capture is in progress");
  // kvcache.ts:118-127: a full context is an error, not a silent overwrite
  if (d->host_position >= d->desc.max_context)
    return eg::fail(d->ctx, EG_ERR_RANGE, "decoder_step: context of %u positions exhausted", d->desc.max_context);
  int st = d->graph ? eg_graph_launch(d->ctx, d->graph) : run_step(d);
  if (st == EG_OK) d->host_position++;
  if (st == EG_OK && token_out) {
    // the one readback per token, into pinned memory: a direct copy, no staging through a
    // bounce buffer as a pageable destination would need
    hipError_t err = hipMemcpyAsync(d->host_token, d->token, sizeof(uint32_t), hipMemcpyDeviceToHost, d->ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(d->ctx->stream);
    if (err != hipSuccess) return eg::hip_fail(d->ctx, err, "decoder_step");
    *token_out = *d->host_token;
  }
  return st;
}

int eg_decoder_capture(eg_decoder* d) {
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "decoder_capture: decoder is NULL");
  if (d->graph) {
    eg_graph_destroy(d->graph);
    d->graph = nullptr;
  }
  int st = eg_graph_begin(d->ctx);
  if (st != EG_OK) return st;
  const int run = run_step(d);
  eg_graph* g = nullptr;
  st = eg_graph_end(d->ctx, &g);
  if (run != EG_OK) {
    if (g) eg_graph_destroy(g);
    return run;
  }
  if (st != EG_OK) return st;
  d->graph = g;
  return EG_OK;
}

}  // extern "C"
