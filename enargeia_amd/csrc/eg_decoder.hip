// The decode-step driver: the native counterpart of the reference's DecodeGraph (launch
// order, graph_decode.ts:185-448) and Session.decodeStep (per-token bookkeeping,
// session.ts:347-375), over the ops of this library.
//
// Per token, per layer
//   q|k|v   one batched GEMV, RMSNorm(input_layernorm) fused into its input stage, biases
//   attn    one fused launch: RoPE, f16 cache append, split-K attention partials
//   o       GEMV whose input stage combines the partials; bias = the residual stream
//   gate|up one GEMV launch over both matrices, RMSNorm(post_attention_layernorm) fused into its
//           input stage, each row pair stored as SiLU(gate) * up
//   down    GEMV on that vector; bias = the residual stream
// then the LM head with the final norm fused and one tail launch that settles the token, advances
// the position and prepares the next step: the new token's embedding row (layer 0's input) and
// the RoPE cos/sin of the next position (read by every attention launch instead of computed
// there). Greedy steps (GREEDY, sample.ts:33) take the LM head's fused argmax partials, which the
// tail reduces; other sampling parameters run the sampler (penalty, temperature, top-p, draw;
// sample.wgsl) between the head and the tail, the decoder's sample step
// (graph_decode.ts:382-385) - an int8 head stores the penalized logits and hands the sampler
// per-workgroup (max, index, normaliser) partials, so the sampler starts at its radix levels. Every per-token value (token id, position, the sampler's
// parameters, its history and the mulberry32 draw state) lives in device memory, so one captured
// hipGraph replays every step with no host work per launch.
#include <algorithm>
#include <cmath>
#include <cstring>
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
  double* rope_table = nullptr;      // [max_context][head_dim / 2] (cos, sin), computed once
  // [4]: next input id, its logit bits (greedy), sampled steps whose sampler gave up (counted by
  // the step tail until the host reads and clears it), unused
  uint32_t* token = nullptr;
  uint32_t* position = nullptr;      // [1]
  // the sample step's state (DecodeGraph.history / setPosition's uniform, graph_decode.ts:150,
  // 398-406; Session's random source, session.ts:75-83)
  uint32_t* history = nullptr;       // [max_context]: Session.tokens, appended by every step
  eg_sample_dims* sp = nullptr;      // {vocab, history_length, temperature, top_p, penalty, random}
  uint32_t* rng = nullptr;           // [1]: mulberry32 state, one draw per step
  eg_sampling_params sampling{0.f, 1.f, 1.f};  // host copy of sp's parameters
  eg_gemv_plan* head_plan = nullptr; // an int4 LM head storing logits for the sampler (vocab % 8 == 0)
  // Host-driven steps (DecodeGraph.setPosition, graph_decode.ts:398-406): the host writes the
  // position, the history length and the draw before each step, and each step starts from the
  // token in `token` (its embedding and RoPE table prepared first), as the reference's Session
  // drives its DecodeGraph. Otherwise steps chain on the device and the draw is taken there.
  bool host_driven = false;
  bool graph_sampled = false, graph_host_driven = false;  // the mode the graph was captured in
  uint32_t* host_staging = nullptr;  // pinned [max_context]: prompt ids on their way to `history`
  // the prompt chain (ForwardGraph, graph.ts:380-567) over chunks of up to `chunk` rows
  // Rows per prompt chunk. The reference runs 256 (DEFAULT_PREFILL_CHUNK, session.ts:30; a
  // browser's buffer limits); here the buffers hold up to kMaxChunk rows (79 KB of activations a
  // row at the Qwen2.5-0.5B shape) and a whole prompt of that length is one chunk, so the
  // projections run as GEMMs of up to 2048 rows, which fill the device, instead of 256.
  uint32_t chunk = 0;
  uint32_t chunk_capacity = 0;
  float *ph[2] = {nullptr, nullptr}; // [chunk][hidden] residual stream, ping-pong
  float* pxn = nullptr;              // [chunk][hidden] normed rows
  float *pq = nullptr, *pk = nullptr, *pv = nullptr;  // projections [chunk][hidden | kv | kv]
  float* pqr = nullptr;              // [chunk][hidden] rotated, scaled q
  float* patt = nullptr;             // [chunk][hidden] attention output
  float* pgu = nullptr;              // [chunk][2 * intermediate] gate | up
  float* pa = nullptr;               // [chunk][intermediate] silu(gate) * up
  // [layers][max_context][kv_heads][head_dim] of f16 bits, or of f32 (cache_f32: the
  // reference's f32 cache variant, SessionOptions.cacheDType)
  void* k_cache = nullptr;
  void* v_cache = nullptr;
  bool cache_f32 = false;
  size_t layer_stride = 0;  // cache elements per layer
  std::vector<eg_gemv_plan*> plans;  // per layer: qkv, o, gate|up (a SwiGLU pair if swiglu), down
  // the layers of a step as one persistent launch (eg_layers.hip), where the shapes and the
  // device allow; NULL: one launch per op
  eg_layers* layers_kernel = nullptr;
  bool swiglu = false;               // gate|up stores silu(gate) * up in gu[0, intermediate)
  eg_graph* graph = nullptr;
  std::vector<void*> allocations;
  uint32_t host_position = 0;  // mirrors position[0]: steps are refused once the cache is full
  uint32_t* host_token = nullptr;  // pinned [3]: the per-token readback lands here (no staging copy)
};

namespace {

// Layer l's rows of a cache (CT: uint16_t for f16 bits, float for an f32 cache).
template <class CT>
CT* layer_cache(const eg_decoder* d, void* base, uint32_t l) {
  return static_cast<CT*>(base) + (size_t)l * d->layer_stride;
}

constexpr uint32_t kMaxChunk = 2048;

int alloc(eg_decoder* d, size_t bytes, void** out) {
  int st = eg_buf_alloc(d->ctx, bytes, out);
  if (st == EG_OK) d->allocations.push_back(*out);
  return st;
}

void release(eg_decoder* d) {
  if (d->host_token) (void)hipHostFree(d->host_token);
  if (d->host_staging) (void)hipHostFree(d->host_staging);
  if (d->graph) eg_graph_destroy(d->graph);
  if (d->head_plan) eg_gemv_plan_destroy(d->ctx, d->head_plan);
  eg::layers_destroy(d->ctx, d->layers_kernel);
  for (eg_gemv_plan* p : d->plans) eg_gemv_plan_destroy(d->ctx, p);
  for (void* p : d->allocations) eg_buf_free(d->ctx, p);
  delete d;
}

bool matrix_ok(const eg_quant_matrix& m, int encoding) {
  return m.packed && m.scales && (encoding == EG_ENC_SIGNED || m.zeros);
}

// Greedy steps fuse the argmax into the LM head; anything else (a temperature, or a penalty,
// which the reference applies before its greedy argmax too) runs the sampler.
bool sampled_mode(const eg_sampling_params& s) { return !(s.temperature <= 0.f && s.repetition_penalty == 1.f); }

eg_embedding_dims embedding_dims_of(const eg_model_desc& m) {
  eg_embedding_dims ed{};
  ed.seq = 1;
  ed.hidden = m.hidden;
  ed.row_begin = 0;
  ed.row_count = m.vocab;
  // an f16 / f32 table has no blocks: the fields describe one block per row
  ed.block_size = m.embed_bits >= 16 ? m.hidden : m.embed_block_size;
  ed.blocks_per_row = m.hidden / ed.block_size;
  ed.grid_width = 1;
  return ed;
}

// The step tail (see eg::launch_step_tail).
int tail(eg_decoder* d, eg::StepTail t) {
  const eg_model_desc& m = d->desc;
  const eg_embedding_dims ed = embedding_dims_of(m);
  t.rope_table = reinterpret_cast<const double2*>(d->rope_table);
  t.rope_positions = m.max_context;
  if (d->layers_kernel)
    eg::layers_sync_words(d->layers_kernel, &t.sync_counters, &t.sync_count, &t.sync_stride, &t.sync_abort);
  return eg::launch_step_tail(d->ctx, t, d->token, d->position, m.embedding.packed, m.embedding.scales,
                              m.embedding.zeros, &ed, m.embed_encoding, m.embed_bits, d->emb, d->rope, m.head_dim,
                              m.rope_theta);
}

eg::StepTail advancing_tail(eg_decoder* d) {
  eg::StepTail t;
  t.advance = true;
  t.history = d->history;
  t.history_length = &d->sp->history_length;
  t.history_capacity = d->desc.max_context;
  return t;
}

// The input of each per-layer plan (qkv, o, gate|up, down) - the per-op launches' and the
// persistent kernel's.
void layer_inputs(const eg_decoder* d, uint32_t l, eg_gemv_input in[4]) {
  const eg_model_desc& m = d->desc;
  const eg_layer_desc& L = d->layers[l];
  for (int j = 0; j < 4; j++) in[j] = eg_gemv_input{};
  in[0].kind = EG_INPUT_RMSNORM;
  in[0].x = l == 0 ? d->emb : d->h[0];
  in[0].x2 = L.input_norm;
  in[0].eps = m.rms_eps;
  in[1].kind = EG_INPUT_ATTENTION;
  in[1].x = d->partials;
  in[1].attention = d->att;
  in[2].kind = EG_INPUT_RMSNORM;
  in[2].x = d->h[1];
  in[2].x2 = L.post_attention_norm;
  in[2].eps = m.rms_eps;
  in[3].kind = d->swiglu ? EG_INPUT_VECTOR : EG_INPUT_SILU_MUL;
  in[3].x = d->gu;
  in[3].x2 = d->swiglu ? nullptr : d->gu + m.intermediate;
}

// The 24 layers of a step on the token whose embedding is in d->emb at position[0].
int run_layers(eg_decoder* d) {
  eg_context* ctx = d->ctx;
  const eg_model_desc& m = d->desc;
  if (d->layers_kernel) return eg::layers_launch(ctx, d->layers_kernel);
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
    st = d->cache_f32 ? eg::attention_decode_rope(ctx, d->position, d->q, d->kv, d->kv + kvn, layer_cache<float>(d, d->k_cache, l),
                                                  layer_cache<float>(d, d->v_cache, l), d->partials, &d->att, d->rope)
                      : eg::attention_decode_rope(ctx, d->position, d->q, d->kv, d->kv + kvn,
                                                  layer_cache<uint16_t>(d, d->k_cache, l),
                                                  layer_cache<uint16_t>(d, d->v_cache, l), d->partials, &d->att, d->rope);
    if (st != EG_OK) return st;
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
    in.kind = d->swiglu ? EG_INPUT_VECTOR : EG_INPUT_SILU_MUL;
    in.x = d->gu;
    in.x2 = d->swiglu ? nullptr : d->gu + m.intermediate;
    if ((st = eg_gemv_plan_launch_input(ctx, P[3], &in)) != EG_OK) return st;  // h[0] = h[1] + down(...)
  }
  return st;
}

// The LM head on `hidden` (the last layer's output row) with the final norm fused, then greedy
// (fused argmax partials reduced in the tail, which also advances the draw state) or sampled
// (logits stored, the sampler draws and writes the token, the tail only settles it).
int run_head(eg_decoder* d, bool sampled, const float* hidden) {
  uint32_t* const rng = d->host_driven ? nullptr : d->rng;  // host-driven: the host's draw is in sp
  eg_context* ctx = d->ctx;
  const eg_model_desc& m = d->desc;
  const eg_quant_matrix& e = m.embedding;
  int st = EG_OK;
  eg_gemv_input in{};
  in.kind = EG_INPUT_RMSNORM;
  in.x = hidden;
  in.x2 = m.final_norm;
  in.eps = m.rms_eps;
  eg::StepTail t = advancing_tail(d);
  t.status = d->token + 2;  // a step that gives up is counted here and moves nothing
  if (!sampled) {
    eg_embedding_dims hd = embedding_dims_of(m);
    hd.grid_width = 65535;
    if ((st = eg::lm_head_argmax_partials(ctx, &in, e.packed, e.scales, e.zeros, d->logits, &hd, m.embed_encoding,
                                          m.embed_bits, &t.groups)) != EG_OK)
      return st;
    t.partials = reinterpret_cast<const uint32_t*>(eg::partials(ctx));
    t.rng = rng;
    return tail(d, t);
  }
  if (m.embed_bits == 8) {
    // the int8 head applies the penalty and leaves the sampler its per-workgroup (max, index,
    // normaliser) partials; the sampler takes the draw, the tail advances the state once the
    // step has its token; a sampler that gives up leaves 0xFFFFFFFF, which the tail counts in
    // token[2], changing nothing
    eg_embedding_dims hd = embedding_dims_of(m);
    if ((st = eg::lm_head_sample_device(ctx, &in, e.packed, e.scales, e.zeros, d->logits, &hd, m.embed_encoding,
                                        m.embed_bits, d->history, d->token, d->sp, rng, nullptr)) != EG_OK)
      return st;
    t.rng = rng;
    return tail(d, t);
  }
  if (d->head_plan) {
    st = eg_gemv_plan_launch_input(ctx, d->head_plan, &in);
  } else {
    eg_embedding_dims hd = embedding_dims_of(m);
    hd.grid_width = 65535;
    uint32_t groups = 0;  // the partials are not used
    st = eg::lm_head_argmax_partials(ctx, &in, e.packed, e.scales, e.zeros, d->logits, &hd, m.embed_encoding,
                                     m.embed_bits, &groups);
  }
  if (st != EG_OK) return st;
  // the sampler takes the draw, the tail advances the state once the step has its token; a
  // sampler that gives up leaves 0xFFFFFFFF, which the tail counts in token[2], changing nothing
  if ((st = eg::launch_sample_device(ctx, d->logits, d->history, d->token, m.vocab, d->sp, rng, nullptr)) != EG_OK)
    return st;
  t.rng = rng;
  return tail(d, t);
}

// A whole decode step: the layers on the current token, then the head.
int run_step(eg_decoder* d, bool sampled) {
  // host-driven: the input is whatever token[0] and position[0] the host wrote
  int st = d->host_driven ? tail(d, eg::StepTail{}) : EG_OK;
  if (st == EG_OK) st = run_layers(d);
  return st != EG_OK ? st : run_head(d, sampled, d->h[0]);
}

// One chunk of the prompt (ForwardGraph.encode over `count` rows at positions begin..,
// graph.ts:380-500, without its tail): the rows' embeddings, then per layer RMSNorm, the q / k / v
// projections with their biases on the matrix cores, RoPE + cache append + causal attention
// (eg_attention_prefill), the o projection with the residual added in its epilogue, RMSNorm,
// gate and up, SiLU(gate) * up, and the down projection with the residual. The chunk's last
// hidden row ends in ph[0].
int run_prefill_chunk(eg_decoder* d, const uint32_t* ids, uint32_t begin, uint32_t count) {
  eg_context* ctx = d->ctx;
  const eg_model_desc& m = d->desc;
  const uint32_t H = m.hidden, I = m.intermediate, kvn = m.kv_heads * m.head_dim;
  int st = eg::embed_rows(ctx, ids, count, m.embedding.packed, m.embedding.scales, m.embedding.zeros, H,
                          m.embed_block_size, m.embed_encoding, m.embed_bits, d->ph[0]);
  auto gemm = [&](const float* x, const eg_quant_matrix& w, const float* bias, const float* residual, float* out,
                  uint32_t n, uint32_t k, uint32_t out_stride, uint32_t out_offset, bool x_bf16) {
    if (st != EG_OK) return;
    eg_matmul_q4_dims dm{};
    dm.m = count;
    dm.n = n;
    dm.k = k;
    dm.use_bias = bias != nullptr;
    dm.block_size = m.block_size;
    dm.blocks_per_row = k / m.block_size;
    dm.out_stride = out_stride;
    dm.out_offset = out_offset;
    st = eg::prefill_gemm(ctx, x, w.packed, w.scales, w.zeros, bias, residual, out, &dm, m.encoding, m.bits, x_bf16);
  };
  for (uint32_t l = 0; l < m.layers && st == EG_OK; l++) {
    const eg_layer_desc& L = d->layers[l];
    // RMSNorm, then q, k and v in one launch (they share the normed rows; the norm folded in)
    const eg::PrefillMatrix qkv[3] = {
        {L.q.packed, L.q.scales, L.q.zeros, L.q_bias, nullptr, d->pq, H, H, 0},
        {L.k.packed, L.k.scales, L.k.zeros, L.k_bias, nullptr, d->pk, kvn, kvn, 0},
        {L.v.packed, L.v.scales, L.v.zeros, L.v_bias, nullptr, d->pv, kvn, kvn, 0}};
    eg_attention_prefill_dims ad{count, begin + count, begin, m.heads, m.kv_heads, m.head_dim, m.max_context,
                                 m.rope_theta};
    uint16_t* kc = layer_cache<uint16_t>(d, d->k_cache, l);
    uint16_t* vc = layer_cache<uint16_t>(d, d->v_cache, l);
    // RoPE and the cache append in the q|k|v launch's epilogue where it can take them (then the
    // attention launches alone), else rope_append's launch before the attention; an f32 cache
    // takes the separate launches (the epilogue stores f16 rows)
    bool fused = false;
    st = eg::check_attention_prefill(ctx, "attention_prefill", &ad);
    if (st == EG_OK && m.head_dim == 64 && !d->cache_f32) {
      const eg::PrefillRope rope{reinterpret_cast<const double2*>(d->rope_table), d->pqr, kc, vc, begin, m.heads,
                                 m.kv_heads};
      st = eg::prefill_qkv_rope(ctx, d->ph[0], count, H, m.block_size, m.encoding, m.bits, qkv, L.input_norm,
                                m.rms_eps, d->pxn, rope, &fused);
    }
    if (st == EG_OK && !fused)
      st = eg::prefill_gemm_multi(ctx, d->ph[0], count, H, m.block_size, m.encoding, m.bits, qkv, 3, L.input_norm,
                                  m.rms_eps, d->pxn);
    if (st != EG_OK) break;
    // the o and down projections take their x as bf16 rows where they stage them (the attention
    // and the SwiGLU pair store them rounded exactly as the staging would)
    const bool xb_o = fused && ctx->prefill_xb16 && eg::prefill_chunked(count, H, H, m.block_size, m.bits, d->patt, L.o.packed);
    const bool xb_down = ctx->prefill_xb16 && eg::prefill_chunked(count, H, I, m.block_size, m.bits, d->pa, L.down.packed);
    if (fused) st = eg::attention_prefill_run(ctx, d->pqr, kc, vc, d->patt, ad, xb_o);
    else if (d->cache_f32)
      st = eg_attention_prefill_f32(ctx, d->pq, d->pk, d->pv, layer_cache<float>(d, d->k_cache, l),
                                    layer_cache<float>(d, d->v_cache, l), d->pqr, d->patt, &ad);
    else st = eg_attention_prefill(ctx, d->pq, d->pk, d->pv, kc, vc, d->pqr, d->patt, &ad);
    gemm(d->patt, L.o, nullptr, d->ph[0], d->ph[1], H, H, H, 0, xb_o);  // ph1 = ph0 + o(attn)
    // RMSNorm and SiLU(gate) * up in one launch of paired gate|up tiles (pgu: the two-launch
    // form's rows)
    const eg::PrefillMatrix gate{L.gate.packed, L.gate.scales, L.gate.zeros, nullptr, nullptr, d->pa, I, I, 0};
    const eg::PrefillMatrix up{L.up.packed, L.up.scales, L.up.zeros, nullptr, nullptr, d->pa, I, I, 0};
    if (st == EG_OK)
      st = eg::prefill_gemm_swiglu(ctx, d->ph[1], count, H, m.block_size, m.encoding, m.bits, gate, up, d->pa, d->pgu,
                                   L.post_attention_norm, m.rms_eps, d->pxn, xb_down);
    gemm(d->pa, L.down, nullptr, d->ph[1], d->ph[0], H, I, H, 0, xb_down);  // ph0 = ph1 + down(...)
  }
  return st;
}

// Writes `count` u32 from host memory to device memory through the pinned staging buffer and
// waits for the copy (the staging buffer is reused by the next call).
int write_ids(eg_decoder* d, uint32_t* dst, const uint32_t* host, uint32_t count) {
  if (count == 0) return EG_OK;
  std::memcpy(d->host_staging, host, (size_t)count * 4);
  hipError_t err = hipMemcpyAsync(dst, d->host_staging, (size_t)count * 4, hipMemcpyHostToDevice, d->ctx->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(d->ctx->stream);
  return err == hipSuccess ? EG_OK : eg::hip_fail(d->ctx, err, "decoder: upload");
}

// The one readback per step: the token the last step produced and the count of sampled steps
// whose sampler gave up (token[0..2], one copy into pinned memory: no staging through a bounce
// buffer as a pageable destination would need). A nonzero count is an error: it is cleared, the
// host's position mirror steps back by it (those steps moved nothing on the device) and the
// caller's next step redoes the step.
int read_token(eg_decoder* d, uint32_t* token_out, const char* op) {
  hipError_t err = hipMemcpyAsync(d->host_token, d->token, 3 * sizeof(uint32_t), hipMemcpyDeviceToHost, d->ctx->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(d->ctx->stream);
  if (err != hipSuccess) return eg::hip_fail(d->ctx, err, op);
  const uint32_t failed = d->host_token[2];
  if (failed != 0) {
    d->host_position -= std::min(failed, d->host_position);
    const uint32_t zero = 0;
    int st = write_ids(d, d->token + 2, &zero, 1);
    if (st != EG_OK) return st;
    return eg::fail(d->ctx, EG_ERR_DEVICE,
                    "%s: %u step(s) gave up: a bounded wait timed out (not every workgroup was resident at once); "
                    "the position, history and draw state are as before those steps, and the next step redoes the "
                    "step",
                    op, failed);
  }
  *token_out = d->host_token[0];
  return EG_OK;
}

int capture(eg_decoder* d);

// Switches between host-driven and device-chained steps; a graph captured in the other mode is
// captured again.
int set_host_driven(eg_decoder* d, bool host) {
  if (d->host_driven == host) return EG_OK;
  d->host_driven = host;
  return d->graph ? capture(d) : EG_OK;
}

int capture(eg_decoder* d) {
  if (d->graph) {
    eg_graph_destroy(d->graph);
    d->graph = nullptr;
  }
  int st = eg_graph_begin(d->ctx);
  if (st != EG_OK) return st;
  const bool sampled = sampled_mode(d->sampling);
  const int run = run_step(d, sampled);
  eg_graph* g = nullptr;
  st = eg_graph_end(d->ctx, &g);
  if (run != EG_OK) {
    if (g) eg_graph_destroy(g);
    return run;
  }
  if (st != EG_OK) return st;
  d->graph = g;
  d->graph_sampled = sampled;
  d->graph_host_driven = d->host_driven;
  return EG_OK;
}

}  // namespace

extern "C" {

int eg_decoder_create(eg_context* ctx, const eg_model_desc* desc, eg_decoder** out_decoder) {
  return eg_decoder_create_cache(ctx, desc, EG_CACHE_F16, out_decoder);
}

int eg_decoder_create_cache(eg_context* ctx, const eg_model_desc* desc, int cache_dtype, eg_decoder** out_decoder) {
  const char* op = "decoder_create";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!desc || !out_decoder || !desc->layer || !desc->final_norm)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  *out_decoder = nullptr;
  if (cache_dtype != EG_CACHE_F16 && cache_dtype != EG_CACHE_F32)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: cache dtype %d (EG_CACHE_F16 or EG_CACHE_F32)", op, cache_dtype);
  const eg_model_desc& m = *desc;
  if (m.layers == 0 || m.hidden == 0 || m.heads == 0 || m.kv_heads == 0 || m.head_dim == 0 || m.intermediate == 0 ||
      m.vocab == 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: a model dimension is zero", op);
  if (m.max_context == 0 || m.max_context % 128 != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: max_context %u is not a positive multiple of 128", op, m.max_context);
  if (m.heads * m.head_dim != m.hidden)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: heads %u x head_dim %u != hidden %u", op, m.heads, m.head_dim, m.hidden);
  // the tied table: codes of 4 or 8 bits with their scales (and zero-points), or an f16 (bits
  // 16) / f32 (bits 32) table as it is (embedding_variants.ts:26-74)
  const bool dense_table = m.embed_bits == 16 || m.embed_bits == 32;
  if (m.embed_bits != 4 && m.embed_bits != 8 && !dense_table)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: embedding bits %d (4, 8, 16 or 32)", op, m.embed_bits);
  if (dense_table ? !m.embedding.packed
                  : !matrix_ok(m.embedding, m.embed_encoding) || m.embed_block_size == 0 ||
                        m.hidden % m.embed_block_size != 0)
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
  d->cache_f32 = cache_dtype == EG_CACHE_F32;
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
  take((size_t)m.max_context * (m.head_dim / 2) * 2 * sizeof(double), &d->rope_table);
  take((size_t)m.heads * m.head_dim * 4, &d->q);
  take(2 * kvn * 4, &d->kv);
  take((size_t)2 * m.intermediate * 4, &d->gu);
  take((size_t)m.kv_heads * chunks * (m.heads / std::max(1u, m.kv_heads)) * (m.head_dim + 2) * 4 + 4, &d->partials);
  take((size_t)m.vocab * 4, &d->logits);
  take(16, &d->token);
  take(4, &d->position);
  take((size_t)m.max_context * 4, &d->history);
  d->chunk_capacity = d->chunk = std::min<uint32_t>(kMaxChunk, m.max_context);
  const size_t rows = d->chunk;
  take(rows * m.hidden * 4, &d->ph[0]);
  take(rows * m.hidden * 4, &d->ph[1]);
  take(rows * m.hidden * 4, &d->pxn);
  take(rows * m.hidden * 4, &d->pq);
  take(rows * kvn * 4, &d->pk);
  take(rows * kvn * 4, &d->pv);
  take(rows * m.hidden * 4, &d->pqr);
  take(rows * m.hidden * 4, &d->patt);
  take(rows * 2 * m.intermediate * 4, &d->pgu);
  take(rows * m.intermediate * 4, &d->pa);
  take(sizeof(eg_sample_dims), &d->sp);
  take(4, &d->rng);
  const size_t cache_bytes = d->layer_stride * m.layers * (d->cache_f32 ? 4 : 2);
  if (st == EG_OK) st = alloc(d, cache_bytes, &d->k_cache);
  if (st == EG_OK) st = alloc(d, cache_bytes, &d->v_cache);
  if (st == EG_OK) st = eg::launch_rope_table(ctx, d->rope_table, m.max_context, m.head_dim, m.rope_theta);
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
    // int4 projections: one launch stores silu(gate) * up (the pair), so the down projection
    // reads a plain vector; otherwise gate and up are stored and down's input stage applies
    // SiLU * up. The choice is the same for every layer (same shapes).
    if (l == 0) d->swiglu = m.bits == 4;
    if (d->swiglu) {
      st = eg_gemv_swiglu_plan_create(ctx, m.hidden, m.block_size, m.encoding, m.bits, gu, &plan);
      if (st != EG_OK && l == 0) d->swiglu = false;  // no pair kernel for this shape
    }
    if (!d->swiglu) st = eg_gemv_plan_create(ctx, m.hidden, m.block_size, m.encoding, m.bits, gu, 2, &plan);
    if (st != EG_OK) break;
    d->plans.push_back(plan);
    eg_gemv_segment dn[1] = {{L.down.packed, L.down.scales, L.down.zeros, d->h[1], d->h[0], m.hidden, 0}};
    st = eg_gemv_plan_create(ctx, m.intermediate, m.block_size, m.encoding, m.bits, dn, 1, &plan);
    if (st != EG_OK) break;
    d->plans.push_back(plan);
  }
  // an int4 LM head storing logits for the sampler: a one-matrix plan with the final norm as its
  // input stage (plans need rows in multiples of 8; other vocabularies use the fused-argmax head
  // and ignore its partials; an int8 head leaves the sampler its partials instead)
  if (st == EG_OK && m.vocab % 8 == 0 && m.embed_bits == 4) {
    eg_gemv_segment head[1] = {{m.embedding.packed, m.embedding.scales, m.embedding.zeros, nullptr, d->logits, m.vocab, 0}};
    st = eg_gemv_plan_create(ctx, m.hidden, m.embed_block_size, m.embed_encoding, m.embed_bits, head, 1, &d->head_plan);
  }
  // (the persistent kernel's attention phase reads an f16 cache)
  if (st == EG_OK && ctx->decode_persistent && !d->cache_f32) {
    std::vector<eg::LayerPlans> lp(m.layers);
    for (uint32_t l = 0; l < m.layers; l++) {
      for (int j = 0; j < 4; j++) lp[l].plan[j] = d->plans[4 * (size_t)l + j];
      layer_inputs(d, l, lp[l].input);
    }
    eg::LayersDesc ld{};
    ld.layers = m.layers;
    ld.plans = lp.data();
    ld.att = d->att;
    ld.position = d->position;
    ld.rope = d->rope;
    ld.q = d->q;
    ld.k = d->kv;
    ld.v = d->kv + kvn;
    ld.partials = d->partials;
    ld.k_cache = static_cast<uint16_t*>(d->k_cache);
    ld.v_cache = static_cast<uint16_t*>(d->v_cache);
    ld.layer_stride = d->layer_stride;
    st = eg::layers_create(ctx, ld, &d->layers_kernel);
  }
  if (st == EG_OK) {
    hipError_t err = hipHostMalloc(reinterpret_cast<void**>(&d->host_token), 4 * sizeof(uint32_t), hipHostMallocDefault);
    if (err != hipSuccess) d->host_token = nullptr;
    if (err == hipSuccess) {
      err = hipHostMalloc(reinterpret_cast<void**>(&d->host_staging), (size_t)m.max_context * 4, hipHostMallocDefault);
      if (err != hipSuccess) d->host_staging = nullptr;
    }
    if (err != hipSuccess) st = eg::hip_fail(ctx, err, op);
  }
  if (st == EG_OK) {
    // GREEDY sampling (sample.ts:33), an empty history, the session's default seed 0x5eed
    // (session.ts:125)
    eg_sample_dims sp{};
    sp.vocab = m.vocab;
    sp.temperature = d->sampling.temperature;
    sp.top_p = d->sampling.top_p;
    sp.repetition_penalty = d->sampling.repetition_penalty;
    static_assert(sizeof(sp) % 4 == 0, "u32 words");
    st = write_ids(d, reinterpret_cast<uint32_t*>(d->sp), reinterpret_cast<const uint32_t*>(&sp), sizeof(sp) / 4);
    const uint32_t seed = 0x5eed;
    if (st == EG_OK) st = write_ids(d, d->rng, &seed, 1);
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
  out->history = d->history;
  out->sample_params = d->sp;
  out->rng = d->rng;
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
  const uint32_t tok[3] = {token, 0, 0};  // clears the count of failed steps
  int st = eg_buf_write(d->ctx, d->token, 0, tok, sizeof(tok));
  if (st == EG_OK) st = eg_buf_write(d->ctx, d->position, 0, &position, 4);
  if (st == EG_OK) st = tail(d, eg::StepTail{});  // this token's embedding, this position's RoPE table
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
  int st = d->graph ? eg_graph_launch(d->ctx, d->graph) : run_step(d, sampled_mode(d->sampling));
  if (st == EG_OK) d->host_position++;
  if (st == EG_OK && token_out) st = read_token(d, token_out, "decoder_step");
  return st;
}

int eg_decoder_capture(eg_decoder* d) {
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "decoder_capture: decoder is NULL");
  return capture(d);
}

int eg_decoder_set_sampling(eg_decoder* d, const eg_sampling_params* params) {
  const char* op = "decoder_set_sampling";
  if (!d || !params) return eg::fail(d ? d->ctx : nullptr, EG_ERR_INVALID, "%s: NULL argument", op);
  if (d->ctx->capturing) return eg::fail(d->ctx, EG_ERR_STATE, "%s: a graph capture is in progress", op);
  const eg_sampling_params& p = *params;
  // DecodeGraph.setSampling (graph_decode.ts:387) takes any values and the sampler handles every
  // finite one as the reference's kernel does (topP <= 0 keeps the argmax fallback, topP >= 1
  // keeps every id); only values no f32 uniform can carry meaningfully are refused
  if (!std::isfinite(p.temperature) || !std::isfinite(p.top_p) || !std::isfinite(p.repetition_penalty))
    return eg::fail(d->ctx, EG_ERR_INVALID, "%s: temperature %g, topP %g and repetitionPenalty %g must be finite", op,
                    (double)p.temperature, (double)p.top_p, (double)p.repetition_penalty);
  const float vals[3] = {p.temperature, p.top_p, p.repetition_penalty};
  uint32_t words[3];
  std::memcpy(words, vals, sizeof(words));
  int st = write_ids(d, reinterpret_cast<uint32_t*>(&d->sp->temperature), words, 3);
  if (st != EG_OK) return st;
  d->sampling = p;
  // a graph captured in the other mode (greedy fused argmax / sampler) is captured again
  if (d->graph && (d->graph_sampled != sampled_mode(p) || d->graph_host_driven != d->host_driven)) st = capture(d);
  return st;
}

int eg_decoder_launches(eg_decoder* d, uint32_t* per_step) {
  if (!d || !per_step) return eg::fail(d ? d->ctx : nullptr, EG_ERR_INVALID, "decoder_launches: NULL argument");
  // the layers (one persistent launch, or 5 per layer), the LM head, the sampler unless GREEDY,
  // the tail, and a host-driven step's input preparation
  *per_step = (d->layers_kernel ? 1u : 5u * d->desc.layers) + 2u + (sampled_mode(d->sampling) ? 1u : 0u) +
              (d->host_driven ? 1u : 0u);
  return EG_OK;
}

int eg_decoder_seed(eg_decoder* d, uint32_t seed) {
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "decoder_seed: decoder is NULL");
  if (d->ctx->capturing) return eg::fail(d->ctx, EG_ERR_STATE, "decoder_seed: a graph capture is in progress");
  int st = write_ids(d, d->rng, &seed, 1);
  if (st == EG_OK) st = set_host_driven(d, false);
  return st;
}

int eg_decoder_set_position(eg_decoder* d, uint32_t position, uint32_t history_length, float random) {
  const char* op = "decoder_set_position";
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "%s: decoder is NULL", op);
  if (d->ctx->capturing) return eg::fail(d->ctx, EG_ERR_STATE, "%s: a graph capture is in progress", op);
  if (position >= d->desc.max_context)  // kvcache.ts:118-127
    return eg::fail(d->ctx, EG_ERR_RANGE, "%s: position %u past the context of %u", op, position, d->desc.max_context);
  if (history_length > d->desc.max_context)
    return eg::fail(d->ctx, EG_ERR_RANGE, "%s: history of %u exceeds %u", op, history_length, d->desc.max_context);
  uint32_t rbits;
  std::memcpy(&rbits, &random, 4);
  int st = write_ids(d, d->position, &position, 1);
  if (st == EG_OK) st = write_ids(d, &d->sp->history_length, &history_length, 1);
  if (st == EG_OK) st = write_ids(d, reinterpret_cast<uint32_t*>(&d->sp->random), &rbits, 1);
  if (st == EG_OK) st = set_host_driven(d, true);
  if (st == EG_OK) d->host_position = position;
  return st;
}

int eg_decoder_set_history(eg_decoder* d, const uint32_t* host_ids, uint32_t count) {
  const char* op = "decoder_set_history";
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "%s: decoder is NULL", op);
  if (d->ctx->capturing) return eg::fail(d->ctx, EG_ERR_STATE, "%s: a graph capture is in progress", op);
  if (count > 0 && !host_ids) return eg::fail(d->ctx, EG_ERR_INVALID, "%s: %u ids from NULL", op, count);
  if (count > d->desc.max_context)
    return eg::fail(d->ctx, EG_ERR_RANGE, "%s: %u ids exceed the history of %u", op, count, d->desc.max_context);
  int st = write_ids(d, d->history, host_ids, count);
  if (st == EG_OK) st = write_ids(d, &d->sp->history_length, &count, 1);
  return st;
}

int eg_decoder_set_prefill_chunk(eg_decoder* d, uint32_t rows) {
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "decoder_set_prefill_chunk: decoder is NULL");
  if (rows == 0 || rows > d->chunk_capacity)
    return eg::fail(d->ctx, EG_ERR_RANGE, "decoder_set_prefill_chunk: %u rows (1..%u)", rows, d->chunk_capacity);
  d->chunk = rows;
  return EG_OK;
}

int eg_decoder_prefill(eg_decoder* d, uint32_t position, const uint32_t* host_ids, uint32_t count,
                       uint32_t* token_out) {
  const char* op = "decoder_prefill";
  if (!d) return eg::fail(nullptr, EG_ERR_INVALID, "%s: decoder is NULL", op);
  if (d->ctx->capturing) return eg::fail(d->ctx, EG_ERR_STATE, "%s: a graph capture is in progress", op);
  if (count == 0 || !host_ids) return eg::fail(d->ctx, EG_ERR_INVALID, "%s: an empty prompt", op);
  // session.ts:326-330: a prompt longer than the remaining context is a RangeError
  if ((uint64_t)position + count > d->desc.max_context)
    return eg::fail(d->ctx, EG_ERR_RANGE, "%s: prompt of %u exceeds the remaining context of %u", op, count,
                    position < d->desc.max_context ? d->desc.max_context - position : 0u);
  for (uint32_t i = 0; i < count; i++)
    if (host_ids[i] >= d->desc.vocab)
      return eg::fail(d->ctx, EG_ERR_INVALID, "%s: token %u at %u outside the vocabulary", op, host_ids[i], i);
  // the history is the prompt (Session.runPrefill: this.tokens = [...prompt]); the chunks read
  // their ids from there. The steps that follow chain on the device.
  int st = set_host_driven(d, false);
  if (st == EG_OK) st = eg_decoder_set_history(d, host_ids, count);
  // the prompt in chunks (ForwardGraph.encodeChunks, graph.ts:610-621)
  uint32_t last_rows = 0;
  for (uint32_t c0 = 0; st == EG_OK && c0 < count; c0 += d->chunk) {
    last_rows = std::min(d->chunk, count - c0);
    st = run_prefill_chunk(d, d->history + c0, position + c0, last_rows);
  }
  // the last position's token: the head on the last row, then the tail advances the position
  // past the prompt (sampleFromPrefill, session.ts:472-495: the decode graph's sample step)
  const uint32_t last = position + count - 1;
  const bool sampled = sampled_mode(d->sampling);
  if (st == EG_OK) st = write_ids(d, d->position, &last, 1);
  if (st == EG_OK && sampled) {
    // The last prompt id and position as the decode step's input (its embedding row and RoPE
    // row): should the sampler give up, nothing advances and the next eg_decoder_step redoes
    // that position as a decode step and samples.
    eg::StepTail input;
    input.token_src = d->history + (count - 1);
    st = tail(d, input);
  }
  if (st == EG_OK) st = run_head(d, sampled, d->ph[0] + (size_t)(last_rows - 1) * d->desc.hidden);
  if (st != EG_OK) return st;
  d->host_position = position + count;
  return token_out ? read_token(d, token_out, op) : EG_OK;
}

}  // extern "C"
