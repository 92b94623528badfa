// Internal plumbing shared by the HIP translation units: the context, error reporting and the
// device-side helpers every kernel uses. Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <unordered_map>

#include "enargeia_hip.h"

struct eg_context {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;  // own_stream or a caller's stream
  int cu_count = 256;
  // Workspace for cross-workgroup reductions (partials, histograms, small state). Every
  // element is written before it is read within one op, so it needs no clearing.
  uint8_t* workspace = nullptr;
  size_t workspace_bytes = 0;
  bool capturing = false;
  // This device's copy of the fixed scratch array of eg_lm_head_argmax_noalloc (resolved by
  // eg::noalloc_scratch_init at creation; shared by every context on the device).
  void* noalloc_scratch = nullptr;
  // GEMV shape override (team, chunks per lane, rows per lane, pipeline depth) from
  // EG_GEMV_SHAPE="t,c,u[,d]", read once at creation; zeros mean the built-in choice. For
  // tuning sweeps.
  int gemv_override[4] = {0, 0, 0, 0};
  // Tiles per wave for GEMVs with a fused input stage (EG_FUSED_TILES_PER_WAVE, default 1: every
  // workgroup recomputes the stage, but the decoder's launches measured faster with more,
  // shorter-lived workgroups than with two tiles per wave).
  uint32_t fused_tiles_per_wave = 1;
  // eg_sample has run on this context: synchronising calls then check the count of its launches
  // that gave up (eg::report_sample_failures).
  bool sample_used = false;
  // Launch stamps (eg_test_launch_stamps): the device buffer the next decode-step launches write
  // their per-wave wall-clock stamps to, its slots, and the next free slot.
  uint64_t* stamps = nullptr;
  uint32_t stamp_capacity = 0;
  uint32_t stamp_next = 0;
  // Groups of 4 waves per prefill GEMM workgroup, each on its own K blocks: 0 = chosen per
  // launch from the tile grid; EG_PREFILL_GROUPS=1, 2 or 4 forces one (for tuning sweeps).
  int prefill_groups = 0;
  // chunk attention's key split: at most this many 64-key tiles per workgroup, and a small grid
  // split up to this many workgroups per CU
  // the SwiGLU pair as one launch of paired gate|up tiles (false: gate | up, then silu_mul_rows)
  bool prefill_pair = true;
  // the prompt chain's RoPE and cache append in the q|k|v launch (false: rope_append's launch)
  bool prefill_rope = true;
  // the prompt chain's GEMM inputs produced as bf16 rows where the GEMM stages them (false: f32)
  bool prefill_xb16 = true;
  // prefill GEMM tiles mapped so each XCD runs whole row tiles where that applies (false: the
  // grid's own order)
  bool prefill_xcd = true;
  uint32_t attention_split_tiles = 8;
  uint32_t attention_split_fill = 1;
  // the decode step's layers as one persistent launch where the shapes allow (EG_DECODE_PERSISTENT=1;
  // off by default: one launch per op measured ~7% faster on MI355X)
  bool decode_persistent = false;
  uint32_t persistent_grid = 0;  // EG_PERSISTENT_GRID: workgroups of that launch (0: the default)
  uint32_t persistent_poll = 1;  // EG_PERSISTENT_POLL: 64-clock sleeps between polls of a wait
  // Resident workgroups per CU of each kernel launched through this context (from
  // hipOccupancyMaxActiveBlocksPerMultiprocessor), so grids can be sized to one full wave of
  // the device.
  std::mutex occupancy_lock;
  std::unordered_map<uint64_t, int> occupancy;  // key: kernel address ^ (LDS bytes << 48)
  char error[512] = {0};
};

struct eg_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

struct eg_layers;  // the persistent decode layers of a decoder (eg_layers.hip)

namespace eg {

int fail(eg_context* ctx, int status, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int hip_fail(eg_context* ctx, hipError_t err, const char* what);

// Workspace layout (bytes from ctx->workspace). Fixed offsets; sizes bound the op limits.
constexpr size_t kStateOffset = 256;           // small per-op state
constexpr size_t kPartialsOffset = 8192;       // per-workgroup partials
constexpr size_t kWorkspaceBytes = 64u << 20;  // 64 MiB

inline uint8_t* state(eg_context* ctx) { return ctx->workspace + kStateOffset; }
inline uint8_t* partials(eg_context* ctx) { return ctx->workspace + kPartialsOffset; }
constexpr size_t kPartialsBytes = kWorkspaceBytes - kPartialsOffset;

// Second stage of every multi-workgroup argmax: one workgroup reduces `groups` partials
// (value bits, index) in a fixed order into result = [index, value bits]. A separate launch
// rather than a last-arriving workgroup. Measured on the 151,936-row LM head (2048 workgroups):
// with an L2 write-back release per workgroup the arrival protocol costs far more than a launch;
// with coherent stores (egd::put / drain), one arrival counter and egd::get reads it added 12 us
// over the GEMV alone (every workgroup's atomic serialises on the one word), and with 16 group
// counters 128 bytes apart 5.7 us - against 3.9 us for this launch.
void launch_argmax_finalize(eg_context* ctx, const uint32_t* partials, uint32_t groups, uint32_t sentinel_index,
                            uint32_t* result);

// The fused LM head + argmax without its finalize launch: the per-workgroup (value, index)
// partials are left in the workspace (eg::partials) and their count in *groups, for a caller
// that reduces them in a launch of its own (the decoder's step tail). Same checks and kernels as
// eg_lm_head_argmax_input.
int lm_head_argmax_partials(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed,
                            const float* scales, const uint32_t* zeros, float* out, const eg_embedding_dims* dims,
                            int encoding, int bits, uint32_t* groups);

// The int8 LM head ahead of the sampler (kSampleStats): each logit penalized and stored in `out`,
// and per workgroup (max of l/T, its lowest index, float64 sum of exp(l/T - that max)) - 16 bytes,
// (value bits, index, sum) - left in `partials` (NULL: the workspace), their count in *groups.
// The parameters come from device memory (sample_dev, so a captured graph follows them) or, when
// that is NULL, from sample_host; the penalty reads `history` (the first history_length ids).
// Workgroup 0 also zeroes clear[0, clear_words) (the sampler's level-0 bins, which the launch after
// this one sums into with no barrier first; NULL: nothing).
int lm_head_sample_partials(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed, const float* scales,
                            const uint32_t* zeros, float* out, const eg_embedding_dims* dims, int encoding, int bits,
                            const eg_sample_dims* sample_dev, const eg_sample_dims* sample_host,
                            const uint32_t* history, uint32_t* partials, size_t partials_bytes, uint32_t* clear,
                            uint32_t clear_words, uint32_t* groups);

// What a decode step's tail does before it prepares the next step (see launch_step_tail).
struct StepTail {
  bool advance = false;                 // false: a reset (token[0] and position[0] as written)
  const uint32_t* partials = nullptr;   // greedy step: the LM head's argmax partials, `groups` of them
  uint32_t groups = 0;
  const uint32_t* token_src = nullptr;  // prompt-fill step or reset: the next input id is *token_src
  // (neither: a sampled step, whose sampler already wrote token[0])
  uint32_t* history = nullptr;          // the new token is appended (not by fill steps) ...
  uint32_t* history_length = nullptr;   // ... at history[*history_length]++, up to the capacity
  uint32_t history_capacity = 0;
  uint32_t* rng = nullptr;              // mulberry32 state: advanced once (the step's draw)
  // A sampled step whose sampler gave up (token[0] outside the vocabulary) has no token: the tail
  // then counts it in *status (nullable) and leaves the position, the history, the draw state
  // and the next step's input (embedding row, RoPE row) as they were, so the next step redoes it.
  uint32_t* status = nullptr;
  // The persistent layers' abort flag (nullable): raised, the step's layers ran without waiting
  // and the step failed as above. Either way the tail zeroes the flag and the arrival counters
  // (sync_count words, sync_stride apart) for the next launch.
  uint32_t* sync_abort = nullptr;
  uint32_t* sync_counters = nullptr;
  uint32_t sync_count = 0, sync_stride = 0;
  // the RoPE cos/sin of positions [0, rope_positions) (launch_rope_table); the next position's
  // row is copied from here (computed in the launch where it is NULL or the position is past it)
  const double2* rope_table = nullptr;
  uint32_t rope_positions = 0;
};

// Fills table[p * head_dim / 2 + i] with the RoPE (cos, sin) of position p and frequency i for
// p < positions: the values launch_step_tail and the attention launch compute, by the same
// function. head_dim 64.
int launch_rope_table(eg_context* ctx, double* table, uint32_t positions, uint32_t head_dim, float theta);

// The decode step's tail, one single-workgroup launch. With `advance` the step's token is
// settled (greedy: reduced from the argmax partials into token[0..1]; fill: copied from
// token_src; sampled: already in token[0]), position[0] advances, the token is appended to the
// history and the draw state advances as asked. Then (also for a reset) the embedding row of
// token[0] is dequantized into `emb` and the RoPE cos/sin of position[0] are written to `rope`
// ([head_dim / 2] pairs of doubles).
int launch_step_tail(eg_context* ctx, const StepTail& t, uint32_t* token, uint32_t* position, const uint32_t* packed,
                     const float* scales, const uint32_t* zeros, const eg_embedding_dims* ed, int encoding, int bits,
                     float* emb, double* rope, uint32_t head_dim, float theta);

// eg_sample's launch with every parameter read from DEVICE memory `params` (the 32-byte
// sample dims: vocab, history_length, temperature, top_p, repetition_penalty, random), so a
// captured graph replays with new values. With `rng` the launch first takes params->random as
// the mulberry32 draw from the state there, WITHOUT advancing it (the caller advances it once
// the step has its token). `vocab` sizes the grid and must equal params->vocab. A launch whose
// bounded waits give up leaves out[0] = 0xFFFFFFFF and adds 1 to *status (status nullable: a
// caller that counts from out[0] itself).
int launch_sample_device(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out, uint32_t vocab,
                         eg_sample_dims* params, uint32_t* rng, uint32_t* status);

// The int8 LM head and the sampler as one sampled token, the parameters in DEVICE memory as for
// launch_sample_device (vocab = dims->row_count, out_offset 0): the head applies the penalty to
// the logits it stores in `logits` and leaves per-workgroup partials (max of l/T, its index, the
// float64 sum of exp(l/T - that max)), from which the sampler takes the global max, its index and
// the normaliser instead of its own penalty pass, slice maxima and first grid barrier. Same token
// semantics, give-up behaviour and status counting as launch_sample_device.
int lm_head_sample_device(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed, const float* scales,
                          const uint32_t* zeros, float* logits, const eg_embedding_dims* dims, int encoding, int bits,
                          const uint32_t* history, uint32_t* out, eg_sample_dims* params, uint32_t* rng,
                          uint32_t* status);

// The test hook's limit on the bounded waits of in-launch synchronisation (the sampler's grid
// barriers, the persistent decode layers' phase waits): 0 = their default (about a second), else
// limit + 1 polls. A word of the context's state, set by eg_test_sample_spin; kernels read it at
// every wait, so captured graphs follow it too.
inline uint32_t* wait_limit_word(eg_context* ctx) { return reinterpret_cast<uint32_t*>(state(ctx) + 2048 + 640); }

// Reports, once, the standalone sampler launches that gave up since the last report: when the
// context has run eg_sample, reads (after the stream has drained) and clears the count the
// sampler keeps in the context's state, and fails with EG_ERR_DEVICE when it is not zero.
// eg_sync and eg_buf_read call it; `op` names the caller in the message.
int report_sample_failures(eg_context* ctx, const char* op);

// eg_attention_decode with the RoPE cos/sin of the current position read from `rope` ([head_dim
// / 2] pairs of doubles, as egd::rope_table computes them) instead of computed in the launch.
int attention_decode_rope(eg_context* ctx, const uint32_t* position, const float* q, const float* k,
                          const float* v, uint16_t* k_cache, uint16_t* v_cache, float* partials,
                          const eg_attention_dims* dims, const double* rope);
int attention_decode_rope(eg_context* ctx, const uint32_t* position, const float* q, const float* k,
                          const float* v, float* k_cache, float* v_cache, float* partials,
                          const eg_attention_dims* dims, const double* rope);

// eg_matmul_q4_prefill with a residual added in the epilogue: out[r * out_stride + col +
// out_offset] = sum_k x[r, k] W[col, k] + bias[col] + residual[same index] (residual nullable;
// it may not alias out). x_bf16: x holds bf16 rows (the chunked staging only).
int prefill_gemm(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales, const uint32_t* zeros,
                 const float* bias, const float* residual, float* out, const eg_matmul_q4_dims* dims, int encoding,
                 int bits, bool x_bf16 = false);

// Several matrices that share x (m rows of k values), the quant block size and the encoding in
// ONE launch - the prompt chain's q|k|v and gate|up: for each matrix s (at most 3),
// out_s[r * out_stride_s + col + out_offset_s] = sum_k x[r, k] W_s[col, k] + bias_s[col]
// (+ residual_s at the same index). Layouts the chunked staging does not take, and a K deep
// enough that a lone matrix would split it, run one prefill_gemm per matrix instead.
struct PrefillMatrix {
  const uint32_t* packed;
  const float* scales;
  const uint32_t* zeros;
  const float* bias;
  const float* residual;
  float* out;
  uint32_t n, out_stride, out_offset;
};
// norm non-NULL: x is RMS-normalised per row first (rmsnorm_rows' x * (1 / rms) * norm, eps) - folded
// into the one launch where it can be, else rmsnorm_rows into `normed` ([m][k]) and the launches
// on that.
int prefill_gemm_multi(eg_context* ctx, const float* x, uint32_t m, uint32_t k, uint32_t block_size, int encoding,
                       int bits, const PrefillMatrix* mats, uint32_t count, const float* norm = nullptr,
                       float eps = 0.f, float* normed = nullptr);
// q | k | v of a prompt chunk with rope_append's work in the launch's epilogue (head_dim 64): q
// rows rotated and scaled by 1/8 into q_rope, k rows rotated and v rows appended to the f16
// caches at positions pos0 + row, cos/sin read from a table of launch_rope_table rows.
struct PrefillRope {
  const double2* table;  // [position][32] (cos, sin), covering pos0 .. pos0 + m - 1
  float* q_rope;         // [m][q_heads][64]
  uint16_t* k_cache;     // [position][kv_heads][64]
  uint16_t* v_cache;
  uint32_t pos0, q_heads, kv_heads;
};
// mats = q, k, v (q_heads * 64, kv_heads * 64, kv_heads * 64 rows). Runs the one fused launch
// (norm, eps, normed as prefill_gemm_multi's) and sets *done, or - when the launch cannot take
// these shapes or the context disables it - launches nothing and leaves *done false.
int prefill_qkv_rope(eg_context* ctx, const float* x, uint32_t m, uint32_t k, uint32_t block_size, int encoding,
                     int bits, const PrefillMatrix* mats, const float* norm, float eps, float* normed,
                     const PrefillRope& rope, bool* done);
// Chunk attention over caches that already hold the chunk's rows, q_rope already written (the
// launches of eg_attention_prefill after its rope_append); dims as that entry point checks them.
// out_bf16: the output rows stored as bf16 (egd::pack_bf16), the o projection's x.
int attention_prefill_run(eg_context* ctx, const float* q_rope, const uint16_t* k_cache, const uint16_t* v_cache,
                          float* out, const eg_attention_prefill_dims& d, bool out_bf16 = false);
// Whether a prefill GEMM over (k, block size, bits, x, packed) takes the chunked staging (the
// launches that can stage bf16 rows of x).
bool prefill_chunked(uint32_t m, uint32_t n, uint32_t k, uint32_t block_size, int bits, const void* x,
                     const uint32_t* packed);
int check_attention_prefill(eg_context* ctx, const char* op, const eg_attention_prefill_dims* dims);
// The SwiGLU pair: out[r][j] = SiLU(x[r] . gate_j + bias) * (x[r] . up_j + bias), j < gate.n, rows
// gate.n apart (the outputs and strides in gate and up are ignored). One launch of paired tiles
// where the staging allows; otherwise gate | up into `scratch` ([m][2 n]) and silu_mul_rows.
// norm, eps, normed: as prefill_gemm_multi's.
int prefill_gemm_swiglu(eg_context* ctx, const float* x, uint32_t m, uint32_t k, uint32_t block_size, int encoding,
                        int bits, const PrefillMatrix& gate, const PrefillMatrix& up, float* out, float* scratch,
                        const float* norm = nullptr, float eps = 0.f, float* normed = nullptr, bool out_bf16 = false);

// Row-wise kernels of the prefill chain (one workgroup per row):
//   embed_rows: out[r] = the dequantized table row of ids[r] (ops.ts:222-233), r < rows;
//   rmsnorm_rows: out[r] = x[r] / sqrt(mean(x[r]^2) + eps) * w (ops.ts:30-51);
//   silu_mul_rows: out[r][j] = silu(x[r][j]) * x[r][n + j] for j < n (gate then up in one row of
//   2n, ops.ts:207-216).
int embed_rows(eg_context* ctx, const uint32_t* ids, uint32_t rows, const uint32_t* packed, const float* scales,
               const uint32_t* zeros, uint32_t hidden, uint32_t block_size, int encoding, int bits, float* out);
// out_bf16: the rows stored as bf16 (egd::pack_bf16), for a GEMM that stages them as they are.
int rmsnorm_rows(eg_context* ctx, const float* x, const float* w, uint32_t rows, uint32_t n, float eps, float* out,
                 bool out_bf16 = false);
int silu_mul_rows(eg_context* ctx, const float* x, uint32_t rows, uint32_t n, float* out, bool out_bf16 = false);

// The decode step's layers as one persistent launch (eg_layers.hip). Per layer, the four GEMV
// plans the per-op launches use (q|k|v, o, the gate|up pair, down) with their inputs; the
// attention's buffers and dims. layers_create leaves *out NULL, with EG_OK, where the shapes or
// the device's occupancy do not fit the persistent kernel (the per-op launches then run).
struct LayerPlans {
  const eg_gemv_plan* plan[4];
  eg_gemv_input input[4];
};
struct LayersDesc {
  uint32_t layers;
  const LayerPlans* plans;
  eg_attention_dims att;
  const uint32_t* position;
  const double* rope;
  const float *q, *k, *v;
  float* partials;
  uint16_t *k_cache, *v_cache;
  size_t layer_stride;  // cache elements per layer
};
int layers_create(eg_context* ctx, const LayersDesc& desc, eg_layers** out);
int layers_launch(eg_context* ctx, eg_layers* layers);
// The arrival counters (`count` words, `stride` words apart) and the abort flag, which the step
// tail reads and zeroes after every launch.
void layers_sync_words(const eg_layers* layers, uint32_t** counters, uint32_t* count, uint32_t* stride,
                       uint32_t** abort);
void layers_destroy(eg_context* ctx, eg_layers* layers);

// Resolves the calling thread's current device's copy of the no-alloc scratch array
// (hipGetSymbolAddress, once per device) into ctx->noalloc_scratch.
int noalloc_scratch_init(eg_context* ctx);

// Workgroups of `kernel` (256 threads, `smem_bytes` of dynamic LDS) resident per CU, cached
// per context; 0 if the runtime cannot say.
int occupancy_of(eg_context* ctx, const void* kernel, uint32_t smem_bytes = 0);

// Validates a launch once the kernel is enqueued (hipGetLastError catches bad configurations
// immediately; faults surface at the next synchronisation).
int check_launch(eg_context* ctx, const char* op);

// Launch stamps: each launch that takes a slot writes (entry, exit) wall-clock stamps of up to
// kStampWaves waves there (egd::WaveStamp); NULL when the context records none.
constexpr uint32_t kStampWaves = 8192;
inline uint64_t* stamp_slot(eg_context* ctx) {
  if (!ctx->stamps || ctx->stamp_next >= ctx->stamp_capacity) return nullptr;
  return ctx->stamps + 2ull * kStampWaves * ctx->stamp_next++;
}

}  // namespace eg

// ---- device helpers ---------------------------------------------------------------------

namespace egd {

// A pointer known to be global memory. Pointers read from device memory (tables) are generic
// to the compiler, which then emits flat loads; flat loads count against both vmcnt and
// lgkmcnt and force coarse waits. Casting to address space 1 restores global loads.
template <typename T>
using gptr = const __attribute__((address_space(1))) T*;
template <typename T>
using gptr_mut = __attribute__((address_space(1))) T*;
// 16 bytes as a native vector (HIP's uint4 is a class, which cannot be copied out of an
// address-space-qualified lvalue).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
template <typename T>
__device__ __forceinline__ gptr<T> as_global(const T* p) {
  return (gptr<T>)p;
}
template <typename T>
__device__ __forceinline__ gptr_mut<T> as_global_mut(T* p) {
  return (gptr_mut<T>)p;
}

// A pointer read from memory that every lane holds: moved to scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

// Raw buffer resources: base address in SGPRs, `bytes` records, 32-bit byte offsets per lane.
// Reads past `bytes` return zero and writes past it are dropped (bounds-checked by hardware).
// Word 3 = 0x00020000: raw 32-bit data for gfx950.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
// `offset` is per lane (VGPR); `soffset` is a wave-uniform byte offset added in the address
// unit (SGPR), so a loop that walks a stream advances it with scalar adds.
__device__ __forceinline__ u32x4 load_b128(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, soffset, 0);
}
// Non-temporal (streaming) loads, for data read exactly once per launch (weight codes and
// scales): the nt cache-policy bit lets the line bypass normal retention, which measures ~10%
// more read bandwidth on MI355X than default-policy loads.
#ifndef EG_WEIGHT_CACHE_POLICY
#define EG_WEIGHT_CACHE_POLICY 2  // the nt bit; 0 (default policy) builds a variant for measurement
#endif
constexpr int kNonTemporal = EG_WEIGHT_CACHE_POLICY;
__device__ __forceinline__ u32x4 load_b128_nt(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, soffset, kNonTemporal);
}
__device__ __forceinline__ uint64_t load_b64(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 v = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, offset, soffset, 0));
  return (uint64_t)v.x | ((uint64_t)v.y << 32);
}
__device__ __forceinline__ uint32_t load_b32_nt(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, offset, soffset, kNonTemporal);
}
__device__ __forceinline__ float load_f32_nt(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, offset, soffset, kNonTemporal));
}
__device__ __forceinline__ uint32_t load_b32(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, offset, soffset, 0);
}
__device__ __forceinline__ float load_f32(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, offset, soffset, 0));
}
__device__ __forceinline__ void store_f32(__amdgpu_buffer_rsrc_t r, uint32_t offset, float v, uint32_t soffset = 0) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, offset, soffset, 0);
}

// The same accesses with an explicit cache policy: AUX = 0 is the default policy; AUX = kCoherent
// (sc1) is the agent-scope coherent form egd::put / egd::get use, for data another workgroup of
// the same launch writes or reads.
constexpr int kCoherent = 16;
template <int AUX>
__device__ __forceinline__ u32x4 load_b128_p(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, offset, soffset, AUX);
}
template <int AUX>
__device__ __forceinline__ uint32_t load_b32_p(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, offset, soffset, AUX);
}
template <int AUX>
__device__ __forceinline__ float load_f32_p(__amdgpu_buffer_rsrc_t r, uint32_t offset, uint32_t soffset = 0) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, offset, soffset, AUX));
}
template <int AUX>
__device__ __forceinline__ void store_f32_p(__amdgpu_buffer_rsrc_t r, uint32_t offset, float v, uint32_t soffset = 0) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, v), r, offset, soffset, AUX);
}

// Opaque AND: keeps the compiler from folding a nibble mask into per-element bitfield
// extracts, so the byte converts (v_cvt_f32_ubyte0..3) consume the masked word directly.
__device__ __forceinline__ uint32_t and_opaque(uint32_t v, uint32_t m) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(v));
  return r;
}
__device__ __forceinline__ float ub0(uint32_t v) { return (float)(v & 0xffu); }
__device__ __forceinline__ float ub1(uint32_t v) { return (float)((v >> 8) & 0xffu); }
__device__ __forceinline__ float ub2(uint32_t v) { return (float)((v >> 16) & 0xffu); }
__device__ __forceinline__ float ub3(uint32_t v) { return (float)(v >> 24); }

// One DPP step: v + (v as seen through dpp_ctrl). Lanes whose source is disabled read 0.
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_add(float v) {
  const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROW_MASK, 0xF, ROW_MASK == 0xF);
  return v + __builtin_bit_cast(float, moved);
}

// Sum across a team of TEAM consecutive lanes (TEAM a power of two <= 64, teams aligned), by
// DPP only: quad permutes, half-row and row mirrors, then row_bcast:15 / row_bcast:31 for
// teams spanning rows of 16 lanes. The total is valid in lane TEAM-1 of each team (in every
// lane of the team when TEAM <= 16). Fixed order, so the result is deterministic.
template <int TEAM>
__device__ __forceinline__ float team_sum(float v) {
  if (TEAM >= 2) v = dpp_add<0xB1>(v);         // quad_perm [1,0,3,2]
  if (TEAM >= 4) v = dpp_add<0x4E>(v);         // quad_perm [2,3,0,1]
  if (TEAM >= 8) v = dpp_add<0x141>(v);        // row_half_mirror
  if (TEAM >= 16) v = dpp_add<0x140>(v);       // row_mirror
  if (TEAM >= 32) v = dpp_add<0x142, 0xA>(v);  // row_bcast:15 into rows 1 and 3
  if (TEAM >= 64) v = dpp_add<0x143, 0xC>(v);  // row_bcast:31 into rows 2 and 3
  return v;
}

// Sum across a team of TEAM consecutive lanes with the total in EVERY lane of the team, so a
// store or compare needs no lane-divergent branch. Within a row of 16 lanes the butterfly is
// DPP (quad permutes, half-row and row mirrors); rows 16 apart are exchanged with a
// ds_swizzle xor-16 (no LDS memory is touched); the two halves of a 64-lane team are joined by
// two readlanes. Every lane adds the same operands in the same order (addition commutes), so
// all lanes hold bit-identical totals, and the order is fixed: deterministic.
template <int TEAM>
__device__ __forceinline__ float team_allsum(float v) {
  if (TEAM >= 2) v = dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  if (TEAM >= 4) v = dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  if (TEAM >= 8) v = dpp_add<0x141>(v);  // row_half_mirror
  if (TEAM >= 16) v = dpp_add<0x140>(v); // row_mirror
  if (TEAM >= 32) {
    // bit mode: and_mask 0x1F, or_mask 0, xor_mask 0x10
    const int o = __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F);
    v = v + __builtin_bit_cast(float, o);
  }
  if (TEAM >= 64) {
    const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    v = lo + hi;
  }
  return v;
}

// Max across a team of TEAM consecutive lanes with the result in every lane: the butterfly of
// team_allsum (DPP within rows of 16, a swizzle across 32, readlanes across 64) with fmaxf.
template <int TEAM>
__device__ __forceinline__ float team_allmax(float v) {
  auto step = [&](float o) { v = fmaxf(v, o); };
  if (TEAM >= 2) step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true)));
  if (TEAM >= 4) step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true)));
  if (TEAM >= 8) step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true)));
  if (TEAM >= 16) step(__builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true)));
  if (TEAM >= 32) step(__builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F)));
  if (TEAM >= 64) {
    const float lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    v = fmaxf(lo, hi);
  }
  return v;
}

// Combining flash-decoding partials (laid out chunk-fastest: o[h][D][chunks], then
// m[h][chunks], then l[h][chunks]) needs, per head, M = max_c m_c and the normaliser
// L = sum_c l_c e^(m_c - M). The products l_c e^(m_c - M) are summed as a balanced pairwise tree
// in chunk order over 64 slots (chunks past the head's count add zeros, which changes no bit):
// the tree a butterfly over a power-of-two group of lanes computes, so a wave that reduces a
// head's chunks across its lanes and a thread that does it alone produce the same bits. At most
// kMaxChunks chunks per head.
constexpr uint32_t kMaxChunks = 64;

// The smallest power of two >= chunks: the lanes one head's statistics span in a butterfly.
__host__ __device__ constexpr uint32_t combine_group(uint32_t chunks) {
  uint32_t g = 1;
  while (g < chunks) g <<= 1;
  return g;
}

// One thread: (M, L) of one head from its m and l rows.
__device__ __forceinline__ void combine_stats(const float* m, const float* l, uint32_t chunks, float& M, float& L) {
  M = -INFINITY;
  for (uint32_t c = 0; c < chunks; c++) M = fmaxf(M, m[c]);
  float t[kMaxChunks];
#pragma unroll
  for (uint32_t c = 0; c < kMaxChunks; c++) t[c] = c < chunks ? l[c] * expf(m[c] - M) : 0.f;
#pragma unroll
  for (uint32_t w = kMaxChunks; w > 1; w >>= 1)
#pragma unroll
    for (uint32_t c = 0; c < w / 2; c++) t[c] = t[2 * c] + t[2 * c + 1];
  L = t[0];
}

// The same statistics with one head's chunks spread over a group of G lanes (G =
// combine_group(chunks), groups aligned within a wave, every lane active): M by a max
// butterfly, e = e^(m - M) per lane, L by the sum butterfly - the pairwise tree combine_stats
// computes on one thread. Lanes past the head's chunks pass valid = false.
template <int G>
__device__ __forceinline__ void group_stats_of(bool valid, float m, float l, float& M, float& e, float& L) {
  M = team_allmax<G>(valid ? m : -INFINITY);
  e = expf(m - M);
  L = team_allsum<G>(valid ? l * e : 0.f);
}
__device__ __forceinline__ void group_stats(uint32_t G, bool valid, float m, float l, float& M, float& e, float& L) {
  switch (G) {
    case 1: group_stats_of<1>(valid, m, l, M, e, L); break;
    case 2: group_stats_of<2>(valid, m, l, M, e, L); break;
    case 4: group_stats_of<4>(valid, m, l, M, e, L); break;
    case 8: group_stats_of<8>(valid, m, l, M, e, L); break;
    case 16: group_stats_of<16>(valid, m, l, M, e, L); break;
    case 32: group_stats_of<32>(valid, m, l, M, e, L); break;
    default: group_stats_of<64>(valid, m, l, M, e, L); break;
  }
}

// One element of the attention output: out[h*D + e] = sum_c o_c[e] * (e^(m_c - M) / L), the
// chunks in order - deterministic, and the same operations as the GEMV input stage's combine.
__device__ __forceinline__ float attention_combine_at(const float* partials, uint32_t i, uint32_t heads,
                                                      uint32_t D, uint32_t chunks) {
  const uint32_t h = i / D;
  const float* o = partials + (size_t)i * chunks;
  const float* m = partials + (size_t)heads * D * chunks + (size_t)h * chunks;
  const float* l = m + (size_t)heads * chunks;
  float M, L;
  combine_stats(m, l, chunks, M, L);
  float acc = 0.f;
  for (uint32_t c = 0; c < chunks; c++) acc = fmaf(o[c], expf(m[c] - M) / L, acc);
  return acc;
}

// A launch's per-wave wall-clock stamps (eg::stamp_slot): lane 0 of each wave stores the wave's
// entry time (s_memrealtime, 100 MHz) at construction and its exit time when the kernel's scope
// ends, wave w of the launch at base[2 w], base[2 w + 1]. Nothing without a slot.
//
// Only the profiling build (EG_LAUNCH_STAMPS defined: libenargeia_hip_prof.so) carries the
// stamps. Even switched off at run time their code costs every kernel: measured on MI355X, the
// config-4 decode step ran 1568 tok/s with it compiled in against 1660 without.
#ifdef EG_LAUNCH_STAMPS
struct WaveStamp {
  uint64_t* p = nullptr;
  __device__ __forceinline__ explicit WaveStamp(uint64_t* base) {
    if (base != nullptr && (threadIdx.x & 63u) == 0) {
      const uint32_t block = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
      const uint32_t w = block * (blockDim.x / 64u) + threadIdx.x / 64u;
      if (w < eg::kStampWaves) {
        p = base + 2u * w;
        p[0] = wall_clock64();
      }
    }
  }
  __device__ __forceinline__ ~WaveStamp() {
    if (p != nullptr) p[1] = wall_clock64();
  }
};
constexpr bool kLaunchStamps = true;
#else
struct WaveStamp {
  __device__ __forceinline__ explicit WaveStamp(uint64_t*) {}
};
constexpr bool kLaunchStamps = false;
#endif

// (value, index) ordering used by every argmax here: larger value wins, ties go to the lower
// index (argmax.wgsl:53-57, sample.wgsl:181-186).
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

template <int WIDTH>
__device__ __forceinline__ void team_argmax(float& v, uint32_t& i) {
#pragma unroll
  for (int m = WIDTH / 2; m > 0; m >>= 1) {
    float ov = __shfl_xor(v, m, 64);
    uint32_t oi = __shfl_xor(i, m, 64);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// mulberry32 (session.ts:75-83): the next draw from `state` as the f32 the reference's uniform
// carries (u / 2^32 rounded to f32; rounding u to 24 bits then scaling by the power of two 2^-32
// rounds identically), without advancing the state ...
__device__ __forceinline__ float mulberry32_peek(uint32_t state) {
  const uint32_t s = state + 0x6D2B79F5u;
  uint32_t t = (s ^ (s >> 15)) * (1u | s);
  t = (t + (t ^ (t >> 7)) * (61u | t)) ^ t;
  return (float)(t ^ (t >> 14)) * 0x1p-32f;
}
// ... and advancing it.
__device__ __forceinline__ float mulberry32_next(uint32_t* state) {
  const float r = mulberry32_peek(*state);
  *state += 0x6D2B79F5u;
  return r;
}

// binary16 <-> f32 (round to nearest even), the KV cache's element type.
__device__ __forceinline__ float half_to_float(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t float_to_half(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Element e (= row * hidden + column) of a tied table as f32, per storage format
// (embedding_variants.ts:46-74 weightAt): bits 4 / 8 are codes with the scale of quant block
// `blk` (minus its zero-point for EG_ENC_OFFSET_ZEROS, two's complement for EG_ENC_SIGNED);
// bits 16 an f16 table (two halves per word, element 2j in the low half, as unpack2x16float
// reads it); bits 32 an f32 table. scales and zeros are not read for 16 and 32.
__device__ __forceinline__ float table_value(const uint32_t* packed, const float* scales, const uint32_t* zeros,
                                            uint64_t e, uint64_t blk, int encoding, int bits) {
  if (bits == 32) return __uint_as_float(packed[e]);
  if (bits == 16) return half_to_float((uint16_t)(packed[e >> 1] >> (16u * (uint32_t)(e & 1u))));
  const uint32_t per_word = 32u / (uint32_t)bits, mask = (1u << bits) - 1u;
  uint32_t code = (packed[e / per_word] >> (bits * (uint32_t)(e % per_word))) & mask;
  float zero;
  if (encoding == EG_ENC_OFFSET_ZEROS) {
    zero = (float)((zeros[blk / per_word] >> (bits * (uint32_t)(blk % per_word))) & mask);
  } else {
    code ^= 1u << (bits - 1);  // two's complement -> offset binary
    zero = (float)(1u << (bits - 1));
  }
  return ((float)code - zero) * scales[blk];
}

// RoPE (ops.ts:87-114): pairs (i, i + D/2) rotated by angle = position * theta^(-2i/D). The
// angle, its cosine and sine are computed once per frequency, in double precision like the CPU
// reference, and the rotation itself is evaluated in double too.
template <int D>
__device__ __forceinline__ void rope_table(double2* cs, uint32_t i, uint32_t position, float theta) {
  const double angle = (double)position / pow((double)theta, (2.0 * i) / D);
  cs[i] = make_double2(cos(angle), sin(angle));
}
// Two floats to a packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32 on gfx950). Every
// bf16 rounding of the prompt chain's x goes through it, whether a GEMM's staging or the kernel
// that produced x does it, so both give the same bits.
__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}

// Data one workgroup hands another inside a launch: agent-scope atomic stores and loads (the sc1
// bit on gfx950), which write through and read past the XCD-private caching of ordinary
// accesses - the instructions the memory model's agent-scope atomics use. A writer drains its
// stores before it counts itself (drain, then a relaxed atomic on a counter); a reader that has
// seen the count reads with get. No L2 write-back or invalidate is involved.
template <typename T>
__device__ __forceinline__ void put(T* p, T v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
template <typename T>
__device__ __forceinline__ T get(const T* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// This wave's memory operations issued so far complete before any issued after (the compiler
// keeps them on their side of it: a signal fence on each side of the wait).
__device__ __forceinline__ void drain() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt 0 (loads and stores), expcnt 7, lgkmcnt 15
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// (a, b) rotated by (cos, sin) in double, each product rounded on its own - no fused multiply-add,
// as a host evaluates a * cos - b * sin and b * cos + a * sin - then rounded to f32. Every RoPE
// here goes through it, so a row rotated in any kernel is the same to the bit.
__device__ __forceinline__ float2 rotate(double a, double b, double2 cs) {
#pragma clang fp contract(off)
  return make_float2((float)(a * cs.x - b * cs.y), (float)(b * cs.x + a * cs.y));
}

template <int D>
__device__ __forceinline__ void rope_apply(float* v, uint32_t i, const double2* cs) {
  const float2 r = rotate(v[i], v[i + D / 2], cs[i]);
  v[i] = r.x;
  v[i + D / 2] = r.y;
}

}  // namespace egd
