// The decode step's 24 layers as ONE persistent launch.
//
// Launched one kernel per op, a decode step is a chain of 120 dependent launches per token (per
// layer: the q|k|v GEMV, the attention, the o GEMV, the gate|up pair, the down GEMV), each a few
// microseconds of latency-bound work followed by ~1.5 us before the next one starts. Here one
// launch of G workgroups - all resident at once, G fixed by the device's occupancy - runs the
// same 120 phases in order. A phase is the same device code as the op's own launch (the GEMV body
// of eg_gemv_kernel.hpp, the attention body of eg_attention.hpp) over a virtual grid of the
// phase's workgroups; workgroup w takes part in phase p when w is below the phase's grid. Between
// phases, instead of a launch boundary:
//   * each taking part workgroup, once its stores have completed, counts itself in the phase's
//     arrival counters (8 of them, one per XCD group w % 8, 128 bytes apart, so the arrivals of
//     the 8 XCDs do not serialise on one word);
//   * a workgroup that takes part in the next phase first issues that phase's weight loads (or,
//     for the attention, its chunk of the KV cache) - inputs of the launch, not of the previous
//     phase - and only then waits for the previous phase's counters to reach their totals, so its
//     weights travel while the previous phase finishes;
//   * everything one phase hands the next (the projections, the attention partials, the residual
//     stream, the SwiGLU vector) is written and read with agent-scope coherent accesses (sc1),
//     which bypass the XCD-private caching of ordinary accesses: no cache write-back or
//     invalidate is needed between phases.
// Every phase waits for the one before it (a strict chain), so a buffer is rewritten only after
// every reader of its previous contents has finished. Waits are bounded: a workgroup whose wait
// times out raises the abort flag, which every wait also reads; the launch then runs to its end
// without waiting (its results are garbage) and the step tail, which reads the flag, treats the
// step as failed and moves nothing. The step tail also zeroes the counters for the next launch.
//
// Results are bit-identical to the per-op launches: every output element is computed by the same
// code, in the same order, whatever grid runs it.
//
// Measured on MI355X (config 4, 2048 context, graph replay with a readback per token) this launch
// is ~7% SLOWER than the per-op launches (1466-1481 tok/s against 1566-1577, over grids of 128 to
// 512 workgroups and poll intervals of 0 to 32 sleeps): a phase hand-off - stores drained, an
// arrival, the next phase's poll seeing it, its coherent input reads - costs as much as the launch
// boundary it replaces. It is therefore opt-in (EG_DECODE_PERSISTENT=1), kept as a tested,
// bit-exact alternative.
#include <algorithm>
#include <vector>

#include "eg_attention.hpp"
#include "eg_gemv_kernel.hpp"

namespace {

using namespace eg_gemv;

constexpr uint32_t kKinds = 5;            // phases per layer: q|k|v, attention, o, gate|up, down
constexpr uint32_t kGroups = 8;           // arrival counters per phase (XCD groups)
constexpr uint32_t kCounterStride = 32;   // words between counters
constexpr uint32_t kSpin = 1u << 20;      // polls of ~1 us: a wait gives up after about a second
constexpr uint32_t kMaxGrid = 512;        // workgroups of the launch at most (two per CU)
// workgroups of the launch by default: one per CU measured fastest on MI355X (config 4: 1466
// tok/s against 1398 at two per CU, 1418 at 384 and 1441 at 128)
constexpr uint32_t kDefaultGrid = 256;
constexpr uint32_t kAttnChunk = 128;      // decode attention: positions per workgroup
constexpr uint32_t kAttnSplit = 4;        // decode attention: workgroups per kv head

// The launch's arguments beside the table of GEMV arguments (kernel parameter `tab`: per layer,
// the q|k|v, o, gate|up and down phases as their own launches would take them - read per layer,
// so what a phase needs is loaded in that phase instead of being held across the whole launch).
struct Persist {
  uint32_t nlayers;
  // the attention phase
  const uint32_t* position;
  const double2* rope;
  const float *q, *k, *v;
  float* partials;
  eg_attention_dims att;
  uint16_t *k_cache, *v_cache;  // layer 0's rows; layer l's are layer_stride elements further
  size_t layer_stride;
  // synchronisation
  uint32_t* counters;  // [nlayers * kKinds][kGroups], kCounterStride words apart
  uint32_t* abort;
  const uint32_t* limit;  // the wait limit (eg::wait_limit_word): 0 = kSpin, else limit + 1
  uint32_t poll_sleep;               // s_sleep 1 (64 clocks) between polls, this many times
  uint32_t grid[kKinds];             // workgroups taking part in each phase kind
  uint32_t expect[kKinds][kGroups];  // of those, per XCD group (w % kGroups)
  uint64_t* stamp;
  // With launch stamps (eg_test_launch_stamps), 4 words per phase p: ~(the first wall-clock time
  // a workgroup passed its wait) at phases[4 p], the last such time at phases[4 p + 1] and the
  // last arrival at phases[4 p + 2] (atomic maxima: the caller zeroes them before the launch)
  uint64_t* phases;
};

__device__ __forceinline__ uint32_t* counter_of(const Persist& p, uint32_t phase, uint32_t g) {
  return p.counters + ((size_t)phase * kGroups + g) * kCounterStride;
}

// Waits, with every thread of the workgroup, until phase `phase` has completed (each of its
// counters at its total), unless the abort flag is up; a wait that times out raises it.
__device__ void wait_for(const Persist& p, uint32_t phase) {
  if (threadIdx.x == 0) {
    const uint32_t kind = phase % kKinds;
    const uint32_t lim = egd::get(p.limit);
    const uint32_t spin = lim ? lim - 1u : kSpin;
    uint32_t n = 0;
    bool waiting = egd::get(p.abort) == 0u;
    if (waiting && spin == 0u) {  // the test hook's limit 0: a wait gives up without polling
      egd::put(p.abort, 1u);
      waiting = false;
    }
    while (waiting) {
      uint32_t v[kGroups];
#pragma unroll
      for (uint32_t g = 0; g < kGroups; g++) v[g] = egd::get(counter_of(p, phase, g));
      bool done = true;
#pragma unroll
      for (uint32_t g = 0; g < kGroups; g++) done = done && v[g] >= p.expect[kind][g];
      if (done) break;
      if (egd::get(p.abort) != 0u) break;
      if (++n > spin) {
        egd::put(p.abort, 1u);
        break;
      }
      for (uint32_t i = 0; i < p.poll_sleep; i++) __builtin_amdgcn_s_sleep(1);
    }
    if (egd::kLaunchStamps && p.phases) {
      const uint64_t now = wall_clock64();
      uint64_t* at = p.phases + 4 * (phase + 1);
      __hip_atomic_fetch_max(at, ~now, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_max(at + 1, now, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  __syncthreads();
}

// This workgroup's part of phase `phase` is done: every wave's stores complete, then one arrival.
__device__ __forceinline__ void publish(const Persist& p, uint32_t phase) {
  egd::drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(counter_of(p, phase, blockIdx.x % kGroups), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (egd::kLaunchStamps && p.phases)
      __hip_atomic_fetch_max(p.phases + 4 * phase + 2, (uint64_t)wall_clock64(), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
  }
}

// The run environment of a GEMV phase (see LaunchEnv in eg_gemv_kernel.hpp).
struct GemvPhaseEnv {
  static constexpr int kAux = egd::kCoherent;
  static constexpr bool kPhase = true;
  const Persist* p;
  uint32_t nblocks, after;  // the phase's workgroups; the phase it waits for (~0u: none)
  __device__ __forceinline__ uint32_t block() const { return blockIdx.x; }
  __device__ __forceinline__ uint32_t blocks() const { return nblocks; }
  __device__ __forceinline__ void wait() const {
    if (after != ~0u) wait_for(*p, after);
  }
};

// The run environment of the attention phase (see AttnLaunchEnv in eg_attention.hpp): virtual
// workgroup w is chunk w % chunks of kv-head share w / chunks.
struct AttnPhaseEnv {
  static constexpr int kAux = egd::kCoherent;
  static constexpr bool kPhase = true;
  const Persist* p;
  uint32_t chunks, after;
  __device__ __forceinline__ uint32_t bx() const { return blockIdx.x % chunks; }
  __device__ __forceinline__ uint32_t by() const { return blockIdx.x / chunks; }
  __device__ __forceinline__ uint32_t gx() const { return chunks; }
  __device__ __forceinline__ uint32_t blocks() const { return p->grid[1]; }
  __device__ __forceinline__ void wait() const { wait_for(*p, after); }
};

template <int ENC>
__global__ __launch_bounds__(256) void layers_kernel(const GemvArgs* __restrict__ tab, Persist p) {
  const egd::WaveStamp stamp(p.stamp);
  const uint32_t w = blockIdx.x;
  for (uint32_t l = 0; l < p.nlayers; l++) {
    const GemvArgs* t = tab + 4 * (size_t)l;
    const uint32_t base = kKinds * l;
    if (w < p.grid[0]) {  // q | k | v, RMSNorm(input_layernorm) in the input stage, biases
      gemv_body<4, ENC, 32, 1, 1, 2, kBatched, EG_INPUT_RMSNORM>(t[0], GemvPhaseEnv{&p, p.grid[0], l ? base - 1 : ~0u});
      publish(p, base);
    }
    if (w < p.grid[1]) {  // attention: RoPE, the cache append, split-K partials
      eg_attn::attention_body<64, kAttnChunk, 2, kAttnSplit>(
          p.position, p.q, p.k, p.v, p.k_cache + l * p.layer_stride, p.v_cache + l * p.layer_stride, p.partials,
          nullptr, nullptr, p.att, p.rope, AttnPhaseEnv{&p, p.att.max_context / kAttnChunk, base});
      publish(p, base + 1);
    }
    if (w < p.grid[2]) {  // o, the partials combined in the input stage, the residual as bias
      gemv_body<4, ENC, 32, 1, 1, 2, kBatched, EG_INPUT_ATTENTION>(t[1], GemvPhaseEnv{&p, p.grid[2], base + 1});
      publish(p, base + 2);
    }
    if (w < p.grid[3]) {  // gate | up as the SwiGLU pair, RMSNorm(post_attention_layernorm) in the input stage
      gemv_body<4, ENC, 32, 1, 2, 2, kSwiGLU, EG_INPUT_RMSNORM>(t[2], GemvPhaseEnv{&p, p.grid[3], base + 2});
      publish(p, base + 3);
    }
    if (w < p.grid[4]) {  // down on the SwiGLU vector, the residual as bias
      gemv_body<4, ENC, 64, 3, 1, 2, kBatched, EG_INPUT_VECTOR>(t[3], GemvPhaseEnv{&p, p.grid[4], base + 3});
      publish(p, base + 4);
    }
  }
}

// Zeroes the arrival counters and the abort flag (at decoder creation; the step tail does it
// after every launch).
__global__ void reset_kernel(uint32_t* counters, uint32_t words, uint32_t* abort) {
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < words; i += gridDim.x * blockDim.x) counters[i] = 0u;
  if (blockIdx.x == 0 && threadIdx.x == 0) *abort = 0u;
}

using LayersKernel = void (*)(const GemvArgs*, Persist);

}  // namespace

// The persistent decode layers of one decoder: the kernel arguments, built once.
struct eg_layers {
  Persist args{};
  LayersKernel kernel = nullptr;
  uint32_t grid = 0;
  uint32_t smem = 0;
  GemvArgs* table = nullptr;    // device: 4 per layer
  uint32_t* counters = nullptr; // device, with the abort flag after them
  uint32_t counter_words = 0;
};

namespace {

bool same_shape(const PlanPhase& ph, int mode, int in_kind, int team, int cpl, int u) {
  return ph.bits == 4 && ph.mode == mode && ph.in_kind == in_kind && ph.team == team && ph.cpl == cpl && ph.u == u &&
         ph.nb == 2;
}

}  // namespace

int eg::layers_create(eg_context* ctx, const LayersDesc& d, eg_layers** out) {
  *out = nullptr;
  if (d.layers == 0 || d.layers > 256) return EG_OK;
  const eg_attention_dims& at = d.att;
  if (at.head_dim != 64 || at.chunk != kAttnChunk || at.max_context % kAttnChunk != 0 ||
      at.heads / at.kv_heads > 2 * kAttnSplit || at.heads % at.kv_heads != 0)
    return EG_OK;  // shapes the persistent kernel does not take: the per-op launches run
  const uint32_t attn_grid = at.max_context / kAttnChunk * at.kv_heads * kAttnSplit;
  std::vector<GemvArgs> host(4 * (size_t)d.layers);
  PlanPhase ph[4];
  int st = EG_OK;
  for (uint32_t l = 0; l < d.layers; l++) {
    const LayerPlans& lp = d.plans[l];
    GemvArgs* a = &host[4 * (size_t)l];
    for (int j = 0; j < 4 && st == EG_OK; j++) st = eg_gemv::plan_phase(ctx, lp.plan[j], &lp.input[j], &a[j], &ph[j]);
    if (st != EG_OK) return st;
    const bool ok = same_shape(ph[0], kBatched, EG_INPUT_RMSNORM, 32, 1, 1) && a[0].seg_count <= kInlineSegments &&
                    same_shape(ph[1], kBatched, EG_INPUT_ATTENTION, 32, 1, 1) && a[1].seg_count <= kInlineSegments &&
                    same_shape(ph[2], kSwiGLU, EG_INPUT_RMSNORM, 32, 1, 2) &&
                    same_shape(ph[3], kBatched, EG_INPUT_VECTOR, 64, 3, 1) && a[3].seg_count <= kInlineSegments &&
                    ph[0].encoding == ph[1].encoding && ph[0].encoding == ph[2].encoding &&
                    ph[0].encoding == ph[3].encoding;
    if (!ok) return EG_OK;  // the per-op launches run
  }
  const LayersKernel kernel =
      ph[0].encoding == EG_ENC_OFFSET_ZEROS ? layers_kernel<EG_ENC_OFFSET_ZEROS> : layers_kernel<EG_ENC_SIGNED>;
  uint32_t smem = 0;
  for (int j = 0; j < 4; j++) smem = std::max(smem, ph[j].smem);
  const int per_cu = eg::occupancy_of(ctx, reinterpret_cast<const void*>(kernel), smem);
  const uint32_t want = ctx->persistent_grid ? std::min(ctx->persistent_grid, kMaxGrid) : kDefaultGrid;
  const uint32_t grid = std::min<uint32_t>(want, (uint32_t)std::max(0, per_cu) * (uint32_t)ctx->cu_count);
  if (grid < attn_grid) return EG_OK;  // the attention phase needs a workgroup per virtual one

  eg_layers* L = new eg_layers();
  Persist& p = L->args;
  p.nlayers = d.layers;
  p.poll_sleep = ctx->persistent_poll;
  p.position = d.position;
  p.rope = reinterpret_cast<const double2*>(d.rope);
  p.q = d.q;
  p.k = d.k;
  p.v = d.v;
  p.partials = d.partials;
  p.att = at;
  p.k_cache = d.k_cache;
  p.v_cache = d.v_cache;
  p.layer_stride = d.layer_stride;
  const uint32_t tiles[kKinds] = {ph[0].tiles, 0, ph[1].tiles, ph[2].tiles, ph[3].tiles};
  for (uint32_t j = 0; j < kKinds; j++) {
    // one tile per wave where the grid allows; every workgroup otherwise
    p.grid[j] = j == 1 ? attn_grid : std::min<uint32_t>(grid, (tiles[j] + kWaves - 1) / kWaves);
    for (uint32_t g = 0; g < kGroups; g++) p.expect[j][g] = p.grid[j] / kGroups + (g < p.grid[j] % kGroups ? 1u : 0u);
  }
  L->kernel = kernel;
  L->grid = grid;
  L->smem = smem;
  L->counter_words = (d.layers * kKinds * kGroups) * kCounterStride;
  void* mem = nullptr;
  st = eg_buf_alloc(ctx, sizeof(GemvArgs) * host.size(), &mem);
  if (st == EG_OK) {
    L->table = static_cast<GemvArgs*>(mem);
    st = eg_buf_write(ctx, L->table, 0, host.data(), sizeof(GemvArgs) * host.size());
  }
  if (st == EG_OK) st = eg_buf_alloc(ctx, ((size_t)L->counter_words + kCounterStride) * 4u, &mem);
  if (st == EG_OK) {
    L->counters = static_cast<uint32_t*>(mem);
    hipLaunchKernelGGL(reset_kernel, dim3(64), dim3(256), 0, ctx->stream, L->counters, L->counter_words,
                       L->counters + L->counter_words);
    st = eg::check_launch(ctx, "layers_create");
  }
  if (st == EG_OK) st = eg_sync(ctx);  // the host table is a local
  if (st != EG_OK) {
    layers_destroy(ctx, L);
    return st;
  }
  p.counters = L->counters;
  p.abort = L->counters + L->counter_words;
  p.limit = eg::wait_limit_word(ctx);
  *out = L;
  return EG_OK;
}

int eg::layers_launch(eg_context* ctx, eg_layers* L) {
  Persist p = L->args;
  p.stamp = eg::stamp_slot(ctx);
  // the per-phase stamps after the waves' own (kMaxGrid workgroups of 4 waves take 4096 words)
  p.phases = egd::kLaunchStamps && p.stamp ? p.stamp + eg::kStampWaves : nullptr;
  hipLaunchKernelGGL(L->kernel, dim3(L->grid), dim3(256), L->smem, ctx->stream, L->table, p);
  return eg::check_launch(ctx, "decode_layers");
}

void eg::layers_sync_words(const eg_layers* L, uint32_t** counters, uint32_t* count, uint32_t* stride,
                           uint32_t** abort) {
  *counters = L->counters;
  *count = L->args.nlayers * kKinds * kGroups;
  *stride = kCounterStride;
  *abort = L->counters + L->counter_words;
}

void eg::layers_destroy(eg_context* ctx, eg_layers* L) {
  if (!L) return;
  if (L->table) eg_buf_free(ctx, L->table);
  if (L->counters) eg_buf_free(ctx, L->counters);
  delete L;
}
