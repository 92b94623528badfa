// sample (sample.wgsl:143-332): repetition penalty in place, then greedy argmax or
// temperature / top-p / seeded draw, all on the GPU; out[0] is the only result.
//
// Semantics kept from the reference:
//   * penalty applied once per distinct history id < vocab (first occurrence), in place:
//     v > 0 ? v / penalty : v * penalty (sample.wgsl:91-113);
//   * temperature <= 0: argmax, ties to the lowest id (:165-195);
//   * p_i = exp(l_i / T - max) / sum, all in f32 (:230-236, :248);
//   * nucleus threshold = 32 bisection steps on [0, 1] with f32 mids (lo + hi) * 0.5 and the
//     rule mass(p >= mid) < topP ? hi = mid : lo = mid (:241-261); threshold 0 when topP >= 1;
//   * target = random * max(kept, 1e-20); the token is the first id, in ascending order, whose
//     running kept mass reaches the target (:266-321); argmax fallback (:324-331).
//
// MI355X design. The reference makes ~36 passes over the vocabulary inside one workgroup. Here
// the vocabulary is split over G workgroups (2048 ids each, G = 75 at 151,936 ids) that are all
// resident at once, and the whole sample is ONE launch whose phases are separated by grid
// barriers (an arrival counter that only grows during the launch and a generation word; every
// wait bounded; what workgroups hand
// each other moves through device-coherent accesses, so a barrier only drains stores and needs
// no cache write-back or invalidate): each workgroup loads its slice's logits once and keeps
// them - and later their probabilities - in registers through every phase:
//   penalty on the slice (a hit mask of the history ids it owns), the slice's (max, argmax)
//     of l/T (of l when greedy) and its sum of exp(l/T - its own max) in float64   | barrier
//   global max (greedy: the token, done); the normaliser sum_g s_g e^(m_g - max)
//   the threshold: the 32 bisection steps compare mass(p >= mid) with topP, and mass(p >= m) is
//     a non-increasing step function of m, so mass(p >= mid) < topP exactly when mid lies above
//     p* = the largest probability whose mass(p >= p*) reaches topP: the steps' path, and the
//     threshold lo it ends on, follow from p* alone. p* is found by radix selection on the bits
//     of p (a p in [0, 1] has 30 significant bits): 3 levels of 10 bits, each a histogram of
//     the masses of the candidates by their next 10 bits, summed over the workgroups with
//     integer atomics; after the barrier every workgroup takes the highest bin whose
//     cumulative mass from the top reaches topP                                  | barrier x 3
//   the slices' kept masses (p >= the threshold): the last level also publishes each slice's
//     mass above its candidate range and lists the candidates themselves (up to 32 per slice),
//     so when the threshold shares the candidates' prefix every workgroup derives them with no
//     further barrier; otherwise (top-p 1, ties filling the list) each slice sums its own
//                                                                                  | barrier
//   the target and the first slice whose kept prefix reaches it; that slice's workgroup finds
//     the id in ascending order.
// Masses are fixed-point integers (p * 2^52, exact for p >= 2^-28) summed with integer adds, so
// every mass is independent of summation order and the result is deterministic. They differ
// from the reference's f32 tree sums only by rounding, which can change a decision only when
// a mass is within ~1e-7 of topP or the target within ~1e-7 of a cumulative boundary.
// A barrier that times out (a workgroup that never became resident) raises an abort flag that
// every wait also reads; every workgroup then leaves, and the last to leave sets the result to
// 0xFFFFFFFF (also stored before the first barrier, the result of every path that never reaches
// the final store) and adds 1 to the launch's status word, which the host reads as an error.
#include <algorithm>

#include "eg_internal.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 8;
constexpr int kWaves = kThreads / 64;
constexpr uint32_t kSlice = kThreads * kPerThread;  // vocabulary ids per workgroup
constexpr uint32_t kMaxGroups = 256;                // vocab <= 524,288 (one group per thread in the final scan)
constexpr int kRadixBits = 10;                      // bits of p selected per level
constexpr int kBins = 1 << kRadixBits;
constexpr int kLevels = 3;                          // 3 x 10 bits: every bit of a p in [0, 1]
constexpr double kFix = 4503599627370496.0;         // 2^52

struct SampleParams {
  uint32_t vocab, history_length;
  float temperature, top_p, repetition_penalty, random;
  uint32_t pad0, pad1;
};
static_assert(sizeof(SampleParams) == 32, "sample dims are 32 bytes");

constexpr uint32_t kCand = 32;  // candidates of the last radix level kept per group
constexpr uint32_t kMaxHeadGroups = 2048;                 // LM-head partials a launch reduces
constexpr uint32_t kHeadPer = kMaxHeadGroups / kThreads;  // per thread
constexpr size_t kHeadPartialsOffset = 1u << 20;          // in the workspace, past the sampler's own data

struct Work {
  uint32_t* max_part;     // 2 u32 per group
  double* sum_part;       // 1 per group
  unsigned long long* bins;  // kLevels x kBins, summed over groups by integer atomics
  uint64_t* kept_part;    // 1 per group
  uint32_t* count_part;   // 1 per group
  uint64_t* above_part;   // 1 per group: mass above the last level's candidate range
  uint32_t* above_count;  // 1 per group: ids above it
  uint32_t* cand_count;   // 1 per group: ids inside it (only the first kCand are stored)
  unsigned long long* cand;  // kCand per group: bits of p << 32 | id
};

__device__ __forceinline__ uint64_t to_fix(float p) { return (uint64_t)__double2ull_rn((double)p * kFix); }

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++) r += scratch[w];
  __syncthreads();
  return r;
}

__device__ __forceinline__ void block_argmax(float& v, uint32_t& i, float* sv, uint32_t* si) {
  egd::team_argmax<64>(v, i);
  if ((threadIdx.x & 63) == 0) {
    sv[threadIdx.x >> 6] = v;
    si[threadIdx.x >> 6] = i;
  }
  __syncthreads();
  v = sv[0];
  i = si[0];
#pragma unroll
  for (int w = 1; w < kWaves; w++)
    if (egd::better(sv[w], si[w], v, i)) {
      v = sv[w];
      i = si[w];
    }
  __syncthreads();
}

// Exclusive prefix sum of one u64 per thread over the workgroup, in thread order; *total gets
// the sum of all. Wave scan by shuffles, then the wave totals.
__device__ unsigned long long block_exclusive_scan(unsigned long long v, unsigned long long* total) {
  __shared__ unsigned long long wsum[kWaves];
  const int lane = threadIdx.x & 63;
  unsigned long long incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const unsigned long long o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) wsum[threadIdx.x >> 6] = incl;
  __syncthreads();
  unsigned long long before = 0, all = 0;
#pragma unroll
  for (int w = 0; w < kWaves; w++) {
    if (w < (int)(threadIdx.x >> 6)) before += wsum[w];
    all += wsum[w];
  }
  __syncthreads();
  if (total) *total = all;
  return before + incl - v;
}

// ---- cross-workgroup data and the grid barrier -----------------------------------------------

// Everything one workgroup hands another inside the launch moves through device-coherent
// accesses (egd::put / egd::get: agent-scope atomic stores and loads), and the only thing a
// barrier then has to order is that every such store of a workgroup has completed before the
// workgroup is counted: each wave drains its stores (egd::drain) before the workgroup's
// s_barrier, and thread 0 counts it after. No L2 write-back or invalidate is needed (the
// release/acquire fences that do them cost ~2.5 us per barrier here), and no ordinary load ever
// reads data another workgroup wrote in this launch.
using egd::drain;
using egd::get;
using egd::put;
__device__ __forceinline__ void put_f64(double* p, double v) {
  put(reinterpret_cast<unsigned long long*>(p), __builtin_bit_cast(unsigned long long, v));
}
__device__ __forceinline__ double get_f64(const double* p) {
  return __builtin_bit_cast(double, get(reinterpret_cast<const unsigned long long*>(p)));
}

// Central barrier over the launch's workgroups: thread 0 of each counts the workgroup once its
// waves have drained their stores. The count only grows during a launch (the last workgroup to
// leave zeroes it), so the launch's barrier b is complete at (b + 1) x groups arrivals; the
// arrival that completes it finds that in its own atomic's result and advances the generation
// word - which only grows, launch after launch - to gen0 + b + 1, gen0 being the value every
// workgroup read at the launch's start; the others poll the generation (a line of its own: polls
// of the counter itself slow the arrivals, measured). On the way through, a workgroup makes one
// atomic round trip, and the last arrival one store. Polls are bounded: past `spin`, or when
// another workgroup has given up, the abort flag is raised and false is returned to every thread.
constexpr uint32_t kSpin = 1u << 20;  // polls of ~1 us: a barrier gives up after about a second

struct GridSync {
  uint32_t* count;  // arrivals since the launch began (zero between launches)
  uint32_t* gen;    // advanced once per completed barrier, never reset
  uint32_t* abort;  // set by a timed-out wait
  uint32_t* exits;  // workgroups done with every barrier of the current launch
  uint32_t* status; // +1 per launch that gave up (nullable: the caller counts from out[0])
  // polls before a wait gives up: kSpin while this word is 0, else its value - 1 (the context's
  // test hook sets it; read at every barrier, so a captured graph follows it too)
  const uint32_t* spin;
};

// `passed` counts the barriers this workgroup has passed in the launch (the same at every thread);
// `gen0` is the generation thread 0 read at the launch's start (the barrier's drain completes that
// read before the first arrival).
__device__ bool grid_barrier(const GridSync& g, uint32_t groups, uint32_t& passed, uint32_t gen0) {
  __shared__ uint32_t ok;
  drain();
  __syncthreads();
  passed++;
  if (threadIdx.x == 0) {
    bool good = true;
    const uint32_t target = passed * groups, release = gen0 + passed;
    const uint32_t w = get(g.spin);  // in flight beside the arrival
    const uint32_t arrived = __hip_atomic_fetch_add(g.count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    if (arrived == target) {
      put(g.gen, release);
    } else {
      const uint32_t spin = w ? w - 1u : kSpin;
      uint32_t n = 0;
      for (;;) {
        const uint32_t c = get(g.gen), stop = get(g.abort);  // one round trip for both
        if ((int32_t)(c - release) >= 0) break;
        if (stop != 0u || ++n > spin) {
          good = false;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
    }
    if (!good) {
      put(g.abort, 1u);
      drain();  // completed before this workgroup's exit count
    }
    ok = good ? 1u : 0u;
  }
  __syncthreads();
  return ok != 0u;
}

// Called by every workgroup once it has passed its last barrier or given up. The last to leave
// settles an aborted launch - out[0] = 0xFFFFFFFF, after every workgroup's own store to it (a
// workgroup can time out at the last barrier after a late arrival has released the others, one
// of which may still store a token), and +1 in the status word - then returns the words to their
// starting state, so the next launch needs no reset launch before it and never starts from a
// count or an abort flag left by an aborted one (the context's state starts zeroed). Thread 0
// makes every store to out[0]; it drains them, as a workgroup that raised the abort flag drained
// that store, before counting its exit.
__device__ void leave(const GridSync& g, uint32_t groups, uint32_t* out) {
  if (threadIdx.x == 0) {
    drain();
    const uint32_t left = __hip_atomic_fetch_add(g.exits, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (left == groups - 1) {
      if (get(g.abort) != 0u) {
        put(out, 0xFFFFFFFFu);
        if (g.status) __hip_atomic_fetch_add(g.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      put(g.count, 0u);
      put(g.abort, 0u);
      put(g.exits, 0u);
    }
  }
}

// ---- the launch --------------------------------------------------------------------------------

// Thread t of workgroup g owns ids g * kSlice + t * kPerThread + [0, kPerThread): thread order is
// id order, which the final scan relies on.
// Every return is taken by a whole workgroup at once.
// `head` (nullable): the LM head's per-workgroup partials (eg::lm_head_sample_partials), head_groups
// of them, which replace the penalty and the slices' first pass.
__device__ __forceinline__ void sample_phases(float* logits, const uint32_t* history, uint32_t* out, SampleParams hp,
                                              SampleParams* dp, const Work& w, const GridSync& gs, uint32_t* rng,
                                              const uint4* head, uint32_t head_groups) {
  const uint32_t G = gridDim.x, g = blockIdx.x, tid = threadIdx.x;
  uint32_t passed = 0;  // grid barriers passed
  const uint32_t gen0 = tid == 0 ? get(gs.gen) : 0u;  // the generation before this launch's barriers
  if (g == 0 && tid == 0) {
    // The give-up result, replaced by the token once one is found. Both are stored coherently
    // (out[0] is written by two workgroups, possibly on different XCDs), and this one completes
    // before the first barrier counts workgroup 0, so it always precedes the token.
    put(out, 0xFFFFFFFFu);
    // This call's draw (one per sampled step, Session.decodeStep session.ts:351) from the
    // mulberry32 state, which the caller advances once the step has its token: taken by
    // workgroup 0 before the first barrier, read by everyone after it.
    if (rng && dp) put(&dp->random, egd::mulberry32_peek(*rng));
  }
  SampleParams p = dp ? *dp : hp;  // `random` is read again after the first barrier (below)
  const uint32_t base = g * kSlice, first = base + tid * kPerThread;
  const uint32_t end = min(base + kSlice, p.vocab);
  float v[kPerThread];
#pragma unroll
  for (int r = 0; r < kPerThread; r += 4) {
    if (first + r + 4 <= p.vocab) {
      const float4 q = *reinterpret_cast<const float4*>(logits + first + r);
      v[r] = q.x;
      v[r + 1] = q.y;
      v[r + 2] = q.z;
      v[r + 3] = q.w;
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) v[r + e] = first + r + e < p.vocab ? logits[first + r + e] : 0.f;
    }
  }
  const bool greedy = p.temperature <= 0.0f;
  float mx;
  uint32_t amax;
  float total;
  if (head) {
    // The LM head applied the penalty and left per-workgroup partials (max of l/T - of l when
    // greedy - its lowest index, float64 sum of exp(l/T - that max)): the global max, its index
    // and the normaliser come from them, with no pass over the slice and no barrier first.
    // Level 0's bins were zeroed by the head launch; the other levels' are cleared here, before
    // workgroup 0's first arrival, which orders them before any of their adds.
    if (g == 0)
      for (int i = kBins + tid; i < kLevels * kBins; i += kThreads) put(&w.bins[i], 0ull);
    if (rng && dp) p.random = egd::mulberry32_peek(*rng);  // the draw workgroup 0 records
    __shared__ float sv[kWaves];
    __shared__ uint32_t si[kWaves];
    __shared__ double scratch[kWaves];
    uint4 hq[kHeadPer];
#pragma unroll
    for (uint32_t r = 0; r < kHeadPer; r++) {
      const uint32_t i = tid + r * kThreads;
      hq[r] = i < head_groups ? head[i] : make_uint4(0u, 0u, 0u, 0u);
    }
    float bv = -1.0e30f;
    uint32_t bi = 0;
#pragma unroll
    for (uint32_t r = 0; r < kHeadPer; r++)
      if (tid + r * kThreads < head_groups && egd::better(__uint_as_float(hq[r].x), hq[r].y, bv, bi)) {
        bv = __uint_as_float(hq[r].x);
        bi = hq[r].y;
      }
    block_argmax(bv, bi, sv, si);
    mx = bv;
    amax = bi;
    if (greedy) {
      if (g == 0 && tid == 0) put(out, amax);
      return;
    }
    double s = 0.0;
#pragma unroll
    for (uint32_t r = 0; r < kHeadPer; r++)
      if (tid + r * kThreads < head_groups)
        s += __builtin_bit_cast(double, (uint64_t)hq[r].z | ((uint64_t)hq[r].w << 32)) *
             exp((double)__uint_as_float(hq[r].x) - (double)mx);
    total = (float)block_sum(s, scratch);
  } else {
    const bool penalize = p.repetition_penalty != 1.0f;
    // the first kHistory x 256 history ids, read beside the logits (one round trip for both)
    constexpr uint32_t kHistory = 4;
    uint32_t hv[kHistory];
#pragma unroll
    for (uint32_t r = 0; r < kHistory; r++) {
      const uint32_t h = tid + r * kThreads;
      hv[r] = penalize && h < p.history_length ? history[h] : 0xFFFFFFFFu;
    }
    if (penalize) {
      // The penalty applies once per distinct history id (the reference applies it at an id's
      // first occurrence only): mark the ids this slice owns, then penalize each marked element
      // once, in registers and in place in memory.
      __shared__ uint8_t hit[kSlice];
      for (uint32_t i = tid; i < kSlice; i += kThreads) hit[i] = 0;
      __syncthreads();
#pragma unroll
      for (uint32_t r = 0; r < kHistory; r++)
        if (hv[r] >= base && hv[r] < end) hit[hv[r] - base] = 1;
      for (uint32_t h = tid + kHistory * kThreads; h < p.history_length; h += kThreads) {
        const uint32_t id = history[h];
        if (id >= base && id < end) hit[id - base] = 1;
      }
      __syncthreads();
#pragma unroll
      for (int r = 0; r < kPerThread; r++) {
        const uint32_t i = first + r;
        if (i < end && hit[i - base]) {
          v[r] = v[r] > 0.0f ? v[r] / p.repetition_penalty : v[r] * p.repetition_penalty;
          logits[i] = v[r];
        }
      }
    }
    {
      // the slice's (max, argmax) of l/T (of l when greedy) and its sum of exp(l/T - that max)
      __shared__ float sv[kWaves];
      __shared__ uint32_t si[kWaves];
      __shared__ double scratch[kWaves];
      float bv = -1.0e30f;
      uint32_t bi = greedy ? 0u : base;
#pragma unroll
      for (int r = 0; r < kPerThread; r++) {
        const uint32_t i = first + r;
        const float x = greedy ? v[r] : v[r] / p.temperature;
        if (i < end && egd::better(x, i, bv, bi)) {
          bv = x;
          bi = i;
        }
      }
      block_argmax(bv, bi, sv, si);
      double s = 0.0;
      if (!greedy) {
#pragma unroll
        for (int r = 0; r < kPerThread; r++)
          if (first + r < end) s += (double)expf(v[r] / p.temperature - bv);
        s = block_sum(s, scratch);
      }
      if (tid == 0) {
        put(&w.max_part[2 * g], __float_as_uint(bv));
        put(&w.max_part[2 * g + 1], bi);
        put_f64(&w.sum_part[g], s);
      }
    }
    // the level bins are summed with atomics: cleared here, before the barrier that orders them
    // before any level adds to them
    if (g == 0)
      for (int i = tid; i < kLevels * kBins; i += kThreads) put(&w.bins[i], 0ull);
    if (!grid_barrier(gs, G, passed, gen0)) return;  // out[0] keeps the give-up result
    if (dp) p.random = __hip_atomic_load(&dp->random, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // this call's draw
    {
      __shared__ float sv[kWaves];
      __shared__ uint32_t si[kWaves];
      __shared__ double scratch[kWaves];
      float bv = -1.0e30f, mg = -1.0e30f;
      uint32_t bi = 0;
      double sg = 0.0;
      if (tid < G) {
        bv = mg = __uint_as_float(get(&w.max_part[2 * tid]));
        bi = get(&w.max_part[2 * tid + 1]);
        sg = get_f64(&w.sum_part[tid]);
      }
      block_argmax(bv, bi, sv, si);
      mx = bv;
      amax = bi;
      if (greedy) {
        if (g == 0 && tid == 0) put(out, amax);
        return;
      }
      // the normaliser: every slice's sum rescaled from its own max to the global one
      total = (float)block_sum(tid < G ? sg * exp((double)mg - (double)mx) : 0.0, scratch);
    }
  }
  // p = exp(l/T - max) / total in registers; ids past the vocabulary get -1 (never kept)
#pragma unroll
  for (int r = 0; r < kPerThread; r++) v[r] = first + r < end ? expf(v[r] / p.temperature - mx) / total : -1.0f;
  float thr = 0.0f;
  // thread t < G: group t's mass and count above the last level's candidate range, and the
  // number of its candidates
  unsigned long long g_above = 0;
  uint32_t g_above_n = 0, g_cand_n = 0;
  bool listed = false;  // the kept set is the ids above the candidate range + listed candidates
  if (p.top_p < 1.0f) {
    // p*: radix selection over the 30 significant bits of p, 10 per level. `prefix` holds the
    // selected bits so far, `above` the mass of every p above the candidates (integer masses).
    __shared__ unsigned long long bins[kBins];
    __shared__ uint32_t sel;
    __shared__ unsigned long long sel_above;
    const double need = (double)p.top_p * kFix;
    uint32_t prefix = 0, cand_prefix = 0;
    unsigned long long above = 0;
    bool last_done = false;  // the last level ran: its candidates and masses above were published
    // topP <= 0: every mass reaches it, so every step moves lo up (p* above everything)
    bool found = need > 0.0;
    if (!found) prefix = 0x7F800000u;  // +inf
    for (int level = 0; level < kLevels && need > 0.0 && found; level++) {
      const int shift = kRadixBits * (kLevels - 1 - level);
      const bool last = level == kLevels - 1;
      __shared__ unsigned long long above_g;
      __shared__ uint32_t above_n, cand_n;
      for (int i = tid; i < kBins; i += kThreads) bins[i] = 0;
      if (tid == 0) {
        sel = 0xFFFFFFFFu;
        above_g = 0;
        above_n = 0;
        cand_n = 0;
      }
      __syncthreads();
      // runs of equal bins summed in registers before the LDS atomic
      int run_bin = -1;
      unsigned long long run_mass = 0, up_mass = 0;
      uint32_t up_n = 0;
#pragma unroll
      for (int r = 0; r < kPerThread; r++) {
        if (!(v[r] >= 0.0f)) continue;
        const uint32_t bits = __float_as_uint(v[r]);
        if ((bits >> (shift + kRadixBits)) != prefix) {
          // the last level also counts what lies above its range and lists its candidates, so
          // the slices' kept masses follow from the selection without another barrier
          if (last && (bits >> (shift + kRadixBits)) > prefix) {
            up_mass += to_fix(v[r]);
            up_n++;
          }
          continue;
        }
        if (last) {
          const uint32_t slot = atomicAdd(&cand_n, 1u);
          if (slot < kCand) put(&w.cand[(size_t)g * kCand + slot], ((unsigned long long)bits << 32) | (first + r));
        }
        const int k = (int)((bits >> shift) & (kBins - 1));
        if (k != run_bin) {
          if (run_bin >= 0) atomicAdd(&bins[run_bin], run_mass);  // integer adds: order-independent
          run_bin = k;
          run_mass = 0;
        }
        run_mass += to_fix(v[r]);
      }
      if (run_bin >= 0) atomicAdd(&bins[run_bin], run_mass);
      if (last) {
#pragma unroll
        for (int m = 32; m > 0; m >>= 1) {
          up_mass += __shfl_xor(up_mass, m, 64);
          up_n += __shfl_xor(up_n, m, 64);
        }
        if ((tid & 63) == 0 && up_n) {
          atomicAdd(&above_g, up_mass);
          atomicAdd(&above_n, up_n);
        }
      }
      __syncthreads();
      unsigned long long* summed = w.bins + (size_t)level * kBins;
      for (int i = tid; i < kBins; i += kThreads)
        if (bins[i]) __hip_atomic_fetch_add(&summed[i], bins[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (last && tid == 0) {
        put(&w.above_part[g], (uint64_t)above_g);
        put(&w.above_count[g], above_n);
        put(&w.cand_count[g], cand_n);
      }
      if (!grid_barrier(gs, G, passed, gen0)) return;
      if (last) {
        // every group's figures for the kept masses below (loaded here, beside the bins)
        last_done = true;
        cand_prefix = prefix;
        if (tid < G) {
          g_above = get(&w.above_part[tid]);
          g_above_n = get(&w.above_count[tid]);
          g_cand_n = get(&w.cand_count[tid]);
        }
      }
      // cum(k) = above + mass of bins >= k; the selected bin is the highest k with cum(k) >=
      // topP (cum grows as k falls). Thread t holds bins kBins - 4 (t + 1) .. kBins - 4 t - 1,
      // so thread order runs from the top bin down and an exclusive scan gives each thread the
      // mass above its bins.
      constexpr int kPer = kBins / kThreads;
      static_assert(kBins % kThreads == 0, "whole bins per thread");
      unsigned long long m[kPer], part = 0;
#pragma unroll
      for (int j = 0; j < kPer; j++) {
        m[j] = get(&summed[kBins - 1 - (tid * kPer + j)]);  // descending bin order
        part += m[j];
      }
      unsigned long long cum = above + block_exclusive_scan(part, nullptr);
#pragma unroll
      for (int j = 0; j < kPer; j++) {
        const unsigned long long prev = cum;
        cum += m[j];
        if ((double)prev < need && (double)cum >= need) {
          sel = (uint32_t)(kBins - 1 - (tid * kPer + j));
          sel_above = prev;  // the mass above the selected bin
        }
      }
      __syncthreads();
      if (sel == 0xFFFFFFFFu) {
        found = false;  // the whole mass falls short of topP (rounding): no p*, threshold 0
      } else {
        above = sel_above;
        prefix = (prefix << kRadixBits) | sel;
      }
      __syncthreads();
    }
    // the 32 bisection steps: mass(p >= mid) < topP exactly when mid > p*
    if (found || need <= 0.0) {
      const float pstar = __uint_as_float(prefix);
      float lo = 0.0f, hi = 1.0f;
      for (int step = 0; step < 32; step++) {
        const float mid = (lo + hi) * 0.5f;
        if (mid > pstar) hi = mid;
        else lo = mid;
      }
      thr = lo;
    }
    // When thr has the candidates' prefix, every id above their range is kept, every id below
    // it is not, and the candidates are decided one by one: the slices' kept masses come from
    // the published figures. Otherwise (thr from a failed selection, or a group with more
    // candidates than it stored) they are summed and exchanged through one more barrier.
    listed = last_done && found && (__float_as_uint(thr) >> kRadixBits) >= cand_prefix;
    listed = !__syncthreads_or(!listed || (tid < G && g_cand_n > kCand));
  }
  // the slice's kept mass and count
  unsigned long long mine = 0;
  uint32_t cnt = 0;
#pragma unroll
  for (int r = 0; r < kPerThread; r++)
    if (v[r] >= thr) {
      mine += to_fix(v[r]);
      cnt++;
    }
  unsigned long long gk = 0;
  uint32_t gc = 0;
  if (listed) {
    if (tid < G) {
      gk = g_above;
      gc = g_above_n;
      for (uint32_t c = 0; c < g_cand_n; c++) {
        const float pc = __uint_as_float((uint32_t)(get(&w.cand[(size_t)tid * kCand + c]) >> 32));
        if (pc >= thr) {
          gk += to_fix(pc);
          gc++;
        }
      }
    }
  } else {
    __shared__ unsigned long long ks[kWaves];
    __shared__ uint32_t cs[kWaves];
    const unsigned long long kept = block_sum(mine, ks);
    const uint32_t count = block_sum(cnt, cs);
    if (tid == 0) {
      put(&w.kept_part[g], (uint64_t)kept);
      put(&w.count_part[g], count);
    }
    if (!grid_barrier(gs, G, passed, gen0)) return;
    if (tid < G) {
      gk = get(&w.kept_part[tid]);
      gc = get(&w.count_part[tid]);
    }
  }
  // Kept mass per slice in id order: the target, then the first slice whose inclusive prefix
  // reaches it (and that keeps something, so a zero target still lands on a kept id). Every
  // workgroup derives the same slice; only that slice's workgroup (or, with none, workgroup 0)
  // goes on.
  __shared__ uint32_t pick_group, pick;
  __shared__ unsigned long long group_prefix;
  unsigned long long all = 0;
  const unsigned long long gbefore = block_exclusive_scan(gk, &all);
  double kd = (double)all / kFix;
  if (kd < 1.0e-20) kd = 1.0e-20;
  const double target_fx = (double)p.random * kd * kFix;
  if (tid == 0) {
    pick_group = 0xFFFFFFFFu;
    pick = 0xFFFFFFFFu;
  }
  __syncthreads();
  if (tid < G && gc > 0 && (double)(gbefore + gk) >= target_fx) atomicMin(&pick_group, tid);
  __syncthreads();
  if (tid == pick_group) group_prefix = gbefore;
  __syncthreads();
  if (pick_group == 0xFFFFFFFFu) {
    if (g == 0 && tid == 0) put(out, amax);
    return;
  }
  if (g != pick_group) return;
  unsigned long long run = group_prefix + block_exclusive_scan(mine, nullptr);
#pragma unroll
  for (int r = 0; r < kPerThread; r++) {
    if (v[r] >= thr) {
      run += to_fix(v[r]);
      if ((double)run >= target_fx) {
        atomicMin(&pick, first + r);
        break;
      }
    }
  }
  __syncthreads();
  if (tid == 0) put(out, pick != 0xFFFFFFFFu ? pick : amax);
}

__global__ __launch_bounds__(kThreads) void sample_kernel(float* logits, const uint32_t* history, uint32_t* out,
                                                          SampleParams hp, SampleParams* dp, Work w, GridSync gs,
                                                          uint32_t* rng, const uint4* head, uint32_t head_groups,
                                                          uint64_t* stamp_slot) {
  const egd::WaveStamp stamp(stamp_slot);
  sample_phases(logits, history, out, hp, dp, w, gs, rng, head, head_groups);
  leave(gs, gridDim.x, out);
}

// The count of eg_sample launches that gave up, and the test hook's poll limit, in the context's
// state (zeroed at creation).
uint32_t* standalone_status(eg_context* ctx) { return reinterpret_cast<uint32_t*>(eg::state(ctx) + 2048 + 512); }
uint32_t* spin_word(eg_context* ctx) { return eg::wait_limit_word(ctx); }

Work workspace(eg_context* ctx, GridSync* gs) {
  Work w;
  uint32_t* sync = reinterpret_cast<uint32_t*>(eg::state(ctx) + 2048);  // four words, 128 bytes apart
  gs->count = sync;
  gs->gen = sync + 32;
  gs->abort = sync + 64;
  gs->exits = sync + 96;
  uint8_t* part = eg::partials(ctx);
  size_t off = 0;
  w.max_part = reinterpret_cast<uint32_t*>(part + off);
  off += (size_t)kMaxGroups * 8;
  w.sum_part = reinterpret_cast<double*>(part + off);
  off += (size_t)kMaxGroups * 8;
  w.kept_part = reinterpret_cast<uint64_t*>(part + off);
  off += (size_t)kMaxGroups * 8;
  w.count_part = reinterpret_cast<uint32_t*>(part + off);
  off += (size_t)kMaxGroups * 4;
  w.bins = reinterpret_cast<unsigned long long*>(part + off);
  off += (size_t)kLevels * kBins * 8;
  w.above_part = reinterpret_cast<uint64_t*>(part + off);
  off += (size_t)kMaxGroups * 8;
  w.above_count = reinterpret_cast<uint32_t*>(part + off);
  off += (size_t)kMaxGroups * 4;
  w.cand_count = reinterpret_cast<uint32_t*>(part + off);
  off += (size_t)kMaxGroups * 4;
  w.cand = reinterpret_cast<unsigned long long*>(part + off);
  off += (size_t)kMaxGroups * kCand * 8;
  static_assert((size_t)kMaxGroups * (44 + kCand * 8) + (size_t)kLevels * kBins * 8 <= eg::kPartialsBytes,
                "sampler partials exceed the workspace");
  return w;
}

// One launch. All its workgroups must be resident at once (G <= kMaxGroups = 256 workgroups of
// 256 threads and ~12 KB of LDS each fit an MI355X); a device that cannot hold them (fewer CUs,
// a partition) is refused here rather than left to the bounded waits.
int launch(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out, const SampleParams& hp,
           SampleParams* dp, uint32_t* rng, uint32_t* status, const uint4* head = nullptr, uint32_t head_groups = 0) {
  const uint32_t groups = (hp.vocab + kSlice - 1) / kSlice;
  const int per_cu = eg::occupancy_of(ctx, reinterpret_cast<const void*>(sample_kernel));
  if (per_cu > 0 && (uint64_t)per_cu * (uint64_t)ctx->cu_count < groups)
    return eg::fail(ctx, EG_ERR_RANGE,
                    "sample: vocab %u needs %u workgroups resident at once; this device holds %d per CU x %d CUs",
                    hp.vocab, groups, per_cu, ctx->cu_count);
  GridSync gs;
  Work w = workspace(ctx, &gs);
  gs.status = status;
  gs.spin = spin_word(ctx);
  hipLaunchKernelGGL(sample_kernel, dim3(groups), dim3(kThreads), 0, ctx->stream, logits, history, out, hp, dp, w, gs,
                     rng, head, head_groups, eg::stamp_slot(ctx));
  return eg::check_launch(ctx, "sample");
}

// The int8 LM head ahead of the sampler (eg::lm_head_sample_partials: penalty, logits, per-
// workgroup partials), then the sampler on its partials. The partials go past the sampler's own
// data in the workspace, and the head launch zeroes the sampler's level-0 bins, which the
// sampler then sums into with no barrier first.
int head_then_sample(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed, const float* scales,
                     const uint32_t* zeros, float* logits, const eg_embedding_dims* dims, int encoding, int bits,
                     const uint32_t* history, uint32_t* out, const SampleParams& hp, SampleParams* dp, uint32_t* rng,
                     uint32_t* status) {
  static_assert((size_t)kMaxGroups * (44 + kCand * 8) + (size_t)kLevels * kBins * 8 <= kHeadPartialsOffset &&
                    kHeadPartialsOffset + (size_t)kMaxHeadGroups * 16 <= eg::kPartialsBytes,
                "the LM head's partials sit past the sampler's data, inside the workspace");
  GridSync gs;
  Work w = workspace(ctx, &gs);
  uint32_t* parts = reinterpret_cast<uint32_t*>(eg::partials(ctx) + kHeadPartialsOffset);
  uint32_t groups = 0;
  int st = eg::lm_head_sample_partials(ctx, input, packed, scales, zeros, logits, dims, encoding, bits,
                                       reinterpret_cast<const eg_sample_dims*>(dp),
                                       dp ? nullptr : reinterpret_cast<const eg_sample_dims*>(&hp), history, parts,
                                       (size_t)kMaxHeadGroups * 16, reinterpret_cast<uint32_t*>(w.bins), kBins * 2,
                                       &groups);
  if (st != EG_OK) return st;
  return launch(ctx, logits, history, out, hp, dp, rng, status, reinterpret_cast<const uint4*>(parts), groups);
}

}  // namespace

int eg::lm_head_sample_device(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed, const float* scales,
                              const uint32_t* zeros, float* logits, const eg_embedding_dims* dims, int encoding,
                              int bits, const uint32_t* history, uint32_t* out, eg_sample_dims* params, uint32_t* rng,
                              uint32_t* status) {
  if (!logits || !out || !params || !dims) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_sample: NULL argument");
  const uint32_t vocab = dims->row_count;
  if (vocab == 0 || (vocab + kSlice - 1) / kSlice > kMaxGroups || dims->out_offset != 0)
    return eg::fail(ctx, EG_ERR_RANGE, "lm_head_sample: vocab %u (offset %u) outside the sampler's range (1..%u)",
                    vocab, dims->out_offset, kMaxGroups * kSlice);
  SampleParams hp{};
  hp.vocab = vocab;
  return head_then_sample(ctx, input, packed, scales, zeros, logits, dims, encoding, bits, history, out, hp,
                          reinterpret_cast<SampleParams*>(params), rng, status);
}

int eg::launch_sample_device(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out, uint32_t vocab,
                             eg_sample_dims* params, uint32_t* rng, uint32_t* status) {
  static_assert(sizeof(eg_sample_dims) == sizeof(SampleParams), "the device block is the 32-byte sample dims");
  if (!logits || !out || !params) return eg::fail(ctx, EG_ERR_INVALID, "sample: NULL argument");
  if (vocab == 0 || (vocab + kSlice - 1) / kSlice > kMaxGroups)
    return eg::fail(ctx, EG_ERR_RANGE, "sample: vocab %u outside the sampler's range (1..%u)", vocab,
                    kMaxGroups * kSlice);
  SampleParams hp{};
  hp.vocab = vocab;
  return launch(ctx, logits, history, out, hp, reinterpret_cast<SampleParams*>(params), rng, status);
}

extern "C" int eg_lm_head_sample(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                                 const uint32_t* zeros, float* out, const uint32_t* history, uint32_t* token,
                                 const eg_embedding_dims* dims, int encoding, int bits, const eg_sample_dims* sample) {
  const char* op = "lm_head_sample";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!x || !out || !token || !dims || !sample) return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  if (sample->history_length > 0 && !history)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: historyLength %u with no history buffer", op, sample->history_length);
  if (sample->vocab != dims->row_count || dims->out_offset != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: sample vocab %u must equal the head's rows %u at offset 0", op,
                    sample->vocab, dims->row_count);
  if (sample->vocab == 0 || (sample->vocab + kSlice - 1) / kSlice > kMaxGroups)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: vocab %u outside the sampler's range (1..%u)", op, sample->vocab,
                    kMaxGroups * kSlice);
  SampleParams hp;
  std::memcpy(&hp, sample, sizeof(hp));
  eg_gemv_input in{};
  in.kind = EG_INPUT_VECTOR;
  in.x = x;
  const int st = head_then_sample(ctx, &in, packed, scales, zeros, out, dims, encoding, bits, history, token, hp,
                                  nullptr, nullptr, standalone_status(ctx));
  if (st == EG_OK) ctx->sample_used = true;
  return st;
}

int eg::report_sample_failures(eg_context* ctx, const char* op) {
  if (!ctx->sample_used) return EG_OK;
  uint32_t* word = standalone_status(ctx);
  uint32_t failed = 0;
  hipError_t err = hipMemcpyAsync(&failed, word, 4, hipMemcpyDeviceToHost, ctx->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
  if (err == hipSuccess && failed != 0) {
    const uint32_t zero = 0;
    err = hipMemcpyAsync(word, &zero, 4, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);  // `zero` is a stack local
  }
  if (err != hipSuccess) return eg::hip_fail(ctx, err, op);
  if (failed != 0)
    return eg::fail(ctx, EG_ERR_DEVICE,
                    "%s: %u sample launch(es) gave up (a grid barrier timed out: not every workgroup was resident "
                    "at once); their out[0] is 0xFFFFFFFF",
                    op, failed);
  return EG_OK;
}

extern "C" int eg_test_sample_spin(eg_context* ctx, int override, uint32_t polls) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "test_sample_spin: ctx is NULL");
  if (ctx->capturing) return eg::fail(ctx, EG_ERR_STATE, "test_sample_spin: a graph capture is in progress");
  const uint32_t word = override ? std::min(polls, 0xFFFFFFFEu) + 1u : 0u;
  hipError_t err = hipMemcpyAsync(spin_word(ctx), &word, 4, hipMemcpyHostToDevice, ctx->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);  // `word` is a stack local
  return err == hipSuccess ? EG_OK : eg::hip_fail(ctx, err, "test_sample_spin");
}

extern "C" int eg_sample(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out,
                         const eg_sample_dims* dims) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "sample: ctx is NULL");
  if (!logits || !out || !dims) return eg::fail(ctx, EG_ERR_INVALID, "sample: NULL argument");
  if (dims->history_length > 0 && !history)
    return eg::fail(ctx, EG_ERR_INVALID, "sample: historyLength %u with no history buffer", dims->history_length);
  if (dims->vocab == 0) return eg::fail(ctx, EG_ERR_INVALID, "sample: vocab is 0");
  if ((dims->vocab + kSlice - 1) / kSlice > kMaxGroups)
    return eg::fail(ctx, EG_ERR_RANGE, "sample: vocab %u exceeds the sampler's limit of %u", dims->vocab,
                    kMaxGroups * kSlice);
  SampleParams hp;
  std::memcpy(&hp, dims, sizeof(hp));
  const int st = launch(ctx, logits, history, out, hp, nullptr, nullptr, standalone_status(ctx));
  if (st == EG_OK) ctx->sample_used = true;
  return st;
}
