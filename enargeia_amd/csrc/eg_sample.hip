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
// the vocabulary is split over G workgroups (4096 ids each) and the work is 7 short launches;
// no launch waits on another workgroup, and each launch starts by re-reducing the previous
// launches' few per-workgroup partials itself, in a fixed order, so every workgroup derives
// the same global values:
//   pass_max   : penalty on this workgroup's slice (a hit mask of the history ids it owns, LDS
//                copy + in-place global write), then the slice's (max, argmax) of l/T (of l
//                when greedy);
//   pass_sum   : global max; the slice's sum of exp(l/T - max) in float64;
//   pass_level : one launch per 8 bisection steps. The 255 mids those 8 steps could visit are
//                the in-order nodes of a depth-8 bisection tree below the current (lo, hi),
//                computed with the same f32 expression; every p in [lo, hi) is binned against
//                them, p >= hi goes to an 'above' bin, and each group adds its bins into one
//                global set with integer atomics. Replaying the 8 steps from the summed bins is
//                exact: mass(p >= mid) is 'above' plus a suffix sum of bins;
//   pass_kept  : the threshold after 32 steps, the slice's kept mass;
//   finalize   : one workgroup: the target, the slice whose prefix reaches it, then the id.
// Masses are fixed-point integers (p * 2^52, exact for p >= 2^-28) summed with integer adds, so
// every mass is independent of summation order and the result is deterministic. They differ
// from the reference's f32 tree sums only by rounding, which can change a decision only when
// a mass is within ~1e-7 of topP or the target within ~1e-7 of a cumulative boundary.
#include "eg_internal.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;
constexpr uint32_t kSlice = kThreads * kPerThread;  // vocabulary ids per workgroup
constexpr uint32_t kMaxGroups = 256;                // vocab <= 1,048,576 (finalize: one group per thread)
constexpr int kBins = 256;
constexpr int kLevels = 4;                          // 4 x 8 = 32 bisection steps
constexpr double kFix = 4503599627370496.0;         // 2^52

struct SampleParams {
  uint32_t vocab, history_length;
  float temperature, top_p, repetition_penalty, random;
  uint32_t pad0, pad1;
};
static_assert(sizeof(SampleParams) == 32, "sample dims are 32 bytes");

struct SampleState {
  float max_scaled;
  uint32_t argmax;
  float total;
  float threshold;
  float lo[kLevels + 1], hi[kLevels + 1];  // bracket each level bins against; [kLevels] = final
};

struct Work {
  SampleState* state;
  uint32_t* max_part;     // 2 u32 per group
  double* sum_part;       // 1 per group
  unsigned long long* bins;  // kLevels x (kBins + 1), summed over groups by integer atomics
  uint64_t* kept_part;    // 1 per group
  uint32_t* count_part;   // 1 per group
};

__device__ __forceinline__ SampleParams load_params(const SampleParams& p, const SampleParams* dev) {
  return dev ? *dev : p;
}

__device__ __forceinline__ float prob(float logit, const SampleParams& p, float mx, float total) {
  return expf(logit / p.temperature - mx) / total;
}

__device__ __forceinline__ uint64_t to_fix(float p) { return (uint64_t)__double2ull_rn((double)p * kFix); }

template <typename T>
__device__ __forceinline__ T block_sum(T v, T* scratch) {
#pragma unroll
  for (int m = 32; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  if ((threadIdx.x & 63) == 0) scratch[threadIdx.x >> 6] = v;
  __syncthreads();
  T r = scratch[0];
#pragma unroll
  for (int w = 1; w < kThreads / 64; w++) r += scratch[w];
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
  for (int w = 1; w < kThreads / 64; w++)
    if (egd::better(sv[w], si[w], v, i)) {
      v = sv[w];
      i = si[w];
    }
  __syncthreads();
}

// ---- the global values every launch re-derives from the partials ------------------------

__device__ void global_max(const Work& w, uint32_t groups, float& mx, uint32_t& amax) {
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  float bv = -1.0e30f;
  uint32_t bi = 0;
  for (uint32_t b = threadIdx.x; b < groups; b += kThreads) {
    const float v = __uint_as_float(w.max_part[2 * b]);
    const uint32_t i = w.max_part[2 * b + 1];
    if (egd::better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  block_argmax(bv, bi, sv, si);
  mx = bv;
  amax = bi;
}

__device__ float global_total(const Work& w, uint32_t groups) {
  __shared__ double scratch[4];
  double t = 0.0;
  for (uint32_t b = threadIdx.x; b < groups; b += kThreads) t += w.sum_part[b];
  return (float)block_sum(t, scratch);
}

// In-order mid j (0..254) of the depth-8 bisection tree below [lo, hi): the f32 mid the
// bisection reaches when its path of left/right choices spells j.
__device__ float tree_mid(uint32_t j, float lo, float hi) {
  const uint32_t target = j + 1;  // 1-based in-order index, root = 128
  uint32_t cur = 128, step = 64;
  float mid = (lo + hi) * 0.5f;
  while (cur != target) {
    if (target < cur) {
      hi = mid;
      cur -= step;
    } else {
      lo = mid;
      cur += step;
    }
    step >>= 1;
    mid = (lo + hi) * 0.5f;
  }
  return mid;
}

// Number of mids <= v (upper bound over a non-decreasing array of kBins - 1 values).
__device__ __forceinline__ int count_le(const float* mids, float v) {
  int a = 0, b = kBins - 1;
  while (a < b) {
    const int m = (a + b) >> 1;
    if (mids[m] <= v) a = m + 1;
    else b = m;
  }
  return a;
}

// Exclusive prefix sum of one u64 per thread over the workgroup, in thread order; *total gets
// the sum of all. Wave scan by shuffles, then the four wave totals.
__device__ unsigned long long block_exclusive_scan(unsigned long long v, unsigned long long* total) {
  __shared__ unsigned long long wsum[kThreads / 64];
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
  for (int w = 0; w < kThreads / 64; w++) {
    if (w < (int)(threadIdx.x >> 6)) before += wsum[w];
    all += wsum[w];
  }
  __syncthreads();
  if (total) *total = all;
  return before + incl - v;
}

// Replays the 8 bisection steps of `level` from its summed bins: (lo, hi) in, (lo, hi) out.
// All threads: the 255 tree mids, the bin column sums, the suffix sums and the mass at every
// tree node in parallel; then the 8-step walk reads one node mass per step.
__device__ void replay_level(const Work& w, uint32_t groups, int level, float top_p, float& lo, float& hi,
                             float* mids, unsigned long long* sums) {
  __shared__ unsigned long long suffix[kBins + 1];
  __shared__ double node_mass[kBins - 1];
  __shared__ float out_lo, out_hi;
  if (threadIdx.x < kBins - 1) mids[threadIdx.x] = tree_mid(threadIdx.x, lo, hi);
  const unsigned long long* summed = w.bins + (size_t)level * (kBins + 1);
  for (int i = threadIdx.x; i <= kBins; i += kThreads) sums[i] = summed[i];
  __syncthreads();
  // suffix[k] = mass of p >= hi (sums[kBins]) plus bins k..kBins-1: total minus an exclusive
  // prefix, so one block scan instead of a serial walk.
  static_assert(kBins == kThreads, "one bin per thread");
  unsigned long long total = 0;
  const unsigned long long before = block_exclusive_scan(sums[threadIdx.x], &total);
  suffix[threadIdx.x] = sums[kBins] + (total - before);
  if (threadIdx.x == 0) suffix[kBins] = sums[kBins];
  __syncthreads();
  if (threadIdx.x < kBins - 1) node_mass[threadIdx.x] = (double)suffix[count_le(mids, mids[threadIdx.x])] / kFix;
  __syncthreads();
  if (threadIdx.x == 0) {
    const double top = (double)top_p;
    float l = lo, h = hi;
    uint32_t cur = 128, step = 64;
    for (int s = 0; s < 8; s++) {
      const float mid = mids[cur - 1];
      if (node_mass[cur - 1] < top) {
        h = mid;
        cur -= step;
      } else {
        l = mid;
        cur += step;
      }
      step >>= 1;
    }
    out_lo = l;
    out_hi = h;
  }
  __syncthreads();
  lo = out_lo;
  hi = out_hi;
}

// ---- launches --------------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void pass_max(float* logits, const uint32_t* history, SampleParams hp,
                                                     const SampleParams* dp, Work w, uint32_t* rng) {
  // This call's draw (one per sampled step, Session.decodeStep session.ts:351), consumed by
  // finalize; no workgroup of this launch reads `random`.
  if (rng && blockIdx.x == 0 && threadIdx.x == 0)
    const_cast<SampleParams*>(dp)->random = egd::mulberry32_next(rng);
  const SampleParams p = load_params(hp, dp);
  __shared__ float slice[kSlice];
  __shared__ float sv[4];
  __shared__ uint32_t si[4];
  const uint32_t base = blockIdx.x * kSlice;
  const uint32_t end = min(base + kSlice, p.vocab);
  for (uint32_t i = threadIdx.x; i < kSlice; i += kThreads) slice[i] = base + i < end ? logits[base + i] : 0.f;
  __syncthreads();
  if (p.repetition_penalty != 1.0f) {
    // The penalty applies once per distinct history id (the reference applies it at an id's
    // first occurrence only): mark the ids this slice owns, then penalize each marked element
    // once. No two threads write the same element.
    __shared__ uint8_t hit[kSlice];
    for (uint32_t i = threadIdx.x; i < kSlice; i += kThreads) hit[i] = 0;
    __syncthreads();
    for (uint32_t h = threadIdx.x; h < p.history_length; h += kThreads) {
      const uint32_t id = history[h];
      if (id >= base && id < end) hit[id - base] = 1;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < end - base; i += kThreads) {
      if (hit[i]) {
        const float v = slice[i];
        const float r = v > 0.0f ? v / p.repetition_penalty : v * p.repetition_penalty;
        slice[i] = r;
        logits[base + i] = r;
      }
    }
    __syncthreads();
  }
  const bool greedy = p.temperature <= 0.0f;
  float bv = -1.0e30f;
  uint32_t bi = greedy ? 0u : base;
  for (uint32_t i = base + threadIdx.x; i < end; i += kThreads) {
    const float v = greedy ? slice[i - base] : slice[i - base] / p.temperature;
    if (egd::better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  block_argmax(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    w.max_part[2 * blockIdx.x] = __float_as_uint(bv);
    w.max_part[2 * blockIdx.x + 1] = bi;
  }
}

__global__ __launch_bounds__(kThreads) void pass_sum(const float* logits, SampleParams hp, const SampleParams* dp,
                                                     Work w) {
  const SampleParams p = load_params(hp, dp);
  if (p.temperature <= 0.0f) return;
  __shared__ double scratch[4];
  float mx;
  uint32_t amax;
  global_max(w, gridDim.x, mx, amax);
  const uint32_t base = blockIdx.x * kSlice;
  const uint32_t end = min(base + kSlice, p.vocab);
  float lv[kPerThread];
#pragma unroll
  for (int r = 0; r < kPerThread; r++) {
    const uint32_t i = base + r * kThreads + threadIdx.x;
    lv[r] = i < end ? logits[i] : 0.f;
  }
  double s = 0.0;
#pragma unroll
  for (int r = 0; r < kPerThread; r++)
    if (base + r * kThreads + threadIdx.x < end) s += (double)expf(lv[r] / p.temperature - mx);
  s = block_sum(s, scratch);
  if (threadIdx.x == 0) w.sum_part[blockIdx.x] = s;
  // The level launches accumulate into these; clear them for this call (a kernel, not a
  // memset, so a captured graph replays it).
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < kLevels * (kBins + 1); i += kThreads) w.bins[i] = 0;
}

__global__ __launch_bounds__(kThreads) void pass_level(const float* logits, int level, SampleParams hp,
                                                       const SampleParams* dp, Work w) {
  const SampleParams p = load_params(hp, dp);
  if (p.temperature <= 0.0f || !(p.top_p < 1.0f)) return;
  __shared__ float mids[kBins - 1];
  __shared__ unsigned long long bins[kBins + 1];
  const uint32_t base = blockIdx.x * kSlice;
  const uint32_t end = min(base + kSlice, p.vocab);
  float lv[kPerThread];  // issued first: independent of everything read below
#pragma unroll
  for (int r = 0; r < kPerThread; r++) {
    const uint32_t i = base + r * kThreads + threadIdx.x;
    lv[r] = i < end ? logits[i] : 0.f;
  }
  float mx;
  uint32_t amax;
  global_max(w, gridDim.x, mx, amax);
  const float total = global_total(w, gridDim.x);
  // The bracket this level bins against: (0, 1) first, then the previous level's bracket
  // replayed through its 8 steps. Workgroup 0 records it for the next launch.
  float lo = 0.0f, hi = 1.0f;
  if (level > 0) {
    lo = w.state->lo[level - 1];
    hi = w.state->hi[level - 1];
    replay_level(w, gridDim.x, level - 1, p.top_p, lo, hi, mids, bins);
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    w.state->lo[level] = lo;
    w.state->hi[level] = hi;
  }
  if (threadIdx.x < kBins - 1) mids[threadIdx.x] = tree_mid(threadIdx.x, lo, hi);
  for (int i = threadIdx.x; i <= kBins; i += kThreads) bins[i] = 0;
  __syncthreads();
  // The mids split [lo, hi) into 256 near-equal steps, so the bin is estimated arithmetically
  // and corrected against the exact f32 mids (usually no step). Runs of equal bins are summed
  // in registers before the LDS atomic (at the first level nearly every p shares bin 0).
  const float scale = (float)kBins / (hi - lo);
  int run_bin = -1;
  unsigned long long run_mass = 0;
  float pv[kPerThread];
#pragma unroll
  for (int r = 0; r < kPerThread; r++) {
    const uint32_t i = base + r * kThreads + threadIdx.x;
    pv[r] = i < end ? prob(lv[r], p, mx, total) : -1.0f;
  }
#pragma unroll
  for (int r = 0; r < kPerThread; r++) {
    const float pr = pv[r];
    if (pr < lo) continue;
    int k;
    if (pr >= hi) {
      k = kBins;
    } else {
      k = min(max((int)((pr - lo) * scale), 0), kBins - 1);  // estimate of #mids <= pr
      while (k < kBins - 1 && mids[k] <= pr) k++;
      while (k > 0 && mids[k - 1] > pr) k--;
    }
    if (k != run_bin) {
      if (run_bin >= 0) atomicAdd(&bins[run_bin], run_mass);  // integer adds: order-independent
      run_bin = k;
      run_mass = 0;
    }
    run_mass += to_fix(pr);
  }
  if (run_bin >= 0) atomicAdd(&bins[run_bin], run_mass);
  __syncthreads();
  // Integer adds commute: the summed bins are the same whatever order the groups arrive in.
  unsigned long long* summed = w.bins + (size_t)level * (kBins + 1);
  for (int i = threadIdx.x; i <= kBins; i += kThreads)
    if (bins[i]) atomicAdd(&summed[i], bins[i]);
}

__global__ __launch_bounds__(kThreads) void pass_kept(const float* logits, SampleParams hp, const SampleParams* dp,
                                                      Work w) {
  const SampleParams p = load_params(hp, dp);
  if (p.temperature <= 0.0f) return;
  __shared__ float mids[kBins - 1];
  __shared__ unsigned long long bins[kBins + 1];
  __shared__ unsigned long long kscratch[4];
  __shared__ uint32_t cscratch[4];
  const uint32_t base = blockIdx.x * kSlice;
  const uint32_t end = min(base + kSlice, p.vocab);
  float lv[kPerThread];  // issued first: independent of everything read below
#pragma unroll
  for (int r = 0; r < kPerThread; r++) {
    const uint32_t i = base + r * kThreads + threadIdx.x;
    lv[r] = i < end ? logits[i] : 0.f;
  }
  float mx;
  uint32_t amax;
  global_max(w, gridDim.x, mx, amax);
  const float total = global_total(w, gridDim.x);
  float lo = 0.0f, hi = 1.0f;
  if (p.top_p < 1.0f) {
    lo = w.state->lo[kLevels - 1];
    hi = w.state->hi[kLevels - 1];
    replay_level(w, gridDim.x, kLevels - 1, p.top_p, lo, hi, mids, bins);
  }
  const float thr = p.top_p < 1.0f ? lo : 0.0f;
  unsigned long long kept = 0;
  uint32_t count = 0;
#pragma unroll
  for (int r = 0; r < kPerThread; r++) {
    const uint32_t i = base + r * kThreads + threadIdx.x;
    if (i >= end) continue;
    const float pr = prob(lv[r], p, mx, total);
    if (pr >= thr) {
      kept += to_fix(pr);
      count++;
    }
  }
  kept = block_sum(kept, kscratch);
  count = block_sum(count, cscratch);
  if (threadIdx.x == 0) {
    w.kept_part[blockIdx.x] = kept;
    w.count_part[blockIdx.x] = count;
    if (blockIdx.x == 0) {
      w.state->max_scaled = mx;
      w.state->argmax = amax;
      w.state->total = total;
      w.state->threshold = thr;
      w.state->lo[kLevels] = lo;
      w.state->hi[kLevels] = hi;
    }
  }
}

// One workgroup: greedy result, or the target and the id where the kept mass reaches it.
__global__ __launch_bounds__(kThreads) void finalize(const float* logits, uint32_t* out, uint32_t groups,
                                                     SampleParams hp, const SampleParams* dp, Work w) {
  const SampleParams p = load_params(hp, dp);
  if (p.temperature <= 0.0f) {
    float mx;
    uint32_t amax;
    global_max(w, groups, mx, amax);
    if (threadIdx.x == 0) out[0] = amax;
    return;
  }
  __shared__ uint32_t group, pick;
  __shared__ unsigned long long group_prefix;
  const SampleState st = *w.state;
  // Kept mass per group in id order: the target, then the first group whose inclusive prefix
  // reaches it (and that keeps something, so a zero target still lands on a kept id).
  unsigned long long all = 0;
  const unsigned long long gk = threadIdx.x < groups ? w.kept_part[threadIdx.x] : 0ull;
  const uint32_t gc = threadIdx.x < groups ? w.count_part[threadIdx.x] : 0u;
  const unsigned long long gbefore = block_exclusive_scan(gk, &all);
  double kd = (double)all / kFix;
  if (kd < 1.0e-20) kd = 1.0e-20;
  const double target_fx = (double)p.random * kd * kFix;
  if (threadIdx.x == 0) {
    group = 0xFFFFFFFFu;
    pick = 0xFFFFFFFFu;
  }
  __syncthreads();
  if (threadIdx.x < groups && gc > 0 && (double)(gbefore + gk) >= target_fx) atomicMin(&group, threadIdx.x);
  __syncthreads();
  if (threadIdx.x == group) group_prefix = gbefore;
  __syncthreads();
  if (group != 0xFFFFFFFFu) {
    // Thread t owns ids [t*16, t*16+16) of the group's slice, so thread order is id order.
    const uint32_t gbase = group * kSlice;
    float pv[kPerThread];
    unsigned long long mine = 0;
#pragma unroll
    for (int r = 0; r < kPerThread; r++) {
      const uint32_t i = gbase + threadIdx.x * kPerThread + r;
      pv[r] = -1.0f;
      if (i < p.vocab) {
        const float pr = prob(logits[i], p, st.max_scaled, st.total);
        if (pr >= st.threshold) {
          pv[r] = pr;
          mine += to_fix(pr);
        }
      }
    }
    unsigned long long run = group_prefix + block_exclusive_scan(mine, nullptr);
#pragma unroll
    for (int r = 0; r < kPerThread; r++) {
      if (pv[r] >= 0.0f) {
        run += to_fix(pv[r]);
        if ((double)run >= target_fx) {
          atomicMin(&pick, gbase + threadIdx.x * kPerThread + r);
          break;
        }
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) out[0] = pick != 0xFFFFFFFFu ? pick : st.argmax;
}

Work workspace(eg_context* ctx) {
  Work w;
  w.state = reinterpret_cast<SampleState*>(eg::state(ctx) + 512);
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
  off += (size_t)kLevels * (kBins + 1) * 8;
  static_assert((size_t)kMaxGroups * 28 + (size_t)kLevels * (kBins + 1) * 8 <= eg::kPartialsBytes,
                "sampler partials exceed the workspace");
  return w;
}

int launch(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out, const SampleParams& hp,
           const SampleParams* dp, bool all_passes, uint32_t* rng = nullptr) {
  const uint32_t groups = (hp.vocab + kSlice - 1) / kSlice;
  Work w = workspace(ctx);
  const dim3 grid(groups), block(kThreads);
  hipLaunchKernelGGL(pass_max, grid, block, 0, ctx->stream, logits, history, hp, dp, w, rng);
  const bool sampled = all_passes || hp.temperature > 0.0f;
  if (sampled) {
    hipLaunchKernelGGL(pass_sum, grid, block, 0, ctx->stream, logits, hp, dp, w);
    if (all_passes || hp.top_p < 1.0f)
      for (int l = 0; l < kLevels; l++)
        hipLaunchKernelGGL(pass_level, grid, block, 0, ctx->stream, logits, l, hp, dp, w);
    hipLaunchKernelGGL(pass_kept, grid, block, 0, ctx->stream, logits, hp, dp, w);
  }
  hipLaunchKernelGGL(finalize, dim3(1), block, 0, ctx->stream, logits, out, groups, hp, dp, w);
  return eg::check_launch(ctx, "sample");
}

}  // namespace

int eg::launch_sample_device(eg_context* ctx, float* logits, const uint32_t* history, uint32_t* out, uint32_t vocab,
                             eg_sample_dims* params, uint32_t* rng) {
  static_assert(sizeof(eg_sample_dims) == sizeof(SampleParams), "the device block is the 32-byte sample dims");
  if (!logits || !out || !params) return eg::fail(ctx, EG_ERR_INVALID, "sample: NULL argument");
  if (vocab == 0 || (vocab + kSlice - 1) / kSlice > kMaxGroups)
    return eg::fail(ctx, EG_ERR_RANGE, "sample: vocab %u outside the sampler's range (1..%u)", vocab,
                    kMaxGroups * kSlice);
  SampleParams hp{};
  hp.vocab = vocab;
  return launch(ctx, logits, history, out, hp, reinterpret_cast<const SampleParams*>(params), true, rng);
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
  return launch(ctx, logits, history, out, hp, nullptr, false);
}
