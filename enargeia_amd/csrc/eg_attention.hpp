// Fused decode attention (RoPE, the cache append, split-K flash-decoding partials), shared by its
// own launch (eg_decode.hip) and the persistent decode kernel (eg_layers.hip). Not part of the
// ABI. The cache element type CT is uint16_t (f16 bits, the reference's f16 cache variant) or
// float (its f32 variant); every cached value is f32 once read.
//
// Reference pieces: rope.wgsl + the f16 cache pack (cache_variants.ts:147-305,
// graph_decode.ts:276-320; the f32 cache's v projection writes the slot itself, :281-283),
// attn_scores / softmax / attn_apply decode (graph_decode.ts:322-345, per dtype
// cache_variants.ts:21-40; CPU semantics ops.ts:87-205).
#pragma once

#include <cmath>
#include <type_traits>

#include "eg_internal.hpp"

namespace eg_attn {

constexpr int kThreads = 256;

using egd::float_to_half;
using egd::half_to_float;
using egd::rope_apply;
using egd::rope_table;

constexpr uint32_t kMaxCombine = 1024;  // heads x chunks the one-workgroup combine holds in LDS

// A value as the cache holds it: f16 bits (round to nearest even) or the f32 itself.
template <class CT>
__device__ __forceinline__ CT to_cache(float x) {
  if constexpr (std::is_same<CT, float>::value) return x;
  else return float_to_half(x);
}

// The whole attention output from the chunk-fastest partials, by one workgroup: per (head,
// chunk) statistics into LDS, each chunk's weight e^(m_c - M) / L, then every output's weighted
// sum of its chunks' o values read as 16-byte vectors. Same operations in the same order as
// egd::attention_combine_at (so the same bits).
__device__ void combine_all(const float* partials, float* out, uint32_t heads, uint32_t D, uint32_t chunks) {
  __shared__ float mval[kMaxCombine], lval[kMaxCombine], wts[kMaxCombine];
  const uint32_t tid = threadIdx.x, hcs = heads * chunks, n = heads * D;
  const float* m = partials + (size_t)heads * D * chunks;
  const float* l = m + hcs;
  for (uint32_t hc = tid; hc < hcs; hc += blockDim.x) {
    mval[hc] = m[hc];
    lval[hc] = l[hc];
  }
  __syncthreads();
  // a head's statistics in a power-of-two group of lanes: M and L are butterflies across it
  // (the order egd::combine_stats reproduces on one thread)
  const uint32_t G = egd::combine_group(chunks);
  for (uint32_t p0 = 0; p0 < heads * G; p0 += blockDim.x) {
    const uint32_t p = p0 + tid, c = p % G, hc = (p / G) * chunks + c;
    const bool valid = p < heads * G && c < chunks;
    float M, e, L;
    egd::group_stats(G, valid, valid ? mval[hc] : 0.f, valid ? lval[hc] : 0.f, M, e, L);
    if (valid) wts[hc] = e / L;
  }
  __syncthreads();
  for (uint32_t i = tid; i < n; i += blockDim.x) {
    const float* o = partials + (size_t)i * chunks;
    const float* w = wts + (i / D) * chunks;
    float acc = 0.f;
    if ((chunks & 3u) == 0) {
      const float4* o4 = reinterpret_cast<const float4*>(o);
#pragma unroll 8
      for (uint32_t q = 0; q < chunks / 4; q++) {
        const float4 v = o4[q];
        acc = fmaf(v.x, w[4 * q + 0], acc);
        acc = fmaf(v.y, w[4 * q + 1], acc);
        acc = fmaf(v.z, w[4 * q + 2], acc);
        acc = fmaf(v.w, w[4 * q + 3], acc);
      }
    } else {
      for (uint32_t c = 0; c < chunks; c++) acc = fmaf(o[c], w[c], acc);
    }
    out[i] = acc;
  }
}

// Everything a workgroup reads from memory, loaded by its threads before anything else: the
// chunk's K and V rows as 16-byte vectors (which rows exist does not depend on the position -
// a chunk always lies inside the cache - so these loads need not wait for it; rows past the
// live history are loaded too and never read), then one query element per thread and the new
// key and value. All of it is in flight at once; the position arrives by a scalar load beside.
template <int D, int CHUNK, int GMAX, class CT = uint16_t>
struct Prefetch {
  static constexpr uint32_t kPer = 16 / sizeof(CT);             // cache elements per 16 bytes
  static constexpr uint32_t kVecs = D / kPer;                   // 16-byte vectors per row
  static constexpr uint32_t kLoads = CHUNK * kVecs / kThreads;  // per thread
  static_assert(CHUNK * kVecs % kThreads == 0, "a chunk's rows split evenly over the threads");
  static_assert(GMAX * D <= kThreads && D <= kThreads, "one query element per thread");
  uint4 k[kLoads], v[kLoads];
  float qv = 0.f, kn = 0.f, vn = 0.f;
  double2 cs = make_double2(0.0, 0.0);  // the RoPE table's entry tid, when one is given
  // The cached rows (and the RoPE row): written before the launch, so a phase of the persistent
  // kernel issues them before waiting for its inputs.
  __device__ __forceinline__ void load_cache(const CT* k_cache, const CT* v_cache, uint32_t j0, uint32_t kv,
                                             uint32_t kv_heads, const double2* rope) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (uint32_t r = 0; r < kLoads; r++) {
      const uint32_t i = tid + r * kThreads, row = i / kVecs, w = i % kVecs;
      const size_t at = ((size_t)(j0 + row) * kv_heads + kv) * D + w * kPer;
      k[r] = *reinterpret_cast<const uint4*>(k_cache + at);
      v[r] = *reinterpret_cast<const uint4*>(v_cache + at);
    }
    if (rope && tid < D / 2) cs = rope[tid];
  }
  // The query and the new key and value: the projection's outputs (AUX: coherent where another
  // workgroup of the same launch wrote them).
  template <int AUX>
  __device__ __forceinline__ void load_inputs(const float* q, uint32_t h0, uint32_t ng, uint32_t kv, const float* kp,
                                              const float* vp) {
    const uint32_t tid = threadIdx.x;
    if (tid < ng * D) qv = egd::load_f32_p<AUX>(egd::buffer(q, (uint32_t)((h0 * D + ng * D) * 4u)), (h0 * D + tid) * 4u);
    if (tid < D) {
      kn = egd::load_f32_p<AUX>(egd::buffer(kp, (kv + 1u) * D * 4u), (kv * D + tid) * 4u);
      vn = egd::load_f32_p<AUX>(egd::buffer(vp, (kv + 1u) * D * 4u), (kv * D + tid) * 4u);
    }
  }
};

// A store of data another workgroup of the same launch reads (AUX = egd::kCoherent: egd::put).
template <int AUX>
__device__ __forceinline__ void store_p(float* p, float v) {
  if constexpr (AUX == egd::kCoherent) egd::put(p, v);
  else *p = v;
}

// The work of one (kv head share, chunk) workgroup: RoPE, the cache append, scores, softmax
// statistics and the partial o, written to po/pm/pl, from what `pre` loaded.
template <int D, int CHUNK, int GMAX, int AUX = 0, class CT = uint16_t>
__device__ __forceinline__ void attend(uint32_t pos, uint32_t j0, uint32_t kv, uint32_t hs, uint32_t ng,
                                       uint32_t chunks, const Prefetch<D, CHUNK, GMAX, CT>& pre, bool rope,
                                       CT* k_cache, CT* v_cache, float* po, float* pm, float* pl,
                                       const eg_attention_dims& d) {
  using Pre = Prefetch<D, CHUNK, GMAX, CT>;
  constexpr bool kF32 = std::is_same<CT, float>::value;
  const uint32_t tid = threadIdx.x;
  const uint32_t live = min((uint32_t)CHUNK, pos + 1 - j0);

  // K rows padded by 16 bytes (144 bytes f16, 272 f32): 16-byte row reads by 16 lanes on 16 rows
  // cover the 64 banks once. V rows unpadded: the f16 P.V loop's 8-byte reads take 4 rows a
  // wave, 2 on each half of the banks (the f32 loop's 16-byte reads, 4 rows on 4 quarters).
  __shared__ __attribute__((aligned(16))) float qs[GMAX][D];          // rotated, pre-scaled queries
  __shared__ float knew[D], vnew[D];                                  // the new key (rotated), value
  __shared__ double2 cs[D / 2];                                       // RoPE cos/sin at `pos`
  __shared__ __attribute__((aligned(16))) CT ks[CHUNK][D + Pre::kPer];  // K rows
  __shared__ __attribute__((aligned(16))) CT vs[CHUNK][D];              // V rows
  __shared__ float p[GMAX][CHUNK];                                    // scores, then exp(score - max)
  __shared__ float mstat[GMAX], lstat[GMAX];
  __shared__ __attribute__((aligned(16))) float half_sum[GMAX][D];    // P.V: the second wave's sums

  const float scale = 1.0f / sqrtf((float)D);
  const bool owns_new = pos < j0 + CHUNK;
  // The cached rows into LDS (every row of the chunk; the row at `pos`, stale in the cache, is
  // replaced by the new one after the next barriers).
#pragma unroll
  for (uint32_t r = 0; r < Pre::kLoads; r++) {
    const uint32_t i = tid + r * kThreads, row = i / Pre::kVecs, w = i % Pre::kVecs;
    uint32_t* kd = reinterpret_cast<uint32_t*>(&ks[row][w * Pre::kPer]);
    uint32_t* vd = reinterpret_cast<uint32_t*>(&vs[row][w * Pre::kPer]);
    kd[0] = pre.k[r].x; kd[1] = pre.k[r].y; kd[2] = pre.k[r].z; kd[3] = pre.k[r].w;
    vd[0] = pre.v[r].x; vd[1] = pre.v[r].y; vd[2] = pre.v[r].z; vd[3] = pre.v[r].w;
  }
  if (tid < ng * D) qs[tid / D][tid % D] = pre.qv;
  if (tid < D) {
    knew[tid] = pre.kn;
    vnew[tid] = pre.vn;
  }
  if (tid < D / 2) {
    if (rope) cs[tid] = pre.cs;  // computed once per step by the step tail, same function
    else rope_table<D>(cs, tid, pos, d.theta);
  }
  __syncthreads();
  for (uint32_t i = tid; i < ng * (D / 2); i += blockDim.x) rope_apply<D>(qs[i / (D / 2)], i % (D / 2), cs);
  if (owns_new && tid < D / 2) rope_apply<D>(knew, tid, cs);
  __syncthreads();
  for (uint32_t i = tid; i < ng * D; i += blockDim.x) qs[i / D][i % D] *= scale;
  // The row at `pos` is the new one: appended to the cache (by the first head share only) and
  // staged from registers.
  if (owns_new && tid < D) {
    const CT kh = to_cache<CT>(knew[tid]), vh = to_cache<CT>(vnew[tid]);
    if (hs == 0) {
      const size_t at = ((size_t)pos * d.kv_heads + kv) * D + tid;
      k_cache[at] = kh;
      v_cache[at] = vh;
    }
    ks[pos - j0][tid] = kh;
    vs[pos - j0][tid] = vh;
  }
  __syncthreads();

  // scores: thread -> one position, a strided subset of the group's heads; the K row in 16-byte
  // pieces, the query in float4s (a broadcast), products summed in element order
  {
    const uint32_t j = tid % CHUNK;
    const uint32_t g0 = tid / CHUNK, gs = kThreads / CHUNK;
    for (uint32_t g = g0; g < ng; g += gs) {
      float s = -INFINITY;
      if (j < live) {
        float acc = 0.f;
        if constexpr (kF32) {
#pragma unroll
          for (int w = 0; w < D / 4; w++) {
            const float4 kk = *reinterpret_cast<const float4*>(&ks[j][4 * w]);
            const float4 qa = *reinterpret_cast<const float4*>(&qs[g][4 * w]);
            acc = fmaf(qa.x, kk.x, acc);
            acc = fmaf(qa.y, kk.y, acc);
            acc = fmaf(qa.z, kk.z, acc);
            acc = fmaf(qa.w, kk.w, acc);
          }
        } else {
#pragma unroll
          for (int w = 0; w < D / 8; w++) {
            const uint4 kk = *reinterpret_cast<const uint4*>(&ks[j][8 * w]);
            const float4 qa = *reinterpret_cast<const float4*>(&qs[g][8 * w]);
            const float4 qb = *reinterpret_cast<const float4*>(&qs[g][8 * w + 4]);
            acc = fmaf(qa.x, half_to_float((uint16_t)kk.x), acc);
            acc = fmaf(qa.y, half_to_float((uint16_t)(kk.x >> 16)), acc);
            acc = fmaf(qa.z, half_to_float((uint16_t)kk.y), acc);
            acc = fmaf(qa.w, half_to_float((uint16_t)(kk.y >> 16)), acc);
            acc = fmaf(qb.x, half_to_float((uint16_t)kk.z), acc);
            acc = fmaf(qb.y, half_to_float((uint16_t)(kk.z >> 16)), acc);
            acc = fmaf(qb.z, half_to_float((uint16_t)kk.w), acc);
            acc = fmaf(qb.w, half_to_float((uint16_t)(kk.w >> 16)), acc);
          }
        }
        s = acc;
      }
      p[g][j] = s;
    }
  }
  __syncthreads();

  // softmax statistics: one wave per head, lanes over the chunk, fixed-order reductions (DPP
  // within rows, a swizzle and readlanes across them)
  const uint32_t wave = tid >> 6, lane = tid & 63u;
  for (uint32_t g = wave; g < ng; g += kThreads / 64) {
    float m = -INFINITY;
    for (uint32_t j = lane; j < CHUNK; j += 64) m = fmaxf(m, p[g][j]);
    m = egd::team_allmax<64>(m);
    float l = 0.f;
    for (uint32_t j = lane; j < CHUNK; j += 64) {
      const float e = j < live ? expf(p[g][j] - m) : 0.f;
      p[g][j] = e;
      l += e;
    }
    l = egd::team_allsum<64>(l);
    if (lane == 0) {
      mstat[g] = m;
      lstat[g] = l;
    }
  }
  __syncthreads();

  // o[g][e] = sum_j p[g][j] * V[j][e]: WPH waves per head, each over its CHUNK / WPH positions;
  // a lane takes 4 consecutive e (lane % 16) and every 4th position (lane / 16), four independent
  // sums; the 4 position phases are added across lanes, then the waves in order.
  {
    constexpr uint32_t kWPH = (kThreads / 64) / GMAX;
    static_assert(kWPH >= 1 && kWPH <= 2 && D == 64, "P.V lane layout");
    const uint32_t g = wave / kWPH, wh = wave % kWPH;
    const uint32_t e4 = 4 * (lane & 15u), ph = lane >> 4;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (g < ng) {
      const uint32_t jb = wh * (CHUNK / kWPH), je = min(live, jb + CHUNK / kWPH);
      for (uint32_t j = jb + ph; j < je; j += 4) {
        const float pj = p[g][j];
        if constexpr (kF32) {
          const float4 vv = *reinterpret_cast<const float4*>(&vs[j][e4]);
          a0 = fmaf(pj, vv.x, a0);
          a1 = fmaf(pj, vv.y, a1);
          a2 = fmaf(pj, vv.z, a2);
          a3 = fmaf(pj, vv.w, a3);
        } else {
          const uint2 vv = *reinterpret_cast<const uint2*>(&vs[j][e4]);
          a0 = fmaf(pj, half_to_float((uint16_t)vv.x), a0);
          a1 = fmaf(pj, half_to_float((uint16_t)(vv.x >> 16)), a1);
          a2 = fmaf(pj, half_to_float((uint16_t)vv.y), a2);
          a3 = fmaf(pj, half_to_float((uint16_t)(vv.y >> 16)), a3);
        }
      }
    }
    a0 += __shfl_xor(a0, 16, 64);
    a1 += __shfl_xor(a1, 16, 64);
    a2 += __shfl_xor(a2, 16, 64);
    a3 += __shfl_xor(a3, 16, 64);
    a0 += __shfl_xor(a0, 32, 64);
    a1 += __shfl_xor(a1, 32, 64);
    a2 += __shfl_xor(a2, 32, 64);
    a3 += __shfl_xor(a3, 32, 64);
    if (kWPH > 1) {
      if (g < ng && wh == 1 && ph == 0)
        *reinterpret_cast<float4*>(&half_sum[g][e4]) = make_float4(a0, a1, a2, a3);
      __syncthreads();
      if (g < ng && wh == 0) {
        const float4 b = *reinterpret_cast<const float4*>(&half_sum[g][e4]);
        a0 += b.x;
        a1 += b.y;
        a2 += b.z;
        a3 += b.w;
      }
    }
    if (g < ng && wh == 0 && ph == 0) {
      float* o = po + (size_t)(g * D + e4) * chunks;
      store_p<AUX>(o, a0);
      store_p<AUX>(o + chunks, a1);
      store_p<AUX>(o + 2 * chunks, a2);
      store_p<AUX>(o + 3 * chunks, a3);
    }
  }
  if (tid < ng) {
    store_p<AUX>(pm + (size_t)tid * chunks, mstat[tid]);
    store_p<AUX>(pl + (size_t)tid * chunks, lstat[tid]);
  }
}

// How the attention body runs: as its own launch (grid chunks x kv_heads * HSPLIT), or as a phase
// of the persistent decode kernel (a virtual grid, a wait for the projection's outputs, coherent
// accesses to what other workgroups of the launch write or read).
struct AttnLaunchEnv {
  static constexpr int kAux = 0;
  static constexpr bool kPhase = false;
  __device__ __forceinline__ uint32_t bx() const { return blockIdx.x; }
  __device__ __forceinline__ uint32_t by() const { return blockIdx.y; }
  __device__ __forceinline__ uint32_t gx() const { return gridDim.x; }
  __device__ __forceinline__ uint32_t blocks() const { return gridDim.x * gridDim.y; }
  __device__ __forceinline__ void wait() const {}
};

// One workgroup: kv head kv = by / HSPLIT and the HSPLIT-th share of its query heads, positions
// [j0, j0 + CHUNK) (bx). Splitting the group's heads over HSPLIT workgroups doubles the
// parallelism of a launch that otherwise has only chunks x kv_heads workgroups; the K/V rows they
// share come from L2.
template <int D, int CHUNK, int GMAX, int HSPLIT, class Env, class CT = uint16_t>
__device__ __forceinline__ void attention_body(const uint32_t* position, const float* q, const float* k,
                                               const float* v, CT* k_cache, CT* v_cache,
                                               float* partials, uint32_t* counter, float* out,
                                               const eg_attention_dims& d, const double2* rope, const Env& env) {
  constexpr int AUX = Env::kAux;
  const uint32_t kv = env.by() / HSPLIT, hs = env.by() % HSPLIT;
  const uint32_t c = env.bx();
  const uint32_t chunks = env.gx();
  const uint32_t group = d.heads / d.kv_heads;
  const uint32_t share = (group + HSPLIT - 1) / HSPLIT;
  const uint32_t gb = min(group, hs * share), ng = min(group, gb + share) - gb;  // heads [gb, gb + ng)
  const uint32_t j0 = c * CHUNK;
  const uint32_t tid = threadIdx.x;
  const uint32_t h0 = kv * group + gb;
  Prefetch<D, CHUNK, GMAX, CT> pre;
  pre.load_cache(k_cache, v_cache, j0, kv, d.kv_heads, rope);
  env.wait();
  pre.template load_inputs<AUX>(q, h0, ng, kv, k, v);
  const uint32_t pos = position[0];
  // partial layout (chunk index fastest): o[h][e][c], then m[h][c], then l[h][c]
  float* po = partials + (size_t)h0 * D * chunks + c;
  float* pm = partials + (size_t)d.heads * D * chunks + (size_t)h0 * chunks + c;
  float* pl = pm + (size_t)d.heads * chunks;
  // Past the live history (or, defensively, a position beyond the cache): an empty partial.
  // No cache row is written unless pos < max_context. Every workgroup still reaches the
  // arrival count below.
  const bool empty = j0 > pos || pos >= d.max_context;
  if (ng > 0 && empty) {
    for (uint32_t i = tid; i < ng * D; i += blockDim.x) store_p<AUX>(po + (size_t)i * chunks, 0.f);
    if (tid < ng) {
      store_p<AUX>(pm + (size_t)tid * chunks, -INFINITY);
      store_p<AUX>(pl + (size_t)tid * chunks, 0.f);
    }
  }
  if (ng > 0 && !empty)
    attend<D, CHUNK, GMAX, AUX, CT>(pos, j0, kv, hs, ng, chunks, pre, rope != nullptr, k_cache, v_cache, po, pm, pl,
                                    d);

  // The combine, once, by the last workgroup to arrive: the fence releases this workgroup's
  // partials device-wide before it counts itself; the last one's fence acquires everyone's.
  if (!Env::kPhase && out) {
    __shared__ uint32_t last;
    __syncthreads();
    if (tid == 0) {
      __threadfence();
      last = atomicAdd(counter, 1u) == env.blocks() - 1;
    }
    __syncthreads();
    if (last) {
      __threadfence();
      combine_all(partials, out, d.heads, D, chunks);
      if (tid == 0) *counter = 0;  // ready for the next launch
    }
  }
}

template <int D, int CHUNK, int GMAX, int HSPLIT, class CT>
__global__ __launch_bounds__(kThreads) void attention_decode_kernel(const uint32_t* position, const float* q,
                                                                    const float* k, const float* v, CT* k_cache,
                                                                    CT* v_cache,
                                                                    float* partials, uint32_t* counter, float* out,
                                                                    eg_attention_dims d, const double2* rope,
                                                                    uint64_t* stamp_slot) {
  const egd::WaveStamp stamp(stamp_slot);
  attention_body<D, CHUNK, GMAX, HSPLIT, AttnLaunchEnv, CT>(position, q, k, v, k_cache, v_cache, partials, counter,
                                                           out, d, rope, AttnLaunchEnv{});
}

}  // namespace eg_attn
