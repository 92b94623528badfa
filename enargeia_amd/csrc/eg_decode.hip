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
  const uint32_t id = token[0];
  if (id < d.row_begin || id - d.row_begin >= d.row_count) return;
  const uint32_t row = id - d.row_begin;
  const uint32_t per_word = 32u / (uint32_t)bits;
  const uint32_t mask = (1u << bits) - 1u;
  for (uint32_t i = threadIdx.x; i < d.hidden; i += blockDim.x) {
    const uint64_t e = (uint64_t)row * d.hidden + i;
    uint32_t code = (packed[e / per_word] >> (bits * (uint32_t)(e % per_word))) & mask;
    const uint32_t blk = row * d.blocks_per_row + i / d.block_size;
    float zero;
    if (encoding == EG_ENC_OFFSET_ZEROS) {
      zero = (float)((zeros[blk / per_word] >> (bits * (blk % per_word))) & mask);
    } else {
      code ^= 1u << (bits - 1);  // two's complement -> offset binary
      zero = (float)(1u << (bits - 1));
    }
    out[d.out_offset + i] = ((float)code - zero) * scales[blk];
  }
}

// ---- fused decode attention ------------------------------------------------------------------

constexpr uint32_t kMaxCombine = 1024;  // heads x chunks the one-workgroup combine holds in LDS

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
template <int D, int CHUNK, int GMAX>
struct Prefetch {
  static constexpr uint32_t kVecs = D / 8;                      // 16-byte vectors per row
  static constexpr uint32_t kLoads = CHUNK * kVecs / kThreads;  // per thread
  static_assert(CHUNK * kVecs % kThreads == 0, "a chunk's rows split evenly over the threads");
  static_assert(GMAX * D <= kThreads && D <= kThreads, "one query element per thread");
  uint4 k[kLoads], v[kLoads];
  float qv = 0.f, kn = 0.f, vn = 0.f;
  double2 cs = make_double2(0.0, 0.0);  // the RoPE table's entry tid, when one is given
  __device__ __forceinline__ void load(const uint16_t* k_cache, const uint16_t* v_cache, uint32_t j0, uint32_t kv,
                                       uint32_t kv_heads, const float* q, uint32_t h0, uint32_t ng, const float* kp,
                                       const float* vp, const double2* rope) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (uint32_t r = 0; r < kLoads; r++) {
      const uint32_t i = tid + r * kThreads, row = i / kVecs, w = i % kVecs;
      const size_t at = ((size_t)(j0 + row) * kv_heads + kv) * D + w * 8;
      k[r] = *reinterpret_cast<const uint4*>(k_cache + at);
      v[r] = *reinterpret_cast<const uint4*>(v_cache + at);
    }
    if (tid < ng * D) qv = q[(size_t)h0 * D + tid];
    if (tid < D) {
      kn = kp[(size_t)kv * D + tid];
      vn = vp[(size_t)kv * D + tid];
    }
    if (rope && tid < D / 2) cs = rope[tid];
  }
};

// The work of one (kv head share, chunk) workgroup: RoPE, the cache append, scores, softmax
// statistics and the partial o, written to po/pm/pl, from what `pre` loaded.
template <int D, int CHUNK, int GMAX>
__device__ __forceinline__ void attend(uint32_t pos, uint32_t j0, uint32_t kv, uint32_t hs, uint32_t ng,
                                       uint32_t chunks, const Prefetch<D, CHUNK, GMAX>& pre, bool rope, uint16_t* k_cache,
                                       uint16_t* v_cache, float* po, float* pm, float* pl,
                                       const eg_attention_dims& d) {
  const uint32_t tid = threadIdx.x;
  const uint32_t live = min((uint32_t)CHUNK, pos + 1 - j0);

  // K rows padded to 144 bytes: 16-byte row reads by 16 lanes on 16 rows cover the 64 banks once.
  // V rows unpadded: the P.V loop's 8-byte reads take 4 rows a wave, 2 on each half of the banks.
  __shared__ __attribute__((aligned(16))) float qs[GMAX][D];          // rotated, pre-scaled queries
  __shared__ float knew[D], vnew[D];                                  // the new key (rotated), value
  __shared__ double2 cs[D / 2];                                       // RoPE cos/sin at `pos`
  __shared__ __attribute__((aligned(16))) uint16_t ks[CHUNK][D + 8];  // K rows (f16)
  __shared__ __attribute__((aligned(16))) uint16_t vs[CHUNK][D];      // V rows (f16)
  __shared__ float p[GMAX][CHUNK];                                    // scores, then exp(score - max)
  __shared__ float mstat[GMAX], lstat[GMAX];
  __shared__ __attribute__((aligned(16))) float half_sum[GMAX][D];    // P.V: the second wave's sums

  const float scale = 1.0f / sqrtf((float)D);
  const bool owns_new = pos < j0 + CHUNK;
  // The cached rows into LDS (every row of the chunk; the row at `pos`, stale in the cache, is
  // replaced by the new one after the next barriers).
#pragma unroll
  for (uint32_t r = 0; r < Prefetch<D, CHUNK, GMAX>::kLoads; r++) {
    const uint32_t i = tid + r * kThreads, row = i / (D / 8), w = i % (D / 8);
    uint32_t* kd = reinterpret_cast<uint32_t*>(&ks[row][w * 8]);
    uint32_t* vd = reinterpret_cast<uint32_t*>(&vs[row][w * 8]);
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
    const uint16_t kh = float_to_half(knew[tid]), vh = float_to_half(vnew[tid]);
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
        const uint2 vv = *reinterpret_cast<const uint2*>(&vs[j][e4]);
        a0 = fmaf(pj, half_to_float((uint16_t)vv.x), a0);
        a1 = fmaf(pj, half_to_float((uint16_t)(vv.x >> 16)), a1);
        a2 = fmaf(pj, half_to_float((uint16_t)vv.y), a2);
        a3 = fmaf(pj, half_to_float((uint16_t)(vv.y >> 16)), a3);
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
      o[0] = a0;
      o[chunks] = a1;
      o[2 * chunks] = a2;
      o[3 * chunks] = a3;
    }
  }
  if (tid < ng) {
    pm[(size_t)tid * chunks] = mstat[tid];
    pl[(size_t)tid * chunks] = lstat[tid];
  }
}

// One workgroup: kv head kv = blockIdx.y / HSPLIT and the HSPLIT-th share of its query heads,
// positions [j0, j0 + CHUNK) (blockIdx.x). Splitting the group's heads over HSPLIT workgroups
// doubles the parallelism of a launch that otherwise has only chunks x kv_heads workgroups; the
// K/V rows they share come from L2.
template <int D, int CHUNK, int GMAX, int HSPLIT>
__global__ __launch_bounds__(kThreads) void attention_decode_kernel(const uint32_t* position, const float* q,
                                                                    const float* k, const float* v,
                                                                    uint16_t* k_cache, uint16_t* v_cache,
                                                                    float* partials, uint32_t* counter, float* out,
                                                                    eg_attention_dims d, const double2* rope,
                                                                    uint64_t* stamp_slot) {
  const egd::WaveStamp stamp(stamp_slot);
  const uint32_t kv = blockIdx.y / HSPLIT, hs = blockIdx.y % HSPLIT;
  const uint32_t c = blockIdx.x;
  const uint32_t chunks = gridDim.x;
  const uint32_t group = d.heads / d.kv_heads;
  const uint32_t share = (group + HSPLIT - 1) / HSPLIT;
  const uint32_t gb = min(group, hs * share), ng = min(group, gb + share) - gb;  // heads [gb, gb + ng)
  const uint32_t j0 = c * CHUNK;
  const uint32_t tid = threadIdx.x;
  const uint32_t h0 = kv * group + gb;
  Prefetch<D, CHUNK, GMAX> pre;
  pre.load(k_cache, v_cache, j0, kv, d.kv_heads, q, h0, ng, k, v, rope);
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
    for (uint32_t i = tid; i < ng * D; i += blockDim.x) po[(size_t)i * chunks] = 0.f;
    if (tid < ng) {
      pm[(size_t)tid * chunks] = -INFINITY;
      pl[(size_t)tid * chunks] = 0.f;
    }
  }
  if (ng > 0 && !empty) attend<D, CHUNK, GMAX>(pos, j0, kv, hs, ng, chunks, pre, rope != nullptr, k_cache, v_cache, po, pm, pl, d);

  // The combine, once, by the last workgroup to arrive: the fence releases this workgroup's
  // partials device-wide before it counts itself; the last one's fence acquires everyone's.
  if (out) {
    __shared__ uint32_t last;
    __syncthreads();
    if (tid == 0) {
      __threadfence();
      last = atomicAdd(counter, 1u) == gridDim.x * gridDim.y - 1;
    }
    __syncthreads();
    if (last) {
      __threadfence();
      combine_all(partials, out, d.heads, D, chunks);
      if (tid == 0) *counter = 0;  // ready for the next launch
    }
  }
}

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

int launch_attention(eg_context* ctx, const char* op, const uint32_t* position, const float* q, const float* k,
                     const float* v, uint16_t* k_cache, uint16_t* v_cache, float* partials, uint32_t* counter,
                     float* out, const eg_attention_dims* dims, const double* rope) {
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
    hipLaunchKernelGGL((attention_decode_kernel<64, 64, 4, 2>), grid, dim3(kThreads), 0, ctx->stream, position, q, k,
                       v, k_cache, v_cache, partials, counter, out, *dims, cs, eg::stamp_slot(ctx));
  } else {
    const dim3 grid(dims->max_context / 128, dims->kv_heads * 4);
    hipLaunchKernelGGL((attention_decode_kernel<64, 128, 2, 4>), grid, dim3(kThreads), 0, ctx->stream, position, q, k,
                       v, k_cache, v_cache, partials, counter, out, *dims, cs, eg::stamp_slot(ctx));
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
      token[0] = bi;
      token[1] = __float_as_uint(bv);
      greedy_id = bi;
    }
  }
  if (tid == 0) {
    // a sampled step whose sampler gave up has no token (0xFFFFFFFF): counted, and nothing moves
    const bool failed = t.advance && !t.partials && !t.token_src && tok0 - d.row_begin >= d.row_count;
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
  if (!token || !packed || !scales || !out || !dims) return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  if (bits != 4 && bits != 8) return eg::fail(ctx, EG_ERR_INVALID, "%s: bits must be 4 or 8", op);
  if (encoding != EG_ENC_OFFSET_ZEROS && encoding != EG_ENC_SIGNED)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: unknown encoding %d", op, encoding);
  if (encoding == EG_ENC_OFFSET_ZEROS && !zeros) return eg::fail(ctx, EG_ERR_INVALID, "%s: zeros is NULL", op);
  if (dims->seq != 1) return eg::fail(ctx, EG_ERR_INVALID, "%s: seq %u (decode gathers one token)", op, dims->seq);
  if (dims->block_size == 0 || dims->hidden % dims->block_size != 0 ||
      dims->blocks_per_row != dims->hidden / dims->block_size)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: hidden %u / block %u / blocksPerRow %u disagree", op, dims->hidden,
                    dims->block_size, dims->blocks_per_row);
  hipLaunchKernelGGL(embed_gather_kernel, dim3(1), dim3(kThreads), 0, ctx->stream, token, packed, scales,
                     encoding == EG_ENC_SIGNED ? nullptr : zeros, out, *dims, encoding, bits);
  return eg::check_launch(ctx, op);
}

int eg_attention_decode(eg_context* ctx, const uint32_t* position, const float* q, const float* k, const float* v,
                        uint16_t* k_cache, uint16_t* v_cache, float* partials, uint32_t* counter, float* out,
                        const eg_attention_dims* dims) {
  return launch_attention(ctx, "attention_decode", position, q, k, v, k_cache, v_cache, partials, counter, out, dims,
                          nullptr);
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
