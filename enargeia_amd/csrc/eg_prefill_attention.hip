// Chunked-prefill attention on the matrix cores: the reference's attn_scores -> softmax ->
// attn_apply over the KV cache (cache_variants.ts:81-145, graph.ts:435-459), with the RoPE and
// cache writes that precede them (rope.wgsl via graph.ts:411-430, k_pack / v_pack).
//
// A chunk of `queries` rows starting at absolute position `query_begin` attends causally over
// keys [0, query_begin + i] of the cache (query i; the reference's mask `j > i + queryBegin`).
//
// Two launches:
//   1. rope_append: RoPE on the chunk's q and k rows (double-precision angles, as the decode
//      path), q pre-scaled by 1/sqrt(D) into q_rope, k and v appended to the f16 caches at
//      positions [query_begin, query_begin + queries).
//   2. attention: flash attention, one workgroup per (64 queries, head), 16 queries per wave.
//      Key tiles of 64 are staged through LDS (K row-major, V transposed); S = Q K^T and
//      O += P V run on v_mfma_f32_16x16x32_f16 (f16 operands - the cache is f16 already, q and
//      the softmax weights are rounded to f16 - with f32 accumulation), the softmax is the
//      online (running max / sum) form in f32, masked scores are the reference's NEG_LARGE.
//      Only key tiles up to the workgroup's last query's causal limit are visited.
//      When those workgroups would leave most CUs idle over a long key range (a late chunk of a
//      long prompt: 4 x 14 workgroups walking up to 32 tiles at 2048 keys), the keys are split
//      over grid.z: each split writes its rows' unnormalised o and (max, sum) to the context's
//      workspace and 3. a combine launch merges the splits in split order.
//
// The f32 cache variant (eg_attention_prefill_f32; cache_variants.ts:21-40 generates the same
// kernels per cache dtype) appends exact f32 rows and runs the attention as f32 FMAs: the
// matrix cores here take f16 or bf16 operands, which would round the f32 keys and values.
#include <algorithm>
#include <type_traits>

#include "eg_internal.hpp"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kD = 64;           // head_dim (the path's models)
constexpr int kQ = 64;           // queries per workgroup
constexpr int kK = 64;           // keys per tile
constexpr int kRow = kK + 8;     // LDS row pitch in f16 (16 bytes of padding)
constexpr float kMasked = -1.0e30f;  // NEG_LARGE, cache_variants.ts

using egd::float_to_half;

// A value as the cache holds it: f16 bits or the f32 itself.
template <class CT>
__device__ __forceinline__ CT to_cache(float x) {
  if constexpr (std::is_same<CT, float>::value) return x;
  else return float_to_half(x);
}

template <class CT>
__global__ __launch_bounds__(256) void rope_append_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, float* __restrict__ q_rope,
                                                          CT* __restrict__ k_cache, CT* __restrict__ v_cache,
                                                          eg_attention_prefill_dims d) {
  const uint32_t i = blockIdx.x;  // query row of the chunk
  const uint32_t pos = d.query_begin + i;
  const uint32_t tid = threadIdx.x;
  __shared__ double2 cs[kD / 2];
  if (tid < kD / 2) egd::rope_table<kD>(cs, tid, pos, d.theta);
  __syncthreads();
  const float scale = 1.0f / sqrtf((float)kD);  // a power of two: exact
  const uint32_t qn = d.heads * (kD / 2), kn = d.kv_heads * (kD / 2);
  for (uint32_t p = tid; p < qn + kn; p += blockDim.x) {
    const bool is_q = p < qn;
    const uint32_t pp = is_q ? p : p - qn;
    const uint32_t head = pp / (kD / 2), e = pp % (kD / 2);
    const float* src = is_q ? q + ((size_t)i * d.heads + head) * kD : k + ((size_t)i * d.kv_heads + head) * kD;
    const float2 rr = egd::rotate(src[e], src[e + kD / 2], cs[e]);
    const float ra = rr.x, rb = rr.y;
    if (is_q) {
      float* dst = q_rope + ((size_t)i * d.heads + head) * kD;
      dst[e] = ra * scale;
      dst[e + kD / 2] = rb * scale;
    } else {
      CT* dst = k_cache + ((size_t)pos * d.kv_heads + head) * kD;
      dst[e] = to_cache<CT>(ra);
      dst[e + kD / 2] = to_cache<CT>(rb);
    }
  }
  for (uint32_t p = tid; p < d.kv_heads * kD; p += blockDim.x)
    v_cache[(size_t)pos * d.kv_heads * kD + p] = to_cache<CT>(v[(size_t)i * d.kv_heads * kD + p]);
}

// The attention over an f32 cache. One workgroup per (query row i, kv head): the group's query
// heads (at most kF32Group) walk the keys [0, query_begin + i] in tiles of 256, one key per
// thread - its scores, products summed in element order - with the online softmax in f32 (the
// tile's max and sum of exp per head by fixed-order wave and cross-wave reductions), then each
// thread's outputs (head g, element e; two per thread) take the tile's weighted V rows in key
// order. Keys past the query's limit weigh 0, as the reference's NEG_LARGE mask makes them.
constexpr uint32_t kF32Tile = 256;
constexpr uint32_t kF32Group = 8;

__global__ __launch_bounds__(256) void attention_f32_kernel(const float* __restrict__ q_rope,
                                                            const float* __restrict__ k_cache,
                                                            const float* __restrict__ v_cache, float* __restrict__ out,
                                                            eg_attention_prefill_dims d) {
  __shared__ __attribute__((aligned(16))) float qs[kF32Group][kD];
  __shared__ float pw[kF32Group][kF32Tile];  // the tile's weights e^(s - M)
  __shared__ float red[4][kF32Group];        // per-wave maxima, then sums
  const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint32_t i = blockIdx.x, kv = blockIdx.y;
  const uint32_t G = d.heads / d.kv_heads, h0 = kv * G;
  const uint32_t limit = d.query_begin + i;  // the last key this query sees
  for (uint32_t t = tid; t < G * kD; t += blockDim.x) qs[t / kD][t % kD] = q_rope[((size_t)i * d.heads + h0) * kD + t];
  __syncthreads();
  float M[kF32Group], L[kF32Group];  // running max and sum per head (the same in every thread)
#pragma unroll
  for (uint32_t g = 0; g < kF32Group; g++) {
    M[g] = -INFINITY;
    L[g] = 0.f;
  }
  // this thread's outputs: (g, e) = (tid / 64, tid % 64) and (4 + tid / 64, tid % 64)
  const uint32_t e = lane, ga = wave, gb = wave + 4;
  float acc_a = 0.f, acc_b = 0.f;
  const size_t row_pitch = (size_t)d.kv_heads * kD;
  for (uint32_t t0 = 0; t0 <= limit; t0 += kF32Tile) {
    const uint32_t key = t0 + tid;
    const bool valid = key <= limit;
    float s[kF32Group];
    {
      float4 kr[kD / 4];
      const float4* src = reinterpret_cast<const float4*>(k_cache + (valid ? key : 0) * row_pitch + kv * kD);
#pragma unroll
      for (int w = 0; w < kD / 4; w++) kr[w] = src[w];
#pragma unroll
      for (uint32_t g = 0; g < kF32Group; g++) {
        float a = 0.f;
        if (g < G) {
#pragma unroll
          for (int w = 0; w < kD / 4; w++) {
            const float4 qv = *reinterpret_cast<const float4*>(&qs[g][4 * w]);
            a = fmaf(qv.x, kr[w].x, a);
            a = fmaf(qv.y, kr[w].y, a);
            a = fmaf(qv.z, kr[w].z, a);
            a = fmaf(qv.w, kr[w].w, a);
          }
        }
        s[g] = valid ? a : -INFINITY;
      }
    }
    // the tile's max per head, then the new running max and the rescale of what came before
    float scale[kF32Group];
#pragma unroll
    for (uint32_t g = 0; g < kF32Group; g++) {
      const float m = egd::team_allmax<64>(s[g]);
      if (lane == 0) red[wave][g] = m;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t g = 0; g < kF32Group; g++) {
      const float mt = fmaxf(fmaxf(red[0][g], red[1][g]), fmaxf(red[2][g], red[3][g]));
      const float mn = fmaxf(M[g], mt);
      scale[g] = g < G ? expf(M[g] - mn) : 0.f;  // e^-inf = 0 on the first tile
      M[g] = mn;
    }
    __syncthreads();  // red is reused below
#pragma unroll
    for (uint32_t g = 0; g < kF32Group; g++) {
      const float p = valid && g < G ? expf(s[g] - M[g]) : 0.f;
      pw[g][tid] = p;
      const float sum = egd::team_allsum<64>(p);
      if (lane == 0) red[wave][g] = sum;
    }
    __syncthreads();
#pragma unroll
    for (uint32_t g = 0; g < kF32Group; g++) L[g] = fmaf(L[g], scale[g], ((red[0][g] + red[1][g]) + red[2][g]) + red[3][g]);
    const uint32_t n = min(kF32Tile, limit + 1 - t0);
    const float* vrow = v_cache + (size_t)t0 * row_pitch + kv * kD + e;
    float sa = 0.f, sb = 0.f;
    for (uint32_t j = 0; j < n; j++) {
      const float vv = vrow[(size_t)j * row_pitch];
      sa = fmaf(pw[ga][j], vv, sa);
      sb = fmaf(pw[gb][j], vv, sb);
    }
    acc_a = fmaf(acc_a, scale[ga], sa);
    acc_b = fmaf(acc_b, scale[gb], sb);
    __syncthreads();  // pw and red are rewritten by the next tile
  }
  if (ga < G) out[((size_t)i * d.heads + h0 + ga) * kD + e] = acc_a / L[ga];
  if (gb < G) out[((size_t)i * d.heads + h0 + gb) * kD + e] = acc_b / L[gb];
}

// Split partials: o [split][query][head][kD] (unnormalised), then m and l [split][query][head].
struct Splits {
  float* o;          // NULL: no split, out written directly
  uint32_t keys;     // keys per split (a multiple of kK)
  uint32_t count;    // splits (grid.z)
};

constexpr float kLog2e = 1.44269504088896340736f;

// One key tile's K and V in registers between its global loads and its LDS stores: K as two
// 16-byte pieces of key tid / 4 (d 16 * (tid % 4) .. +16), V as 4 d values (4 * (tid % 16) .. +4)
// of the 4 keys 4 * (tid / 16) .. +4. The caches are read through buffer resources that end at
// the workgroup's last key: rows past it read as zeros without touching memory (a V row there
// must be finite - its weight is 0 - and no branch is needed).
struct KVTile {
  egd::u32x4 k[2];
  uint64_t v[4];
};

struct KVStream {
  __amdgpu_buffer_rsrc_t k, v;
  uint32_t koff, voff, pitch;  // this thread's byte offsets in tile 0; bytes between cache rows
};

__device__ __forceinline__ void load_tile(KVTile& t, const KVStream& st, uint32_t j0) {
  const uint32_t base = j0 * st.pitch;
  t.k[0] = egd::load_b128(st.k, st.koff + base);
  t.k[1] = egd::load_b128(st.k, st.koff + base + 16u);
#pragma unroll
  for (int i = 0; i < 4; i++) t.v[i] = egd::load_b64(st.v, st.voff + base + i * st.pitch);
}

// LDS row of key r in Ks: bit 2 flipped where bit 4 is set, so the 16 rows one S^T operand read
// touches (keys 0-3, 8-11, 16-19, 24-27 of a half tile, plus 4 for odd blocks) fall in 16
// different groups of 4 banks.
__device__ __forceinline__ uint32_t ks_row(uint32_t r) { return r ^ (((r >> 4) & 1u) << 2); }

// K row-major, V transposed: the 4 x 4 block of V (keys 4a .. 4a+3, d c .. c+3) becomes 4 rows of
// Vt, one 8-byte store each.
__device__ __forceinline__ void store_tile(const KVTile& t, uint16_t (*Ks)[kRow], uint16_t (*Vt)[kRow], uint32_t tid) {
  {
    const uint32_t r = ks_row(tid >> 2), c = (tid & 3u) * 16u;
    *reinterpret_cast<egd::u32x4*>(&Ks[r][c]) = t.k[0];
    *reinterpret_cast<egd::u32x4*>(&Ks[r][c + 8]) = t.k[1];
  }
  const uint32_t a = tid >> 4, c = (tid & 15u) * 4u;
  // t.v[i] = (d c, c+1 | c+2, c+3) of key 4a + i; row c + e of Vt takes element e of each key
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int sh = 32 * (e >> 1);
    const uint32_t k0 = (uint32_t)(t.v[0] >> sh), k1 = (uint32_t)(t.v[1] >> sh);
    const uint32_t k2 = (uint32_t)(t.v[2] >> sh), k3 = (uint32_t)(t.v[3] >> sh);
    // element e is the low (e even) or high (e odd) half of word e / 2
    const uint2 row = (e & 1) ? make_uint2((k0 >> 16) | (k1 & 0xFFFF0000u), (k2 >> 16) | (k3 & 0xFFFF0000u))
                              : make_uint2((k0 & 0xFFFFu) | (k1 << 16), (k2 & 0xFFFFu) | (k3 << 16));
    *reinterpret_cast<uint2*>(&Vt[c + e][4 * a]) = row;
  }
}

// Flash attention in the transposed form: S^T = K Q^T and O^T += V^T P^T, so that each lane holds
// ONE query's scores (the MFMA D layout puts a column in a lane) and P goes from the S^T
// accumulators straight into the B operand of the second product, with no LDS round trip.
//
// Key order inside a tile: row m = 4g + e of S^T block n (n < 4, g = m / 4, e = m % 4) is key
// 32 (n / 2) + 8 g + 4 (n % 2) + e, so a lane (column lr, group g = lane / 16) holds, for each half
// h of the tile, the 8 consecutive keys 32 h + 8 g .. +8 - exactly the 8 k-slots of its P^T operand
// in the second product, whose V^T operand then reads 8 consecutive keys of a Vt row.
__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ q_rope,
                                                        const uint16_t* __restrict__ k_cache,
                                                        const uint16_t* __restrict__ v_cache, float* __restrict__ out,
                                                        eg_attention_prefill_dims d, Splits sp, uint32_t out_bf16) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[2][kK][kRow];  // [buffer][key][d]
  __shared__ __attribute__((aligned(16))) uint16_t Vt[2][kD][kRow];  // [buffer][d][key]
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  const uint32_t lr = lane & 15u, lg = lane >> 4;  // MFMA lane coordinates
  const uint32_t h = blockIdx.y, kv = h / (d.heads / d.kv_heads);
  // the last query blocks (the longest causal walks) first, so they do not start last
  const uint32_t q0 = (gridDim.x - 1 - blockIdx.x) * kQ;
  const uint32_t query = q0 + wave * 16 + lr;  // this lane's query (its column of S^T and O^T)

  // Q^T fragments (B operand of S^T = K Q^T): query lr, d 32 ks + 8 lg .. +8.
  half8 qb[2];
  {
    const bool in = query < d.queries;
    const float4* src = reinterpret_cast<const float4*>(q_rope + ((size_t)(in ? query : 0) * d.heads + h) * kD + 8 * lg);
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const float4 a = in ? src[8 * ks] : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 b = in ? src[8 * ks + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
      qb[ks] = half8{(_Float16)a.x, (_Float16)a.y, (_Float16)a.z, (_Float16)a.w,
                     (_Float16)b.x, (_Float16)b.y, (_Float16)b.z, (_Float16)b.w};
    }
  }

  // O^T blocks (d 16 nd .. +16) in the D layout: lane holds d 16 nd + 4 lg + e of its query.
  f32x4 o[4];
#pragma unroll
  for (int n = 0; n < 4; n++) o[n] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kMasked;  // the query's running max (the same in the 4 lanes holding it)
  float l = 0.f;      // this lane's share of the running sum (its 16 keys of each tile)

  const uint32_t last_query = min(q0 + (uint32_t)kQ, d.queries) - 1;
  uint32_t key_end = d.query_begin + last_query + 1;  // the keys any row of this group sees
  uint32_t key_begin = 0;
  if (sp.o) {  // this split's keys
    key_begin = blockIdx.z * sp.keys;
    key_end = min(key_end, key_begin + sp.keys);
  }
  const uint32_t ntiles = key_end > key_begin ? (key_end - key_begin + kK - 1) / kK : 0;
  const uint32_t limit = d.query_begin + query;  // the last key this query sees
  // a tile wholly at or below the wave's first query's limit (and inside the keys) needs no mask
  const uint32_t open_end = min(d.query_begin + q0 + wave * 16 + 1, key_end);
  // this lane's A-operand rows of S^T blocks n (even, odd): key 32 (n / 2) + 8 (lr / 4) + 4 (n % 2)
  // + lr % 4, at its swizzled LDS row
  const uint32_t krow = 8 * (lr >> 2) + (lr & 3u);
  const uint32_t krows[2] = {ks_row(krow), ks_row(krow + 4)};

  const uint32_t pitch = d.kv_heads * kD * 2u;
  const KVStream kst{egd::buffer(k_cache, key_end * pitch), egd::buffer(v_cache, key_end * pitch),
                     (tid >> 2) * pitch + kv * kD * 2u + (tid & 3u) * 32u,
                     (tid >> 4) * 4u * pitch + kv * kD * 2u + (tid & 15u) * 8u, pitch};
  KVTile kvt;
  if (ntiles) {
    load_tile(kvt, kst, key_begin);
    store_tile(kvt, Ks[0], Vt[0], tid);
  }
  __syncthreads();
  for (uint32_t t = 0; t < ntiles; t++) {
    const uint32_t j0 = key_begin + t * kK, buf = t & 1u;
    // the next tile's loads stay in flight through this tile's products
    if (t + 1 < ntiles) load_tile(kvt, kst, j0 + kK);

    f32x4 s[4];
#pragma unroll
    for (int n = 0; n < 4; n++) {
      s[n] = f32x4{0.f, 0.f, 0.f, 0.f};
      const uint32_t row = 32 * (n >> 1) + krows[n & 1];
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const half8 ka = *reinterpret_cast<const half8*>(&Ks[buf][row][32 * ks + 8 * lg]);
        s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qb[ks], s[n], 0, 0, 0);
      }
    }

    // Causal mask (tiles that cross a limit or the last key) and the online softmax: the lane's
    // 16 scores, then the max over the 4 lanes holding the query (lanes lr, lr + 16, lr + 32,
    // lr + 48).
    if (j0 + kK > open_end) {
#pragma unroll
      for (int n = 0; n < 4; n++)
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const uint32_t j = j0 + 32 * (n >> 1) + 8 * lg + 4 * (n & 1) + e;
          if (!(j <= limit && j < key_end)) s[n][e] = kMasked;
        }
    }
    float mx = kMasked;
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
      for (int e = 0; e < 4; e++) mx = fmaxf(mx, s[n][e]);
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx);
    const float alpha = __builtin_amdgcn_exp2f((m - mnew) * kLog2e);
    // a query with no visible key yet (a split wholly past its causal limit) keeps nothing: its
    // exponent offset is pushed past f32's range below zero
    const float ml = mnew == kMasked ? 3.0e38f : mnew * kLog2e;
    float sum = 0.f;
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float p = __builtin_amdgcn_exp2f(fmaf(s[n][e], kLog2e, -ml));
        s[n][e] = p;
        sum += p;
      }
    l = l * alpha + sum;
    // the accumulators are rescaled only when some query of the wave found a larger max
    if (__builtin_amdgcn_ballot_w64(mnew > m) != 0) {
#pragma unroll
      for (int n = 0; n < 4; n++) o[n] *= alpha;
    }
    m = mnew;

    // O^T += V^T P^T over the two halves of the tile.
#pragma unroll
    for (int hh = 0; hh < 2; hh++) {
      const half8 pb = half8{(_Float16)s[2 * hh][0],     (_Float16)s[2 * hh][1],     (_Float16)s[2 * hh][2],
                             (_Float16)s[2 * hh][3],     (_Float16)s[2 * hh + 1][0], (_Float16)s[2 * hh + 1][1],
                             (_Float16)s[2 * hh + 1][2], (_Float16)s[2 * hh + 1][3]};
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const half8 va = *reinterpret_cast<const half8*>(&Vt[buf][16 * n + lr][32 * hh + 8 * lg]);
        o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va, pb, o[n], 0, 0, 0);
      }
    }
    // the other buffer was last read in the previous iteration, before the barrier that ended it
    if (t + 1 < ntiles) store_tile(kvt, Ks[buf ^ 1u], Vt[buf ^ 1u], tid);
    __syncthreads();
  }

  // the query's sum over its 4 lanes
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (query >= d.queries) return;
  if (sp.o) {
    const size_t row = ((size_t)blockIdx.z * d.queries + query) * d.heads + h;
#pragma unroll
    for (int n = 0; n < 4; n++)
      *reinterpret_cast<float4*>(&sp.o[row * kD + 16 * n + 4 * lg]) = make_float4(o[n][0], o[n][1], o[n][2], o[n][3]);
    if (lg == 0) {
      float* mlp = sp.o + (size_t)sp.count * d.queries * d.heads * kD;
      mlp[row] = m;
      mlp[(size_t)sp.count * d.queries * d.heads + row] = l;
    }
    return;
  }
  const float inv = 1.0f / l;
  const size_t at = ((size_t)query * d.heads + h) * kD + 4 * lg;
#pragma unroll
  for (int n = 0; n < 4; n++) {
    const float4 v = make_float4(o[n][0] * inv, o[n][1] * inv, o[n][2] * inv, o[n][3] * inv);
    if (out_bf16) *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(out) + at + 16 * n) =
        make_uint2(egd::pack_bf16(v.x, v.y), egd::pack_bf16(v.z, v.w));
    else *reinterpret_cast<float4*>(out + at + 16 * n) = v;
  }
}

// The splits merged: out = sum_z o_z e^(m_z - M) / sum_z l_z e^(m_z - M), M = max_z m_z, splits
// in order (an empty split has m = NEG_LARGE and l = 0, weight 0). One thread per 4 elements of a
// row. A row's splits past its causal limit are empty (z > zmax: the split's first key is past the
// row's last) and are not read. Up to kFastSplits splits, the statistics and values of the
// others are loaded at once (no chain of dependent round trips); more splits take the loop. Both
// add in split order: the same result.
constexpr uint32_t kFastSplits = 8;

__device__ __forceinline__ float4 merged(const float* __restrict__ part, const float* m, const float* l, size_t total,
                                         uint32_t rows, size_t row, size_t idx, uint32_t splits, uint32_t zmax) {
  float M = kMasked, L = 0.f;
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (splits <= kFastSplits) {
    float mz[kFastSplits], lz[kFastSplits];
    float4 vz[kFastSplits];
#pragma unroll
    for (uint32_t z = 0; z < kFastSplits; z++) {
      if (z <= zmax) {
        mz[z] = m[(size_t)z * rows + row];
        lz[z] = l[(size_t)z * rows + row];
        vz[z] = reinterpret_cast<const float4*>(part + (size_t)z * total)[idx];
      }
    }
#pragma unroll
    for (uint32_t z = 0; z < kFastSplits; z++)
      if (z <= zmax) M = fmaxf(M, mz[z]);
#pragma unroll
    for (uint32_t z = 0; z < kFastSplits; z++) {
      if (z <= zmax && lz[z] > 0.f) {
        const float w = expf(mz[z] - M);
        L = fmaf(lz[z], w, L);
        acc.x = fmaf(vz[z].x, w, acc.x);
        acc.y = fmaf(vz[z].y, w, acc.y);
        acc.z = fmaf(vz[z].z, w, acc.z);
        acc.w = fmaf(vz[z].w, w, acc.w);
      }
    }
  } else {
    for (uint32_t z = 0; z <= zmax; z++) M = fmaxf(M, m[(size_t)z * rows + row]);
    for (uint32_t z = 0; z <= zmax; z++) {
      const float lzz = l[(size_t)z * rows + row];
      if (!(lzz > 0.f)) continue;
      const float w = expf(m[(size_t)z * rows + row] - M);
      L = fmaf(lzz, w, L);
      const float4 v = reinterpret_cast<const float4*>(part + (size_t)z * total)[idx];
      acc.x = fmaf(v.x, w, acc.x);
      acc.y = fmaf(v.y, w, acc.y);
      acc.z = fmaf(v.z, w, acc.z);
      acc.w = fmaf(v.w, w, acc.w);
    }
  }
  return make_float4(acc.x / L, acc.y / L, acc.z / L, acc.w / L);
}

__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                      uint32_t rows, uint32_t splits, uint32_t out_bf16, uint32_t heads,
                                                      uint32_t query_begin, uint32_t split_keys) {
  const size_t total = (size_t)rows * kD;
  const float* m = part + (size_t)splits * total;
  const float* l = m + (size_t)splits * rows;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total / 4; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t row = idx / (kD / 4);
    const uint32_t zmax = min(splits - 1, (query_begin + (uint32_t)(row / heads)) / split_keys);
    const float4 v = merged(part, m, l, total, rows, row, idx, splits, zmax);
    if (out_bf16) reinterpret_cast<uint2*>(out)[idx] = make_uint2(egd::pack_bf16(v.x, v.y), egd::pack_bf16(v.z, v.w));
    else reinterpret_cast<float4*>(out)[idx] = v;
  }
}

}  // namespace

// The dims checks of eg_attention_prefill (pointers aside).
int eg::check_attention_prefill(eg_context* ctx, const char* op, const eg_attention_prefill_dims* dims) {
  const eg_attention_prefill_dims& d = *dims;
  if (d.head_dim != (uint32_t)kD)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: head_dim %u is not supported (64)", op, d.head_dim);
  if (d.kv_heads == 0 || d.heads == 0 || d.heads % d.kv_heads != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: heads %u are not a multiple of kv_heads %u", op, d.heads, d.kv_heads);
  if (d.queries == 0) return EG_OK;
  if (d.keys != d.query_begin + d.queries)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: keys %u != query_begin %u + queries %u", op, d.keys, d.query_begin,
                    d.queries);
  if ((uint64_t)d.query_begin + d.queries > d.max_context)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: positions up to %llu exceed the cache's %u", op,
                    (unsigned long long)d.query_begin + d.queries, d.max_context);
  if ((uint64_t)d.max_context * d.kv_heads * d.head_dim * 2 >= (1ull << 31))
    return eg::fail(ctx, EG_ERR_RANGE, "%s: a cache of %u positions x %u kv heads exceeds 2 GiB", op, d.max_context,
                    d.kv_heads);
  if (d.heads > 65535 || (d.queries + kQ - 1) / kQ > 0x7FFFFFFFu)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u heads over the grid limit", op, d.heads);
  return EG_OK;
}

int eg::attention_prefill_run(eg_context* ctx, const float* q_rope, const uint16_t* k_cache, const uint16_t* v_cache,
                              float* out, const eg_attention_prefill_dims& d, bool out_bf16) {
  const char* op = "attention_prefill";
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15u)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: the caches must be 16-byte aligned", op);
  if ((reinterpret_cast<uintptr_t>(q_rope) | reinterpret_cast<uintptr_t>(out)) & 15u)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: q_rope and out must be 16-byte aligned", op);
  if (d.queries == 0) return EG_OK;
  // Keys split over a long key range, within the workspace: where the (query block, head) grid
  // leaves most CUs idle, into splits of at least 4 key tiles, about one workgroup per CU in all;
  // and so that no workgroup walks more than 8 tiles - the causal limit makes the last query
  // blocks of a long chunk the longest, and with the split their keys spread over more
  // workgroups while the early blocks' later splits are empty.
  const uint32_t blocks = (d.queries + kQ - 1) / kQ;
  const uint64_t grid = (uint64_t)blocks * d.heads;
  const uint32_t tiles = (d.keys + kK - 1) / kK;
  const uint32_t cap = ctx->attention_split_tiles;
  const uint64_t target = (uint64_t)ctx->cu_count * ctx->attention_split_fill;
  uint32_t splits = 1;
  if (tiles >= 8) {
    if (grid < target) splits = (uint32_t)std::min<uint64_t>((target + grid - 1) / grid, tiles / 4);
    splits = std::max(splits, (tiles + cap - 1) / cap);
  }
  const uint64_t rows = (uint64_t)d.queries * d.heads;
  while (splits > 1 && (uint64_t)splits * rows * (kD + 2) * 4 > eg::kPartialsBytes) splits--;
  Splits sp{nullptr, 0, 1};
  if (splits > 1) {
    sp.keys = ((tiles + splits - 1) / splits) * kK;
    sp.count = (d.keys + sp.keys - 1) / sp.keys;
    sp.o = reinterpret_cast<float*>(eg::partials(ctx));
  }
  hipLaunchKernelGGL(attention_kernel, dim3(blocks, d.heads, sp.count), dim3(256), 0, ctx->stream, q_rope, k_cache,
                     v_cache, out, d, sp, out_bf16 ? 1u : 0u);
  if (sp.o) {
    const uint64_t total = rows * kD;
    const uint32_t cblocks = (uint32_t)std::min<uint64_t>((total / 4 + 255) / 256, (uint64_t)ctx->cu_count * 8);
    hipLaunchKernelGGL(combine_kernel, dim3(cblocks), dim3(256), 0, ctx->stream, sp.o, out, (uint32_t)rows, sp.count,
                       out_bf16 ? 1u : 0u, d.heads, d.query_begin, sp.keys);
  }
  return eg::check_launch(ctx, op);
}

extern "C" int eg_attention_prefill(eg_context* ctx, const float* q, const float* k, const float* v, uint16_t* k_cache,
                                    uint16_t* v_cache, float* q_rope, float* out,
                                    const eg_attention_prefill_dims* dims) {
  const char* op = "attention_prefill";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!dims || !q || !k || !v || !k_cache || !v_cache || !q_rope || !out)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  int st = eg::check_attention_prefill(ctx, op, dims);
  if (st != EG_OK || dims->queries == 0) return st;
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15u)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: the caches must be 16-byte aligned", op);
  if ((reinterpret_cast<uintptr_t>(q_rope) | reinterpret_cast<uintptr_t>(out)) & 15u)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: q_rope and out must be 16-byte aligned", op);
  const eg_attention_prefill_dims& d = *dims;
  hipLaunchKernelGGL(rope_append_kernel<uint16_t>, dim3(d.queries), dim3(256), 0, ctx->stream, q, k, v, q_rope,
                     k_cache, v_cache, d);
  return eg::attention_prefill_run(ctx, q_rope, k_cache, v_cache, out, d);
}

extern "C" int eg_attention_prefill_f32(eg_context* ctx, const float* q, const float* k, const float* v, float* k_cache,
                                        float* v_cache, float* q_rope, float* out,
                                        const eg_attention_prefill_dims* dims) {
  const char* op = "attention_prefill_f32";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!dims || !q || !k || !v || !k_cache || !v_cache || !q_rope || !out)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  int st = eg::check_attention_prefill(ctx, op, dims);
  if (st != EG_OK || dims->queries == 0) return st;
  const eg_attention_prefill_dims& d = *dims;
  if (d.heads / d.kv_heads > kF32Group)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: %u query heads per kv head (at most %u)", op, d.heads / d.kv_heads,
                    kF32Group);
  if (d.kv_heads > 65535) return eg::fail(ctx, EG_ERR_RANGE, "%s: %u kv heads exceed the grid", op, d.kv_heads);
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache) |
       reinterpret_cast<uintptr_t>(q_rope)) & 15u)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: the caches and q_rope must be 16-byte aligned", op);
  hipLaunchKernelGGL(rope_append_kernel<float>, dim3(d.queries), dim3(256), 0, ctx->stream, q, k, v, q_rope, k_cache,
                     v_cache, d);
  hipLaunchKernelGGL(attention_f32_kernel, dim3(d.queries, d.kv_heads), dim3(256), 0, ctx->stream, q_rope, k_cache,
                     v_cache, out, d);
  return eg::check_launch(ctx, op);
}
