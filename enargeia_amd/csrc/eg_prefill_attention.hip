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
#include <algorithm>

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

__global__ __launch_bounds__(256) void rope_append_kernel(const float* __restrict__ q, const float* __restrict__ k,
                                                          const float* __restrict__ v, float* __restrict__ q_rope,
                                                          uint16_t* __restrict__ k_cache,
                                                          uint16_t* __restrict__ v_cache,
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
    const double a = src[e], b = src[e + kD / 2];
    const float ra = (float)(a * cs[e].x - b * cs[e].y);
    const float rb = (float)(b * cs[e].x + a * cs[e].y);
    if (is_q) {
      float* dst = q_rope + ((size_t)i * d.heads + head) * kD;
      dst[e] = ra * scale;
      dst[e + kD / 2] = rb * scale;
    } else {
      uint16_t* dst = k_cache + ((size_t)pos * d.kv_heads + head) * kD;
      dst[e] = float_to_half(ra);
      dst[e + kD / 2] = float_to_half(rb);
    }
  }
  for (uint32_t p = tid; p < d.kv_heads * kD; p += blockDim.x)
    v_cache[(size_t)pos * d.kv_heads * kD + p] = float_to_half(v[(size_t)i * d.kv_heads * kD + p]);
}

// Split partials: o [split][query][head][kD] (unnormalised), then m and l [split][query][head].
struct Splits {
  float* o;          // NULL: no split, out written directly
  uint32_t keys;     // keys per split (a multiple of kK)
  uint32_t count;    // splits (grid.z)
};

__global__ __launch_bounds__(256) void attention_kernel(const float* __restrict__ q_rope,
                                                        const uint16_t* __restrict__ k_cache,
                                                        const uint16_t* __restrict__ v_cache, float* __restrict__ out,
                                                        eg_attention_prefill_dims d, Splits sp) {
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kK][kRow];     // [key][d]
  __shared__ __attribute__((aligned(16))) uint16_t Vt[kD][kRow];     // [d][key]
  __shared__ __attribute__((aligned(16))) uint16_t Ps[4][16][kRow];  // per wave: [query][key]
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  const uint32_t lr = lane & 15u, lg = lane >> 4;  // MFMA lane coordinates
  const uint32_t h = blockIdx.y, kv = h / (d.heads / d.kv_heads);
  const uint32_t q0 = blockIdx.x * kQ;
  const uint32_t row0 = q0 + wave * 16;

  // Q fragments (A operand of S = Q K^T): lane holds query row0 + lr, d 8*lg + 32*ks .. +8.
  half8 qa[2];
  {
    const uint32_t r = row0 + lr;
#pragma unroll
    for (int ks = 0; ks < 2; ks++)
#pragma unroll
      for (int e = 0; e < 8; e++)
        qa[ks][e] = r < d.queries ? (_Float16)q_rope[((size_t)r * d.heads + h) * kD + 32 * ks + 8 * lg + e]
                                  : (_Float16)0.f;
  }

  // O blocks (d 16*n .. 16*n+15) in the MFMA D layout: lane holds rows 4*lg + e, column lr.
  f32x4 o[4];
  float m[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    o[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[e] = kMasked;
    l[e] = 0.f;
  }

  const uint32_t last_query = min(q0 + (uint32_t)kQ, d.queries) - 1;
  uint32_t key_end = d.query_begin + last_query + 1;  // the keys any row of this group sees
  uint32_t key_begin = 0;
  if (sp.o) {  // this split's keys
    key_begin = blockIdx.z * sp.keys;
    key_end = min(key_end, key_begin + sp.keys);
  }
  const size_t pitch = (size_t)d.kv_heads * kD;             // f16 elements between cache rows
  for (uint32_t j0 = key_begin; j0 < key_end; j0 += kK) {
    __syncthreads();  // the previous tile's K, V and P are consumed
    {
      const uint32_t r = tid >> 2, c = (tid & 3u) * 16u;  // 64 keys x 4 pieces of 16 elements
      const uint32_t j = j0 + r;
      uint4 kk[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
      uint4 vv[2] = {make_uint4(0, 0, 0, 0), make_uint4(0, 0, 0, 0)};
      if (j < key_end) {
        const uint4* ks = reinterpret_cast<const uint4*>(k_cache + (size_t)j * pitch + kv * kD + c);
        const uint4* vs = reinterpret_cast<const uint4*>(v_cache + (size_t)j * pitch + kv * kD + c);
        kk[0] = ks[0];
        kk[1] = ks[1];
        vv[0] = vs[0];
        vv[1] = vs[1];
      }
      *reinterpret_cast<uint4*>(&Ks[r][c]) = kk[0];
      *reinterpret_cast<uint4*>(&Ks[r][c + 8]) = kk[1];
      const uint16_t* vh = reinterpret_cast<const uint16_t*>(vv);
#pragma unroll
      for (int e = 0; e < 16; e++) Vt[c + e][r] = vh[e];
    }
    __syncthreads();

    // S = Q K^T, 16 queries x 64 keys per wave.
    f32x4 s[4];
#pragma unroll
    for (int n = 0; n < 4; n++) {
      s[n] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 2; ks++) {
        const half8 kb = *reinterpret_cast<const half8*>(&Ks[16 * n + lr][32 * ks + 8 * lg]);
        s[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(qa[ks], kb, s[n], 0, 0, 0);
      }
    }

    // Causal mask and the online softmax, per row (4 per lane; a row's 64 keys live in the 16
    // lanes sharing lg, 4 per lane).
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t i = row0 + 4 * lg + e;
      float mx = kMasked;
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const uint32_t j = j0 + 16 * n + lr;
        const float v = (j <= d.query_begin + i && j < d.keys) ? s[n][e] : kMasked;
        s[n][e] = v;
        mx = fmaxf(mx, v);
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float mnew = fmaxf(m[e], mx);
      const float alpha = expf(m[e] - mnew);
      // a row with no visible key yet (a split wholly past its causal limit) keeps nothing
      const bool none = mnew == kMasked;
      float sum = 0.f;
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const float p = none ? 0.f : expf(s[n][e] - mnew);
        s[n][e] = p;
        sum += p;
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) sum += __shfl_xor(sum, off, 64);
      l[e] = l[e] * alpha + sum;
      m[e] = mnew;
#pragma unroll
      for (int n = 0; n < 4; n++) o[n][e] *= alpha;
    }

    // P (f16) through LDS into the A-operand layout, then O += P V.
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
      for (int e = 0; e < 4; e++) Ps[wave][4 * lg + e][16 * n + lr] = float_to_half(s[n][e]);
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's P writes are in LDS
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int ks = 0; ks < 2; ks++) {
      const half8 pa = *reinterpret_cast<const half8*>(&Ps[wave][lr][32 * ks + 8 * lg]);
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const half8 vb = *reinterpret_cast<const half8*>(&Vt[16 * n + lr][32 * ks + 8 * lg]);
        o[n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pa, vb, o[n], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int e = 0; e < 4; e++) {
    const uint32_t i = row0 + 4 * lg + e;
    if (i >= d.queries) continue;
    if (sp.o) {
      const size_t row = ((size_t)blockIdx.z * d.queries + i) * d.heads + h;
#pragma unroll
      for (int n = 0; n < 4; n++) sp.o[row * kD + 16 * n + lr] = o[n][e];
      if (lr == 0) {
        float* ml = sp.o + (size_t)sp.count * d.queries * d.heads * kD;
        ml[row] = m[e];
        ml[(size_t)sp.count * d.queries * d.heads + row] = l[e];
      }
      continue;
    }
    const float inv = 1.0f / l[e];
#pragma unroll
    for (int n = 0; n < 4; n++) out[((size_t)i * d.heads + h) * kD + 16 * n + lr] = o[n][e] * inv;
  }
}

// The splits merged: out = sum_z o_z e^(m_z - M) / sum_z l_z e^(m_z - M), M = max_z m_z, splits
// in order (an empty split has m = NEG_LARGE and l = 0, weight 0).
__global__ __launch_bounds__(256) void combine_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                      uint32_t rows, uint32_t splits) {
  const size_t total = (size_t)rows * kD;
  const float* m = part + (size_t)splits * total;
  const float* l = m + (size_t)splits * rows;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t row = idx / kD;
    float M = kMasked;
    for (uint32_t z = 0; z < splits; z++) M = fmaxf(M, m[(size_t)z * rows + row]);
    float L = 0.f, acc = 0.f;
    for (uint32_t z = 0; z < splits; z++) {
      const float w = l[(size_t)z * rows + row] > 0.f ? expf(m[(size_t)z * rows + row] - M) : 0.f;
      L = fmaf(l[(size_t)z * rows + row], w, L);
      acc = fmaf(part[(size_t)z * total + idx], w, acc);
    }
    out[idx] = acc / L;
  }
}

}  // namespace

extern "C" int eg_attention_prefill(eg_context* ctx, const float* q, const float* k, const float* v, uint16_t* k_cache,
                                    uint16_t* v_cache, float* q_rope, float* out,
                                    const eg_attention_prefill_dims* dims) {
  const char* op = "attention_prefill";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!dims || !q || !k || !v || !k_cache || !v_cache || !q_rope || !out)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
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
  if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15u)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: the caches must be 16-byte aligned", op);
  if (d.heads > 65535 || (d.queries + kQ - 1) / kQ > 0x7FFFFFFFu)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u heads over the grid limit", op, d.heads);
  hipLaunchKernelGGL(rope_append_kernel, dim3(d.queries), dim3(256), 0, ctx->stream, q, k, v, q_rope, k_cache,
                     v_cache, d);
  // Keys split over a long key range, within the workspace: where the (query block, head) grid
  // leaves most CUs idle, into splits of at least 4 key tiles, about one workgroup per CU in all;
  // and so that no workgroup walks more than 8 tiles - the causal limit makes the last query
  // blocks of a long chunk the longest, and with the split their keys spread over more
  // workgroups while the early blocks' later splits are empty.
  const uint32_t blocks = (d.queries + kQ - 1) / kQ;
  const uint64_t grid = (uint64_t)blocks * d.heads;
  const uint32_t tiles = (d.keys + kK - 1) / kK;
  uint32_t splits = 1;
  if (tiles >= 8) {
    if (grid < (uint64_t)ctx->cu_count)
      splits = (uint32_t)std::min<uint64_t>((ctx->cu_count + grid - 1) / grid, tiles / 4);
    splits = std::max(splits, (tiles + 7) / 8);
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
                     v_cache, out, d, sp);
  if (sp.o) {
    const uint64_t total = rows * kD;
    const uint32_t cblocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, (uint64_t)ctx->cu_count * 8);
    hipLaunchKernelGGL(combine_kernel, dim3(cblocks), dim3(256), 0, ctx->stream, sp.o, out, (uint32_t)rows, sp.count);
  }
  return eg::check_launch(ctx, op);
}
