// Decode-shape (M=1) quantized GEMV: the host side (shape choice, validation, launches, batched
// plans) and the kernels for inputs given as a vector. The kernel template and its design notes
// are in eg_gemv_kernel.hpp; the fused input stages are instantiated in eg_gemv_rmsnorm.hip,
// eg_gemv_silu.hip and eg_gemv_attention.hip.
//
// Reference ops: matmul_q4_decode (matmul_q4_decode.wgsl:56-101) and lm_head_q4/q8
// (embedding_variants.ts:135-180).
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "eg_gemv_kernel.hpp"

namespace {

using namespace eg_gemv;

// Fallback for layouts the chunked kernel does not take (K or block_size not a multiple of
// the chunk, unaligned streams, very long rows): one wave per row, the reference's exact
// per-element indexing (matmul_q4_decode.wgsl:66-83), wave butterfly instead of the LDS tree.
template <bool ARGMAX>
__global__ __launch_bounds__(256) void gemv_generic_kernel(
    const float* __restrict__ x, const uint32_t* __restrict__ packed, const float* __restrict__ scales,
    const uint32_t* __restrict__ zeros, const float* __restrict__ bias, float* out, uint32_t n, uint32_t k,
    uint32_t block_size, uint32_t blocks_per_row, uint32_t out_offset, int bits, int encoding,
    uint32_t* partials) {
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t wave = blockIdx.x * kWaves + (threadIdx.x >> 6);
  const uint32_t total_waves = gridDim.x * kWaves;
  const uint32_t per_word = 32u / (uint32_t)bits;
  const uint32_t mask = (1u << bits) - 1u;
  float best_v = -1.0e30f;
  uint32_t best_i = out_offset;
  for (uint32_t row = wave; row < n; row += total_waves) {
    float acc = 0.f;
    for (uint32_t i = lane; i < k; i += 64) {
      const size_t flat = (size_t)row * k + i;
      uint32_t code = (packed[flat / per_word] >> (bits * (flat % per_word))) & mask;
      const uint32_t blk = row * blocks_per_row + i / block_size;
      float zero;
      if (encoding == EG_ENC_OFFSET_ZEROS) {
        zero = (float)((zeros[blk / per_word] >> (bits * (blk % per_word))) & mask);
      } else {
        code ^= 1u << (bits - 1);
        zero = (float)(1u << (bits - 1));
      }
      acc = fmaf(((float)code - zero) * scales[blk], x[i], acc);
    }
    acc = egd::team_sum<64>(acc);
    if (lane == 63) {
      const float v = bias ? acc + bias[row] : acc;
      if (out) out[row + out_offset] = v;
      if (ARGMAX && egd::better(v, row + out_offset, best_v, best_i)) {
        best_v = v;
        best_i = row + out_offset;
      }
    }
  }
  if (ARGMAX) {
    __shared__ float wv[kWaves];
    __shared__ uint32_t wi[kWaves];
    egd::team_argmax<64>(best_v, best_i);
    if (lane == 0) {
      wv[threadIdx.x >> 6] = best_v;
      wi[threadIdx.x >> 6] = best_i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      float bv = wv[0];
      uint32_t bi = wi[0];
      for (int q = 1; q < kWaves; q++)
        if (egd::better(wv[q], wi[q], bv, bi)) {
          bv = wv[q];
          bi = wi[q];
        }
      partials[2 * blockIdx.x] = __float_as_uint(bv);
      partials[2 * blockIdx.x + 1] = bi;
    }
  }
}

// The LM head over an f16 (BITS 16) or f32 (BITS 32) tied table (the 'f16' / 'f32' dtypes of
// embedding_variants.ts:46-74, 135-180): out[n] = sum_k x[k] table[n][k]. With no codes to
// unpack the launch streams the table: one wave per row, two rows per step (their loads issued
// together), grid-stride over the rows; x in LDS, RMS-normalised there when the final norm is
// fused (NORM, the quantized input stage's arithmetic and order, so the same bits); the row as
// 16-byte vectors (VEC; 8 halves or 4 floats, element 2j of an f16 pair in the low half), each
// lane's products summed in element order, then the wave's DPP sum. VEC false reads element by
// element (a row that is not a whole number of vectors, or an unaligned table). ARGMAX leaves
// one (value bits, index) partial per workgroup, as gemv_generic_kernel does.
constexpr uint32_t kDenseMaxK = 16384;  // x in LDS: 64 KiB

template <int BITS>
__device__ __forceinline__ float dense_dot(const uint4 w, const float* xv, float acc) {
  if constexpr (BITS == 32) {
    const float4 a = *reinterpret_cast<const float4*>(xv);
    acc = fmaf(__uint_as_float(w.x), a.x, acc);
    acc = fmaf(__uint_as_float(w.y), a.y, acc);
    acc = fmaf(__uint_as_float(w.z), a.z, acc);
    return fmaf(__uint_as_float(w.w), a.w, acc);
  } else {
    const float4 a = *reinterpret_cast<const float4*>(xv), b = *reinterpret_cast<const float4*>(xv + 4);
    acc = fmaf(egd::half_to_float((uint16_t)w.x), a.x, acc);
    acc = fmaf(egd::half_to_float((uint16_t)(w.x >> 16)), a.y, acc);
    acc = fmaf(egd::half_to_float((uint16_t)w.y), a.z, acc);
    acc = fmaf(egd::half_to_float((uint16_t)(w.y >> 16)), a.w, acc);
    acc = fmaf(egd::half_to_float((uint16_t)w.z), b.x, acc);
    acc = fmaf(egd::half_to_float((uint16_t)(w.z >> 16)), b.y, acc);
    acc = fmaf(egd::half_to_float((uint16_t)w.w), b.z, acc);
    return fmaf(egd::half_to_float((uint16_t)(w.w >> 16)), b.w, acc);
  }
}

template <int BITS, bool ARGMAX, bool NORM, bool VEC>
__global__ __launch_bounds__(256) void dense_head_kernel(const float* __restrict__ x, const float* __restrict__ norm_w,
                                                         float eps, const uint32_t* __restrict__ table, float* out,
                                                         uint32_t n, uint32_t k, uint32_t out_offset,
                                                         uint32_t* partials) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  const uint32_t tid = threadIdx.x, lane = tid & 63u;
  if (NORM) {  // k is a multiple of 4, x and the weight 16-byte aligned (checked on the host)
    __shared__ float red[kWaves];
    const uint32_t n4 = k / 4;
    const float4* x4 = reinterpret_cast<const float4*>(x);
    const float4* w4 = reinterpret_cast<const float4*>(norm_w);
    float ss = 0.f;
    for (uint32_t i = tid; i < n4; i += blockDim.x) {
      const float4 v = x4[i];
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if (lane == 0) red[tid >> 6] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) total += red[w];
    const float inv = 1.0f / sqrtf(total / (float)k + eps);
    for (uint32_t i = tid; i < n4; i += blockDim.x) {
      const float4 v = x4[i], g = w4[i];
      reinterpret_cast<float4*>(xs)[i] = make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w);
    }
  } else {
    for (uint32_t i = tid; i < k; i += blockDim.x) xs[i] = x[i];
  }
  __syncthreads();
  constexpr uint32_t kEpv = 128u / BITS;  // elements per 16-byte vector
  constexpr int kBatch = 2;               // vectors per lane and row issued before any is used
  const uint32_t wave = blockIdx.x * kWaves + (tid >> 6), waves = gridDim.x * kWaves;
  float best_v = -1.0e30f;
  uint32_t best_i = out_offset;
  for (uint32_t r0 = wave; r0 < n; r0 += 2 * waves) {
    const uint32_t rows[2] = {r0, r0 + waves};
    float acc[2] = {0.f, 0.f};
    if (VEC) {
      const uint32_t vecs = k / kEpv;
      for (uint32_t v0 = lane; v0 < vecs; v0 += 64u * kBatch) {
        uint4 w[2][kBatch];
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
          for (int b = 0; b < kBatch; b++) {
            const uint32_t v = v0 + 64u * b;
            w[r][b] = rows[r] < n && v < vecs ? reinterpret_cast<const uint4*>(table)[(size_t)rows[r] * vecs + v]
                                              : make_uint4(0u, 0u, 0u, 0u);
          }
#pragma unroll
        for (int r = 0; r < 2; r++)
#pragma unroll
          for (int b = 0; b < kBatch; b++) {
            const uint32_t v = v0 + 64u * b;
            if (v < vecs) acc[r] = dense_dot<BITS>(w[r][b], xs + v * kEpv, acc[r]);
          }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 2; r++)
        if (rows[r] < n)
          for (uint32_t i = lane; i < k; i += 64)
            acc[r] = fmaf(egd::table_value(table, nullptr, nullptr, (uint64_t)rows[r] * k + i, 0, 0, BITS), xs[i],
                          acc[r]);
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const float v = egd::team_sum<64>(acc[r]);
      if (lane == 63 && rows[r] < n) {
        if (out) out[rows[r] + out_offset] = v;
        if (ARGMAX && egd::better(v, rows[r] + out_offset, best_v, best_i)) {
          best_v = v;
          best_i = rows[r] + out_offset;
        }
      }
    }
  }
  if (ARGMAX) {
    __shared__ float wv[kWaves];
    __shared__ uint32_t wi[kWaves];
    egd::team_argmax<64>(best_v, best_i);
    if (lane == 0) {
      wv[tid >> 6] = best_v;
      wi[tid >> 6] = best_i;
    }
    __syncthreads();
    if (tid == 0) {
      float bv = wv[0];
      uint32_t bi = wi[0];
      for (int q = 1; q < kWaves; q++)
        if (egd::better(wv[q], wi[q], bv, bi)) {
          bv = wv[q];
          bi = wi[q];
        }
      partials[2 * blockIdx.x] = __float_as_uint(bv);
      partials[2 * blockIdx.x + 1] = bi;
    }
  }
}

// Instantiated (TEAM, CPL, U, NB) shapes: one chunk slot per lane for rows of up to 64 chunks
// (TEAM the next power of two), a full-wave team with 2-4 slots for longer rows. The library
// picks NB = 2 (a deeper pipeline costs resident waves and duplicate tail tiles) except for
// the long walks of choose_shape; the other NB 3-4 variants stay selectable through
// EG_GEMV_SHAPE for tuning.
#define EG_SHAPES(X)                                                                                      \
  X(8, 1, 1, 2) X(8, 1, 2, 2) X(8, 1, 4, 2) X(16, 1, 1, 2) X(16, 1, 2, 2) X(16, 1, 4, 2) X(32, 1, 1, 2)    \
  X(32, 1, 2, 2) X(32, 1, 2, 3) X(32, 1, 2, 4) X(32, 1, 4, 2) X(64, 1, 1, 2) X(64, 1, 2, 2) X(64, 1, 4, 2) \
  X(64, 1, 4, 3) X(64, 2, 1, 2) X(64, 2, 2, 2) X(64, 3, 1, 2) X(64, 3, 1, 3) X(64, 3, 1, 4) X(64, 3, 2, 2) \
  X(64, 4, 1, 2)

template <int BITS, int ENC, int MODE>
KernelFn pick(int team, int cpl, int u, int nb) {
#define EG_CASE(T, P, UU, D) \
  if (team == T && cpl == P && u == UU && nb == D) return gemv_kernel<BITS, ENC, T, P, UU, D, MODE, EG_INPUT_VECTOR>;
  EG_SHAPES(EG_CASE)
#undef EG_CASE
  return nullptr;
}

// kSampleStats (int8 heads): the shapes at pipeline depth 2
template <int ENC>
KernelFn pick_stats(int team, int cpl, int u, int nb) {
#define EG_CASE(T, P, UU, D)                                 \
  if constexpr (D == 2)                                      \
    if (team == T && cpl == P && u == UU && nb == D)         \
      return gemv_kernel<8, ENC, T, P, UU, D, kSampleStats, EG_INPUT_VECTOR>;
  EG_SHAPES(EG_CASE)
#undef EG_CASE
  return nullptr;
}

template <int BITS, int ENC>
KernelFn pick_mode(int mode, int team, int cpl, int u, int nb) {
  if constexpr (BITS == 8)
    if (mode == kSampleStats) return pick_stats<ENC>(team, cpl, u, nb);
  if (mode == kArgmax) return pick<BITS, ENC, kArgmax>(team, cpl, u, nb);
  if (mode == kArgmaxOnly) return pick<BITS, ENC, kArgmaxOnly>(team, cpl, u, nb);
  if (mode == kBatched) return pick<BITS, ENC, kBatched>(team, cpl, u, nb);
  return pick<BITS, ENC, kPlain>(team, cpl, u, nb);
}

KernelFn pick_kernel(int bits, int enc, int mode, int team, int cpl, int u, int nb, int in_kind = EG_INPUT_VECTOR) {
  if (in_kind != EG_INPUT_VECTOR) return pick_fused(bits, enc, mode, in_kind, team, cpl, u, nb);
  if (bits == 4 && enc == EG_ENC_OFFSET_ZEROS) return pick_mode<4, EG_ENC_OFFSET_ZEROS>(mode, team, cpl, u, nb);
  if (bits == 4 && enc == EG_ENC_SIGNED) return pick_mode<4, EG_ENC_SIGNED>(mode, team, cpl, u, nb);
  if (bits == 8 && enc == EG_ENC_OFFSET_ZEROS) return pick_mode<8, EG_ENC_OFFSET_ZEROS>(mode, team, cpl, u, nb);
  return pick_mode<8, EG_ENC_SIGNED>(mode, team, cpl, u, nb);
}

struct Shape {
  int team = 0, cpl = 0, u = 0, nb = 2;
  uint32_t tiles = 0;
};

// One tile per wave while the matrix is small; otherwise exactly the workgroups the device
// holds at once (occupancy x CUs), each wave then walking its own contiguous range of tiles.
// Sizing to residency matters because the ranges are equal: a second, late-starting round of
// workgroups would double the tail.
// A fused input stage is recomputed by every workgroup; those launches give each wave
// `tiles_per_wave` tiles (the context's setting, 1 by default: measured, the decoder's launches
// finish sooner with more workgroups than with fewer that amortise the stage).
uint32_t grid_for(eg_context* ctx, KernelFn fn, uint32_t tiles, uint32_t smem_bytes, uint32_t tiles_per_wave = 1) {
  int occ = eg::occupancy_of(ctx, reinterpret_cast<const void*>(fn), smem_bytes);
  if (occ <= 0) occ = 2;
  const uint64_t per_block = (uint64_t)kWaves * (tiles_per_wave ? tiles_per_wave : 1);
  uint64_t blocks = ((uint64_t)tiles + per_block - 1) / per_block;
  const uint64_t cap = (uint64_t)ctx->cu_count * (uint64_t)occ;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (uint32_t)blocks;
}

// One chunk slot per lane while rows have <= 64 chunks (x costs 32 VGPRs), two rows per lane
// per tile (four for full-wave teams); longer rows take the full wave and 2-4 slots, with
// fewer rows per tile to stay within ~128 VGPRs. `row_multiple` (batched plans) is the row count every segment divides.
Shape choose_shape(uint32_t n, uint32_t chunks, const eg_context* ctx, uint32_t row_multiple = 0) {
  Shape sh;
  if (chunks == 0 || chunks > 256) return sh;
  if (chunks <= 64) {
    sh.team = 8;
    while ((uint32_t)sh.team < chunks) sh.team *= 2;
    sh.cpl = 1;
    // measured on MI355X: int8 rows of 56 chunks / int4 rows of 28 stream best with 4 / 2 rows
    // per lane; a matrix whose one-row-per-lane tiles all fit in about one resident wave of the
    // device (the decoder's per-layer projections) is faster with one - each wave's chain of
    // dependent steps is then a single tile
    const uint32_t rpw = 64u / sh.team;
    const uint32_t cus = ctx ? (uint32_t)ctx->cu_count : 256u;
    sh.u = sh.team == 64 ? 4 : (n + rpw - 1) / rpw <= 16u * cus ? 1 : 2;
  } else {
    sh.team = 64;
    sh.cpl = (int)((chunks + 63) / 64);
    sh.u = sh.cpl == 2 ? 2 : 1;
  }
  if (ctx && ctx->gemv_override[0]) {
    sh.team = ctx->gemv_override[0];
    sh.cpl = ctx->gemv_override[1];
    sh.u = ctx->gemv_override[2];
    sh.nb = ctx->gemv_override[3];
    if ((uint32_t)(sh.team * sh.cpl) < chunks) return Shape{};
  }
  const uint32_t rpw = 64u / sh.team;
  if (row_multiple)
    while (sh.u > 1 && row_multiple % (rpw * sh.u) != 0) sh.u /= 2;
  if (row_multiple && row_multiple % (rpw * sh.u) != 0) return Shape{};
  // A plain launch shifts its last partial tile back inside the matrix, so a tile may not
  // have more rows than the matrix.
  while (sh.u > 1 && rpw * sh.u > n) sh.u /= 2;
  if (rpw * sh.u > n) return Shape{};
  const uint32_t tile_rows = rpw * sh.u;
  sh.tiles = (n + tile_rows - 1) / tile_rows;
  // Over many tiles per wave, three-slot rows (K = 4864 int4: 152 chunks) and two-row 32-lane
  // tiles (K = 896 int4) stream best with three load buffers (measured, interleaved: the
  // 24-matrix K = 4864 launch 13.9 us against 15.1 with two and 14.2 with four; the K = 896 one
  // 26.8 against 27.5 with two); launches with a fused input stage always take two.
  const bool long_walk = sh.tiles > 16u * (ctx ? (uint32_t)ctx->cu_count : 256u);
  if (!(ctx && ctx->gemv_override[0]) && long_walk &&
      ((sh.cpl == 3 && sh.u == 1) || (sh.team == 32 && sh.cpl == 1 && sh.u == 2)))
    sh.nb = 3;
  return sh;
}

struct QuantView {
  const char* op;
  const float* x;
  const uint32_t* packed;
  const float* scales;
  const uint32_t* zeros;
  const float* bias;
  float* out;
  uint32_t n, k, block_size, blocks_per_row, out_offset;
  int encoding, bits;
  uint32_t* result;  // non-null for the fused argmax
  const eg_gemv_input* input = nullptr;  // fused input stage; NULL: x as given
  uint32_t* groups_out = nullptr;  // fused argmax: skip the finalize, report the partials' count here
  uint32_t* partials = nullptr;    // fused argmax: where the partials go (NULL: the context workspace)
  size_t partials_bytes = 0;       // its size
  // the sampling statistics (kSampleStats, with `result` and `groups_out`): the parameters from
  // device memory (sample_dev) or as given (sample_host), and the history the penalty reads
  const eg_sample_dims* sample_dev = nullptr;
  const eg_sample_dims* sample_host = nullptr;
  const uint32_t* history = nullptr;
  uint32_t* clear = nullptr;  // zeroed by workgroup 0 (clear_words words)
  uint32_t clear_words = 0;
  bool table = false;  // an LM head: f16 (bits 16) and f32 (bits 32) tables are taken too
};

// LDS the input stage needs beyond x and the segment table.
uint32_t input_scratch_bytes(const GemvArgs& a) {
  return a.in_kind == EG_INPUT_ATTENTION ? a.att_heads * a.att_chunks * 4u : 0u;
}

// Validates an input stage against the GEMV's K and copies it into the kernel arguments.
int apply_input(eg_context* ctx, const char* op, const eg_gemv_input* in, uint32_t k, GemvArgs& a) {
  a.in_kind = EG_INPUT_VECTOR;
  if (!in) return EG_OK;
  a.in_kind = in->kind;
  a.x = in->x;
  a.x2 = in->x2;
  a.eps = in->eps;
  if (!in->x) return eg::fail(ctx, EG_ERR_INVALID, "%s: input x is NULL", op);
  switch (in->kind) {
    case EG_INPUT_VECTOR:
      if (reinterpret_cast<uintptr_t>(in->x) & 15u)
        return eg::fail(ctx, EG_ERR_INVALID, "%s: x is not 16-byte aligned", op);
      return EG_OK;
    case EG_INPUT_RMSNORM:
    case EG_INPUT_SILU_MUL:
      if (!in->x2) return eg::fail(ctx, EG_ERR_INVALID, "%s: the input stage needs x2", op);
      if (in->kind == EG_INPUT_RMSNORM && !(in->eps >= 0.f))
        return eg::fail(ctx, EG_ERR_INVALID, "%s: eps must be >= 0", op);
      return EG_OK;
    case EG_INPUT_ATTENTION: {
      const eg_attention_dims& d = in->attention;
      if (d.kv_heads == 0 || d.heads % d.kv_heads != 0 || d.chunk == 0 || d.max_context % d.chunk != 0)
        return eg::fail(ctx, EG_ERR_INVALID, "%s: bad attention layout", op);
      if (d.heads * d.head_dim != k)
        return eg::fail(ctx, EG_ERR_INVALID, "%s: attention output %u x %u does not match k = %u", op, d.heads,
                        d.head_dim, k);
      if ((uint64_t)d.heads * egd::combine_group(d.max_context / d.chunk) > kMaxCombine ||
          d.max_context / d.chunk > egd::kMaxChunks)
        return eg::fail(ctx, EG_ERR_RANGE, "%s: %u heads x %u chunks exceed the combine stage's %u (at most %u chunks)",
                        op, d.heads, d.max_context / d.chunk, kMaxCombine, egd::kMaxChunks);
      a.att_heads = d.heads;
      a.att_kv_heads = d.kv_heads;
      a.att_head_dim = d.head_dim;
      a.att_chunks = d.max_context / d.chunk;
      return EG_OK;
    }
    default:
      return eg::fail(ctx, EG_ERR_INVALID, "%s: unknown input kind %d", op, in->kind);
  }
}

int validate(eg_context* ctx, const QuantView& v) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", v.op);
  if (v.bits != 4 && v.bits != 8) return eg::fail(ctx, EG_ERR_INVALID, "%s: bits must be 4 or 8, got %d", v.op, v.bits);
  if (v.encoding != EG_ENC_OFFSET_ZEROS && v.encoding != EG_ENC_SIGNED)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: unknown encoding %d", v.op, v.encoding);
  if (!v.x || !v.packed || !v.scales) return eg::fail(ctx, EG_ERR_INVALID, "%s: x, packed and scales are required", v.op);
  if (v.encoding == EG_ENC_OFFSET_ZEROS && !v.zeros)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: the offset encoding needs a zero-point stream", v.op);
  if (!v.out && !v.result) return eg::fail(ctx, EG_ERR_INVALID, "%s: out is NULL", v.op);
  if (v.block_size == 0 || v.k % v.block_size != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: reduction axis %u is not a multiple of %u", v.op, v.k, v.block_size);
  if (v.blocks_per_row != v.k / v.block_size)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: blocksPerRow %u does not equal k / blockSize = %u", v.op,
                    v.blocks_per_row, v.k / v.block_size);
  const uint64_t elements = (uint64_t)v.n * v.k;
  if (elements % (32 / v.bits) != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: %llu codes do not fill whole 32-bit words", v.op,
                    (unsigned long long)elements);
  // Streams are addressed with 32-bit byte offsets.
  if (elements * (uint64_t)v.bits / 8 >= (1ull << 32) || (uint64_t)v.n * v.blocks_per_row * 4 >= (1ull << 32) ||
      ((uint64_t)v.out_offset + v.n) * 4 >= (1ull << 32))
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u x %u exceeds the 4 GiB stream range", v.op, v.n, v.k);
  return EG_OK;
}

// An LM head over an f16 or f32 table (dense_head_kernel).
int launch_dense(eg_context* ctx, const QuantView& v) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", v.op);
  if (!v.x || !v.packed) return eg::fail(ctx, EG_ERR_INVALID, "%s: x and the table are required", v.op);
  if (!v.out && !v.result) return eg::fail(ctx, EG_ERR_INVALID, "%s: out is NULL", v.op);
  if (v.sample_dev || v.sample_host)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: the sampling statistics need an int8 head", v.op);
  const bool norm = v.input && v.input->kind == EG_INPUT_RMSNORM;
  if (v.input && v.input->kind != EG_INPUT_VECTOR && !norm)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: an f16 / f32 head takes x as given or after an RMSNorm", v.op);
  if (v.k > kDenseMaxK)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: hidden %u over the %u an f16 / f32 head holds", v.op, v.k, kDenseMaxK);
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  if (norm && (!v.input->x2 || v.k % 4 != 0 || !aligned(v.x) || !aligned(v.input->x2)))
    return eg::fail(ctx, EG_ERR_INVALID,
                    "%s: the fused RMSNorm needs its weight, hidden a multiple of 4 and 16-byte aligned vectors", v.op);
  if (((uint64_t)v.out_offset + v.n) * 4 >= (1ull << 32))
    return eg::fail(ctx, EG_ERR_RANGE, "%s: rows up to %llu exceed the output range", v.op,
                    (unsigned long long)v.out_offset + v.n);
  if (v.n == 0) return v.result ? eg::fail(ctx, EG_ERR_INVALID, "%s: argmax over zero rows", v.op) : EG_OK;
  const bool argmax = v.result != nullptr;
  const bool vec = aligned(v.packed) && ((uint64_t)v.k * v.bits) % 128 == 0;
  uint64_t blocks = ((uint64_t)v.n + 2 * kWaves - 1) / (2 * kWaves);
  blocks = std::min<uint64_t>(blocks, (uint64_t)ctx->cu_count * 8);
  uint32_t* partials = v.partials ? v.partials : reinterpret_cast<uint32_t*>(eg::partials(ctx));
  const size_t partials_cap = v.partials ? v.partials_bytes : eg::kPartialsBytes;
  if (argmax && blocks * 8 > partials_cap)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %llu workgroups' partials exceed the %zu-byte buffer", v.op,
                    (unsigned long long)blocks, partials_cap);
  using Fn = void (*)(const float*, const float*, float, const uint32_t*, float*, uint32_t, uint32_t, uint32_t,
                      uint32_t*);
#define EG_DENSE(B, A, N) (vec ? (Fn)dense_head_kernel<B, A, N, true> : (Fn)dense_head_kernel<B, A, N, false>)
#define EG_DENSE_B(B) (argmax ? (norm ? EG_DENSE(B, true, true) : EG_DENSE(B, true, false)) \
                              : (norm ? EG_DENSE(B, false, true) : EG_DENSE(B, false, false)))
  const Fn fn = v.bits == 16 ? EG_DENSE_B(16) : EG_DENSE_B(32);
#undef EG_DENSE_B
#undef EG_DENSE
  hipLaunchKernelGGL(fn, dim3((unsigned)blocks), dim3(256), std::max<uint32_t>(v.k, 4) * 4u, ctx->stream, v.x,
                     norm ? v.input->x2 : nullptr, norm ? v.input->eps : 0.f, v.packed, v.out, v.n, v.k,
                     v.out_offset, partials);
  if (argmax && v.groups_out) *v.groups_out = (uint32_t)blocks;
  else if (argmax) eg::launch_argmax_finalize(ctx, partials, (uint32_t)blocks, v.out_offset, v.result);
  return eg::check_launch(ctx, v.op);
}

int launch(eg_context* ctx, const QuantView& v) {
  if (v.bits == 16 || v.bits == 32) {
    if (v.table) return launch_dense(ctx, v);
    return eg::fail(ctx, EG_ERR_INVALID, "%s: bits must be 4 or 8, got %d", v.op, v.bits);
  }
  int st = validate(ctx, v);
  if (st != EG_OK) return st;
  if (v.n == 0) {
    if (v.result || v.sample_dev || v.sample_host) return eg::fail(ctx, EG_ERR_INVALID, "%s: argmax over zero rows", v.op);
    return EG_OK;
  }
  const bool stats = v.sample_dev || v.sample_host;
  const bool argmax = v.result != nullptr || stats;
  const uint32_t epc = 128u / v.bits;
  const bool fused = v.input && v.input->kind != EG_INPUT_VECTOR;
  const bool aligned = (reinterpret_cast<uintptr_t>(v.packed) & 15u) == 0 &&
                       (fused || (reinterpret_cast<uintptr_t>(v.x) & 15u) == 0);
  const uint32_t chunks = v.k / epc;
  Shape shape;
  if (aligned && v.k % epc == 0 && v.block_size % epc == 0)
    shape = choose_shape(v.n, chunks, ctx);
  uint32_t* partials = v.partials ? v.partials : reinterpret_cast<uint32_t*>(eg::partials(ctx));
  const size_t partials_cap = v.partials ? v.partials_bytes : eg::kPartialsBytes;
  // one (value bits, index) partial per workgroup - (value, index, float64 sum) for the sampling
  // statistics - checked before anything is launched
  auto partials_fit = [&](uint64_t groups) {
    return !argmax || groups * (stats ? 16 : 8) <= partials_cap ? EG_OK
                                                 : eg::fail(ctx, EG_ERR_RANGE,
                                                            "%s: %llu workgroups' partials exceed the %zu-byte buffer",
                                                            v.op, (unsigned long long)groups, partials_cap);
  };
  uint32_t grid = 0;
  const int mode = stats ? kSampleStats : argmax ? (v.out ? kArgmax : kArgmaxOnly) : kPlain;
  const int in_kind = v.input ? v.input->kind : EG_INPUT_VECTOR;
  KernelFn fn = shape.team ? pick_kernel(v.bits, v.encoding, mode, shape.team, shape.cpl, shape.u,
                                         in_kind != EG_INPUT_VECTOR || stats ? 2 : shape.nb, in_kind)
                           : nullptr;
  if (fused && !fn)
    return eg::fail(ctx, EG_ERR_INVALID,
                    "%s: no kernel for this shape with a fused input stage (k and the block must be multiples of %u)",
                    v.op, epc);
  if (stats && (!fn || !v.out || !v.groups_out))
    return eg::fail(ctx, EG_ERR_INVALID,
                    "%s: the sampling statistics need an int8 head whose k and block are multiples of %u", v.op,
                    epc);
  if (fn) {
    GemvArgs a{};
    a.x = v.x;
    st = apply_input(ctx, v.op, v.input, v.k, a);
    if (st != EG_OK) return st;
    a.w = reinterpret_cast<const uint4*>(v.packed);
    a.scales = v.scales;
    a.zeros = v.zeros;
    a.bias = v.bias;
    a.out = v.out;
    a.n = v.n;
    a.chunks = chunks;
    a.chunks_per_block = v.block_size / epc;
    a.blocks_per_row = v.blocks_per_row;
    a.out_offset = v.out_offset;
    a.partials = partials;
    a.segs = nullptr;
    a.seg_count = 0;
    a.total_passes = shape.tiles;
    a.any_bias = v.bias != nullptr;
    const uint32_t smem = chunks * epc * 4u + input_scratch_bytes(a) + (stats ? kStatsLdsBytes : 0u);
    grid = grid_for(ctx, fn, shape.tiles, smem, a.in_kind != EG_INPUT_VECTOR ? ctx->fused_tiles_per_wave : 1);
    if (stats) {
      // every workgroup's nominal rows within the kernel's per-workgroup record (kStatsRows; a
      // tile to spare)
      const uint32_t tile_rows = (64u / shape.team) * shape.u;
      const uint32_t tiles_per_group = (kStatsRows - tile_rows) / tile_rows;
      grid = std::max<uint32_t>(grid, (shape.tiles + tiles_per_group - 1) / tiles_per_group);
      a.stats.sample_dev = v.sample_dev;
      if (v.sample_host) {
        a.stats.temperature = v.sample_host->temperature;
        a.stats.repetition_penalty = v.sample_host->repetition_penalty;
        a.stats.history_length = v.sample_host->history_length;
      }
      a.stats.history = v.history;
      a.stats.clear = v.clear;
      a.stats.clear_words = v.clear ? v.clear_words : 0u;
    }
    if ((st = partials_fit(grid)) != EG_OK) return st;
    a.stamp = eg::stamp_slot(ctx);
    hipLaunchKernelGGL(fn, dim3(grid), dim3(256), smem, ctx->stream, a);
  } else {
    uint64_t blocks = (v.n + kWaves - 1) / kWaves;
    const uint64_t cap = (uint64_t)ctx->cu_count * 8;
    if (blocks > cap) blocks = cap;
    grid = (uint32_t)blocks;
    if ((st = partials_fit(grid)) != EG_OK) return st;
    if (argmax)
      hipLaunchKernelGGL(gemv_generic_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, v.x,
                         v.packed, v.scales, v.zeros, v.bias, v.out, v.n, v.k, v.block_size, v.blocks_per_row,
                         v.out_offset, v.bits, v.encoding, partials);
    else
      hipLaunchKernelGGL(gemv_generic_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, v.x,
                         v.packed, v.scales, v.zeros, v.bias, v.out, v.n, v.k, v.block_size, v.blocks_per_row,
                         v.out_offset, v.bits, v.encoding, partials);
  }
  if (argmax && v.groups_out) *v.groups_out = grid;
  else if (argmax) eg::launch_argmax_finalize(ctx, partials, grid, v.out_offset, v.result);
  return eg::check_launch(ctx, v.op);
}

}  // namespace

// ---- the fixed scratch of eg_lm_head_argmax_noalloc ----------------------------------------
// A file-scope device array: every GPU the library runs on holds its own copy, at its own
// address, until the process ends. In host code `scratch` names the symbol, not device memory,
// so it is never passed to a kernel: eg::noalloc_scratch_init resolves this device's copy with
// hipGetSymbolAddress once per device (at eg_create, with the device current) and the entry
// point hands kernels that address. 64 KiB = 8192 (value bits, index) partials, four times the
// largest grid the LM head launches (256 CUs x 8 resident workgroups).
constexpr size_t kNoAllocScratchBytes = 64u << 10;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_lock;
std::unordered_map<int, void*> g_scratch_address;  // device -> its copy of `scratch`
}  // namespace

int eg::noalloc_scratch_init(eg_context* ctx) {
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  auto it = g_scratch_address.find(ctx->device);
  if (it == g_scratch_address.end()) {
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr) {
      ctx->noalloc_scratch = nullptr;
      return eg::hip_fail(ctx, err != hipSuccess ? err : hipErrorInvalidSymbol, "eg_create: hipGetSymbolAddress(scratch)");
    }
    it = g_scratch_address.emplace(ctx->device, ptr).first;
  }
  ctx->noalloc_scratch = it->second;
  return EG_OK;
}

extern "C" {

int eg_matmul_q4_decode(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                        const uint32_t* zeros, const float* bias, float* out, const eg_matmul_q4_dims* dims,
                        int encoding, int bits) {
  if (!dims) return eg::fail(ctx, EG_ERR_INVALID, "matmul_q4_decode: dims is NULL");
  if (dims->use_bias && !bias) return eg::fail(ctx, EG_ERR_INVALID, "matmul_q4_decode: useBias set but bias is NULL");
  QuantView v{"matmul_q4_decode", x, packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros,
              dims->use_bias ? bias : nullptr, out, dims->n, dims->k, dims->block_size, dims->blocks_per_row,
              dims->out_offset, encoding, bits, nullptr};
  if (!out) return eg::fail(ctx, EG_ERR_INVALID, "matmul_q4_decode: out is NULL");
  return launch(ctx, v);
}

int eg_lm_head(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales, const uint32_t* zeros,
               float* out, const eg_embedding_dims* dims, int encoding, int bits) {
  if (!dims) return eg::fail(ctx, EG_ERR_INVALID, "lm_head: dims is NULL");
  if (!out) return eg::fail(ctx, EG_ERR_INVALID, "lm_head: out is NULL");
  QuantView v{bits == 4 ? "lm_head_q4" : "lm_head_q8", x, packed, scales,
              encoding == EG_ENC_SIGNED ? nullptr : zeros, nullptr, out, dims->row_count, dims->hidden,
              dims->block_size, dims->blocks_per_row, dims->out_offset, encoding, bits, nullptr};
  v.table = true;
  return launch(ctx, v);
}

int eg_lm_head_argmax(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                      const uint32_t* zeros, float* out, uint32_t* result, const eg_embedding_dims* dims,
                      int encoding, int bits) {
  if (!dims) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_argmax: dims is NULL");
  if (!result) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_argmax: result is NULL");
  QuantView v{"lm_head_argmax", x, packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros, nullptr, out,
              dims->row_count, dims->hidden, dims->block_size, dims->blocks_per_row, dims->out_offset, encoding,
              bits, result};
  v.table = true;
  if (ctx) {
    const uint64_t max_groups = eg::kPartialsBytes / 8;
    if ((uint64_t)ctx->cu_count * 8 > max_groups)
      return eg::fail(ctx, EG_ERR_RANGE, "lm_head_argmax: workspace too small for the grid");
  }
  return launch(ctx, v);
}

int eg_lm_head_argmax_noalloc(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                              const uint32_t* zeros, float* out, uint32_t* result, const eg_embedding_dims* dims,
                              int encoding, int bits) {
  const char* op = "lm_head_argmax_noalloc";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!dims) return eg::fail(ctx, EG_ERR_INVALID, "%s: dims is NULL", op);
  if (!result) return eg::fail(ctx, EG_ERR_INVALID, "%s: result is NULL", op);
  if (!ctx->noalloc_scratch) return eg::fail(ctx, EG_ERR_STATE, "%s: the device's scratch address is unknown", op);
  QuantView v{op, x, packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros, nullptr, out, dims->row_count,
              dims->hidden, dims->block_size, dims->blocks_per_row, dims->out_offset, encoding, bits, result};
  v.partials = static_cast<uint32_t*>(ctx->noalloc_scratch);
  v.partials_bytes = kNoAllocScratchBytes;
  v.table = true;
  return launch(ctx, v);
}

int eg_lm_head_argmax_input(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed,
                            const float* scales, const uint32_t* zeros, float* out, uint32_t* result,
                            const eg_embedding_dims* dims, int encoding, int bits) {
  if (!dims) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_argmax: dims is NULL");
  if (!result) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_argmax: result is NULL");
  if (!input) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_argmax: input is NULL");
  QuantView v{"lm_head_argmax", input->x, packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros, nullptr, out,
              dims->row_count, dims->hidden, dims->block_size, dims->blocks_per_row, dims->out_offset, encoding,
              bits, result, input};
  v.table = true;
  return launch(ctx, v);
}

}  // extern "C"

int eg::lm_head_argmax_partials(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed,
                                const float* scales, const uint32_t* zeros, float* out, const eg_embedding_dims* dims,
                                int encoding, int bits, uint32_t* groups) {
  if (!dims || !input || !groups) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_argmax: NULL argument");
  uint32_t* partials = ctx ? reinterpret_cast<uint32_t*>(eg::partials(ctx)) : nullptr;
  QuantView v{"lm_head_argmax", input->x, packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros, nullptr, out,
              dims->row_count, dims->hidden, dims->block_size, dims->blocks_per_row, dims->out_offset, encoding,
              bits, partials, input, groups};
  v.table = true;
  return launch(ctx, v);
}

int eg::lm_head_sample_partials(eg_context* ctx, const eg_gemv_input* input, const uint32_t* packed,
                                const float* scales, const uint32_t* zeros, float* out, const eg_embedding_dims* dims,
                                int encoding, int bits, const eg_sample_dims* sample_dev,
                                const eg_sample_dims* sample_host, const uint32_t* history, uint32_t* partials,
                                size_t partials_bytes, uint32_t* clear, uint32_t clear_words, uint32_t* groups) {
  if (!dims || !input || !groups || !out || (!sample_dev && !sample_host))
    return eg::fail(ctx, EG_ERR_INVALID, "lm_head_sample: NULL argument");
  if (bits != 8) return eg::fail(ctx, EG_ERR_INVALID, "lm_head_sample: an int8 head (bits 8), not %d", bits);
  QuantView v{"lm_head_sample", input->x, packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros, nullptr, out,
              dims->row_count, dims->hidden, dims->block_size, dims->blocks_per_row, dims->out_offset, encoding,
              bits, nullptr, input, groups, partials, partials ? partials_bytes : 0};
  v.sample_dev = sample_dev;
  v.sample_host = sample_host;
  v.history = history;
  v.clear = clear;
  v.clear_words = clear_words;
  return launch(ctx, v);
}

// ---- batched plans ------------------------------------------------------------------------

struct eg_gemv_plan {
  // Device copy of the table, followed (plans of more than kInlineSegments matrices) by the
  // segment of every pass, 16 bits each: a wave finds its first segment in two scalar loads,
  // whatever the launch's grid.
  DevSegment* table = nullptr;
  const uint32_t* seg_index = nullptr;
  DevSegment inline_table[kInlineSegments] = {};  // host copy, passed in the arguments when count <= kInlineSegments
  uint32_t any_bias = 0;                           // some segment has a bias
  uint32_t count = 0;
  uint32_t swiglu_rows = 0;  // a SwiGLU pair (eg_gemv_swiglu_plan_create): the rows of each matrix
  uint32_t k = 0, block_size = 0, chunks = 0, total_passes = 0, grid = 0, smem = 0;
  int encoding = 0, bits = 0, team = 0, cpl = 0, u = 0, nb = 2;
};

extern "C" {

int eg_gemv_plan_create(eg_context* ctx, uint32_t k, uint32_t block_size, int encoding, int bits,
                        const eg_gemv_segment* segments, uint32_t count, eg_gemv_plan** out_plan) {
  const char* op = "gemv_plan";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!out_plan || !segments || count == 0) return eg::fail(ctx, EG_ERR_INVALID, "%s: empty segment table", op);
  if (count > kMaxSegments)
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u segments, at most %u per plan", op, count, kMaxSegments);
  *out_plan = nullptr;
  if (bits != 4 && bits != 8) return eg::fail(ctx, EG_ERR_INVALID, "%s: bits must be 4 or 8", op);
  if (encoding != EG_ENC_OFFSET_ZEROS && encoding != EG_ENC_SIGNED)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: unknown encoding %d", op, encoding);
  const uint32_t epc = 128u / bits;
  if (block_size == 0 || k % block_size != 0 || block_size % epc != 0 || k % epc != 0 || k / epc > 256)
    return eg::fail(ctx, EG_ERR_INVALID,
                    "%s: k %u / block %u must be multiples of %u codes with at most %u codes per row", op, k,
                    block_size, epc, 256 * epc);
  uint64_t rows_total = 0;
  for (uint32_t i = 0; i < count; i++) {
    const eg_gemv_segment& g = segments[i];
    if (!g.packed || !g.scales || !g.out || (encoding == EG_ENC_OFFSET_ZEROS && !g.zeros))
      return eg::fail(ctx, EG_ERR_INVALID, "%s: segment %u is missing a stream", op, i);
    if (g.rows == 0 || g.rows % 8 != 0)
      return eg::fail(ctx, EG_ERR_INVALID, "%s: segment %u has %u rows, not a positive multiple of 8", op, i, g.rows);
    if ((reinterpret_cast<uintptr_t>(g.packed) & 15u) != 0)
      return eg::fail(ctx, EG_ERR_INVALID, "%s: segment %u codes are not 16-byte aligned", op, i);
    if ((uint64_t)g.rows * (k / block_size) * 4 >= (1ull << 32) || (uint64_t)g.rows * k * bits / 8 >= (1ull << 32) ||
        ((uint64_t)g.out_offset + g.rows) * 4 >= (1ull << 32))
      return eg::fail(ctx, EG_ERR_RANGE, "%s: segment %u exceeds the 4 GiB stream range", op, i);
    rows_total += g.rows;
  }
  const uint32_t chunks = k / epc;
  uint32_t row_gcd = 0;
  for (uint32_t i = 0; i < count; i++) row_gcd = std::gcd(row_gcd, segments[i].rows);
  Shape shape = choose_shape((uint32_t)std::min<uint64_t>(rows_total, 0xFFFFFFFFu), chunks, ctx, row_gcd);
  if (shape.team == 0) return eg::fail(ctx, EG_ERR_INVALID, "%s: no kernel shape for k %u and these row counts", op, k);
  const uint32_t tile_rows = (64u / shape.team) * shape.u;
  DevSegment* host = new DevSegment[count];
  uint32_t pass = 0;
  for (uint32_t i = 0; i < count; i++) {
    const eg_gemv_segment& g = segments[i];
    pass += g.rows / tile_rows;
    host[i] = DevSegment{reinterpret_cast<const uint4*>(g.packed), g.scales,
                         encoding == EG_ENC_SIGNED ? nullptr : g.zeros, g.bias, g.out, pass, g.rows, g.out_offset, {0, 0, 0}};
  }
  eg_gemv_plan* plan = new eg_gemv_plan();
  for (uint32_t i = 0; i < count && i < kInlineSegments; i++) plan->inline_table[i] = host[i];
  for (uint32_t i = 0; i < count; i++) plan->any_bias |= segments[i].bias != nullptr;
  // table, then the pass index (count < 2^16: kMaxSegments)
  static_assert(kMaxSegments <= 0x10000u, "segment numbers are stored in 16 bits");
  std::vector<uint8_t> blob(sizeof(DevSegment) * count);
  std::memcpy(blob.data(), host, blob.size());
  if (count > kInlineSegments) {
    std::vector<uint16_t> index((pass + 1u) & ~1u, (uint16_t)(count - 1));
    for (uint32_t i = 0, p = 0; i < count; i++)
      for (; p < host[i].pass_end; p++) index[p] = (uint16_t)i;
    const size_t at = blob.size();
    blob.resize(at + index.size() * sizeof(uint16_t));
    std::memcpy(blob.data() + at, index.data(), index.size() * sizeof(uint16_t));
  }
  hipError_t err = hipMalloc(&plan->table, blob.size());
  if (err == hipSuccess) err = hipMemcpy(plan->table, blob.data(), blob.size(), hipMemcpyHostToDevice);
  if (err != hipSuccess) {
    delete[] host;
    if (plan->table) (void)hipFree(plan->table);
    delete plan;
    return eg::hip_fail(ctx, err, "gemv_plan_create");
  }
  if (count > kInlineSegments) plan->seg_index = reinterpret_cast<const uint32_t*>(plan->table + count);
  plan->count = count;
  plan->k = k;
  plan->block_size = block_size;
  plan->chunks = chunks;
  plan->total_passes = pass;
  plan->encoding = encoding;
  plan->bits = bits;
  plan->team = shape.team;
  plan->cpl = shape.cpl;
  plan->u = shape.u;
  plan->nb = shape.nb;
  KernelFn fn = pick_kernel(bits, encoding, kBatched, shape.team, shape.cpl, shape.u, shape.nb);
  plan->smem = k * 4u;
  plan->grid = fn ? grid_for(ctx, fn, pass, plan->smem) : 0;
  delete[] host;
  *out_plan = plan;
  return EG_OK;
}

int eg_gemv_swiglu_plan_create(eg_context* ctx, uint32_t k, uint32_t block_size, int encoding, int bits,
                               const eg_gemv_segment* pair, eg_gemv_plan** out_plan) {
  const char* op = "gemv_swiglu_plan";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!out_plan || !pair) return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  *out_plan = nullptr;
  if (bits != 4) return eg::fail(ctx, EG_ERR_INVALID, "%s: int4 weights only, got %d bits", op, bits);
  const eg_gemv_segment &g = pair[0], &u = pair[1];
  if (g.rows != u.rows) return eg::fail(ctx, EG_ERR_INVALID, "%s: gate has %u rows, up %u", op, g.rows, u.rows);
  if (g.bias || u.bias) return eg::fail(ctx, EG_ERR_INVALID, "%s: the pair takes no biases", op);
  // the streams, alignment and ranges of each matrix, as a two-matrix plan checks them (the
  // pair stores through the gate's output only)
  eg_gemv_segment both[2] = {g, u};
  both[1].out = g.out;
  both[1].out_offset = g.out_offset;
  eg_gemv_plan* plan = nullptr;
  int st = eg_gemv_plan_create(ctx, k, block_size, encoding, bits, both, 2, &plan);
  if (st != EG_OK) return st;
  // one team per row of each matrix: two rows (gate r, up r) per lane pair of slots
  int u2 = 2;
  const uint32_t rpw = 64u / plan->team;
  if (plan->cpl > 2 || g.rows % rpw != 0) u2 = 0;
  if (!u2 || !pick_kernel(bits, encoding, kSwiGLU, plan->team, plan->cpl, u2, 2, EG_INPUT_RMSNORM)) {
    eg_gemv_plan_destroy(ctx, plan);
    return eg::fail(ctx, EG_ERR_INVALID, "%s: no SwiGLU kernel for k %u and %u rows", op, k, g.rows);
  }
  plan->u = u2;
  plan->swiglu_rows = g.rows;
  plan->total_passes = g.rows / rpw;
  plan->grid = 0;  // a pair always has its input stage: the grid is sized at launch
  *out_plan = plan;
  return EG_OK;
}

int eg_gemv_plan_launch(eg_context* ctx, const eg_gemv_plan* plan, const float* x) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "gemv_plan_launch: ctx is NULL");
  eg_gemv_input in{};
  in.kind = EG_INPUT_VECTOR;
  in.x = x;
  return eg_gemv_plan_launch_input(ctx, plan, &in);
}

int eg_gemv_plan_launch_input(eg_context* ctx, const eg_gemv_plan* plan, const eg_gemv_input* input) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "gemv_plan_launch: ctx is NULL");
  if (!plan || !input || !input->x) return eg::fail(ctx, EG_ERR_INVALID, "gemv_plan_launch: NULL argument");
  GemvArgs a{};
  int st = apply_input(ctx, "gemv_plan_launch", input, plan->k, a);
  if (st != EG_OK) return st;
  a.chunks = plan->chunks;
  a.chunks_per_block = plan->block_size / (128u / plan->bits);
  a.blocks_per_row = plan->k / plan->block_size;
  a.segs = plan->table;
  a.seg_index = plan->seg_index;
  a.seg_count = plan->count;
  if (plan->count <= kInlineSegments)
    for (uint32_t i = 0; i < plan->count; i++) a.inline_segs[i] = plan->inline_table[i];
  a.total_passes = plan->total_passes;
  a.any_bias = plan->any_bias;
  const bool pair = plan->swiglu_rows != 0;
  if (pair && a.in_kind != EG_INPUT_RMSNORM)
    return eg::fail(ctx, EG_ERR_INVALID, "gemv_plan_launch: a SwiGLU pair takes the RMSNORM input stage");
  a.n = plan->swiglu_rows;
  KernelFn fn = pick_kernel(plan->bits, plan->encoding, pair ? kSwiGLU : kBatched, plan->team, plan->cpl, plan->u,
                            a.in_kind != EG_INPUT_VECTOR ? 2 : plan->nb, a.in_kind);
  if (!fn) return eg::fail(ctx, EG_ERR_INVALID, "gemv_plan_launch: no kernel for this plan's shape");
  const uint32_t extra = input_scratch_bytes(a);
  const uint32_t grid = a.in_kind != EG_INPUT_VECTOR
                            ? grid_for(ctx, fn, plan->total_passes, plan->smem + extra, ctx->fused_tiles_per_wave)
                            : plan->grid;
  const uint32_t smem = plan->smem + extra;
  a.stamp = eg::stamp_slot(ctx);
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), smem, ctx->stream, a);
  return eg::check_launch(ctx, "gemv_plan_launch");
}

}  // extern "C"

int eg_gemv::plan_phase(eg_context* ctx, const eg_gemv_plan* plan, const eg_gemv_input* input, GemvArgs* args,
                        PlanPhase* phase) {
  if (!plan || !input || !input->x || !args || !phase)
    return eg::fail(ctx, EG_ERR_INVALID, "gemv_plan_phase: NULL argument");
  GemvArgs a{};
  int st = apply_input(ctx, "gemv_plan_phase", input, plan->k, a);
  if (st != EG_OK) return st;
  a.chunks = plan->chunks;
  a.chunks_per_block = plan->block_size / (128u / plan->bits);
  a.blocks_per_row = plan->k / plan->block_size;
  a.segs = plan->table;
  a.seg_index = plan->seg_index;
  a.seg_count = plan->count;
  if (plan->count <= kInlineSegments)
    for (uint32_t i = 0; i < plan->count; i++) a.inline_segs[i] = plan->inline_table[i];
  a.total_passes = plan->total_passes;
  a.any_bias = plan->any_bias;
  const bool pair = plan->swiglu_rows != 0;
  a.n = plan->swiglu_rows;
  *args = a;
  phase->bits = plan->bits;
  phase->encoding = plan->encoding;
  phase->mode = pair ? kSwiGLU : kBatched;
  phase->in_kind = a.in_kind;
  phase->team = plan->team;
  phase->cpl = plan->cpl;
  phase->u = plan->u;
  phase->nb = a.in_kind != EG_INPUT_VECTOR ? 2 : plan->nb;
  phase->tiles = plan->total_passes;
  phase->smem = plan->smem + input_scratch_bytes(a);
  return EG_OK;
}

extern "C" {

int eg_gemv_plan_destroy(eg_context* ctx, eg_gemv_plan* plan) {
  if (!plan) return EG_OK;
  if (plan->table) {
    hipError_t err = hipFree(plan->table);
    if (err != hipSuccess) {
      delete plan;
      return eg::hip_fail(ctx, err, "gemv_plan_destroy");
    }
  }
  delete plan;
  return EG_OK;
}

}  // extern "C"
