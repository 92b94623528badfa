// matmul_q4_prefill (matmul_q4_prefill.wgsl:77-162) on the matrix cores:
//   out[r*out_stride + col + out_offset] = sum_k x[r,k] * W[col,k] (+ bias[col])
//
// The prefill chunk (M = 128-256 queries) is the one dense contraction on the path. Each
// workgroup owns a 64 x 64 output tile and a slice of K; its 4 waves each own 32 x 32 = 2 x 2
// tiles of v_mfma_f32_16x16x32_bf16. K is staged 64 at a time through LDS:
//   * x (f32) is rounded to bf16 (round-to-nearest-even) on the way into LDS;
//   * W is dequantized while staging, as the reference's prefill kernel does: 16 int4 codes
//     (8 bytes, one scale and zero-point) per thread, dequantized in f32, then bf16 - so the
//     codes cross HBM as int4 and each weight is unpacked once per tile, not once per MFMA
//     that reads it.
// The loop is latency-bound at these sizes (a few MFMAs per staged block), so:
//   * global loads run two blocks ahead of the LDS staging, in three register stages;
//   * K is split over grid.z when the tile grid alone would leave the device idle (the down
//     projection has 4 x 14 tiles at M = 256): each split writes f32 partials into the context's
//     workspace and a second launch sums the splits in index order, plus the bias - the result
//     does not depend on how the work was scheduled.
// Rows are padded by 16 bytes in LDS so the 16 lanes that read one column of A (or B) hit
// different banks. Accumulation is f32 inside the MFMA.
// Layouts the chunked staging cannot take (K or block size not a multiple of 32 codes, a block
// size that is not a power of two, int8 codes, unaligned streams, K not a multiple of 4) stage
// element by element with the reference's indexing.
#include <algorithm>

#include "eg_internal.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;   // M and N tile
constexpr int kBK = 64;     // K staged per iteration
constexpr int kPad = 8;     // bf16 elements of padding per LDS row
constexpr int kLds = kBK + kPad;
constexpr int kStages = 3;  // register stages of the chunked staging pipeline

// One matrix of a launch: its streams, outputs and the end of its range of 64-column tiles along
// grid.x. A multi-matrix launch holds several that share x, M, K, the quant block size and the
// encoding; the usual launch holds one.
struct PrefillMat {
  const uint32_t* packed;
  const float* scales;
  const uint32_t* zeros;
  const float* bias;
  const float* residual;  // nullable: out = acc + bias + residual[r * out_stride + col + out_offset]
  float* out;
  uint32_t n, out_stride, out_offset, tiles_end;
};
constexpr uint32_t kMaxSegs = 3;

struct PrefillArgs {
  const float* x;
  float* partials;  // split-K: [splits][m][n] f32; NULL when grid.z == 1
  uint32_t m, k, block_size, blocks_per_row, k_per_split;
  int bits;
  uint32_t block_shift;  // log2(block_size) (the chunked staging takes power-of-two blocks)
  uint32_t nmats;        // matrices in mats (> 1: no K split)
  const float* norm;     // NORM launches: x is RMS-normalised per row with these weights (no K split)
  float eps;
  // ROPE launches (q | k | v, 64-column tiles = heads): q rows rotated and scaled by 1/8 into
  // q_rope [row][q heads][64], k rows rotated and v rows as they are into the f16 caches at
  // positions rope_pos0 + row ([pos][kv_heads][64]); rope = the cos/sin table [pos][32]
  const double2* rope;
  float* q_rope;
  uint16_t* k_cache;
  uint16_t* v_cache;
  uint32_t rope_pos0, q_heads, kv_heads;
  uint32_t out_bf16;  // PAIR launches: SiLU(g) * u stored as bf16 (the next GEMM's x, bit-for-bit
                      // what its staging would round it to)
  uint32_t xcd_rows;  // grid.y a multiple of 8, grid.z 1: tiles mapped so that each XCD runs whole
                      // row tiles (below)
  PrefillMat mats[kMaxSegs];
};

// The matrix that owns tile column `tx` and the first tile column of its range. The matrix is
// read in place from the kernel arguments (the arguments are never written: a written copy with
// an indexed array member would be kept in scratch memory).
__device__ __forceinline__ uint32_t select_matrix(const PrefillArgs& a, uint32_t tx) {
  uint32_t s = 0;
#pragma unroll
  for (uint32_t i = 0; i + 1 < kMaxSegs; i++)
    if (i + 1 < a.nmats && tx >= a.mats[i].tiles_end) s = i + 1;
  return s;
}

__device__ __forceinline__ uint16_t bf16_bits(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0x7FFFFFu) ? 0x40u : 0u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

using egd::pack_bf16;

// One 64 x 64 block of x and of W held in registers between its global loads and its LDS
// stores (chunked layout): x as 4 float4 per thread; W as 16 codes (8 bytes) per thread - row
// tid / 4, codes 16 * (tid % 4) .. +16 of the block - with their block's scale and zero-point.
struct Staged {
  float4 x[4];
  float4 g;  // NORM: the norm weights of the 4 x columns
  uint2 q;
  float s;
  float z;
};

// The four streams as buffer resources: an out-of-range offset reads zeros without touching
// memory, so a block's edge needs no branch (a branch around a load makes the compiler wait
// for it on the spot, which would serialize the stages).
struct Streams {
  __amdgpu_buffer_rsrc_t x, w, s, z, g;
};
constexpr uint32_t kOutside = 0x80000000u;  // an offset past every stream (streams < 2 GiB here)

// This thread's part of every staged block, fixed for the launch: its 4 x vectors (rows
// m0 + tid/16 + 16i, columns 4 * (tid % 16) of the block) and its 16 codes (row n0 + tid/4,
// columns 16 * (tid % 4) of the block). A block's loads are then these bases plus the block's
// column, with no per-block multiplies.
struct StageBase {
  uint32_t x[4];    // byte offset of row r_i, column c (block 0), or kOutside when the row is outside
  uint32_t xc;      // column of the x vectors within a block
  uint32_t w;       // byte offset of the codes (block 0), or kOutside when the row is outside
  uint32_t kc;      // column of the codes within a block
  uint32_t sblk;    // the row's first quant block index
};

template <bool XB16>
__device__ __forceinline__ StageBase stage_base(const PrefillArgs& a, const PrefillMat& w, uint32_t m0, uint32_t n0) {
  const uint32_t tid = threadIdx.x & 255u;  // the thread within its group of 4 waves
  StageBase b;
  b.xc = (tid & 15u) * 4u;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t row = m0 + (tid >> 4) + 16u * i;
    b.x[i] = row < a.m ? (row * a.k + b.xc) * (XB16 ? 2u : 4u) : kOutside;
  }
  const uint32_t nrow = n0 + (tid >> 2);
  b.kc = 16u * (tid & 3u);
  b.w = nrow < w.n ? (nrow * a.k + b.kc) / 2u : kOutside;
  b.sblk = nrow * a.blocks_per_row;
  return b;
}

template <int ENC, bool NORM, bool XB16>
__device__ __forceinline__ void load_block(const PrefillArgs& a, const Streams& r, const StageBase& b, uint32_t k0,
                                           Staged& st) {
  const bool xin = k0 + b.xc < a.k;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (XB16) {  // 4 bf16 values, kept as their bits in x and y
      const uint64_t v = egd::load_b64(r.x, xin && b.x[i] != kOutside ? b.x[i] + k0 * 2u : kOutside);
      st.x[i] = make_float4(__uint_as_float((uint32_t)v), __uint_as_float((uint32_t)(v >> 32)), 0.f, 0.f);
    } else {
      const egd::u32x4 v = egd::load_b128(r.x, xin && b.x[i] != kOutside ? b.x[i] + k0 * 4u : kOutside);
      st.x[i] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    }
  }
  if (NORM) {
    const egd::u32x4 v = egd::load_b128(r.g, xin ? (k0 + b.xc) * 4u : kOutside);
    st.g = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
  const bool in = b.w != kOutside && k0 + b.kc < a.k;
  const uint32_t blk = b.sblk + ((k0 + b.kc) >> a.block_shift);
  const uint64_t codes = egd::load_b64(r.w, in ? b.w + k0 / 2u : kOutside);
  st.q = make_uint2((uint32_t)codes, (uint32_t)(codes >> 32));
  st.s = egd::load_f32(r.s, in ? blk * 4u : kOutside);
  if (ENC == EG_ENC_OFFSET_ZEROS) {
    const uint32_t zw = egd::load_b32(r.z, in ? (blk / 8u) * 4u : kOutside);
    st.z = (float)((zw >> (4 * (blk % 8))) & 0xFu);
  } else {
    st.z = 8.f;
  }
}

template <int ENC, bool NORM, bool XB16>
__device__ __forceinline__ void store_block(const Staged& st, uint16_t (*As)[kLds], uint16_t (*Bs)[kLds]) {
  const uint32_t tid = threadIdx.x & 255u;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t idx = tid + i * 256u;
    const uint32_t r = idx >> 4, c = (idx & 15u) * 4u;
    if (XB16) {
      *reinterpret_cast<uint2*>(&As[r][c]) = make_uint2(__float_as_uint(st.x[i].x), __float_as_uint(st.x[i].y));
      continue;
    }
    // NORM: x times its column's norm weight here, the row's 1 / rms in the epilogue
    const float4 v = NORM ? make_float4(st.x[i].x * st.g.x, st.x[i].y * st.g.y, st.x[i].z * st.g.z, st.x[i].w * st.g.w)
                          : st.x[i];
    *reinterpret_cast<uint2*>(&As[r][c]) = make_uint2(pack_bf16(v.x, v.y), pack_bf16(v.z, v.w));
  }
  // (code - zero) * scale in f32, exactly the reference's dequantElement, then bf16. Each word's
  // low and high nibbles are masked in place (the high ones stay 16x, their scale is divided
  // by 16: exact) and each byte converts straight to f32. Two's-complement codes are flipped
  // to offset binary c = q + 8 in the same mask, and c * s - 8 * s is one fused multiply-add:
  // the product is exact inside it and 8 * s is exact, so the single rounding is that of
  // (c - 8) * s. Offset-binary codes keep the subtraction: (c - z) * s.
  const uint32_t d[2] = {st.q.x, st.q.y};
  const float s16 = st.s * 0.0625f;
  uint32_t packed[8];
#pragma unroll
  for (int w = 0; w < 2; w++) {
    uint32_t lo, hi;
    if (ENC == EG_ENC_SIGNED) {
      lo = (d[w] & 0x0F0F0F0Fu) ^ 0x08080808u;
      hi = (d[w] & 0xF0F0F0F0u) ^ 0x80808080u;
    } else {
      lo = egd::and_opaque(d[w], 0x0F0F0F0Fu);
      hi = egd::and_opaque(d[w], 0xF0F0F0F0u);
    }
    float v[8];
    const float cl[4] = {egd::ub0(lo), egd::ub1(lo), egd::ub2(lo), egd::ub3(lo)};
    const float ch[4] = {egd::ub0(hi), egd::ub1(hi), egd::ub2(hi), egd::ub3(hi)};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (ENC == EG_ENC_SIGNED) {
        const float off = -8.f * st.s;
        v[2 * j] = fmaf(cl[j], st.s, off);
        v[2 * j + 1] = fmaf(ch[j], s16, off);
      } else {
        v[2 * j] = (cl[j] - st.z) * st.s;
        v[2 * j + 1] = (ch[j] - 16.f * st.z) * s16;
      }
    }
#pragma unroll
    for (int e = 0; e < 8; e += 2) packed[(w * 8 + e) / 2] = pack_bf16(v[e], v[e + 1]);
  }
  uint4* dst = reinterpret_cast<uint4*>(&Bs[tid >> 2][16u * (tid & 3u)]);
  dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
  dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

// Element-by-element staging for the layouts the chunked path does not take.
template <int ENC>
__device__ void stage_elements(const PrefillArgs& a, const PrefillMat& w, uint32_t m0, uint32_t n0, uint32_t k0,
                               uint16_t (*As)[kLds], uint16_t (*Bs)[kLds]) {
  const uint32_t tid = threadIdx.x & 255u;
  const uint32_t per_word = 32u / (uint32_t)a.bits, mask = (1u << a.bits) - 1u;
#pragma unroll 4
  for (uint32_t e = tid; e < kTile * kBK; e += 256) {
    const uint32_t r = e / kBK, c = e % kBK;
    const uint32_t row = m0 + r, kk = k0 + c;
    const float v = (row < a.m && kk < a.k) ? a.x[(size_t)row * a.k + kk] : 0.f;
    As[r][c] = bf16_bits(v);
  }
#pragma unroll 4
  for (uint32_t e = tid; e < kTile * kBK; e += 256) {
    const uint32_t r = e / kBK, c = e % kBK;
    const uint32_t nrow = n0 + r, kk = k0 + c;
    float v = 0.f;
    if (nrow < w.n && kk < a.k) {
      const size_t flat = (size_t)nrow * a.k + kk;
      uint32_t code = (w.packed[flat / per_word] >> (a.bits * (flat % per_word))) & mask;
      const uint32_t blk = nrow * a.blocks_per_row + kk / a.block_size;
      int32_t z;
      if (ENC == EG_ENC_OFFSET_ZEROS) {
        z = (int32_t)((w.zeros[blk / per_word] >> (a.bits * (blk % per_word))) & mask);
      } else {
        code ^= 1u << (a.bits - 1);
        z = 1 << (a.bits - 1);
      }
      v = (float)((int32_t)code - z) * w.scales[blk];
    }
    Bs[r][c] = bf16_bits(v);
  }
}

// v rounded to bf16 as pack_bf16 rounds it (round to nearest even).
__device__ __forceinline__ uint16_t bf16_of(float v) { return (uint16_t)(pack_bf16(v, 0.f) & 0xFFFFu); }

// SiLU(g) * u with SiLU(g) = g / (1 + e^-g), the prompt chain's silu_mul_rows formula.
__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

// KG groups of 4 waves share a workgroup and a tile: group g stages and multiplies the 64-deep
// blocks g, g + KG, ... of the workgroup's K range into its own accumulators (its own LDS
// buffers; one barrier pair per KG blocks), and the groups' sums are added in group order at the
// end. With one workgroup per CU (the tile grids here hold ~1 per CU) a single group leaves
// every SIMD one wave, so each block's staging, LDS round trip, barriers and MFMAs run back to
// back; KG groups put KG waves on each SIMD and cut the serial chain by KG.
//
// PAIR (the gate|up SwiGLU pair, chunked staging only): tile column t holds rows 32t .. 32t+31 of
// mats[0] (gate) in its first 32 columns and the same rows of mats[1] (up) in the last 32 - waves
// 0-1 of a group stage gate rows, waves 2-3 up rows - and the epilogue stores SiLU(gate) * up for
// the 32 columns into mats[0].out.
//
// NORM (chunked staging, no K split): x is a residual row, RMS-normalised on the way in - each
// staged x value times its column's norm weight before the bf16 rounding, each thread summing
// the squares of the x it stages; the rows' sums meet in LDS after the K loop and the epilogue
// scales each output row by 1 / sqrt(sum / K + eps) (rmsnorm_rows' formula, with the row's
// scale applied after the products instead of before them).
//
// ROPE (chunked staging; mats = q, k, v with head_dim 64, so a tile is one head): the epilogue
// takes each row's (e, e + 32) pairs from the LDS sums, adds the biases, rotates them in double
// precision with the table's cos/sin of the row's position - rope_append's arithmetic - and
// stores q * RoPE / 8 in f32 and k, v in f16 into the caches.
//
// XB16 (chunked staging, no NORM): x holds bf16 values (a producer stored them rounded as the
// staging would), staged as they are.
//
// S: register stages of the chunked staging (blocks in flight per group: S - 1). Four groups fit
// four waves per SIMD only within 128 VGPRs: they keep one block in flight. Measured on the
// config-3 shapes, deeper staging does not pay: one group at S = 5 runs as S = 3, at S = 8 (one
// wave per SIMD) 18.5 -> 27.4 us for gate M = 256; two groups at S = 4 and four at S = 3 are
// slower than their defaults.
template <int ENC, bool CHUNKED, int KG, bool PAIR = false, bool NORM = false, bool ROPE = false, bool XB16 = false,
          int S = (KG >= 4 ? 2 : kStages)>
__global__ __launch_bounds__(256 * KG) void prefill_kernel(PrefillArgs a) {
  // No contraction of separate operations into fused multiply-adds (the explicit fmaf calls stay):
  // every epilogue then rounds the row's norm scale and the bias addition on their own, so the
  // launches that fold different work into their epilogues give the same values.
#pragma clang fp contract(off)
  // staging buffers of every group; after the K loop they hold the groups' f32 sums
  constexpr uint32_t kStageBytes = 2u * kTile * kLds * 2u;  // As + Bs of one group
  static_assert(kStageBytes >= kTile * kTile * 4u, "a group's buffers hold its 64 x 64 f32 sums");
  __shared__ __attribute__((aligned(16))) uint8_t lds[KG * kStageBytes];
  __shared__ float row_ss[NORM ? KG : 1][kTile];  // NORM: each group's sums of squares per row
  const uint32_t group = threadIdx.x >> 8;
  uint16_t(*As)[kLds] = reinterpret_cast<uint16_t(*)[kLds]>(lds + group * kStageBytes);
  uint16_t(*Bs)[kLds] = reinterpret_cast<uint16_t(*)[kLds]>(lds + group * kStageBytes + kTile * kLds * 2u);
  const uint32_t tid = threadIdx.x & 255u, wave = tid >> 6, lane = tid & 63u;
  // The tile (tx, ty). Workgroups are dispatched to the 8 XCDs in turn (workgroup L of the grid
  // on XCD L % 8), each with its own L2. With xcd_rows the workgroups of one XCD take whole row
  // tiles (row tiles k, k + 8, ... on XCD k, every column tile of each), so a row tile's x is
  // fetched into one L2 instead of up to eight; otherwise the grid's own order.
  uint32_t tx = blockIdx.x, ty = blockIdx.y;
  if (a.xcd_rows) {
    const uint32_t L = blockIdx.x + gridDim.x * blockIdx.y, k = L % 8u, j = L / 8u;
    ty = k + 8u * (j / gridDim.x);
    tx = j % gridDim.x;
  }
  // the matrix whose rows this thread stages (wave-uniform), and the tile's first row of it
  const uint32_t half = PAIR ? __builtin_amdgcn_readfirstlane(wave >> 1) : 0u;
  const PrefillMat& w = a.mats[PAIR ? half : select_matrix(a, tx)];
  const uint32_t m0 = ty * kTile;
  const uint32_t n0 = PAIR ? 32u * tx - 32u * half : (tx - (w.tiles_end - ((w.n + kTile - 1) / kTile))) * kTile;
  const uint32_t wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const uint32_t kbeg = blockIdx.z * a.k_per_split, kend = min(a.k, kbeg + a.k_per_split);

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto mfma_block = [&]() {
#pragma unroll
    for (int ks = 0; ks < kBK / 32; ks++) {
      const uint32_t kofs = ks * 32 + 8 * (lane >> 4);
      bf16x8 af[2], bfr[2];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const uint4 ua = *reinterpret_cast<const uint4*>(&As[wm + i * 16 + (lane & 15)][kofs]);
        af[i] = __builtin_bit_cast(bf16x8, ua);
        const uint4 ub = *reinterpret_cast<const uint4*>(&Bs[wn + i * 16 + (lane & 15)][kofs]);
        bfr[i] = __builtin_bit_cast(bf16x8, ub);
      }
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
  };

  const uint32_t nblk = (kend - kbeg + kBK - 1) / kBK;
  // this group's blocks: group + KG * i for i < iters (the last ones past nblk are skipped; the
  // groups run the same number of iterations so the barriers match)
  const uint32_t iters = (nblk + KG - 1) / KG;
  auto block_of = [&](uint32_t i) { return group + KG * i; };
  if (CHUNKED) {
    // kStages register stages: block b lives in stage b % kStages and is stored to LDS while
    // blocks b+1 .. b+kStages-1 are in flight (an iteration is ~0.3 us of staging and MFMAs;
    // HBM latency is several of those). The steady-state loop covers whole groups of kStages
    // blocks with no branch at all - loads unconditional, clamped to the last block - so the
    // compiler's wait before each store counts exactly the loads issued after that stage's; the
    // remaining blocks are already in flight and drain in a loop that issues no loads.
    const Streams rs{egd::buffer(a.x, a.m * a.k * (XB16 ? 2u : 4u)), egd::buffer(w.packed, w.n * a.k / 2u),
                     egd::buffer(w.scales, w.n * a.blocks_per_row * 4u),
                     egd::buffer(w.zeros, ((w.n * a.blocks_per_row + 7u) / 8u) * 4u),
                     egd::buffer(NORM ? a.norm : nullptr, NORM ? a.k * 4u : 0u)};
    const StageBase sb = stage_base<XB16>(a, w, m0, n0);
    Staged st[S];
    float ss[4] = {0.f, 0.f, 0.f, 0.f};  // NORM: squares of this thread's x, rows tid / 16 + 16 i
    auto square = [&](const Staged& v) {
#pragma unroll
      for (int i = 0; i < 4; i++) {
        ss[i] = fmaf(v.x[i].x, v.x[i].x, ss[i]);
        ss[i] = fmaf(v.x[i].y, v.x[i].y, ss[i]);
        ss[i] = fmaf(v.x[i].z, v.x[i].z, ss[i]);
        ss[i] = fmaf(v.x[i].w, v.x[i].w, ss[i]);
      }
    };
#pragma unroll
    for (int u = 0; u + 1 < S; u++)
      load_block<ENC, NORM, XB16>(a, rs, sb, kbeg + min(block_of((uint32_t)u), nblk - 1) * kBK, st[u]);
    const uint32_t full = iters / S;
    for (uint32_t g = 0; g < full; g++) {
#pragma unroll
      for (int u = 0; u < S; u++) {
        const uint32_t it = g * S + u;
        store_block<ENC, NORM, XB16>(st[u], As, Bs);
        if (NORM && block_of(it) < nblk) square(st[u]);
        __syncthreads();
        load_block<ENC, NORM, XB16>(a, rs, sb, kbeg + min(block_of(it + S - 1), nblk - 1) * kBK, st[(u + S - 1) % S]);
        if (block_of(it) < nblk) mfma_block();
        __syncthreads();
      }
    }
    const uint32_t rest = iters - full * S;
#pragma unroll
    for (int u = 0; u + 1 < S; u++) {
      if ((uint32_t)u < rest) {
        store_block<ENC, NORM, XB16>(st[u], As, Bs);
        if (NORM && block_of(full * S + u) < nblk) square(st[u]);
        __syncthreads();
        if (block_of(full * S + u) < nblk) mfma_block();
        __syncthreads();
      }
    }
    if (NORM) {
      // the 16 threads of a row group (lanes 16 q .. 16 q + 15 of a wave) hold the row's columns
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) ss[i] += __shfl_xor(ss[i], off, 64);
      if ((tid & 15u) == 0)
#pragma unroll
        for (int i = 0; i < 4; i++) row_ss[NORM ? group : 0][(tid >> 4) + 16 * i] = ss[i];
      __syncthreads();
    }
  } else {
    for (uint32_t it = 0; it < iters; it++) {
      const uint32_t blk = min(block_of(it), nblk - 1);
      stage_elements<ENC>(a, w, m0, n0, kbeg + blk * kBK, As, Bs);
      __syncthreads();
      if (block_of(it) < nblk) mfma_block();
      __syncthreads();
    }
  }
  // NORM: 1 / rms of tile row r, the groups' sums of squares added in group order
  auto inv_rms = [&](uint32_t r) {
    float t = row_ss[0][r];
#pragma unroll
    for (int g = 1; g < (NORM ? KG : 1); g++) t += row_ss[NORM ? g : 0][r];
    return 1.0f / sqrtf(t / (float)a.k + a.eps);
  };
  if (KG > 1 || PAIR || ROPE) {
    // every group's sums into its own buffers (the last barrier above ended the staging), then
    // the groups added in order by the thread that stores the element
    float* sums = reinterpret_cast<float*>(lds + group * kStageBytes);
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int j = 0; j < 2; j++)
#pragma unroll
        for (int e = 0; e < 4; e++)
          sums[(wm + i * 16 + 4 * (lane >> 4) + e) * kTile + wn + j * 16 + (lane & 15)] = acc[i][j][e];
    __syncthreads();
    if (ROPE) {
      const uint32_t s = select_matrix(a, tx), hd = n0 / kTile;
      auto sum = [&](uint32_t r, uint32_t c) {
        float v = reinterpret_cast<const float*>(lds)[r * kTile + c];
#pragma unroll
        for (int k = 1; k < KG; k++) v += reinterpret_cast<const float*>(lds + k * kStageBytes)[r * kTile + c];
        if (NORM) v *= inv_rms(r);
        return v + (w.bias ? w.bias[n0 + c] : 0.f) + 0.f;
      };
      if (s == 2) {  // v: the rows as they are, f16
        for (uint32_t idx = threadIdx.x; idx < kTile * kTile; idx += 256u * KG) {
          const uint32_t r = idx / kTile, c = idx % kTile, row = m0 + r;
          if (row >= a.m) continue;
          a.v_cache[((size_t)(a.rope_pos0 + row) * a.kv_heads + hd) * kTile + c] = egd::float_to_half(sum(r, c));
        }
        return;
      }
      for (uint32_t idx = threadIdx.x; idx < kTile * 32u; idx += 256u * KG) {
        const uint32_t r = idx / 32u, e = idx % 32u, row = m0 + r;
        if (row >= a.m) continue;
        const double2 cs = a.rope[(size_t)(a.rope_pos0 + row) * 32u + e];
        const float2 rr = egd::rotate(sum(r, e), sum(r, e + 32u), cs);
        const float r0 = rr.x, r1 = rr.y;
        if (s == 0) {
          float* dst = a.q_rope + ((size_t)row * a.q_heads + hd) * kTile;
          dst[e] = r0 * 0.125f;
          dst[e + 32u] = r1 * 0.125f;
        } else {
          uint16_t* dst = a.k_cache + ((size_t)(a.rope_pos0 + row) * a.kv_heads + hd) * kTile;
          dst[e] = egd::float_to_half(r0);
          dst[e + 32u] = egd::float_to_half(r1);
        }
      }
      return;
    }
    if (PAIR) {
      const PrefillMat& g = a.mats[0];
      const PrefillMat& u = a.mats[1];
      for (uint32_t idx = threadIdx.x; idx < kTile * 32u; idx += 256u * KG) {
        const uint32_t r = idx / 32u, c = idx % 32u, row = m0 + r, col = 32u * tx + c;
        if (row >= a.m || col >= g.n) continue;
        float gv = reinterpret_cast<const float*>(lds)[r * kTile + c];
        float uv = reinterpret_cast<const float*>(lds)[r * kTile + c + 32u];
#pragma unroll
        for (int k = 1; k < KG; k++) {
          gv += reinterpret_cast<const float*>(lds + k * kStageBytes)[r * kTile + c];
          uv += reinterpret_cast<const float*>(lds + k * kStageBytes)[r * kTile + c + 32u];
        }
        if (NORM) {
          const float inv = inv_rms(r);
          gv *= inv;
          uv *= inv;
        }
        gv = gv + (g.bias ? g.bias[col] : 0.f) + 0.f;
        uv = uv + (u.bias ? u.bias[col] : 0.f) + 0.f;
        const size_t o = (size_t)row * g.out_stride + col + g.out_offset;
        if (a.out_bf16) reinterpret_cast<uint16_t*>(g.out)[o] = bf16_of(silu_mul(gv, uv));
        else g.out[o] = silu_mul(gv, uv);
      }
      return;
    }
    for (uint32_t idx = threadIdx.x; idx < kTile * kTile; idx += 256u * KG) {
      const uint32_t r = idx / kTile, c = idx % kTile, row = m0 + r, col = n0 + c;
      if (row >= a.m || col >= w.n) continue;
      float v = reinterpret_cast<const float*>(lds)[idx];
#pragma unroll
      for (int g = 1; g < KG; g++) v += reinterpret_cast<const float*>(lds + g * kStageBytes)[idx];
      if (NORM) v *= inv_rms(r);
      if (a.partials) {
        a.partials[((size_t)blockIdx.z * a.m + row) * w.n + col] = v;
      } else {
        const size_t o = (size_t)row * w.out_stride + col + w.out_offset;
        w.out[o] = v + (w.bias ? w.bias[col] : 0.f) + (w.residual ? w.residual[o] : 0.f);
      }
    }
    return;
  }

  // D layout of the 16x16 MFMA: lane l holds rows 4*(l/16) + e, column l % 16.
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint32_t col = n0 + wn + j * 16 + (lane & 15);
      if (col >= w.n) continue;
      const float b = (a.partials == nullptr && w.bias) ? w.bias[col] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t r = wm + i * 16 + 4 * (lane >> 4) + e, row = m0 + r;
        if (row >= a.m) continue;
        if (a.partials) {
          a.partials[((size_t)blockIdx.z * a.m + row) * w.n + col] = acc[i][j][e];
        } else {
          const size_t o = (size_t)row * w.out_stride + col + w.out_offset;
          w.out[o] = (NORM ? acc[i][j][e] * inv_rms(r) : acc[i][j][e]) + b + (w.residual ? w.residual[o] : 0.f);
        }
      }
    }
}

// The split-K sum: splits added in index order, then the bias.
__global__ __launch_bounds__(256) void prefill_reduce_kernel(const float* __restrict__ partials,
                                                             const float* __restrict__ bias,
                                                             const float* __restrict__ residual, float* out, uint32_t m,
                                                             uint32_t n, uint32_t splits, uint32_t out_stride,
                                                             uint32_t out_offset) {
  const size_t total = (size_t)m * n;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    float acc = 0.f;
    for (uint32_t z = 0; z < splits; z++) acc += partials[(size_t)z * total + i];
    const uint32_t row = (uint32_t)(i / n), col = (uint32_t)(i % n);
    const size_t o = (size_t)row * out_stride + col + out_offset;
    out[o] = acc + (bias ? bias[col] : 0.f) + (residual ? residual[o] : 0.f);
  }
}

// Whether a launch maps whole row tiles to each XCD: its grid has no K split and a multiple of 8
// row tiles, and its column tiles are not a multiple of 8 (with a multiple of 8 the grid's own
// order already keeps each column tile on one XCD, which suits the wide launches whose weight
// tiles outweigh their x tiles).
uint32_t xcd_rows_for(const eg_context* ctx, dim3 grid) {
  return ctx->prefill_xcd && grid.z == 1 && grid.y % 8 == 0 && grid.x % 8 != 0 ? 1u : 0u;
}

// One launch of the chunked staging with kg groups of 4 waves per workgroup.
template <bool PAIR, bool NORM, bool ROPE = false, bool XB16 = false>
void launch_chunked(int encoding, int kg, dim3 grid, hipStream_t stream, const PrefillArgs& a) {
  const dim3 block(256 * kg);
#define EG_KG(ENC)                                                                                                  \
  do {                                                                                                              \
    if (kg == 4) hipLaunchKernelGGL((prefill_kernel<ENC, true, 4, PAIR, NORM, ROPE, XB16>), grid, block, 0, stream, a);    \
    else if (kg == 2) hipLaunchKernelGGL((prefill_kernel<ENC, true, 2, PAIR, NORM, ROPE, XB16>), grid, block, 0, stream, a); \
    else hipLaunchKernelGGL((prefill_kernel<ENC, true, 1, PAIR, NORM, ROPE, XB16>), grid, block, 0, stream, a);            \
  } while (0)
  if (encoding == EG_ENC_SIGNED) EG_KG(EG_ENC_SIGNED);
  else EG_KG(EG_ENC_OFFSET_ZEROS);
#undef EG_KG
}

}  // namespace

bool eg::prefill_chunked(uint32_t m, uint32_t n, uint32_t k, uint32_t bs, int bits, const void* x,
                         const uint32_t* packed) {
  return bits == 4 && k % 32 == 0 && bs % 16 == 0 && (bs & (bs - 1)) == 0 && k % 4 == 0 &&
         (uint64_t)m * k * 4 < kOutside && (uint64_t)n * k / 2 < kOutside &&
         (reinterpret_cast<uintptr_t>(packed) & 7u) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

int eg::prefill_gemm(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                     const uint32_t* zeros, const float* bias, const float* residual, float* out,
                     const eg_matmul_q4_dims* dims, int encoding, int bits, bool x_bf16) {
  const char* op = "matmul_q4_prefill";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!dims || !x || !packed || !scales || !out) return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  if (bits != 4 && bits != 8) return eg::fail(ctx, EG_ERR_INVALID, "%s: bits must be 4 or 8, got %d", op, bits);
  if (encoding != EG_ENC_OFFSET_ZEROS && encoding != EG_ENC_SIGNED)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: unknown encoding %d", op, encoding);
  if (encoding == EG_ENC_OFFSET_ZEROS && !zeros)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: the offset encoding needs a zero-point stream", op);
  if (dims->use_bias && !bias) return eg::fail(ctx, EG_ERR_INVALID, "%s: useBias set but bias is NULL", op);
  const uint32_t m = dims->m, n = dims->n, k = dims->k, bs = dims->block_size;
  if (bs == 0 || k % bs != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: reduction axis %u is not a multiple of %u", op, k, bs);
  if (dims->blocks_per_row != k / bs)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: blocksPerRow %u does not equal k / blockSize = %u", op,
                    dims->blocks_per_row, k / bs);
  if (m > 1 && dims->out_stride < n)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: outStride %u is less than n %u", op, dims->out_stride, n);
  if (((uint64_t)n * k) % (32 / bits) != 0)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: codes do not fill whole 32-bit words", op);
  if ((uint64_t)m * k >= (1ull << 40) || (uint64_t)n * dims->blocks_per_row >= (1ull << 32))
    return eg::fail(ctx, EG_ERR_RANGE, "%s: %u x %u x %u exceeds the index range", op, m, n, k);
  if (m == 0 || n == 0) return EG_OK;
  const uint32_t tiles_n = (n + kTile - 1) / kTile, tiles_m = (m + kTile - 1) / kTile;
  if (tiles_m > 65535) return eg::fail(ctx, EG_ERR_RANGE, "%s: m %u needs %u row tiles, over 65535", op, m, tiles_m);
  // Groups per workgroup: a grid of at least one tile per CU runs one-group workgroups (three
  // fit on a CU, so a second round of tiles overlaps the first); a smaller grid runs four groups
  // per workgroup (one per CU), whose 16 waves work through the tile's K blocks four at a time
  // (measured at M = 128: gate 11.4 -> 8.3 us; at M = 256 the 304 gate tiles would need a
  // second round of 1024-thread workgroups: 14.6 -> 16.3 us).
  const uint64_t tiles = (uint64_t)tiles_n * tiles_m;
  const uint64_t blocks = (k + kBK - 1) / kBK;
  const int kg = ctx->prefill_groups ? ctx->prefill_groups : (tiles >= (uint64_t)ctx->cu_count ? 1 : 4);
  // Split K only where the tile grid leaves most CUs idle over a long reduction (the down
  // projection: 4 x 14 tiles at M = 256, 76 blocks deep): the partial sums cost a second
  // launch, so the split must save more block iterations than that launch costs. Four-group
  // workgroups keep the split grid within one workgroup per CU and at least two blocks per
  // group. The f32 partials live in the context's workspace.
  uint64_t splits = 1;
  if (blocks >= 32 && tiles < (uint64_t)ctx->cu_count)
    splits = kg == 1 ? std::min<uint64_t>((ctx->cu_count + tiles - 1) / tiles, blocks / 8)
                     : std::min<uint64_t>(ctx->cu_count / tiles, blocks / (2 * (uint64_t)kg));
  splits = std::min<uint64_t>(splits, std::max<uint64_t>(1, eg::kPartialsBytes / ((uint64_t)m * n * 4)));
  splits = std::max<uint64_t>(1, std::min<uint64_t>(splits, 65535));
  uint32_t k_per_split = (uint32_t)((((uint64_t)k + splits - 1) / splits + kBK - 1) / kBK * kBK);
  splits = (k + k_per_split - 1) / k_per_split;
  const bool split = splits > 1;
  PrefillArgs a{x, split ? reinterpret_cast<float*>(eg::partials(ctx)) : nullptr, m, k, bs, dims->blocks_per_row,
                k_per_split, bits, (uint32_t)__builtin_ctz(bs), 1u, nullptr, 0.f, nullptr, nullptr, nullptr, nullptr,
                0u, 0u, 0u, 0u, 0u, {}};
  a.mats[0] = PrefillMat{packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros, dims->use_bias ? bias : nullptr,
                         residual, out, n, dims->out_stride, dims->out_offset, tiles_n};
  const dim3 grid(tiles_n, tiles_m, (uint32_t)splits);
  a.xcd_rows = xcd_rows_for(ctx, grid);
  const bool chunked = eg::prefill_chunked(m, n, k, bs, bits, x, packed);
  if (x_bf16 && !chunked)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: bf16 rows of x need the chunked staging", op);
  const dim3 block(256 * kg);
#define EG_PREFILL_LAUNCH(ENC, CH)                                                                        \
  do {                                                                                                    \
    if (kg == 4) hipLaunchKernelGGL((prefill_kernel<ENC, CH, 4>), grid, block, 0, ctx->stream, a);        \
    else if (kg == 2) hipLaunchKernelGGL((prefill_kernel<ENC, CH, 2>), grid, block, 0, ctx->stream, a);   \
    else hipLaunchKernelGGL((prefill_kernel<ENC, CH, 1>), grid, block, 0, ctx->stream, a);                \
  } while (0)
  if (x_bf16) {
    launch_chunked<false, false, false, true>(encoding, kg, grid, ctx->stream, a);
  } else if (encoding == EG_ENC_SIGNED) {
    if (chunked) EG_PREFILL_LAUNCH(EG_ENC_SIGNED, true);
    else EG_PREFILL_LAUNCH(EG_ENC_SIGNED, false);
  } else {
    if (chunked) EG_PREFILL_LAUNCH(EG_ENC_OFFSET_ZEROS, true);
    else EG_PREFILL_LAUNCH(EG_ENC_OFFSET_ZEROS, false);
  }
#undef EG_PREFILL_LAUNCH
  if (split) {
    const uint64_t total = (uint64_t)m * n;
    const uint32_t blocks = (uint32_t)std::min<uint64_t>((total + 255) / 256, (uint64_t)ctx->cu_count * 8);
    hipLaunchKernelGGL(prefill_reduce_kernel, dim3(blocks), dim3(256), 0, ctx->stream, a.partials, a.mats[0].bias, residual,
                       out, m, n, (uint32_t)splits, dims->out_stride, dims->out_offset);
  }
  return eg::check_launch(ctx, op);
}

namespace {

// Whether matrices sharing x run in ONE launch: the chunked staging takes every one of them and
// no K split is wanted. Sets the total of their 64-column tiles.
bool one_launch(const float* x, uint32_t m, uint32_t k, uint32_t block_size, int encoding, int bits,
                const eg::PrefillMatrix* mats, uint32_t count, uint64_t* tiles_n) {
  bool ok = count >= 1 && count <= kMaxSegs && m > 0 && x && bits == 4 &&
            (encoding == EG_ENC_SIGNED || encoding == EG_ENC_OFFSET_ZEROS) && block_size >= 16 &&
            (block_size & (block_size - 1)) == 0 && k % block_size == 0 && k % 32 == 0 &&
            (k + kBK - 1) / kBK < 32 && (uint64_t)m * k * 4 < kOutside && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  *tiles_n = 0;
  for (uint32_t i = 0; ok && i < count; i++) {
    const eg::PrefillMatrix& w = mats[i];
    ok = w.n > 0 && w.packed && w.scales && w.out && (encoding == EG_ENC_SIGNED || w.zeros) &&
         (m == 1 || w.out_stride >= w.n) && (uint64_t)w.n * k / 2 < kOutside &&
         (uint64_t)w.n * (k / block_size) < (1ull << 32) && (reinterpret_cast<uintptr_t>(w.packed) & 7u) == 0;
    *tiles_n += (w.n + kTile - 1) / kTile;
  }
  return ok && *tiles_n <= 0x7FFFFFFFull && (m + kTile - 1) / kTile <= 65535;
}

// Groups per workgroup for a tile grid: one where the grid holds at least a tile per CU, else four.
int groups_for(const eg_context* ctx, uint64_t tiles) {
  return ctx->prefill_groups ? ctx->prefill_groups : (tiles >= (uint64_t)ctx->cu_count ? 1 : 4);
}

// Whether a launch folds the rows' RMSNorm in: only with four-group workgroups (a grid under one
// tile per CU, latency-bound), where the extra staging work (the weight multiply and the squares,
// 32 VALU operations per thread and block) is hidden; a launch that fills the device is bound by
// that work, and a separate rmsnorm_rows launch costs less there (measured at 2048 rows: the
// gate|up pair 94 -> 128 us with the norm folded in, against 5.5 us for rmsnorm_rows).
bool fold_norm(const eg_context* ctx, uint64_t tiles, const float* norm) {
  return norm && (reinterpret_cast<uintptr_t>(norm) & 15u) == 0 && groups_for(ctx, tiles) == 4;
}

// The matrices (one_launch accepted them) as one chunked launch; norm non-NULL folds the rows'
// RMSNorm into it.
int launch_multi(eg_context* ctx, const float* x, uint32_t m, uint32_t k, uint32_t block_size, int encoding, int bits,
                 const eg::PrefillMatrix* mats, uint32_t count, uint64_t tiles_n, const float* norm, float eps,
                 const eg::PrefillRope* rope = nullptr, bool x_bf16 = false) {
  PrefillArgs a{x, nullptr, m, k, block_size, k / block_size, k, bits, (uint32_t)__builtin_ctz(block_size), count,
                norm, eps, nullptr, nullptr, nullptr, nullptr, 0u, 0u, 0u, 0u, 0u, {}};
  if (rope) {
    a.rope = rope->table;
    a.q_rope = rope->q_rope;
    a.k_cache = rope->k_cache;
    a.v_cache = rope->v_cache;
    a.rope_pos0 = rope->pos0;
    a.q_heads = rope->q_heads;
    a.kv_heads = rope->kv_heads;
  }
  uint32_t end = 0;
  for (uint32_t i = 0; i < count; i++) {
    const eg::PrefillMatrix& w = mats[i];
    end += (w.n + kTile - 1) / kTile;
    a.mats[i] = PrefillMat{w.packed, w.scales, encoding == EG_ENC_SIGNED ? nullptr : w.zeros, w.bias, w.residual,
                           w.out, w.n, w.out_stride, w.out_offset, end};
  }
  const uint64_t tiles_m = (m + kTile - 1) / kTile;
  const int kg = groups_for(ctx, tiles_n * tiles_m);
  const dim3 grid((uint32_t)tiles_n, (uint32_t)tiles_m, 1);
  a.xcd_rows = xcd_rows_for(ctx, grid);
  if (rope) {
    if (norm) launch_chunked<false, true, true>(encoding, kg, grid, ctx->stream, a);
    else if (x_bf16) launch_chunked<false, false, true, true>(encoding, kg, grid, ctx->stream, a);
    else launch_chunked<false, false, true>(encoding, kg, grid, ctx->stream, a);
  } else if (norm) {
    launch_chunked<false, true>(encoding, kg, grid, ctx->stream, a);
  } else if (x_bf16) {
    launch_chunked<false, false, false, true>(encoding, kg, grid, ctx->stream, a);
  } else {
    launch_chunked<false, false>(encoding, kg, grid, ctx->stream, a);
  }
  return eg::check_launch(ctx, "matmul_q4_prefill");
}

}  // namespace

int eg::prefill_gemm_multi(eg_context* ctx, const float* x, uint32_t m, uint32_t k, uint32_t block_size,
                           int encoding, int bits, const PrefillMatrix* mats, uint32_t count, const float* norm,
                           float eps, float* normed) {
  const char* op = "matmul_q4_prefill";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (count > 0 && !mats) return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL matrix list", op);
  uint64_t tiles_n = 0;
  const uint64_t tiles_m = (m + kTile - 1) / kTile;
  if (norm) {
    // RMSNorm folded into the one launch where that pays (fold_norm); otherwise rmsnorm_rows
    // into `normed` (as bf16 rows when the one launch stages them) and the launches below on it
    const bool one = one_launch(x, m, k, block_size, encoding, bits, mats, count, &tiles_n);
    if (one && fold_norm(ctx, tiles_n * tiles_m, norm))
      return launch_multi(ctx, x, m, k, block_size, encoding, bits, mats, count, tiles_n, norm, eps);
    if (!normed) return eg::fail(ctx, EG_ERR_INVALID, "%s: RMSNorm needs a buffer for the normed rows", op);
    const bool xb = one && ctx->prefill_xb16;
    const int st = eg::rmsnorm_rows(ctx, x, norm, m, k, eps, normed, xb);
    if (st != EG_OK) return st;
    if (xb) return launch_multi(ctx, normed, m, k, block_size, encoding, bits, mats, count, tiles_n, nullptr, 0.f,
                                nullptr, true);
    x = normed;
  }
  auto one = [&](const PrefillMatrix& w) {
    eg_matmul_q4_dims dm{};
    dm.m = m;
    dm.n = w.n;
    dm.k = k;
    dm.use_bias = w.bias != nullptr;
    dm.block_size = block_size;
    dm.blocks_per_row = block_size ? k / block_size : 0;
    dm.out_stride = w.out_stride;
    dm.out_offset = w.out_offset;
    return eg::prefill_gemm(ctx, x, w.packed, w.scales, w.zeros, w.bias, w.residual, w.out, &dm, encoding, bits);
  };
  // One launch where the chunked staging takes every matrix and no matrix would split K;
  // otherwise (and for anything the single path must reject with its own message) one each.
  if (count < 2 || !one_launch(x, m, k, block_size, encoding, bits, mats, count, &tiles_n)) {
    for (uint32_t i = 0; i < count; i++) {
      const int st = one(mats[i]);
      if (st != EG_OK) return st;
    }
    return EG_OK;
  }
  (void)tiles_m;
  return launch_multi(ctx, x, m, k, block_size, encoding, bits, mats, count, tiles_n, nullptr, 0.f);
}

int eg::prefill_qkv_rope(eg_context* ctx, const float* x, uint32_t m, uint32_t k, uint32_t block_size, int encoding,
                         int bits, const PrefillMatrix* mats, const float* norm, float eps, float* normed,
                         const PrefillRope& rope, bool* done) {
  *done = false;
  if (!ctx || !mats || !ctx->prefill_rope || m == 0) return EG_OK;
  uint64_t tiles_n = 0;
  if (!rope.table || !rope.q_rope || !rope.k_cache || !rope.v_cache || mats[0].n != rope.q_heads * kTile ||
      mats[1].n != rope.kv_heads * kTile || mats[2].n != rope.kv_heads * kTile ||
      !one_launch(x, m, k, block_size, encoding, bits, mats, 3, &tiles_n))
    return EG_OK;
  const uint64_t tiles_m = (m + kTile - 1) / kTile;
  bool xb = false;
  if (norm && !fold_norm(ctx, tiles_n * tiles_m, norm)) {
    if (!normed) return eg::fail(ctx, EG_ERR_INVALID, "matmul_q4_prefill: RMSNorm needs a buffer for the normed rows");
    xb = ctx->prefill_xb16;
    const int st = eg::rmsnorm_rows(ctx, x, norm, m, k, eps, normed, xb);
    if (st != EG_OK) return st;
    x = normed;
    norm = nullptr;
  }
  *done = true;
  return launch_multi(ctx, x, m, k, block_size, encoding, bits, mats, 3, tiles_n, norm, eps, &rope, xb);
}

int eg::prefill_gemm_swiglu(eg_context* ctx, const float* x, uint32_t m, uint32_t k, uint32_t block_size,
                            int encoding, int bits, const PrefillMatrix& gate, const PrefillMatrix& up, float* out,
                            float* scratch, const float* norm, float eps, float* normed, bool out_bf16) {
  const char* op = "matmul_q4_prefill";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!out || !scratch || gate.n != up.n)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: SwiGLU pair needs matching gate and up and two outputs", op);
  const uint32_t n = gate.n;
  // the pair as ONE launch of paired tiles where the chunked staging takes both and K is short
  const PrefillMatrix pair[2] = {{gate.packed, gate.scales, gate.zeros, gate.bias, nullptr, out, n, n, 0},
                                 {up.packed, up.scales, up.zeros, up.bias, nullptr, out, n, n, 0}};
  uint64_t tiles_n = 0;
  if (n == 0 || m == 0 || !ctx->prefill_pair || !one_launch(x, m, k, block_size, encoding, bits, pair, 2, &tiles_n)) {
    // otherwise gate | up side by side in the scratch rows, then SiLU(gate) * up
    const PrefillMatrix gu[2] = {{gate.packed, gate.scales, gate.zeros, gate.bias, nullptr, scratch, n, 2 * n, 0},
                                 {up.packed, up.scales, up.zeros, up.bias, nullptr, scratch, n, 2 * n, n}};
    int st = eg::prefill_gemm_multi(ctx, x, m, k, block_size, encoding, bits, gu, 2, norm, eps, normed);
    if (st == EG_OK && m > 0 && n > 0) st = eg::silu_mul_rows(ctx, scratch, m, n, out, out_bf16);
    return st;
  }
  const uint32_t tiles_x = (n + 31) / 32;
  const uint64_t tiles_m = (m + kTile - 1) / kTile;
  const int kg = groups_for(ctx, (uint64_t)tiles_x * tiles_m);
  bool xb = false;
  if (norm && !fold_norm(ctx, (uint64_t)tiles_x * tiles_m, norm)) {
    if (!normed) return eg::fail(ctx, EG_ERR_INVALID, "%s: RMSNorm needs a buffer for the normed rows", op);
    xb = ctx->prefill_xb16;
    const int st = eg::rmsnorm_rows(ctx, x, norm, m, k, eps, normed, xb);
    if (st != EG_OK) return st;
    x = normed;
    norm = nullptr;
  }
  PrefillArgs a{x, nullptr, m, k, block_size, k / block_size, k, bits, (uint32_t)__builtin_ctz(block_size), 2u,
                norm, eps, nullptr, nullptr, nullptr, nullptr, 0u, 0u, 0u, out_bf16 ? 1u : 0u, 0u, {}};
  for (int i = 0; i < 2; i++) {
    const PrefillMatrix& w = pair[i];
    a.mats[i] = PrefillMat{w.packed, w.scales, encoding == EG_ENC_SIGNED ? nullptr : w.zeros, w.bias, nullptr,
                           w.out, n, n, 0, tiles_x};
  }
  const dim3 grid(tiles_x, (uint32_t)tiles_m, 1);
  a.xcd_rows = xcd_rows_for(ctx, grid);
  if (norm) launch_chunked<true, true>(encoding, kg, grid, ctx->stream, a);
  else if (xb) launch_chunked<true, false, false, true>(encoding, kg, grid, ctx->stream, a);
  else launch_chunked<true, false>(encoding, kg, grid, ctx->stream, a);
  return eg::check_launch(ctx, op);
}

extern "C" int eg_matmul_q4_prefill_swiglu(eg_context* ctx, const float* x, const uint32_t* gate_packed,
                                           const float* gate_scales, const uint32_t* gate_zeros,
                                           const uint32_t* up_packed, const float* up_scales, const uint32_t* up_zeros,
                                           float* out, float* scratch, const eg_matmul_q4_dims* dims, int encoding,
                                           int bits) {
  const char* op = "matmul_q4_prefill_swiglu";
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!dims || !x || !gate_packed || !gate_scales || !up_packed || !up_scales || !out || !scratch)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  if (dims->use_bias || dims->out_offset != 0 || (dims->m > 1 && dims->out_stride != dims->n))
    return eg::fail(ctx, EG_ERR_INVALID, "%s: no bias, out_stride n and out_offset 0 are required", op);
  if (dims->block_size == 0 || dims->k % dims->block_size != 0 || dims->blocks_per_row != dims->k / dims->block_size)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: k %u, block size %u and blocks per row %u disagree", op, dims->k,
                    dims->block_size, dims->blocks_per_row);
  if (dims->n % 4 != 0 || (reinterpret_cast<uintptr_t>(scratch) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u))
    return eg::fail(ctx, EG_ERR_INVALID, "%s: n %u must be a multiple of 4 and out, scratch 16-byte aligned", op,
                    dims->n);
  const eg::PrefillMatrix gate{gate_packed, gate_scales, gate_zeros, nullptr, nullptr, out, dims->n, dims->n, 0};
  const eg::PrefillMatrix up{up_packed, up_scales, up_zeros, nullptr, nullptr, out, dims->n, dims->n, 0};
  return eg::prefill_gemm_swiglu(ctx, x, dims->m, dims->k, dims->block_size, encoding, bits, gate, up, out, scratch);
}

extern "C" int eg_matmul_q4_prefill(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                                    const uint32_t* zeros, const float* bias, float* out,
                                    const eg_matmul_q4_dims* dims, int encoding, int bits) {
  return eg::prefill_gemm(ctx, x, packed, scales, zeros, bias, nullptr, out, dims, encoding, bits);
}
