// Decode-shape (M=1) quantized GEMV for the projections and the tied LM head.
//
// Reference ops: matmul_q4_decode (matmul_q4_decode.wgsl:56-101) and lm_head_q4/q8
// (embedding_variants.ts:135-180). Same math, same three weight streams, read verbatim:
//   out[row + out_offset] = sum_k x[k] * (code[row,k] - zero[blk]) * scale[blk] (+ bias[row])
//
// MI355X design (not the reference's one-workgroup-per-row tree):
//   * A 16-byte chunk of a row (32 int4 or 16 int8 codes) is the unit of work; a chunk never
//     straddles a quant block because block_size is a multiple of the chunk length on this
//     path, so each chunk needs exactly one scale and one zero-point.
//   * A team of TEAM lanes owns one row; lane t of the team owns chunks t, t+TEAM, ... (CPL of
//     them). The x values those chunks multiply are loaded ONCE into VGPRs and reused for every
//     row the lane visits, so activations cost no memory traffic in the steady state. A wave
//     holds 64/TEAM rows; consecutive lanes read consecutive 16-byte chunks of a row, so each
//     load instruction moves TEAM*16 contiguous bytes per row (128 B at TEAM=8, 1 KiB at 64).
//   * Dequantization is in registers: the word is split into low/high nibble bytes with one
//     opaque AND each, and v_cvt_f32_ubyte0..3 convert each byte straight to f32 - 2.4 VALU
//     ops per int4 weight, below the ~3 ops/byte of issue the HBM rate allows.
//     sum (code - zero) * x * scale is evaluated as scale * (sum code*x - zero * sum x), with
//     sum x per chunk precomputed; two's-complement codes are XORed to offset-binary first.
//   * The row total is a butterfly over the team (fixed order: deterministic); no atomics.
//   * The fused-argmax variant keeps a (value, index) best per lane and reduces it per
//     workgroup; a one-workgroup second launch reduces those partials to the greedy token, so
//     the logits never need a second pass.
#include <algorithm>
#include <cstdlib>
#include <numeric>

#include "eg_internal.hpp"

namespace {

constexpr int kWaves = 4;  // waves per workgroup (256 threads)
constexpr uint32_t kMaxSegments = 256;  // matrices per batched plan (the table lives in LDS)
constexpr uint32_t kMaxCombine = 1024;  // heads x chunks of an attention-combine input stage

// One matrix of a batched launch, as the kernel sees it: its pointers and the range of wave
// passes (RPW rows each) it occupies in the launch's pass space.
struct DevSegment {
  const uint4* w;
  const float* scales;
  const uint32_t* zeros;
  const float* bias;
  float* out;
  uint32_t pass_end;  // exclusive end of this segment's passes (cumulative)
  uint32_t rows;
  uint32_t out_offset;
  uint32_t pad[3];
};
// 64 bytes: the table is copied into LDS with 16-byte loads.
static_assert(sizeof(DevSegment) == 64, "DevSegment is copied as 16-byte vectors");
constexpr uint32_t kTableLoads = kMaxSegments * sizeof(DevSegment) / 16 / 256;  // per thread

struct GemvArgs {
  const float* x;
  const uint4* w;          // code stream viewed as 16-byte chunks, row-major
  const float* scales;
  const uint32_t* zeros;   // offset encoding only
  const float* bias;       // nullable
  float* out;              // nullable in the argmax variant
  uint32_t n;              // rows
  uint32_t chunks;         // 16-byte chunks per row
  uint32_t chunks_per_block;
  uint32_t blocks_per_row;
  uint32_t out_offset;
  uint32_t* partials;      // argmax: (value bits, index) per workgroup
  const DevSegment* segs;  // batched launches only
  uint32_t seg_count;
  uint32_t total_passes;   // tiles over all rows (all segments)
  // input stage (eg_input_kind): how each workgroup produces x in LDS
  int in_kind;
  const float* x2;         // norm weight / up
  float eps;
  uint32_t att_heads, att_kv_heads, att_head_dim, att_chunks;
};

template <int BITS>
struct Codes;

template <>
struct Codes<4> {
  static constexpr int kPerChunk = 32;
  static constexpr uint32_t kSignFlip = 0x88888888u;
  static constexpr int kZeroPerWord = 8;
  // sum over the 32 codes of a chunk of code * x, codes as unsigned nibbles.
  static __device__ __forceinline__ float dot(const uint4& q, const float (&x)[32]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t lo = egd::and_opaque(d[i], 0x0F0F0F0Fu);
      const uint32_t hi = egd::and_opaque(d[i] >> 4, 0x0F0F0F0Fu);
      const float* xv = x + 8 * i;
      a0 = fmaf(egd::ub0(lo), xv[0], a0);
      a1 = fmaf(egd::ub0(hi), xv[1], a1);
      a0 = fmaf(egd::ub1(lo), xv[2], a0);
      a1 = fmaf(egd::ub1(hi), xv[3], a1);
      a0 = fmaf(egd::ub2(lo), xv[4], a0);
      a1 = fmaf(egd::ub2(hi), xv[5], a1);
      a0 = fmaf(egd::ub3(lo), xv[6], a0);
      a1 = fmaf(egd::ub3(hi), xv[7], a1);
    }
    return a0 + a1;
  }
};

template <>
struct Codes<8> {
  static constexpr int kPerChunk = 16;
  static constexpr uint32_t kSignFlip = 0x80808080u;
  static constexpr int kZeroPerWord = 4;
  static __device__ __forceinline__ float dot(const uint4& q, const float (&x)[16]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float* xv = x + 4 * i;
      a0 = fmaf(egd::ub0(d[i]), xv[0], a0);
      a1 = fmaf(egd::ub1(d[i]), xv[1], a1);
      a0 = fmaf(egd::ub2(d[i]), xv[2], a0);
      a1 = fmaf(egd::ub3(d[i]), xv[3], a1);
    }
    return a0 + a1;
  }
};

// kPlain: one matrix, logits/outputs stored. kArgmax: also a per-workgroup (max, index)
// partial. kArgmaxOnly: the partial without storing the outputs. kBatched: a segment table of
// matrices that share x and K.
enum Mode { kPlain = 0, kArgmax = 1, kBatched = 2, kArgmaxOnly = 3 };

template <int BITS, int U, int CPL>
struct Loads {
  egd::u32x4 q[U][CPL];
  float s[U][CPL];
  uint32_t zw[U][CPL];
  float b[U];
};

// The input stage: every workgroup writes the K-element input vector into LDS (xs), from x
// as given or through a fused producer - RMSNorm (the reduction is per workgroup, fixed order,
// so every workgroup computes the same bits), SiLU(gate) * up, or the attention combine.
__device__ __forceinline__ void produce_input(const GemvArgs& a, float* xs, uint32_t n, float* scratch) {
  // Every global read below is a 16-byte vector in a loop the compiler unrolls, so a thread has
  // several loads in flight instead of one round trip per element (the producers read data the
  // previous launch wrote, often from another XCD's L2: each round trip is long).
  const uint32_t tid = threadIdx.x;
  const uint32_t n4 = n / 4;  // n is a multiple of 32
  const float4* x4 = reinterpret_cast<const float4*>(a.x);
  const float4* y4 = reinterpret_cast<const float4*>(a.x2);
  float4* out4 = reinterpret_cast<float4*>(xs);
  if (a.in_kind == EG_INPUT_RMSNORM) {
    __shared__ float red[kWaves];
    float ss = 0.f;
#pragma unroll 4
    for (uint32_t i = tid; i < n4; i += blockDim.x) {
      const float4 v = x4[i];
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((tid & 63u) == 0) red[tid >> 6] = ss;
    __syncthreads();
    float total = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; w++) total += red[w];
    const float inv = 1.0f / sqrtf(total / (float)n + a.eps);
#pragma unroll 4
    for (uint32_t i = tid; i < n4; i += blockDim.x) {
      const float4 v = x4[i], w = y4[i];
      out4[i] = make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w);
    }
  } else if (a.in_kind == EG_INPUT_SILU_MUL) {
#pragma unroll 4
    for (uint32_t i = tid; i < n4; i += blockDim.x) {
      const float4 g = x4[i], u = y4[i];
      out4[i] = make_float4(g.x / (1.0f + expf(-g.x)) * u.x, g.y / (1.0f + expf(-g.y)) * u.y,
                            g.z / (1.0f + expf(-g.z)) * u.z, g.w / (1.0f + expf(-g.w)) * u.w);
    }
  } else if (a.in_kind == EG_INPUT_ATTENTION) {
    // Three phases, none walking the chunks with dependent global loads: every (head, chunk)
    // pair's (max, sum) is loaded once into LDS; each pair's weight e^(m_c - M) / L is formed
    // from LDS; then every output sums its chunks' partial o values (contiguous, read as
    // vectors) with those weights - the same operations in the same order as
    // egd::attention_combine_at.
    const uint32_t heads = a.att_heads, chunks = a.att_chunks, D = a.att_head_dim;
    const uint32_t hcs = heads * chunks;
    const float* m = a.x + (size_t)heads * D * chunks;
    const float* l = m + hcs;
    float* mval = scratch;
    float* lval = scratch + hcs;
    float* wts = scratch + 2 * hcs;
    for (uint32_t hc = tid; hc < hcs; hc += blockDim.x) {
      mval[hc] = m[hc];
      lval[hc] = l[hc];
    }
    __syncthreads();
    for (uint32_t hc = tid; hc < hcs; hc += blockDim.x) {
      const uint32_t b = (hc / chunks) * chunks;
      float M = -INFINITY;
      for (uint32_t c = 0; c < chunks; c++) M = fmaxf(M, mval[b + c]);
      float L = 0.f;
      for (uint32_t c = 0; c < chunks; c++) L = fmaf(lval[b + c], expf(mval[b + c] - M), L);
      wts[hc] = expf(mval[hc] - M) / L;
    }
    __syncthreads();
    const uint32_t c4 = chunks / 4;
    for (uint32_t i = tid; i < n; i += blockDim.x) {
      const float* o = a.x + (size_t)i * chunks;
      const float* w = wts + (i / D) * chunks;
      float acc = 0.f;
      if ((chunks & 3u) == 0) {
        const float4* o4 = reinterpret_cast<const float4*>(o);
#pragma unroll 8
        for (uint32_t q = 0; q < c4; q++) {
          const float4 v = o4[q];
          acc = fmaf(v.x, w[4 * q + 0], acc);
          acc = fmaf(v.y, w[4 * q + 1], acc);
          acc = fmaf(v.z, w[4 * q + 2], acc);
          acc = fmaf(v.w, w[4 * q + 3], acc);
        }
      } else {
        for (uint32_t c = 0; c < chunks; c++) acc = fmaf(o[c], w[c], acc);
      }
      xs[i] = acc;
    }
  } else {
    // x as given: every load issued before any LDS write (8 per thread covers the longest
    // rows, 256 chunks of 32 codes); reads past x return zeros without touching memory.
    constexpr uint32_t kMaxLoads = 256 * 32 / 4 / 256;
    const auto src = egd::buffer(a.x, n4 * 16u);
    egd::u32x4 v[kMaxLoads];
#pragma unroll
    for (uint32_t r = 0; r < kMaxLoads; r++) v[r] = egd::load_b128(src, (tid + r * 256u) * 16u);
    egd::u32x4* dst = reinterpret_cast<egd::u32x4*>(xs);
#pragma unroll
    for (uint32_t r = 0; r < kMaxLoads; r++)
      if (tid + r * 256u < n4) dst[tid + r * 256u] = v[r];
  }
}

// One wave computes a tile of RPW * U rows per step: RPW teams of TEAM lanes side by side,
// each team owning U rows (spaced RPW apart so that, for every (u, j), the wave's load is RPW
// consecutive rows x TEAM consecutive 16-byte chunks).
//
// Each wave owns a contiguous range of tiles (so a batched launch looks its segment up once,
// not per tile) and walks it NB tiles at a time with NB load buffers: the loads of tiles
// i+1 .. i+NB-1 are in flight while tile i is computed. The bytes a CU keeps in flight are
// what bounds a streaming kernel's bandwidth (latency x rate), and they cost VGPRs: x takes
// CPL * EPC per lane, each buffer U * (5 * CPL + 1) more, so long rows (large x) trade
// resident waves for a deeper pipeline per wave.
// The steady-state loop has no memory operation under a branch, which lets the compiler wait
// for exactly the tile it is about to use:
//   * loads are unconditional - out-of-range rows read the last row, out-of-range chunk slots
//     read chunk 0 (x is zero there), and a wave whose count is not a multiple of NB re-reads
//     its last tile (an L2 hit) instead of branching around the spare buffers;
//   * stores are unconditional - the team total is in every lane of the team, every lane
//     stores it, and a clamped or repeated row stores the value that row already has.
template <int BITS, int ENC, int TEAM, int CPL, int U, int NB, int MODE>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  using C = Codes<BITS>;
  constexpr int EPC = C::kPerChunk;
  constexpr int RPW = 64 / TEAM;
  constexpr int TILE = RPW * U;
  constexpr bool kStore = MODE != kArgmaxOnly;
  constexpr bool kBest = MODE == kArgmax || MODE == kArgmaxOnly;
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t t = lane % TEAM;
  const uint32_t slot = lane / TEAM;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(blockIdx.x * kWaves + (threadIdx.x >> 6));
  const uint32_t total_waves = gridDim.x * kWaves;

  // Dynamic LDS: x (chunks * EPC floats), then (batched) the segment table. The workgroup
  // copies x in once, so the activations cross L2 once per workgroup rather than once per
  // wave; each lane then keeps the chunks it owns in VGPRs for every row it visits.
  extern __shared__ __align__(16) uint8_t smem[];
  const uint32_t x_words = a.chunks * EPC;
  DevSegment* table = reinterpret_cast<DevSegment*>(smem + x_words * 4u);
  float* scratch = reinterpret_cast<float*>(smem + x_words * 4u + (MODE == kBatched ? a.seg_count : 0u) *
                                                                      (uint32_t)sizeof(DevSegment));
  // The segment table's loads are all issued up front (kTableLoads per thread at most, reads
  // past the table return zeros), so copying it costs one L2 round trip that overlaps the
  // input stage's, not one per element.
  egd::u32x4 tv[MODE == kBatched ? kTableLoads : 1];
  const uint32_t table_vecs = a.seg_count * (uint32_t)(sizeof(DevSegment) / 16);
  if (MODE == kBatched) {
    const auto src = egd::buffer(a.segs, table_vecs * 16u);
#pragma unroll
    for (uint32_t r = 0; r < kTableLoads; r++) tv[r] = egd::load_b128(src, (threadIdx.x + r * 256u) * 16u);
  }
  produce_input(a, reinterpret_cast<float*>(smem), x_words, scratch);
  if (MODE == kBatched) {
    egd::u32x4* dst = reinterpret_cast<egd::u32x4*>(table);
#pragma unroll
    for (uint32_t r = 0; r < kTableLoads; r++)
      if (threadIdx.x + r * 256u < table_vecs) dst[threadIdx.x + r * 256u] = tv[r];
  }
  __syncthreads();

  // This lane's activations: chunk slot j covers x[c*EPC, c*EPC + EPC).
  float xr[CPL][EPC];
  float sx[CPL];
  uint32_t cj[CPL], bj[CPL];
#pragma unroll
  for (int j = 0; j < CPL; j++) {
    const uint32_t c = t + j * TEAM;
    const bool valid = c < a.chunks;
    cj[j] = valid ? c : 0u;
    bj[j] = cj[j] / a.chunks_per_block;
    sx[j] = 0.f;
    const egd::u32x4* xs = reinterpret_cast<const egd::u32x4*>(smem) + (size_t)cj[j] * (EPC / 4);
#pragma unroll
    for (int e = 0; e < EPC / 4; e++) {
      const egd::u32x4 v = xs[e];
      xr[j][4 * e + 0] = valid ? __uint_as_float(v.x) : 0.f;
      xr[j][4 * e + 1] = valid ? __uint_as_float(v.y) : 0.f;
      xr[j][4 * e + 2] = valid ? __uint_as_float(v.z) : 0.f;
      xr[j][4 * e + 3] = valid ? __uint_as_float(v.w) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < EPC; e++) sx[j] += xr[j][e];
  }

  // Byte offsets of this lane's loads relative to its tile's first row: constant for the whole
  // launch. The tile's own offset is wave-uniform and rides in the buffer instruction's scalar
  // offset, so walking tiles costs scalar adds, not per-lane address arithmetic.
  uint32_t qoff[U][CPL], soff[U][CPL], roff[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t lrow = u * RPW + slot;
    roff[u] = lrow * 4u;
#pragma unroll
    for (int j = 0; j < CPL; j++) {
      qoff[u][j] = (lrow * a.chunks + cj[j]) * 16u;
      soff[u][j] = (lrow * a.blocks_per_row + bj[j]) * 4u;
    }
  }

  // This wave's tiles: [begin, end), contiguous. (readfirstlane: the 64-bit divisions run on
  // the vector unit, and the tile offsets derived from these must be known wave-uniform.)
  const uint32_t begin =
      __builtin_amdgcn_readfirstlane((uint32_t)(((uint64_t)a.total_passes * wave) / total_waves));
  const uint32_t end =
      __builtin_amdgcn_readfirstlane((uint32_t)(((uint64_t)a.total_passes * (wave + 1)) / total_waves));

  // The matrix the issue side is walking (one for a plain launch; the current segment of a
  // batched one). Rows are a multiple of TILE in a batched plan; a plain launch's last partial
  // tile is shifted back to end at the last row (rows >= TILE), recomputing a few rows with
  // identical results, so every access stays inside its stream.
  struct Seg {
    __amdgpu_buffer_rsrc_t w, s, z, b, o;
    uint32_t rows, out_offset, first, end, has_bias;
  };
  auto make_seg = [&](const uint4* w, const float* scales, const uint32_t* zeros, const float* bias, float* out,
                      uint32_t rows, uint32_t out_offset, uint32_t first, uint32_t seg_end) {
    const uint32_t blocks = rows * a.blocks_per_row;
    Seg r;
    r.w = egd::buffer(w, rows * a.chunks * 16u);
    r.s = egd::buffer(scales, blocks * 4u);
    r.z = egd::buffer(zeros, ((blocks + C::kZeroPerWord - 1) / C::kZeroPerWord) * 4u);
    r.has_bias = bias != nullptr;
    // Without a bias the (discarded) bias load reads the scale stream, which has >= 1 entry per row.
    r.b = r.has_bias ? egd::buffer(bias, rows * 4u) : r.s;
    r.o = egd::buffer(out, (out_offset + rows) * 4u);
    r.rows = rows;
    r.out_offset = out_offset;
    r.first = first;
    r.end = seg_end;
    return r;
  };

  // Batched: a segment is read from the LDS table into scalar registers (an LDS read waits on
  // lgkmcnt, so switching segments never waits for the tile loads in flight, as a global load
  // of the table would).
  Seg cur = make_seg(a.w, a.scales, a.zeros, a.bias, a.out, a.n, a.out_offset, 0, a.total_passes);
  uint32_t seg = 0;
  auto load_segment = [&](uint32_t sidx) {
    const DevSegment& d = table[sidx];
    const uint32_t rows = __builtin_amdgcn_readfirstlane(d.rows);
    const uint32_t seg_end = __builtin_amdgcn_readfirstlane(d.pass_end);
    cur = make_seg(egd::uniform(d.w), egd::uniform(d.scales), egd::uniform(d.zeros), egd::uniform(d.bias),
                   egd::uniform(d.out), rows, __builtin_amdgcn_readfirstlane(d.out_offset), seg_end - rows / TILE,
                   seg_end);
  };
  if (MODE == kBatched && begin < end) {
    // The first segment whose pass_end exceeds `begin` = the number of segments ending at or
    // before it (pass_end increases): 64 entries per LDS read, counted with a ballot.
    uint32_t count = 0;
    for (uint32_t e0 = 0; e0 < a.seg_count; e0 += 64) {
      const uint32_t e = e0 + lane;
      const bool done = e < a.seg_count && table[e < a.seg_count ? e : 0].pass_end <= begin;
      count += (uint32_t)__builtin_popcountll(__builtin_amdgcn_ballot_w64(done));
    }
    seg = __builtin_amdgcn_readfirstlane(count);
    load_segment(seg);
  }

  // What computing a tile needs once its loads are in flight: where its rows are stored.
  struct Pending {
    __amdgpu_buffer_rsrc_t o;
    uint32_t row0, out_offset, has_bias;
  };
  const uint32_t last = end - 1;

  // Issues the loads of tile `tl` (clamped to the wave's last tile; tiles are visited in
  // increasing order, so the segment cursor only moves forward).
  auto issue = [&](uint32_t tl, Loads<BITS, U, CPL>& L, Pending& P) {
    tl = min(tl, last);
    if (MODE == kBatched)
      while (tl >= cur.end) load_segment(++seg);
    // (readfirstlane pins the value to a scalar register: a scalar offset left in a vector
    // register would make the compiler wrap every load in a per-lane loop.)
    const uint32_t row0 = __builtin_amdgcn_readfirstlane(min((tl - cur.first) * TILE, cur.rows - TILE));
    const uint32_t sq = row0 * (a.chunks * 16u);
    const uint32_t ss = row0 * (a.blocks_per_row * 4u);
#pragma unroll
    for (int u = 0; u < U; u++) {
      L.b[u] = egd::load_f32(cur.b, roff[u], row0 * 4u);
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        L.q[u][j] = egd::load_b128_nt(cur.w, qoff[u][j], sq);
        L.s[u][j] = egd::load_f32_nt(cur.s, soff[u][j], ss);
        if (ENC == EG_ENC_OFFSET_ZEROS) {
          const uint32_t blk = (row0 + u * RPW + slot) * a.blocks_per_row + bj[j];
          L.zw[u][j] = egd::load_b32(cur.z, (blk / C::kZeroPerWord) * 4u);
        }
      }
    }
    P.o = cur.o;
    P.row0 = row0;
    P.out_offset = cur.out_offset;
    P.has_bias = cur.has_bias;
  };

  float best_v = -1.0e30f;
  uint32_t best_i = a.out_offset;

  auto compute = [&](const Loads<BITS, U, CPL>& L, const Pending& P) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      // The bias starts lane 0's partial (linearQ4 starts its sum from the bias too).
      float acc = (t == 0 && P.has_bias) ? L.b[u] : 0.f;
      const uint32_t row = P.row0 + u * RPW + slot;
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        uint4 q = make_uint4(L.q[u][j].x, L.q[u][j].y, L.q[u][j].z, L.q[u][j].w);
        float z;
        if (ENC == EG_ENC_OFFSET_ZEROS) {
          const uint32_t blk = row * a.blocks_per_row + bj[j];
          z = (float)((L.zw[u][j] >> (BITS * (blk % C::kZeroPerWord))) & ((1u << BITS) - 1u));
        } else {
          q.x ^= C::kSignFlip;
          q.y ^= C::kSignFlip;
          q.z ^= C::kSignFlip;
          q.w ^= C::kSignFlip;
          z = (float)(1 << (BITS - 1));
        }
        acc = fmaf(L.s[u][j], C::dot(q, xr[j]) - z * sx[j], acc);
      }
      const float v = egd::team_allsum<TEAM>(acc);
      if (kStore) egd::store_f32(P.o, roff[u], v, (P.row0 + P.out_offset) * 4u);
      if (kBest) {
        const uint32_t idx = row + P.out_offset;
        const bool take = egd::better(v, idx, best_v, best_i);
        best_v = take ? v : best_v;
        best_i = take ? idx : best_i;
      }
    }
  };

  // The wave's range is one software pipeline over NB load buffers, NB tiles per iteration,
  // with a single exit at the bottom: while tile i is computed, the loads of tiles
  // i+1 .. i+NB-1 are in flight. Each buffer carries where its rows go, so the pipeline runs
  // straight through segment boundaries (a boundary costs a few scalar LDS reads, not a drain
  // of the loads in flight). A count that is not a multiple of NB computes the wave's last
  // tile again (same loads, same stores) rather than leaving the loop mid-body. With no path
  // leaving the loop between an issue and its consumer, the compiler's wait counts stay exact -
  // computing a tile waits only for that tile's loads, never for a later tile's.
  // sched_barrier(0) after each issue keeps the scheduler from sinking the next tile's loads
  // into the current tile's math.
  if (begin < end) {
    Loads<BITS, U, CPL> L[NB];
    Pending P[NB];
    uint32_t tile = begin;
    const uint32_t groups = (end - begin + NB - 1) / NB;
#pragma unroll
    for (int b = 0; b + 1 < NB; b++) issue(tile + b, L[b], P[b]);
    for (uint32_t g = 0; g < groups; g++) {
#pragma unroll
      for (int b = 0; b < NB; b++) {
        const int nx = (b + NB - 1) % NB;
        issue(tile + b + NB - 1, L[nx], P[nx]);
        __builtin_amdgcn_sched_barrier(0);
        compute(L[b], P[b]);
      }
      tile += NB;
    }
    // The last NB-1 issues are duplicates that nothing consumes; they complete before the
    // wave ends.
    __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt 0, expcnt 7, lgkmcnt 15
  }

  if (kBest) {
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
      for (int k = 1; k < kWaves; k++)
        if (egd::better(wv[k], wi[k], bv, bi)) {
          bv = wv[k];
          bi = wi[k];
        }
      a.partials[2 * blockIdx.x + 0] = __float_as_uint(bv);
      a.partials[2 * blockIdx.x + 1] = bi;
    }
  }
}

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

using KernelFn = void (*)(GemvArgs);

// Instantiated (TEAM, CPL, U, NB) shapes: one chunk slot per lane for rows of up to 64 chunks
// (TEAM the next power of two), a full-wave team with 2-4 slots for longer rows. The library
// picks NB = 2 (measured fastest on MI355X: a deeper pipeline costs resident waves and
// duplicate tail tiles); NB 3-4 variants of the main shapes stay selectable through
// EG_GEMV_SHAPE for tuning.
#define EG_SHAPES(X)                                                                                      \
  X(8, 1, 1, 2) X(8, 1, 2, 2) X(8, 1, 4, 2) X(16, 1, 1, 2) X(16, 1, 2, 2) X(16, 1, 4, 2) X(32, 1, 1, 2)    \
  X(32, 1, 2, 2) X(32, 1, 2, 3) X(32, 1, 2, 4) X(32, 1, 4, 2) X(64, 1, 1, 2) X(64, 1, 2, 2) X(64, 1, 4, 2) \
  X(64, 1, 4, 3) X(64, 2, 1, 2) X(64, 2, 2, 2) X(64, 3, 1, 2) X(64, 3, 1, 3) X(64, 3, 1, 4) X(64, 3, 2, 2) \
  X(64, 4, 1, 2)

template <int BITS, int ENC, int MODE>
KernelFn pick(int team, int cpl, int u, int nb) {
#define EG_CASE(T, P, UU, D) \
  if (team == T && cpl == P && u == UU && nb == D) return gemv_kernel<BITS, ENC, T, P, UU, D, MODE>;
  EG_SHAPES(EG_CASE)
#undef EG_CASE
  return nullptr;
}

template <int BITS, int ENC>
KernelFn pick_mode(int mode, int team, int cpl, int u, int nb) {
  if (mode == kArgmax) return pick<BITS, ENC, kArgmax>(team, cpl, u, nb);
  if (mode == kArgmaxOnly) return pick<BITS, ENC, kArgmaxOnly>(team, cpl, u, nb);
  if (mode == kBatched) return pick<BITS, ENC, kBatched>(team, cpl, u, nb);
  return pick<BITS, ENC, kPlain>(team, cpl, u, nb);
}

KernelFn pick_kernel(int bits, int enc, int mode, int team, int cpl, int u, int nb) {
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
// A fused input stage is recomputed by every workgroup, so those launches give each wave
// `tiles_per_wave` tiles to amortise it (fewer, longer-lived workgroups).
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
    sh.u = sh.team == 64 ? 4 : 2;  // measured on MI355X: int8 rows of 56 chunks / int4 rows of 28
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
};

// LDS the input stage needs beyond x and the segment table.
uint32_t input_scratch_bytes(const GemvArgs& a) {
  return a.in_kind == EG_INPUT_ATTENTION ? 3u * a.att_heads * a.att_chunks * 4u : 0u;
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
      if ((uint64_t)d.heads * (d.max_context / d.chunk) > kMaxCombine)
        return eg::fail(ctx, EG_ERR_RANGE, "%s: %u heads x %u chunks exceed the combine stage's %u", op, d.heads,
                        d.max_context / d.chunk, kMaxCombine);
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

int launch(eg_context* ctx, const QuantView& v) {
  int st = validate(ctx, v);
  if (st != EG_OK) return st;
  if (v.n == 0) {
    if (v.result) return eg::fail(ctx, EG_ERR_INVALID, "%s: argmax over zero rows", v.op);
    return EG_OK;
  }
  const bool argmax = v.result != nullptr;
  const uint32_t epc = 128u / v.bits;
  const bool fused = v.input && v.input->kind != EG_INPUT_VECTOR;
  const bool aligned = (reinterpret_cast<uintptr_t>(v.packed) & 15u) == 0 &&
                       (fused || (reinterpret_cast<uintptr_t>(v.x) & 15u) == 0);
  const uint32_t chunks = v.k / epc;
  Shape shape;
  if (aligned && v.k % epc == 0 && v.block_size % epc == 0)
    shape = choose_shape(v.n, chunks, ctx);
  uint32_t* partials = reinterpret_cast<uint32_t*>(eg::partials(ctx));
  uint32_t grid = 0;
  const int mode = argmax ? (v.out ? kArgmax : kArgmaxOnly) : kPlain;
  KernelFn fn = shape.team ? pick_kernel(v.bits, v.encoding, mode, shape.team, shape.cpl, shape.u, shape.nb) : nullptr;
  if (fused && !fn)
    return eg::fail(ctx, EG_ERR_INVALID, "%s: a fused input stage needs k and the block a multiple of %u", v.op, epc);
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
    const uint32_t smem = chunks * epc * 4u + input_scratch_bytes(a);
    grid = grid_for(ctx, fn, shape.tiles, smem, a.in_kind != EG_INPUT_VECTOR ? ctx->fused_tiles_per_wave : 1);
    hipLaunchKernelGGL(fn, dim3(grid), dim3(256), smem, ctx->stream, a);
  } else {
    uint64_t blocks = (v.n + kWaves - 1) / kWaves;
    const uint64_t cap = (uint64_t)ctx->cu_count * 8;
    if (blocks > cap) blocks = cap;
    grid = (uint32_t)blocks;
    if (argmax)
      hipLaunchKernelGGL(gemv_generic_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, v.x,
                         v.packed, v.scales, v.zeros, v.bias, v.out, v.n, v.k, v.block_size, v.blocks_per_row,
                         v.out_offset, v.bits, v.encoding, partials);
    else
      hipLaunchKernelGGL(gemv_generic_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, ctx->stream, v.x,
                         v.packed, v.scales, v.zeros, v.bias, v.out, v.n, v.k, v.block_size, v.blocks_per_row,
                         v.out_offset, v.bits, v.encoding, partials);
  }
  if (argmax) eg::launch_argmax_finalize(ctx, partials, grid, v.out_offset, v.result);
  return eg::check_launch(ctx, v.op);
}

}  // namespace

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
  if (ctx) {
    const uint64_t max_groups = eg::kPartialsBytes / 8;
    if ((uint64_t)ctx->cu_count * 8 > max_groups)
      return eg::fail(ctx, EG_ERR_RANGE, "lm_head_argmax: workspace too small for the grid");
  }
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
  return launch(ctx, v);
}

}  // extern "C"

// ---- batched plans ------------------------------------------------------------------------

struct eg_gemv_plan {
  DevSegment* table = nullptr;  // device copy
  uint32_t count = 0;
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
  hipError_t err = hipMalloc(&plan->table, sizeof(DevSegment) * count);
  if (err == hipSuccess) err = hipMemcpy(plan->table, host, sizeof(DevSegment) * count, hipMemcpyHostToDevice);
  delete[] host;
  if (err != hipSuccess) {
    if (plan->table) hipFree(plan->table);
    delete plan;
    return eg::hip_fail(ctx, err, "gemv_plan_create");
  }
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
  plan->smem = k * 4u + count * (uint32_t)sizeof(DevSegment);
  plan->grid = fn ? grid_for(ctx, fn, pass, plan->smem) : 0;
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
  a.seg_count = plan->count;
  a.total_passes = plan->total_passes;
  KernelFn fn = pick_kernel(plan->bits, plan->encoding, kBatched, plan->team, plan->cpl, plan->u, plan->nb);
  if (!fn) return eg::fail(ctx, EG_ERR_INVALID, "gemv_plan_launch: no kernel for this plan's shape");
  const uint32_t extra = input_scratch_bytes(a);
  const uint32_t grid = a.in_kind != EG_INPUT_VECTOR
                            ? grid_for(ctx, fn, plan->total_passes, plan->smem + extra, ctx->fused_tiles_per_wave)
                            : plan->grid;
  hipLaunchKernelGGL(fn, dim3(grid), dim3(256), plan->smem + extra, ctx->stream, a);
  return eg::check_launch(ctx, "gemv_plan_launch");
}

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
