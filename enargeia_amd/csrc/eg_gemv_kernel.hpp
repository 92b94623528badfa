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
//   * Dequantization is in registers: the word is split into low and high nibble bytes in
//     place (one masked flip each - a single v_bitop3 - the high nibbles left unshifted and
//     their x values pre-divided by 16), and v_cvt_f32_ubyte0..3 convert each byte straight to
//     f32: about 2.1 VALU ops per int4 weight. The VALU issue rate and the HBM rate are close
//     on this path (16 lane-ops per clock per SIMD against ~3.3 bytes), so every op counts.
//     sum (code - zero) * x * scale is evaluated as scale * (sum code*x - zero * sum x), with
//     sum x per chunk precomputed; two's-complement codes are flipped to offset binary.
//   * The row total is a butterfly over the team (fixed order: deterministic); no atomics.
//   * The fused-argmax variant keeps a (value, index) best per lane and reduces it per
//     workgroup; a one-workgroup second launch reduces those partials to the greedy token, so
//     the logits never need a second pass.
//
// This header holds the kernel template; eg_gemv.hip instantiates it for inputs given as a
// vector (and holds the host side); eg_gemv_rmsnorm.hip, eg_gemv_silu.hip and
// eg_gemv_attention.hip instantiate it for the fused input stages.
#pragma once

#include <algorithm>
#include <type_traits>
#include <cstdlib>
#include <numeric>

#include "eg_internal.hpp"

namespace eg_gemv {

constexpr int kWaves = 4;  // waves per workgroup (256 threads)
constexpr uint32_t kMaxSegments = 256;  // matrices per batched plan
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
// 64 bytes: one entry is one 16-dword scalar load.
static_assert(sizeof(DevSegment) == 64, "DevSegment is read as 16 dwords");
// Plans of up to this many matrices carry their table in the kernel arguments, so a wave knows
// its first segment with no memory round trip (the decoder's q|k|v and gate|up plans are 3 and
// 2 matrices); larger tables stay in global memory and are read with scalar loads. Three, not
// more: the argument block's size shows in the decode step (its 97 GEMV launches a token ran
// 0.3% faster at three entries than at four, and ~1% slower with 48 bytes more; MI355X).
constexpr uint32_t kInlineSegments = 3;

// kSampleStats: the sampling parameters - from device memory (sample_dev, the 32-byte sample
// dims, so a captured graph replays with new values) or, when that is NULL, the values here - the
// history the penalty reads, and words workgroup 0 zeroes (clear[0, clear_words), nullable).
struct SampleStatsArgs {
  const eg_sample_dims* sample_dev;
  const uint32_t* history;
  uint32_t* clear;
  float temperature, repetition_penalty;
  uint32_t history_length, clear_words;
};

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
  union {
    DevSegment inline_segs[kInlineSegments];  // the table itself when seg_count <= kInlineSegments
    // kSampleStats launches, never batched, keep their arguments in the table's place, so no
    // launch's argument block grows for them
    SampleStatsArgs stats;
  };
  const uint32_t* seg_index;  // seg_count > kInlineSegments: the segment of each pass, 16 bits per pass
  uint32_t total_passes;   // tiles over all rows (all segments)
  // input stage (eg_input_kind): how each workgroup produces x in LDS
  int in_kind;
  uint32_t any_bias;       // some matrix of the launch has a bias (informational)
  const float* x2;         // norm weight / up
  float eps;
  uint32_t att_heads, att_kv_heads, att_head_dim, att_chunks;
  uint64_t* stamp;         // launch stamps (egd::WaveStamp), nullable
};

template <int BITS>
struct Codes;

// Dot products of one 16-byte chunk of codes with the lane's x values, the encoding handled
// inside: two's-complement codes are flipped to offset binary (value + 2^(BITS-1)) on the way.
//
// The codes enter the products as binary16 subnormals: a code masked in place into the low ten
// bits of a 16-bit half reads, as an f16, as code * 2^-24 exactly (a nibble in bits 4-7 as
// 16 * code * 2^-24), and v_fma_mix_f32 multiplies that half by an f32 x and adds an f32
// accumulator - one instruction per weight where a byte convert and an FMA took two. x is
// pre-scaled by the inverse power of two (x_scale), so every product is exactly code * x and the
// sums are those of float(code) * x in the same order, bit for bit. Needs f16 subnormals kept
// (the kernels' default float mode: .amdhsa_float_denorm_mode_16_64 3). Measured on MI355X
// against the convert + FMA form: outputs bitwise equal, the config-1 batched launches 28.1 ->
// 27.6 us (K = 896) and 14.3 -> 13.9 us (K = 4864) - they are bound by the loads in flight
// more than by the VALU.
using half2v = _Float16 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ half2v as_halves(uint32_t v) { return __builtin_bit_cast(half2v, v); }

template <>
struct Codes<4> {
  static constexpr int kPerChunk = 32;
  static constexpr int kZeroPerWord = 8;
  // x as the dot expects it: times 2^24 for the low nibble of each byte (even elements), times
  // 2^20 for the high nibble (odd elements, whose codes read as 16 * code * 2^-24).
  static __device__ __forceinline__ float x_scale(int e) { return (e & 1) ? 1048576.0f : 16777216.0f; }
  // sum over the 32 codes of (unsigned code) * x. Per word: one shift, four masked halves (the
  // signed flip folded in: v_bitop3 on gfx950), eight fma_mix - about 1.6 VALU ops per weight.
  template <int ENC>
  static __device__ __forceinline__ float dot(const uint4& q, const float (&x)[32]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t d8 = d[i] >> 8;
      // m0: elements 0 | 4 (low nibbles of bytes 0 | 2), m1: 1 | 5 (their high nibbles),
      // m2: 2 | 6 (low nibbles of bytes 1 | 3), m3: 3 | 7
      uint32_t m0 = d[i] & 0x000F000Fu, m1 = d[i] & 0x00F000F0u, m2 = d8 & 0x000F000Fu, m3 = d8 & 0x00F000F0u;
      if (ENC == EG_ENC_SIGNED) {
        m0 ^= 0x00080008u;
        m1 ^= 0x00800080u;
        m2 ^= 0x00080008u;
        m3 ^= 0x00800080u;
      }
      const half2v c0 = as_halves(m0), c1 = as_halves(m1), c2 = as_halves(m2), c3 = as_halves(m3);
      const float* xv = x + 8 * i;
      a0 = fmaf((float)c0.x, xv[0], a0);
      a1 = fmaf((float)c1.x, xv[1], a1);
      a0 = fmaf((float)c2.x, xv[2], a0);
      a1 = fmaf((float)c3.x, xv[3], a1);
      a0 = fmaf((float)c0.y, xv[4], a0);
      a1 = fmaf((float)c1.y, xv[5], a1);
      a0 = fmaf((float)c2.y, xv[6], a0);
      a1 = fmaf((float)c3.y, xv[7], a1);
    }
    return a0 + a1;
  }
};

template <>
struct Codes<8> {
  static constexpr int kPerChunk = 16;
  static constexpr int kZeroPerWord = 4;
  // x times 2^24: every byte reads as code * 2^-24
  static __device__ __forceinline__ float x_scale(int) { return 16777216.0f; }
  template <int ENC>
  static __device__ __forceinline__ float dot(const uint4& q, const float (&x)[16]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      // m0: bytes 0 | 2, m1: bytes 1 | 3
      uint32_t m0 = d[i] & 0x00FF00FFu, m1 = (d[i] >> 8) & 0x00FF00FFu;
      if (ENC == EG_ENC_SIGNED) {
        m0 ^= 0x00800080u;
        m1 ^= 0x00800080u;
      }
      const half2v c0 = as_halves(m0), c1 = as_halves(m1);
      const float* xv = x + 4 * i;
      a0 = fmaf((float)c0.x, xv[0], a0);
      a1 = fmaf((float)c1.x, xv[1], a1);
      a0 = fmaf((float)c0.y, xv[2], a0);
      a1 = fmaf((float)c1.y, xv[3], a1);
    }
    return a0 + a1;
  }
};

// kPlain: one matrix, logits/outputs stored. kArgmax: also a per-workgroup (max, index)
// partial. kArgmaxOnly: the partial without storing the outputs. kBatched: a segment table of
// matrices that share x and K. kSwiGLU: two matrices of equal shape (gate, up; the argument
// table's first two entries) whose row r is computed by the same team, which stores
// silu(gate_r) * up_r (ops.ts:207-216) - so the SiLU is evaluated once per row, in the
// producer, instead of by every workgroup of the down projection's input stage. kSampleStats:
// the LM head ahead of the sampler (sample.wgsl:143-236 up to its normaliser) - each row's logit
// penalized (once per distinct history id: v > 0 ? v / penalty : v * penalty) and stored, and a
// per-workgroup partial (max of l/T, its lowest index, sum of exp(l/T - that max) in float64;
// l itself and no sum at temperature <= 0) in place of the sampler's per-slice pass.
enum Mode { kPlain = 0, kArgmax = 1, kBatched = 2, kArgmaxOnly = 3, kSwiGLU = 4, kSampleStats = 5 };

// kSampleStats: rows of a workgroup's record (one per thread of the epilogue; the host sizes the
// grid so that every workgroup's rows fit), and the dynamic LDS the mode adds after x: the record,
// the history bitmap, and the epilogue's (value, index) and float64 slots per wave. (In dynamic
// LDS rather than __shared__ arrays: any static LDS makes the compiler plan these kernels for
// fewer waves, and the int8 head took 99 VGPRs instead of 75.)
constexpr uint32_t kStatsRows = 256;
constexpr uint32_t kStatsLdsBytes = kStatsRows * 4 + kStatsRows / 32 * 4 + 4 * 8 + 4 * 8;

template <int BITS, int U, int CPL>
struct Loads {
  egd::u32x4 q[U][CPL];
  float s[U][CPL];
  uint32_t zw[U][CPL];
  float b;  // lane t < U of a team: the bias of the team's row t
};

// How a GEMV body runs. LaunchEnv: as its own launch - its grid, nothing to wait for, default
// cache policy. The persistent decode kernel (eg_layers.hip) runs the same body as one phase of a
// longer launch with an environment of its own: a virtual grid (the phase's workgroups), a wait
// for the phase's inputs (called once the first tiles' weights are in flight), and coherent
// accesses (kAux = egd::kCoherent) to everything another workgroup of the launch writes or reads -
// the input vector, the residual bias, the outputs.
struct LaunchEnv {
  static constexpr int kAux = 0;
  static constexpr bool kPhase = false;
  __device__ __forceinline__ uint32_t block() const { return blockIdx.x; }
  __device__ __forceinline__ uint32_t blocks() const { return gridDim.x; }
  __device__ __forceinline__ void wait() const {}
};

// Where float4 i of x (P float4 per 16-byte chunk of codes: 8 for int4, 4 for int8) sits in LDS:
// chunk-transposed, piece e of every chunk side by side (x_slot = e * chunks + chunk). A lane
// reads its chunk's pieces in order, so at each read the lanes of a team touch consecutive 16-byte
// slots - no bank conflicts - where a row-major x would put every lane 128 (int4) or 64 (int8)
// bytes apart, on the same banks.
template <int P>
__device__ __forceinline__ uint32_t x_slot(uint32_t i, uint32_t chunks) {
  return (i % P) * chunks + i / P;
}

// The input stage: every workgroup writes the K-element input vector into LDS (xs), from x
// as given or through a fused producer - RMSNorm (the reduction is per workgroup, fixed order,
// so every workgroup computes the same bits), SiLU(gate) * up, or the attention combine. IN
// selects the stage at compile time, so each kernel carries only its own stage's registers.
//
// Each stage makes ONE round trip to memory in the common case: every global read it needs is
// issued before any of them is used (16-byte buffer loads into registers; reads past the end
// of a stream return zeros without touching memory), because the producers read what the
// previous launch wrote, from L2 or beyond, and a chain of dependent round trips is what a
// small launch's duration is made of. Inputs longer than a stage's register batch take a
// second, looped pass for the remainder.
// `early` runs right after the stage has issued its loads and before it uses any of them: the
// kernel issues its first tiles' weight loads there, so the weights are in flight while the
// stage waits for its own reads and computes. (A wave's reads complete in issue order, so the
// stage still waits only for its own loads; a workgroup barrier does not wait for reads.)
// Env::kAux is the cache policy of the reads of x (and of the attention partials), which a phase
// of the persistent kernel reads after another workgroup wrote them.
template <int IN, int P, class Env, typename Early>
__device__ __forceinline__ void produce_input(const GemvArgs& a, float* xs, uint32_t n, float* scratch,
                                              Early&& early) {
  constexpr int AUX = Env::kAux;
  const uint32_t tid = threadIdx.x;
  const uint32_t n4 = n / 4;  // n is a multiple of 32
  // x goes into LDS chunk-transposed (see x_slot): float4 i of x at x_slot(i)
  float4* xs4 = reinterpret_cast<float4*>(xs);
  const uint32_t xchunks = n4 / P;  // 16-byte chunks of codes per row
  auto put4 = [&](uint32_t i, const float4& v) { xs4[x_slot<P>(i, xchunks)] = v; };
  auto f4 = [](const egd::u32x4& v) {
    return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  };
  if (IN == EG_INPUT_RMSNORM) {
    // x and the norm weight for up to kVec * 1024 inputs in one batch
    constexpr uint32_t kVec = 2;
    const auto xb = egd::buffer(a.x, n4 * 16u), wb = egd::buffer(a.x2, n4 * 16u);
    egd::u32x4 xv[kVec], wv[kVec];
#pragma unroll
    for (uint32_t r = 0; r < kVec; r++) {
      xv[r] = egd::load_b128_p<AUX>(xb, (tid + r * 256u) * 16u);
      wv[r] = egd::load_b128(wb, (tid + r * 256u) * 16u);
    }
    early();
    __shared__ float red[kWaves];
    float ss = 0.f;
#pragma unroll
    for (uint32_t r = 0; r < kVec; r++) {
      const float4 v = f4(xv[r]);
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
    for (uint32_t i = tid + kVec * 256u; i < n4; i += blockDim.x) {
      const float4 v = f4(egd::load_b128_p<AUX>(xb, i * 16u));
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
#pragma unroll
    for (uint32_t r = 0; r < kVec; r++) {
      const uint32_t i = tid + r * 256u;
      const float4 v = f4(xv[r]), w = f4(wv[r]);
      if (i < n4) put4(i, make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w));
    }
    for (uint32_t i = tid + kVec * 256u; i < n4; i += blockDim.x) {
      const float4 v = f4(egd::load_b128_p<AUX>(xb, i * 16u)), w = f4(egd::load_b128(wb, i * 16u));
      put4(i, make_float4(v.x * inv * w.x, v.y * inv * w.y, v.z * inv * w.z, v.w * inv * w.w));
    }
  } else if (IN == EG_INPUT_SILU_MUL) {
    // gate and up for up to kVec * 1024 inputs in one batch (the intermediate width 4864 is 4.75
    // vectors per thread)
    constexpr uint32_t kVec = 5;
    const auto gb = egd::buffer(a.x, n4 * 16u), ub = egd::buffer(a.x2, n4 * 16u);
    egd::u32x4 gv[kVec], uv[kVec];
#pragma unroll
    for (uint32_t r = 0; r < kVec; r++) {
      gv[r] = egd::load_b128_p<AUX>(gb, (tid + r * 256u) * 16u);
      uv[r] = egd::load_b128_p<AUX>(ub, (tid + r * 256u) * 16u);
    }
    early();
    auto silu_mul = [](const float4& g, const float4& u) {
      return make_float4(g.x / (1.0f + expf(-g.x)) * u.x, g.y / (1.0f + expf(-g.y)) * u.y,
                         g.z / (1.0f + expf(-g.z)) * u.z, g.w / (1.0f + expf(-g.w)) * u.w);
    };
#pragma unroll
    for (uint32_t r = 0; r < kVec; r++) {
      const uint32_t i = tid + r * 256u;
      if (i < n4) put4(i, silu_mul(f4(gv[r]), f4(uv[r])));
    }
    for (uint32_t i = tid + kVec * 256u; i < n4; i += blockDim.x)
      put4(i, silu_mul(f4(egd::load_b128_p<AUX>(gb, i * 16u)), f4(egd::load_b128_p<AUX>(ub, i * 16u))));
  } else if (IN == EG_INPUT_ATTENTION) {
    // The combine of the attention partials (chunk-fastest: o[h][D][chunks], m[h][chunks],
    // l[h][chunks]): every (head, chunk) pair's weight e^(m_c - M) / L goes into LDS, then every
    // output sums its chunks' partial o values with those weights - the same operations as
    // egd::attention_combine_at. A head's statistics sit in a power-of-two group of lanes
    // (G >= chunks), so M and L are butterflies across the group (L in egd::combine_stats's
    // pairwise tree order): one exp per lane instead of a serial loop over the chunks. In the
    // common case (<= 16 chunks of a multiple of 4, <= 1024 outputs) the statistics and every
    // output's o values are all loaded at once, 4 outputs x 4 vectors per thread.
    const uint32_t heads = a.att_heads, chunks = a.att_chunks, D = a.att_head_dim;
    const uint32_t hcs = heads * chunks;
    const uint32_t G = egd::combine_group(chunks);  // <= 64 and heads * G <= kMaxCombine (host-checked)
    const float* m = a.x + (size_t)heads * D * chunks;
    const float* l = m + hcs;
    float* wts = scratch;
    constexpr uint32_t kOut = 4, kQ = 4;  // outputs per thread, 16-byte vectors per output
    const bool batched = (chunks & 3u) == 0 && chunks <= 4 * kQ && n <= kOut * 256u;
    const uint32_t q4 = chunks / 4;
    const auto ob = egd::buffer(a.x, n * chunks * 4u);
    const auto mb = egd::buffer(m, hcs * 4u), lb = egd::buffer(l, hcs * 4u);
    // statistics: thread p = tid + 256 r holds head p / G, chunk p % G (chunks past the head's
    // count, and groups past the last head, read nothing: m = -inf, l = 0). Issued before the o
    // values, so the weights are computed while those are still arriving (a wave's reads
    // complete in issue order).
    constexpr uint32_t kStat = kMaxCombine / 256;
    float mv[kStat], lv[kStat];
    uint32_t sidx[kStat];
    bool sval[kStat];
#pragma unroll
    for (uint32_t r = 0; r < kStat; r++) {
      const uint32_t p = tid + r * 256u, c = p % G;
      sval[r] = p < heads * G && c < chunks;
      sidx[r] = (p / G) * chunks + c;
      const uint32_t off = sval[r] ? sidx[r] * 4u : 0xFFFFFFF0u;  // past the stream: reads zero
      mv[r] = __uint_as_float(egd::load_b32_p<AUX>(mb, off));
      lv[r] = __uint_as_float(egd::load_b32_p<AUX>(lb, off));
    }
    egd::u32x4 ov[kOut][kQ];
    if (batched) {
#pragma unroll
      for (uint32_t r = 0; r < kOut; r++)
#pragma unroll
        for (uint32_t q = 0; q < kQ; q++)
          ov[r][q] = q < q4 ? egd::load_b128_p<AUX>(ob, ((tid + r * 256u) * chunks + 4u * q) * 4u) : egd::u32x4{0, 0, 0, 0};
    }
    early();
#pragma unroll
    for (uint32_t r = 0; r < kStat; r++) {
      if (r * 256u < heads * G) {  // workgroup-uniform: only the rounds that hold a head
        float M, e, L;
        egd::group_stats(G, sval[r], mv[r], lv[r], M, e, L);
        if (sval[r]) wts[sidx[r]] = e / L;
      }
    }
    __syncthreads();
    if (batched) {
#pragma unroll
      for (uint32_t r = 0; r < kOut; r++) {
        const uint32_t i = tid + r * 256u;
        // the head's weights: one 16-byte LDS read per 4 chunks, the same address in every lane
        // of the wave (a head is 64 consecutive outputs), so a broadcast
        const float4* w = reinterpret_cast<const float4*>(wts + (i / D) * chunks);
        float acc = 0.f;
#pragma unroll
        for (uint32_t q = 0; q < kQ; q++) {
          if (q < q4) {
            const float4 v = f4(ov[r][q]), wq = w[q];
            acc = fmaf(v.x, wq.x, acc);
            acc = fmaf(v.y, wq.y, acc);
            acc = fmaf(v.z, wq.z, acc);
            acc = fmaf(v.w, wq.w, acc);
          }
        }
        if (i < n) xs[x_slot<P>(i / 4, xchunks) * 4 + i % 4] = acc;
      }
    } else {
      for (uint32_t i = tid; i < n; i += blockDim.x) {
        const float* w = wts + (i / D) * chunks;
        float acc = 0.f;
        for (uint32_t c = 0; c < chunks; c++) acc = fmaf(egd::load_f32_p<AUX>(ob, (i * chunks + c) * 4u), w[c], acc);
        xs[x_slot<P>(i / 4, xchunks) * 4 + i % 4] = acc;
      }
    }
  } else {
    // x as given: every load issued before any LDS write (8 per thread covers the longest
    // rows, 256 chunks of 32 codes).
    constexpr uint32_t kMaxLoads = 256 * 32 / 4 / 256;
    const auto src = egd::buffer(a.x, n4 * 16u);
    egd::u32x4 v[kMaxLoads];
#pragma unroll
    for (uint32_t r = 0; r < kMaxLoads; r++) v[r] = egd::load_b128_p<AUX>(src, (tid + r * 256u) * 16u);
    early();
    egd::u32x4* dst = reinterpret_cast<egd::u32x4*>(xs);
#pragma unroll
    for (uint32_t r = 0; r < kMaxLoads; r++)
      if (tid + r * 256u < n4) dst[x_slot<P>(tid + r * 256u, xchunks)] = v[r];
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
template <int BITS, int ENC, int TEAM, int CPL, int U, int NB, int MODE, int IN, class Env>
__device__ __forceinline__ void gemv_body(const GemvArgs& a, const Env& env) {
  constexpr int AUX = Env::kAux;
  using C = Codes<BITS>;
  constexpr int EPC = C::kPerChunk;
  constexpr int RPW = 64 / TEAM;
  // kSwiGLU: slot u = 0 of a tile reads the gate matrix and u = 1 the up matrix at the same rows,
  // so a tile produces RPW outputs; otherwise RPW * U rows of one matrix.
  constexpr bool kPair = MODE == kSwiGLU;
  static_assert(!kPair || U == 2, "a SwiGLU tile pairs one gate row with one up row");
  constexpr int TILE = kPair ? RPW : RPW * U;
  constexpr bool kStats = MODE == kSampleStats;
  constexpr bool kStore = MODE != kArgmaxOnly && !kStats;
  constexpr bool kBest = MODE == kArgmax || MODE == kArgmaxOnly;
  static_assert(!kStats || (!Env::kPhase && MODE != kBatched), "the sampling statistics are a launch of their own");
  const uint32_t lane = threadIdx.x & 63u;
  const uint32_t t = lane % TEAM;
  const uint32_t slot = lane / TEAM;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(env.block() * kWaves + (threadIdx.x >> 6));
  const uint32_t total_waves = env.blocks() * kWaves;

  // Dynamic LDS: x (chunks * EPC floats), then the input stage's scratch. The workgroup copies
  // x in once, so the activations cross L2 once per workgroup rather than once per wave; each
  // lane then keeps the chunks it owns in VGPRs for every row it visits.
  extern __shared__ __align__(16) uint8_t smem[];
  const uint32_t x_words = a.chunks * EPC;
  float* scratch = reinterpret_cast<float*>(smem + x_words * 4u);

  // This lane's chunk slots: slot j covers chunk cj[j] of each row (chunk 0 past the row's end,
  // where x is zero), in quant block bj[j].
  uint32_t cj[CPL], bj[CPL];
#pragma unroll
  for (int j = 0; j < CPL; j++) {
    const uint32_t c = t + j * TEAM;
    cj[j] = c < a.chunks ? c : 0u;
    bj[j] = cj[j] / a.chunks_per_block;
  }

  // Byte offsets of this lane's loads relative to its tile's first row: constant for the whole
  // launch. The tile's own offset is wave-uniform and rides in the buffer instruction's scalar
  // offset, so walking tiles costs scalar adds, not per-lane address arithmetic.
  uint32_t qoff[U][CPL], soff[U][CPL], roff[U];
#pragma unroll
  for (int u = 0; u < U; u++) {
    const uint32_t lrow = (kPair ? 0u : (uint32_t)u * RPW) + slot;
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
  // A wave with no tiles (more waves than tiles) still issues its first loads - of a valid
  // tile, computed by nobody - so that no load sits under a branch (see `run`).
  const uint32_t first = begin < end ? begin : min(begin, a.total_passes - 1u);
  const uint32_t last = begin < end ? end - 1 : first;

  // The matrix the issue side is walking (one for a plain launch; the current segment of a
  // batched one). Rows are a multiple of TILE in a batched plan; a plain launch's last partial
  // tile is shifted back to end at the last row (rows >= TILE), recomputing a few rows with
  // identical results, so every access stays inside its stream.
  struct Seg {
    __amdgpu_buffer_rsrc_t w, s, z, b, o;
    uint32_t rows, out_offset, first, end;
  };
  auto make_seg = [&](const uint4* w, const float* scales, const uint32_t* zeros, const float* bias, float* out,
                      uint32_t rows, uint32_t out_offset, uint32_t first, uint32_t seg_end) {
    const uint32_t blocks = rows * a.blocks_per_row;
    Seg r;
    r.w = egd::buffer(w, rows * a.chunks * 16u);
    r.s = egd::buffer(scales, blocks * 4u);
    r.z = egd::buffer(zeros, ((blocks + C::kZeroPerWord - 1) / C::kZeroPerWord) * 4u);
    // Without a bias the stream is empty: its loads read zeros without touching memory.
    r.b = bias != nullptr ? egd::buffer(bias, rows * 4u) : egd::buffer(scales, 0u);
    r.o = egd::buffer(out, (out_offset + rows) * 4u);
    r.rows = rows;
    r.out_offset = out_offset;
    r.first = first;
    r.end = seg_end;
    return r;
  };

  // Batched: a segment is read into scalar registers from the kernel arguments (small plans)
  // or with a scalar load from the table in global memory (scalar loads count on lgkmcnt, so
  // switching segments never waits for the tile loads in flight, as a vector load would). The
  // table is read-only for the launch, so the constant address space is accurate.
  Seg cur = kPair ? make_seg(a.inline_segs[0].w, a.inline_segs[0].scales, a.inline_segs[0].zeros, nullptr,
                             a.inline_segs[0].out, a.n, a.inline_segs[0].out_offset, 0, a.total_passes)
                  : make_seg(a.w, a.scales, a.zeros, a.bias, a.out, a.n, a.out_offset, 0, a.total_passes);
  // kSwiGLU: the up matrix (its output pointer unused: the pair stores through cur)
  const Seg up = kPair ? make_seg(a.inline_segs[1].w, a.inline_segs[1].scales, a.inline_segs[1].zeros, nullptr,
                                  a.inline_segs[0].out, a.n, 0, 0, a.total_passes)
                       : cur;
  uint32_t seg = 0;
  auto use_segment = [&](const uint4* w, const float* scales, const uint32_t* zeros, const float* bias, float* out,
                         uint32_t rows, uint32_t pass_end, uint32_t out_offset) {
    rows = __builtin_amdgcn_readfirstlane(rows);
    const uint32_t seg_end = __builtin_amdgcn_readfirstlane(pass_end);
    cur = make_seg(egd::uniform(w), egd::uniform(scales), egd::uniform(zeros), egd::uniform(bias), egd::uniform(out),
                   rows, __builtin_amdgcn_readfirstlane(out_offset), seg_end - rows / TILE, seg_end);
  };
  auto load_segment = [&](uint32_t sidx) {
    if (a.seg_count > kInlineSegments) {
      typedef const __attribute__((address_space(4))) DevSegment ConstSegment;
      ConstSegment* d = (ConstSegment*)(a.segs + sidx);
      use_segment(d->w, d->scales, d->zeros, d->bias, d->out, d->rows, d->pass_end, d->out_offset);
    } else {
      // kernel-argument table: a select per field over the few entries keeps every value scalar
      auto sel = [&](auto DevSegment::*field) {
        auto v = a.inline_segs[0].*field;
#pragma unroll
        for (uint32_t i = 1; i < kInlineSegments; i++) v = sidx == i ? a.inline_segs[i].*field : v;
        return v;
      };
      use_segment(sel(&DevSegment::w), sel(&DevSegment::scales), sel(&DevSegment::zeros), sel(&DevSegment::bias),
                  sel(&DevSegment::out), sel(&DevSegment::rows), sel(&DevSegment::pass_end),
                  sel(&DevSegment::out_offset));
    }
  };
  // The segment holding the wave's first tile: looked up in the plan's pass index (two
  // dependent scalar loads, which overlap the input stage's reads), or - small plans - the
  // number of argument-table segments ending at or before that tile (pass_end increases).
  auto find_first_segment = [&]() {
    uint32_t count = 0;
    if (a.seg_count > kInlineSegments) {
      typedef const __attribute__((address_space(4))) uint32_t ConstWord;
      const uint32_t w = *(ConstWord*)(a.seg_index + (first >> 1));
      count = (w >> ((first & 1u) * 16u)) & 0xFFFFu;
    } else {
#pragma unroll
      for (uint32_t i = 0; i < kInlineSegments; i++) count += (i < a.seg_count && a.inline_segs[i].pass_end <= first);
    }
    seg = __builtin_amdgcn_readfirstlane(count);
    load_segment(seg);
  };

  // What computing a tile needs once its loads are in flight: where its rows are stored (and,
  // for a phase's first tiles, whose bias loads wait for the phase's inputs, where it is read).
  struct Pending {
    __amdgpu_buffer_rsrc_t o, b;
    uint32_t row0, out_offset;
  };

  // Issues the loads of tile `tl` (clamped to the wave's last tile; tiles are visited in
  // increasing order, so the segment cursor only moves forward). The biases of a tile's rows
  // take one load instruction: lane t < U of each team reads its row t's (lanes past U re-read
  // row U-1's, unused).
  const uint32_t boff = ((t < (uint32_t)U ? t : (uint32_t)(U - 1)) * RPW + slot) * 4u;
  auto issue = [&](uint32_t tl, Loads<BITS, U, CPL>& L, Pending& P, bool with_bias = true) {
    tl = min(tl, last);
    if (MODE == kBatched)
      while (tl >= cur.end) load_segment(++seg);
    // (readfirstlane pins the value to a scalar register: a scalar offset left in a vector
    // register would make the compiler wrap every load in a per-lane loop.)
    const uint32_t row0 = __builtin_amdgcn_readfirstlane(min((tl - cur.first) * TILE, cur.rows - TILE));
    const uint32_t sq = row0 * (a.chunks * 16u);
    const uint32_t ss = row0 * (a.blocks_per_row * 4u);
    if (with_bias) L.b = egd::load_f32_p<AUX>(cur.b, boff, row0 * 4u);
#pragma unroll
    for (int u = 0; u < U; u++) {
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const Seg& m = kPair && u == 1 ? up : cur;
        L.q[u][j] = egd::load_b128_nt(m.w, qoff[u][j], sq);
        L.s[u][j] = egd::load_f32_nt(m.s, soff[u][j], ss);
        if (ENC == EG_ENC_OFFSET_ZEROS) {
          const uint32_t blk = (row0 + (kPair ? 0u : (uint32_t)u * RPW) + slot) * a.blocks_per_row + bj[j];
          L.zw[u][j] = egd::load_b32(m.z, (blk / C::kZeroPerWord) * 4u);
        }
      }
    }
    P.o = cur.o;
    P.b = cur.b;
    P.row0 = row0;
    P.out_offset = cur.out_offset;
  };

  // This lane's activations: chunk slot j covers x[cj*EPC, cj*EPC + EPC), zero past the row
  // (filled from LDS once the input stage has written x there).
  float xr[CPL][EPC];
  float sx[CPL];
  auto load_x = [&]() {
#pragma unroll
    for (int j = 0; j < CPL; j++) {
      const bool valid = t + j * TEAM < a.chunks;
      sx[j] = 0.f;
      const egd::u32x4* xs = reinterpret_cast<const egd::u32x4*>(smem) + cj[j];  // piece e at e * chunks
#pragma unroll
      for (int e = 0; e < EPC / 4; e++) {
        const egd::u32x4 v = xs[(size_t)e * a.chunks];
        xr[j][4 * e + 0] = valid ? __uint_as_float(v.x) : 0.f;
        xr[j][4 * e + 1] = valid ? __uint_as_float(v.y) : 0.f;
        xr[j][4 * e + 2] = valid ? __uint_as_float(v.z) : 0.f;
        xr[j][4 * e + 3] = valid ? __uint_as_float(v.w) : 0.f;
      }
#pragma unroll
      for (int e = 0; e < EPC; e++) sx[j] += xr[j][e];
#pragma unroll
      for (int e = 0; e < EPC; e++) xr[j][e] *= C::x_scale(e);
    }
  };

  float best_v = -1.0e30f;
  uint32_t best_i = a.out_offset;

  // kSampleStats: the tile loop only records each row's logit in stats_x, for the workgroup's
  // nominal rows [stats_lo, stats_hi) - its tiles' rows before a last partial tile's shift back;
  // the rows that tile recomputes below stats_lo belong to the workgroup before and are left to
  // it - and the epilogue does the rest, one row per thread: the penalty (`hit`: the history ids
  // among the rows), the store, l/T and the partial.
  // The parameters (device memory or the arguments) and the first kStatsHistory x 256 history
  // ids are read before the input stage, so their round trips overlap its own and the first
  // tiles' weights.
  static_assert(!kStats || kStatsRows == kWaves * 64, "the epilogue takes one row per thread");
  static_assert(kStatsLdsBytes == kStatsRows * 4 + kStatsRows / 32 * 4 + kWaves * 8 + kWaves * 8, "stats LDS");
  constexpr uint32_t kStatsHistory = 4;
  float* const stats_x = scratch;  // the mode takes no input stage with scratch of its own
  uint32_t* const hit = reinterpret_cast<uint32_t*>(stats_x + kStatsRows);
  uint32_t stats_lo = 0, stats_hi = 0, hist_len = 0;
  float temp = 0.0f, pen = 1.0f;
  uint32_t hv[kStats ? kStatsHistory : 1];
  if constexpr (kStats) {
    // (wave-uniform values pinned to scalar registers, as begin and end below)
    stats_lo = __builtin_amdgcn_readfirstlane(
        (uint32_t)(((uint64_t)a.total_passes * (env.block() * kWaves)) / total_waves) * TILE);
    stats_hi = __builtin_amdgcn_readfirstlane(
        min((uint32_t)(((uint64_t)a.total_passes * ((env.block() + 1) * kWaves)) / total_waves) * TILE, a.n));
    temp = a.stats.temperature;
    pen = a.stats.repetition_penalty;
    hist_len = a.stats.history_length;
    if (a.stats.sample_dev) {
      temp = a.stats.sample_dev->temperature;
      pen = a.stats.sample_dev->repetition_penalty;
      hist_len = a.stats.sample_dev->history_length;
    }
    temp = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, temp)));
    pen = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(uint32_t, pen)));
    hist_len = __builtin_amdgcn_readfirstlane(hist_len);
#pragma unroll
    for (uint32_t r = 0; r < kStatsHistory; r++) {
      const uint32_t h = threadIdx.x + r * blockDim.x;
      hv[r] = pen != 1.0f && a.stats.history && h < hist_len ? a.stats.history[h] : 0xFFFFFFFFu;
    }
    for (uint32_t i = threadIdx.x; i < kStatsRows / 32; i += blockDim.x) hit[i] = 0u;
    if (a.stats.clear && env.block() == 0)
      for (uint32_t i = threadIdx.x; i < a.stats.clear_words; i += blockDim.x) a.stats.clear[i] = 0u;
  }

  auto compute = [&](const Loads<BITS, U, CPL>& L, const Pending& P) {
    float pair[2];  // kSwiGLU: the gate and up totals of the team's row
    float rec[U];   // kSampleStats: the tile's row values (lane t < U of each team records row t)
#pragma unroll
    for (int u = 0; u < U; u++) {
      // The bias starts lane u's partial (linearQ4 starts its sum from the bias too; zero
      // where the matrix has none).
      float acc = t == (uint32_t)u ? L.b : 0.f;
      const uint32_t row = P.row0 + (kPair ? 0u : (uint32_t)u * RPW) + slot;
#pragma unroll
      for (int j = 0; j < CPL; j++) {
        const uint4 q = make_uint4(L.q[u][j].x, L.q[u][j].y, L.q[u][j].z, L.q[u][j].w);
        float z;
        if (ENC == EG_ENC_OFFSET_ZEROS) {
          const uint32_t blk = row * a.blocks_per_row + bj[j];
          z = (float)((L.zw[u][j] >> (BITS * (blk % C::kZeroPerWord))) & ((1u << BITS) - 1u));
        } else {
          z = (float)(1 << (BITS - 1));
        }
        acc = fmaf(L.s[u][j], C::template dot<ENC>(q, xr[j]) - z * sx[j], acc);
      }
      float v = egd::team_allsum<TEAM>(acc);
      if (kPair) {
        pair[u & 1] = v;
        continue;
      }
      if constexpr (kStats) rec[u] = v;
      if (kStore) egd::store_f32_p<AUX>(P.o, roff[u], v, (P.row0 + P.out_offset) * 4u);
      if (kBest) {
        const uint32_t idx = row + P.out_offset;
        const bool take = egd::better(v, idx, best_v, best_i);
        best_v = take ? v : best_v;
        best_i = take ? idx : best_i;
      }
    }
    if constexpr (kStats) {
      // one LDS write per tile: lane t < U of each team records its team's row t (a shifted
      // tile's rows below stats_lo wrap and are left out)
      float mine = rec[0];
#pragma unroll
      for (int u = 1; u < U; u++) mine = t == (uint32_t)u ? rec[u] : mine;
      const uint32_t rel = P.row0 + (t < (uint32_t)U ? t : 0u) * RPW + slot - stats_lo;
      if (t < (uint32_t)U && rel < kStatsRows) stats_x[rel] = mine;
    }
    if (kPair) {
      const float g = pair[0];
      egd::store_f32_p<AUX>(P.o, roff[0], g / (1.0f + expf(-g)) * pair[1], (P.row0 + P.out_offset) * 4u);
    }
  };

  // The wave's range is one software pipeline over NB load buffers, NB tiles per iteration,
  // with a single exit at the bottom: while tile i is computed, the loads of tiles
  // i+1 .. i+NB-1 are in flight. The first NB-1 tiles are issued from inside the input stage,
  // right after its own reads, so they travel while the stage waits and computes. Each buffer
  // carries where its rows go, so the pipeline runs straight through segment boundaries (a
  // boundary costs a few scalar reads, not a drain of the loads in flight). The loop runs whole
  // groups of NB tiles; the last count % NB tiles, already in flight, are computed after it. No
  // load sits under a branch - a wave without tiles issues its first ones anyway, and issues
  // past the last tile re-read it - so the compiler's wait counts stay exact: the input stage
  // waits only for its own reads, and computing a tile waits only for that tile's loads.
  // sched_barrier(0) after each issue keeps the scheduler from sinking the next tile's loads
  // into the current tile's math.
  Loads<BITS, U, CPL> L[NB];
  Pending P[NB];
  auto start = [&]() {
    if (MODE == kBatched) find_first_segment();
#pragma unroll
    for (int b = 0; b + 1 < NB; b++) issue(first + b, L[b], P[b], !Env::kPhase);
    __builtin_amdgcn_sched_barrier(0);
  };
  if constexpr (Env::kPhase) {
    // A phase: the first tiles' weights go out before the wait for the phase's inputs, and
    // travel while it lasts; their biases (a residual another workgroup writes) and x after it.
    start();
    env.wait();
#pragma unroll
    for (int b = 0; b + 1 < NB; b++) L[b].b = egd::load_f32_p<AUX>(P[b].b, boff, P[b].row0 * 4u);
    produce_input<IN, EPC / 4, Env>(a, reinterpret_cast<float*>(smem), x_words, scratch, [] {});
  } else {
    produce_input<IN, EPC / 4, Env>(a, reinterpret_cast<float*>(smem), x_words, scratch, start);
  }
  __syncthreads();
  load_x();
  if constexpr (kStats) {
    // the history ids among the workgroup's rows (the penalty's set: each id once); the epilogue's
    // barrier orders these marks before their reads
#pragma unroll
    for (uint32_t r = 0; r < kStatsHistory; r++) {
      const uint32_t rel = hv[r] - stats_lo;
      if (rel < stats_hi - stats_lo) atomicOr(&hit[rel >> 5], 1u << (rel & 31u));
    }
    if (pen != 1.0f && a.stats.history)
      for (uint32_t h = threadIdx.x + kStatsHistory * blockDim.x; h < hist_len; h += blockDim.x) {
        const uint32_t rel = a.stats.history[h] - stats_lo;
        if (rel < stats_hi - stats_lo) atomicOr(&hit[rel >> 5], 1u << (rel & 31u));
      }
  }
  const uint32_t count = end - begin;
  const uint32_t groups = count / NB;
  uint32_t tile = begin;
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
  // The last count % NB tiles are already in flight in buffers 0 .. NB-2 (issued by the last
  // group, or by the input stage when the wave has fewer than NB tiles): compute them, with no
  // load under the branch.
  const uint32_t rem = count - groups * NB;
#pragma unroll
  for (int b = 0; b + 1 < NB; b++)
    if ((uint32_t)b < rem) compute(L[b], P[b]);
  // Issues past the wave's last tile (clamped to it) are duplicates that nothing consumes;
  // they complete before the wave ends.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // gfx9 encoding: vmcnt 0, expcnt 7, lgkmcnt 15

  if constexpr (kStats) {
    // The epilogue, thread i on row stats_lo + i.
    __syncthreads();  // the record and the marks complete
    const uint32_t i = threadIdx.x, row = stats_lo + i;
    const bool valid = row < stats_hi;
    float v = valid ? stats_x[i] : 0.0f;
    if (valid && ((hit[i >> 5] >> (i & 31u)) & 1u)) v = v > 0.0f ? v / pen : v * pen;
    if (valid) a.out[a.out_offset + row] = v;
    const float x = temp > 0.0f ? v / temp : v;  // what the argmax ranks: l/T, or l when greedy
    float bv = valid ? x : -1.0e30f;
    uint32_t bi = valid ? a.out_offset + row : a.out_offset;
    float* const wv = reinterpret_cast<float*>(hit + kStatsRows / 32);
    uint32_t* const wi = reinterpret_cast<uint32_t*>(wv + kWaves);
    double* const ws = reinterpret_cast<double*>(wi + kWaves);  // 8-byte aligned: 1,088 bytes in
    egd::team_argmax<64>(bv, bi);
    if (lane == 0) {
      wv[threadIdx.x >> 6] = bv;
      wi[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    bv = wv[0];
    bi = wi[0];
    for (int k = 1; k < kWaves; k++)
      if (egd::better(wv[k], wi[k], bv, bi)) {
        bv = wv[k];
        bi = wi[k];
      }
    // sum of exp(l/T - the workgroup's max) over its rows in float64 (the sampler's per-slice
    // statement, sample.wgsl:230-236, over this workgroup's rows)
    double e = valid && temp > 0.0f ? (double)expf(x - bv) : 0.0;
#pragma unroll
    for (int m = 32; m > 0; m >>= 1) e += __shfl_xor(e, m, 64);
    if (lane == 0) ws[threadIdx.x >> 6] = e;
    __syncthreads();
    if (threadIdx.x == 0) {
      double sum = 0.0;
      for (int k = 0; k < kWaves; k++) sum += ws[k];
      const uint64_t sb = __builtin_bit_cast(uint64_t, sum);
      a.partials[4 * env.block() + 0] = __float_as_uint(bv);
      a.partials[4 * env.block() + 1] = bi;
      a.partials[4 * env.block() + 2] = (uint32_t)sb;
      a.partials[4 * env.block() + 3] = (uint32_t)(sb >> 32);
    }
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
      a.partials[2 * env.block() + 0] = __float_as_uint(bv);
      a.partials[2 * env.block() + 1] = bi;
    }
  }
}

// (kSampleStats kernels take 90-105 VGPRs, four waves per SIMD against the plain head's six;
// held to six waves they spill around the tile loop, and the config-2 head took 39 us instead of
// ~27. Measured on MI355X.)
template <int BITS, int ENC, int TEAM, int CPL, int U, int NB, int MODE, int IN>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
  const egd::WaveStamp stamp(a.stamp);
  gemv_body<BITS, ENC, TEAM, CPL, U, NB, MODE, IN>(a, LaunchEnv{});
}

using KernelFn = void (*)(GemvArgs);

// Fused input stages are instantiated for the shapes the library's shape choice produces (one
// chunk slot per lane for rows of up to 64 chunks, a full-wave team with 2-4 slots for longer
// rows; the pipeline depth is 2) and for the modes that take an input stage (batched plans and
// the fused LM-head argmax). Each stage has its own translation unit, so they compile in
// parallel: eg_gemv_rmsnorm.hip, eg_gemv_silu.hip, eg_gemv_attention.hip.
#define EG_FUSED_SHAPES(X)                                                                                    \
  X(8, 1, 1) X(8, 1, 2) X(16, 1, 1) X(16, 1, 2) X(32, 1, 1) X(32, 1, 2) X(64, 1, 1) X(64, 1, 2) X(64, 1, 4) \
  X(64, 2, 1) X(64, 2, 2) X(64, 3, 1) X(64, 4, 1)

// The shapes a SwiGLU pair takes (two rows per tile slot pair: U = 2).
#define EG_SWIGLU_SHAPES(X) X(8, 1, 2) X(16, 1, 2) X(32, 1, 2) X(64, 1, 2) X(64, 2, 2)

template <int IN, int BITS, int ENC, int MODE>
KernelFn pick_fused_shape(int team, int cpl, int u) {
  if constexpr (MODE == kSwiGLU) {
#define EG_SWIGLU_CASE(T, P, UU) \
  if (team == T && cpl == P && u == UU) return gemv_kernel<BITS, ENC, T, P, UU, 2, kSwiGLU, IN>;
    EG_SWIGLU_SHAPES(EG_SWIGLU_CASE)
#undef EG_SWIGLU_CASE
  } else {
#define EG_FUSED_CASE(T, P, UU) \
  if (team == T && cpl == P && u == UU) return gemv_kernel<BITS, ENC, T, P, UU, 2, MODE, IN>;
    EG_FUSED_SHAPES(EG_FUSED_CASE)
#undef EG_FUSED_CASE
  }
  return nullptr;
}

template <int IN, int BITS, int ENC>
KernelFn pick_fused_mode(int mode, int team, int cpl, int u) {
  if (mode == kBatched) return pick_fused_shape<IN, BITS, ENC, kBatched>(team, cpl, u);
  if (mode == kArgmax) return pick_fused_shape<IN, BITS, ENC, kArgmax>(team, cpl, u);
  if (mode == kArgmaxOnly) return pick_fused_shape<IN, BITS, ENC, kArgmaxOnly>(team, cpl, u);
  if constexpr (IN == EG_INPUT_RMSNORM && BITS == 4)  // the int4 gate|up pair after the post-attention norm
    if (mode == kSwiGLU) return pick_fused_shape<IN, BITS, ENC, kSwiGLU>(team, cpl, u);
  if constexpr (IN == EG_INPUT_RMSNORM && BITS == 8)  // the int8 LM head after the final norm, ahead of the sampler
    if (mode == kSampleStats) return pick_fused_shape<IN, BITS, ENC, kSampleStats>(team, cpl, u);
  return nullptr;
}

template <int IN>
KernelFn pick_fused_format(int bits, int enc, int mode, int team, int cpl, int u) {
  if (bits == 4 && enc == EG_ENC_OFFSET_ZEROS) return pick_fused_mode<IN, 4, EG_ENC_OFFSET_ZEROS>(mode, team, cpl, u);
  if (bits == 4 && enc == EG_ENC_SIGNED) return pick_fused_mode<IN, 4, EG_ENC_SIGNED>(mode, team, cpl, u);
  if (bits == 8 && enc == EG_ENC_OFFSET_ZEROS) return pick_fused_mode<IN, 8, EG_ENC_OFFSET_ZEROS>(mode, team, cpl, u);
  return pick_fused_mode<IN, 8, EG_ENC_SIGNED>(mode, team, cpl, u);
}

// One per input-stage translation unit.
KernelFn pick_rmsnorm(int bits, int enc, int mode, int team, int cpl, int u);
KernelFn pick_silu_mul(int bits, int enc, int mode, int team, int cpl, int u);
KernelFn pick_attention(int bits, int enc, int mode, int team, int cpl, int u);

// A plan's launch on an input as the persistent decode kernel runs it (one of its phases): the
// kernel arguments eg_gemv_plan_launch_input would pass, the plan's shape and mode, its tiles,
// and the dynamic LDS the body needs. Defined in eg_gemv.hip.
struct PlanPhase {
  int bits, encoding, mode, in_kind, team, cpl, u, nb;
  uint32_t tiles, smem;
};
int plan_phase(eg_context* ctx, const eg_gemv_plan* plan, const eg_gemv_input* input, GemvArgs* args,
               PlanPhase* phase);

// The kernel for a fused input stage (in_kind RMSNORM, SILU_MUL or ATTENTION) of one
// (format, mode, shape), or nullptr where none is instantiated.
inline KernelFn pick_fused(int bits, int enc, int mode, int in_kind, int team, int cpl, int u, int nb) {
  if (nb != 2) return nullptr;
  if (in_kind == EG_INPUT_RMSNORM) return pick_rmsnorm(bits, enc, mode, team, cpl, u);
  if (in_kind == EG_INPUT_SILU_MUL) return pick_silu_mul(bits, enc, mode, team, cpl, u);
  if (in_kind == EG_INPUT_ATTENTION) return pick_attention(bits, enc, mode, team, cpl, u);
  return nullptr;
}

}  // namespace eg_gemv
