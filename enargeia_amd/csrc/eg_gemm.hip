// matmul_q4_prefill (matmul_q4_prefill.wgsl:77-162) on the matrix cores:
//   out[r*out_stride + col + out_offset] = sum_k x[r,k] * W[col,k] (+ bias[col])
//
// The prefill chunk (M = 128-256 queries) is the one dense contraction on the path. Each
// workgroup owns a 64 x 64 output tile; its 4 waves each own 32 x 32 = 2 x 2 tiles of
// v_mfma_f32_16x16x32_bf16. K is staged 64 at a time through LDS:
//   * x (f32) is rounded to bf16 (round-to-nearest-even) on the way into LDS;
//   * W is dequantized while staging, as the reference's prefill kernel does: one 16-byte chunk
//     (32 int4 codes, one scale and zero-point) per thread, (code - zero) * scale in f32, then
//     bf16 - so the codes cross HBM as int4 and each weight is unpacked once per tile, not once
//     per MFMA that reads it.
// Rows are padded by 16 bytes in LDS so the 16 lanes that read one column of A (or B) hit
// different banks. Accumulation is f32 inside the MFMA; the bias is added at the store.
// Layouts the chunked staging cannot take (K or block size not a multiple of 32 codes,
// int8 codes, unaligned streams) stage W element by element with the reference's indexing.
#include "eg_internal.hpp"

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 64;   // M and N tile
constexpr int kBK = 64;     // K staged per iteration
constexpr int kPad = 8;     // bf16 elements of padding per LDS row
constexpr int kLds = kBK + kPad;

struct PrefillArgs {
  const float* x;
  const uint32_t* packed;
  const float* scales;
  const uint32_t* zeros;
  const float* bias;
  float* out;
  uint32_t m, n, k, block_size, blocks_per_row, out_stride, out_offset;
  int bits;
};

__device__ __forceinline__ uint16_t bf16_bits(float v) {
  uint32_t u = __float_as_uint(v);
  if ((u & 0x7F800000u) == 0x7F800000u) return (uint16_t)((u >> 16) | ((u & 0x7FFFFFu) ? 0x40u : 0u));
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

template <int ENC, bool CHUNKED>
__global__ __launch_bounds__(256) void prefill_kernel(PrefillArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t As[kTile][kLds];
  __shared__ __attribute__((aligned(16))) uint16_t Bs[kTile][kLds];
  const uint32_t m0 = blockIdx.y * kTile, n0 = blockIdx.x * kTile;
  const uint32_t tid = threadIdx.x, wave = tid >> 6, lane = tid & 63u;
  const uint32_t wm = (wave >> 1) * 32, wn = (wave & 1) * 32;
  const uint32_t per_word = 32u / (uint32_t)a.bits, mask = (1u << a.bits) - 1u;

  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (uint32_t k0 = 0; k0 < a.k; k0 += kBK) {
    // x tile: 64 rows x 64 k, consecutive threads on consecutive k (coalesced).
#pragma unroll 4
    for (uint32_t e = tid; e < kTile * kBK; e += 256) {
      const uint32_t r = e / kBK, c = e % kBK;
      const uint32_t row = m0 + r, kk = k0 + c;
      const float v = (row < a.m && kk < a.k) ? a.x[(size_t)row * a.k + kk] : 0.f;
      As[r][c] = bf16_bits(v);
    }
    // W tile: 64 output features x 64 k, dequantized to bf16.
    if (CHUNKED) {
      if (tid < 128) {
        const uint32_t r = tid >> 1, half = tid & 1u;
        const uint32_t nrow = n0 + r, kk = k0 + half * 32;
        uint16_t* dst = &Bs[r][half * 32];
        if (nrow < a.n && kk < a.k) {
          const uint4 q = *reinterpret_cast<const uint4*>(a.packed + ((size_t)nrow * a.k + kk) / 8);
          const uint32_t blk = nrow * a.blocks_per_row + kk / a.block_size;
          const float s = a.scales[blk];
          int32_t z;
          if (ENC == EG_ENC_OFFSET_ZEROS) z = (int32_t)((a.zeros[blk / 8] >> (4 * (blk % 8))) & 0xFu);
          else z = 8;
          const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
          for (int w = 0; w < 4; w++) {
            const uint32_t word = ENC == EG_ENC_SIGNED ? d[w] ^ 0x88888888u : d[w];
#pragma unroll
            for (int e = 0; e < 8; e++) {
              const int32_t code = (int32_t)((word >> (4 * e)) & 0xFu);
              dst[w * 8 + e] = bf16_bits((float)(code - z) * s);
            }
          }
        } else {
#pragma unroll
          for (int e = 0; e < 32; e++) dst[e] = 0;
        }
      }
    } else {
#pragma unroll 4
      for (uint32_t e = tid; e < kTile * kBK; e += 256) {
        const uint32_t r = e / kBK, c = e % kBK;
        const uint32_t nrow = n0 + r, kk = k0 + c;
        float v = 0.f;
        if (nrow < a.n && kk < a.k) {
          const size_t flat = (size_t)nrow * a.k + kk;
          uint32_t code = (a.packed[flat / per_word] >> (a.bits * (flat % per_word))) & mask;
          const uint32_t blk = nrow * a.blocks_per_row + kk / a.block_size;
          int32_t z;
          if (ENC == EG_ENC_OFFSET_ZEROS) {
            z = (int32_t)((a.zeros[blk / per_word] >> (a.bits * (blk % per_word))) & mask);
          } else {
            code ^= 1u << (a.bits - 1);
            z = 1 << (a.bits - 1);
          }
          v = (float)((int32_t)code - z) * a.scales[blk];
        }
        Bs[r][c] = bf16_bits(v);
      }
    }
    __syncthreads();
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
    __syncthreads();
  }

  // D layout of the 16x16 MFMA: lane l holds rows 4*(l/16) + e, column l % 16.
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const uint32_t col = n0 + wn + j * 16 + (lane & 15);
      if (col >= a.n) continue;
      const float b = a.bias ? a.bias[col] : 0.f;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const uint32_t row = m0 + wm + i * 16 + 4 * (lane >> 4) + e;
        if (row < a.m) a.out[(size_t)row * a.out_stride + col + a.out_offset] = acc[i][j][e] + b;
      }
    }
}

}  // namespace

extern "C" int eg_matmul_q4_prefill(eg_context* ctx, const float* x, const uint32_t* packed, const float* scales,
                                    const uint32_t* zeros, const float* bias, float* out,
                                    const eg_matmul_q4_dims* dims, int encoding, int bits) {
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
  const dim3 grid((n + kTile - 1) / kTile, (m + kTile - 1) / kTile);
  if (grid.y > 65535) return eg::fail(ctx, EG_ERR_RANGE, "%s: m %u needs %u row tiles, over 65535", op, m, grid.y);
  PrefillArgs a{x, packed, scales, encoding == EG_ENC_SIGNED ? nullptr : zeros, dims->use_bias ? bias : nullptr,
                out, m, n, k, bs, dims->blocks_per_row, dims->out_stride, dims->out_offset, bits};
  const bool chunked = bits == 4 && k % 32 == 0 && bs % 32 == 0 && (reinterpret_cast<uintptr_t>(packed) & 15u) == 0;
  if (encoding == EG_ENC_SIGNED) {
    if (chunked) hipLaunchKernelGGL((prefill_kernel<EG_ENC_SIGNED, true>), grid, dim3(256), 0, ctx->stream, a);
    else hipLaunchKernelGGL((prefill_kernel<EG_ENC_SIGNED, false>), grid, dim3(256), 0, ctx->stream, a);
  } else {
    if (chunked) hipLaunchKernelGGL((prefill_kernel<EG_ENC_OFFSET_ZEROS, true>), grid, dim3(256), 0, ctx->stream, a);
    else hipLaunchKernelGGL((prefill_kernel<EG_ENC_OFFSET_ZEROS, false>), grid, dim3(256), 0, ctx->stream, a);
  }
  return eg::check_launch(ctx, op);
}
