// Row-wise kernels of the prompt chain (the prefill graph's embed, rmsnorm and silu_mul stages,
// graph.ts:380-500, over a chunk of up to 256 rows): one workgroup per row, vectorized 16-byte
// accesses, the same arithmetic as the decode path's GEMV input stages (f32 sum of squares,
// 1 / sqrt(mean + eps); silu(g) = g / (1 + e^-g)) so prompt rows and decode rows are computed
// alike. They sit between the prefill GEMMs, which consume their outputs as bf16 MFMA operands.
#include "eg_internal.hpp"

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void embed_rows_kernel(const uint32_t* ids, const uint32_t* packed,
                                                              const float* scales, const uint32_t* zeros,
                                                              uint32_t hidden, uint32_t block_size, int encoding,
                                                              int bits, float* out) {
  const uint32_t r = blockIdx.x;
  const uint32_t id = ids[r];
  const uint32_t bpr = bits >= 16 ? 0 : hidden / block_size;
  for (uint32_t i = threadIdx.x; i < hidden; i += kThreads) {
    const uint64_t blk = bits >= 16 ? 0 : (uint64_t)id * bpr + i / block_size;
    out[(size_t)r * hidden + i] = egd::table_value(packed, scales, zeros, (uint64_t)id * hidden + i, blk, encoding, bits);
  }
}

__device__ __forceinline__ float block_total(float v) {
  __shared__ float red[kThreads / 64];
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  if ((threadIdx.x & 63u) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float t = 0.f;
#pragma unroll
  for (int w = 0; w < kThreads / 64; w++) t += red[w];
  return t;
}

// n is a multiple of 4 (checked on the host).
// Four results stored as f32, or as bf16 (egd::pack_bf16) for a GEMM that stages them as they are.
template <bool B16>
__device__ __forceinline__ void store4(float* out, size_t i, float4 v) {
  if (B16) reinterpret_cast<uint2*>(out)[i] = make_uint2(egd::pack_bf16(v.x, v.y), egd::pack_bf16(v.z, v.w));
  else reinterpret_cast<float4*>(out)[i] = v;
}

template <bool B16>
__global__ __launch_bounds__(kThreads) void rmsnorm_rows_kernel(const float* x, const float* w, uint32_t n, float eps,
                                                                float* out) {
  const uint32_t r = blockIdx.x;
  const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)r * n);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  float ss = 0.f;
  for (uint32_t i = threadIdx.x; i < n / 4; i += kThreads) {
    const float4 v = x4[i];
    ss = fmaf(v.x, v.x, ss);
    ss = fmaf(v.y, v.y, ss);
    ss = fmaf(v.z, v.z, ss);
    ss = fmaf(v.w, v.w, ss);
  }
  const float inv = 1.0f / sqrtf(block_total(ss) / (float)n + eps);
  for (uint32_t i = threadIdx.x; i < n / 4; i += kThreads) {
    const float4 v = x4[i], g = w4[i];
    store4<B16>(out, (size_t)r * (n / 4) + i, make_float4(v.x * inv * g.x, v.y * inv * g.y, v.z * inv * g.z, v.w * inv * g.w));
  }
}

template <bool B16>
__global__ __launch_bounds__(kThreads) void silu_mul_rows_kernel(const float* x, uint32_t n, float* out) {
  const uint32_t r = blockIdx.x;
  const float4* g4 = reinterpret_cast<const float4*>(x + (size_t)r * 2 * n);
  const float4* u4 = g4 + n / 4;
  for (uint32_t i = threadIdx.x; i < n / 4; i += kThreads) {
    const float4 g = g4[i], u = u4[i];
    store4<B16>(out, (size_t)r * (n / 4) + i,
                make_float4(g.x / (1.0f + expf(-g.x)) * u.x, g.y / (1.0f + expf(-g.y)) * u.y,
                            g.z / (1.0f + expf(-g.z)) * u.z, g.w / (1.0f + expf(-g.w)) * u.w));
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

int eg::embed_rows(eg_context* ctx, const uint32_t* ids, uint32_t rows, const uint32_t* packed, const float* scales,
                   const uint32_t* zeros, uint32_t hidden, uint32_t block_size, int encoding, int bits, float* out) {
  if (rows == 0) return EG_OK;
  if (rows > 65535 || (bits < 16 && (block_size == 0 || hidden % block_size != 0)))
    return eg::fail(ctx, EG_ERR_INVALID, "embed_rows: %u rows of %u in blocks of %u", rows, hidden, block_size);
  hipLaunchKernelGGL(embed_rows_kernel, dim3(rows), dim3(kThreads), 0, ctx->stream, ids, packed, scales,
                     encoding == EG_ENC_SIGNED ? nullptr : zeros, hidden, block_size, encoding, bits, out);
  return eg::check_launch(ctx, "embed_rows");
}

int eg::rmsnorm_rows(eg_context* ctx, const float* x, const float* w, uint32_t rows, uint32_t n, float eps,
                     float* out, bool out_bf16) {
  if (rows == 0) return EG_OK;
  if (rows > 65535 || n % 4 != 0 || !aligned16(x) || !aligned16(w) || !aligned16(out))
    return eg::fail(ctx, EG_ERR_INVALID, "rmsnorm_rows: %u rows of %u (a multiple of 4, 16-byte aligned)", rows, n);
  if (out_bf16) hipLaunchKernelGGL(rmsnorm_rows_kernel<true>, dim3(rows), dim3(kThreads), 0, ctx->stream, x, w, n, eps, out);
  else hipLaunchKernelGGL(rmsnorm_rows_kernel<false>, dim3(rows), dim3(kThreads), 0, ctx->stream, x, w, n, eps, out);
  return eg::check_launch(ctx, "rmsnorm_rows");
}

int eg::silu_mul_rows(eg_context* ctx, const float* x, uint32_t rows, uint32_t n, float* out, bool out_bf16) {
  if (rows == 0) return EG_OK;
  if (rows > 65535 || n % 4 != 0 || !aligned16(x) || !aligned16(out))
    return eg::fail(ctx, EG_ERR_INVALID, "silu_mul_rows: %u rows of %u (a multiple of 4, 16-byte aligned)", rows, n);
  if (out_bf16) hipLaunchKernelGGL(silu_mul_rows_kernel<true>, dim3(rows), dim3(kThreads), 0, ctx->stream, x, n, out);
  else hipLaunchKernelGGL(silu_mul_rows_kernel<false>, dim3(rows), dim3(kThreads), 0, ctx->stream, x, n, out);
  return eg::check_launch(ctx, "silu_mul_rows");
}
