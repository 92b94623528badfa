// argmax (argmax.wgsl:28-66): index of the largest of logits[offset, offset + count), ties to
// the lowest index, -1e30 sentinel. out[0] = index relative to offset, out[1] = value bits.
//
// The reference reduces the whole vocabulary in one 256-thread workgroup. Here the vocabulary
// is split over many workgroups (one (max, lowest index) partial each), and a one-workgroup
// second launch reduces the partials in index order: the same deterministic pair.
#include "eg_internal.hpp"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 16;

__device__ __forceinline__ void block_best(float& bv, uint32_t& bi, float* wv, uint32_t* wi) {
  egd::team_argmax<64>(bv, bi);
  if ((threadIdx.x & 63u) == 0) {
    wv[threadIdx.x >> 6] = bv;
    wi[threadIdx.x >> 6] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < kThreads / 64; k++)
      if (egd::better(wv[k], wi[k], wv[0], wi[0])) {
        wv[0] = wv[k];
        wi[0] = wi[k];
      }
  }
  __syncthreads();
  bv = wv[0];
  bi = wi[0];
}

__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* __restrict__ logits, uint32_t count,
                                                          uint32_t* partials) {
  float bv = -1.0e30f;
  uint32_t bi = 0;
  const uint32_t per_block = kThreads * kPerThread;
  for (uint32_t base = blockIdx.x * per_block; base < count; base += gridDim.x * per_block) {
#pragma unroll
    for (int r = 0; r < kPerThread; r++) {
      const uint32_t i = base + r * kThreads + threadIdx.x;
      if (i < count) {
        const float v = logits[i];
        if (egd::better(v, i, bv, bi)) {
          bv = v;
          bi = i;
        }
      }
    }
  }
  __shared__ float wv[kThreads / 64];
  __shared__ uint32_t wi[kThreads / 64];
  block_best(bv, bi, wv, wi);
  if (threadIdx.x == 0) {
    partials[2 * blockIdx.x] = __float_as_uint(bv);
    partials[2 * blockIdx.x + 1] = bi;
  }
}

// Up to kFinalPerThread partials per thread are loaded at once (one round trip for the largest
// grids, 2048 partials); more take a loop.
constexpr uint32_t kFinalPerThread = 8;

__global__ __launch_bounds__(kThreads) void finalize_kernel(const uint32_t* partials, uint32_t groups,
                                                            uint32_t sentinel_index, uint32_t* result) {
  float bv = -1.0e30f;
  uint32_t bi = sentinel_index;
  const auto pb = egd::buffer(partials, groups * 8u);  // past the partials: zeros, masked below
  uint64_t pv[kFinalPerThread];
#pragma unroll
  for (uint32_t r = 0; r < kFinalPerThread; r++) pv[r] = egd::load_b64(pb, (threadIdx.x + r * kThreads) * 8u);
#pragma unroll
  for (uint32_t r = 0; r < kFinalPerThread; r++) {
    const float v = __uint_as_float((uint32_t)pv[r]);
    const uint32_t i = (uint32_t)(pv[r] >> 32);
    if (threadIdx.x + r * kThreads < groups && egd::better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  for (uint32_t b = threadIdx.x + kFinalPerThread * kThreads; b < groups; b += kThreads) {
    const float v = __uint_as_float(partials[2 * b]);
    const uint32_t i = partials[2 * b + 1];
    if (egd::better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  __shared__ float wv[kThreads / 64];
  __shared__ uint32_t wi[kThreads / 64];
  block_best(bv, bi, wv, wi);
  if (threadIdx.x == 0) {
    result[0] = bi;
    result[1] = __float_as_uint(bv);
  }
}

}  // namespace

void eg::launch_argmax_finalize(eg_context* ctx, const uint32_t* partials, uint32_t groups, uint32_t sentinel_index,
                                uint32_t* result) {
  hipLaunchKernelGGL(finalize_kernel, dim3(1), dim3(kThreads), 0, ctx->stream, partials, groups, sentinel_index,
                     result);
}

extern "C" int eg_argmax(eg_context* ctx, const float* logits, uint32_t* out, const eg_argmax_dims* dims) {
  if (!ctx) return eg::fail(nullptr, EG_ERR_INVALID, "argmax: ctx is NULL");
  if (!logits || !out || !dims) return eg::fail(ctx, EG_ERR_INVALID, "argmax: NULL argument");
  if (dims->count == 0) return eg::fail(ctx, EG_ERR_INVALID, "argmax: count is 0");
  const uint32_t per_block = kThreads * kPerThread;
  uint64_t blocks = (dims->count + per_block - 1) / per_block;
  const uint64_t cap = (uint64_t)ctx->cu_count * 2;
  if (blocks > cap) blocks = cap;
  uint32_t* partials = reinterpret_cast<uint32_t*>(eg::partials(ctx));
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, ctx->stream, logits + dims->offset,
                     dims->count, partials);
  eg::launch_argmax_finalize(ctx, partials, (uint32_t)blocks, 0, out);
  return eg::check_launch(ctx, "argmax");
}
