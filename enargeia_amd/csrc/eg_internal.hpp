// Internal plumbing shared by the HIP translation units: the context, error reporting and the
// device-side helpers every kernel uses. Not part of the ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "../../include/enargeia_hip.h"

struct eg_context {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;  // own_stream or a caller's stream
  int cu_count = 256;
  // Workspace for cross-workgroup reductions (partials, histograms, arrival counters).
  // Counters are zeroed once at creation and left at zero by every kernel that uses them,
  // so no memset is ever recorded into a captured graph.
  uint8_t* workspace = nullptr;
  size_t workspace_bytes = 0;
  bool capturing = false;
  char error[512] = {0};
};

struct eg_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace eg {

int fail(eg_context* ctx, int status, const char* fmt, ...) __attribute__((format(printf, 3, 4)));
int hip_fail(eg_context* ctx, hipError_t err, const char* what);

// Workspace layout (bytes from ctx->workspace). Fixed offsets; sizes bound the op limits.
constexpr size_t kCountersOffset = 0;          // 64 u32 arrival counters
constexpr size_t kStateOffset = 256;           // 4 KiB of small per-op state
constexpr size_t kPartialsOffset = 8192;       // per-workgroup partials
constexpr size_t kWorkspaceBytes = 16u << 20;  // 16 MiB

enum Counter : int {
  kCounterLmHeadArgmax = 0,
  kCounterArgmax = 1,
  kCounterSampleBase = 8,  // the sampler uses kCounterSampleBase .. +15
};

inline uint32_t* counters(eg_context* ctx) {
  return reinterpret_cast<uint32_t*>(ctx->workspace + kCountersOffset);
}
inline uint8_t* state(eg_context* ctx) { return ctx->workspace + kStateOffset; }
inline uint8_t* partials(eg_context* ctx) { return ctx->workspace + kPartialsOffset; }
constexpr size_t kPartialsBytes = kWorkspaceBytes - kPartialsOffset;

// Validates a launch once the kernel is enqueued (hipGetLastError catches bad configurations
// immediately; faults surface at the next synchronisation).
int check_launch(eg_context* ctx, const char* op);

}  // namespace eg

// ---- device helpers ---------------------------------------------------------------------

namespace egd {

// Opaque AND: keeps the compiler from folding a nibble mask into per-element bitfield
// extracts, so the byte converts (v_cvt_f32_ubyte0..3) consume the masked word directly.
__device__ __forceinline__ uint32_t and_opaque(uint32_t v, uint32_t m) {
  uint32_t r;
  asm("v_and_b32 %0, %1, %2" : "=v"(r) : "v"(m), "v"(v));
  return r;
}
__device__ __forceinline__ float ub0(uint32_t v) { return (float)(v & 0xffu); }
__device__ __forceinline__ float ub1(uint32_t v) { return (float)((v >> 8) & 0xffu); }
__device__ __forceinline__ float ub2(uint32_t v) { return (float)((v >> 16) & 0xffu); }
__device__ __forceinline__ float ub3(uint32_t v) { return (float)(v >> 24); }

// Sum across a team of TEAM consecutive lanes (power of two <= 64); every lane of the team
// receives the total. Fixed butterfly order, so the result is deterministic.
template <int TEAM>
__device__ __forceinline__ float team_sum(float v) {
#pragma unroll
  for (int m = TEAM / 2; m > 0; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// (value, index) ordering used by every argmax here: larger value wins, ties go to the lower
// index (argmax.wgsl:53-57, sample.wgsl:181-186).
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return v > bv || (v == bv && i < bi);
}

template <int WIDTH>
__device__ __forceinline__ void team_argmax(float& v, uint32_t& i) {
#pragma unroll
  for (int m = WIDTH / 2; m > 0; m >>= 1) {
    float ov = __shfl_xor(v, m, 64);
    uint32_t oi = __shfl_xor(i, m, 64);
    if (better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

// Arrival at a per-op counter after a workgroup published its partial results. Returns true
// in exactly one workgroup, the last to arrive, which may then read every workgroup's
// partials. Each thread releases its own partial writes at agent scope (written back past
// this XCD's L2) before thread 0 counts the arrival; the last workgroup acquires at agent
// scope (stale L2 lines invalidated) before reading. The last arrival resets the counter to
// zero for the next launch. Call from all threads of the workgroup.
__device__ __forceinline__ bool last_arrival(uint32_t* counter, uint32_t expected) {
  __shared__ uint32_t is_last;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    is_last = (prev == expected - 1) ? 1u : 0u;
    if (is_last) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const bool last = is_last != 0;
  if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  return last;
}

}  // namespace egd
