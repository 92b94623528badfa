// Context, buffers, errors and graph capture: the part of the ABI that replaces the
// reference's gpu layer (src/gpu/device.ts, pool.ts, readback.ts) for this path.
#include <algorithm>
#include <cstdlib>

#include "eg_internal.hpp"

namespace {
thread_local char g_thread_error[512] = {0};

__global__ void zero_fill_kernel(uint8_t* dst, size_t bytes) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  // 16-byte body when aligned, byte tail otherwise.
  if ((reinterpret_cast<uintptr_t>(dst) & 15u) == 0) {
    uint4* d4 = reinterpret_cast<uint4*>(dst);
    size_t n4 = bytes / 16;
    for (size_t j = i; j < n4; j += stride) d4[j] = make_uint4(0, 0, 0, 0);
    for (size_t j = n4 * 16 + i; j < bytes; j += stride) dst[j] = 0;
  } else {
    for (size_t j = i; j < bytes; j += stride) dst[j] = 0;
  }
}
}  // namespace

namespace eg {

int fail(eg_context* ctx, int status, const char* fmt, ...) {
  char* buf = ctx ? ctx->error : g_thread_error;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, 512, fmt, ap);
  va_end(ap);
  if (ctx) std::memcpy(g_thread_error, ctx->error, 512);
  return status;
}

int hip_fail(eg_context* ctx, hipError_t err, const char* what) {
  int status = err == hipErrorOutOfMemory ? EG_ERR_NOMEM : EG_ERR_DEVICE;
  return fail(ctx, status, "%s: %s (%s)", what, hipGetErrorString(err), hipGetErrorName(err));
}

int occupancy_of(eg_context* ctx, const void* kernel, uint32_t smem_bytes) {
  const uint64_t key = reinterpret_cast<uint64_t>(kernel) ^ ((uint64_t)smem_bytes << 48);
  std::lock_guard<std::mutex> guard(ctx->occupancy_lock);
  auto it = ctx->occupancy.find(key);
  if (it != ctx->occupancy.end()) return it->second;
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, 256, smem_bytes) != hipSuccess) {
    (void)hipGetLastError();
    blocks = 0;
  }
  ctx->occupancy.emplace(key, blocks);
  return blocks;
}

int check_launch(eg_context* ctx, const char* op) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return hip_fail(ctx, err, op);
  return EG_OK;
}

}  // namespace eg

using eg::fail;
using eg::hip_fail;

extern "C" {

int eg_abi_version(void) { return EG_ABI_VERSION; }

const char* eg_last_error(const eg_context* ctx) { return ctx ? ctx->error : g_thread_error; }

int eg_create(int device, eg_context** out_ctx) {
  if (!out_ctx) return fail(nullptr, EG_ERR_INVALID, "eg_create: out_ctx is NULL");
  *out_ctx = nullptr;
  int count = 0;
  hipError_t err = hipGetDeviceCount(&count);
  if (err != hipSuccess) return hip_fail(nullptr, err, "eg_create: hipGetDeviceCount");
  if (device < 0 || device >= count)
    return fail(nullptr, EG_ERR_INVALID, "eg_create: device %d out of range (%d devices)", device, count);
  err = hipSetDevice(device);
  if (err != hipSuccess) return hip_fail(nullptr, err, "eg_create: hipSetDevice");

  eg_context* ctx = new eg_context();
  ctx->device = device;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess) ctx->cu_count = prop.multiProcessorCount;
  // Default priority only; non-blocking so it does not serialise against the null stream.
  err = hipStreamCreateWithFlags(&ctx->own_stream, hipStreamNonBlocking);
  if (err != hipSuccess) {
    delete ctx;
    return hip_fail(nullptr, err, "eg_create: hipStreamCreateWithFlags");
  }
  ctx->stream = ctx->own_stream;
  if (const char* shape = std::getenv("EG_GEMV_SHAPE")) {
    int t = 0, c = 0, u = 0, d = 2;
    const int got = std::sscanf(shape, "%d,%d,%d,%d", &t, &c, &u, &d);
    if (got >= 3 && (t == 8 || t == 16 || t == 32 || t == 64) && c >= 1 && c <= 4 && (u == 1 || u == 2 || u == 4) &&
        d >= 2 && d <= 8) {
      ctx->gemv_override[0] = t;
      ctx->gemv_override[1] = c;
      ctx->gemv_override[2] = u;
      ctx->gemv_override[3] = d;
    }
  }
  if (const char* tpw = std::getenv("EG_FUSED_TILES_PER_WAVE")) {
    const int v = std::atoi(tpw);
    if (v >= 1 && v <= 64) ctx->fused_tiles_per_wave = (uint32_t)v;
  }
  if (const char* pp = std::getenv("EG_PREFILL_PAIR")) ctx->prefill_pair = std::atoi(pp) != 0;
  if (const char* pr = std::getenv("EG_PREFILL_ROPE")) ctx->prefill_rope = std::atoi(pr) != 0;
  if (const char* xb = std::getenv("EG_PREFILL_XB16")) ctx->prefill_xb16 = std::atoi(xb) != 0;
  if (const char* xc = std::getenv("EG_PREFILL_XCD")) ctx->prefill_xcd = std::atoi(xc) != 0;
  if (const char* dp = std::getenv("EG_DECODE_PERSISTENT")) ctx->decode_persistent = std::atoi(dp) != 0;
  if (const char* pg = std::getenv("EG_PERSISTENT_GRID")) ctx->persistent_grid = (uint32_t)std::max(0, std::atoi(pg));
  if (const char* pp = std::getenv("EG_PERSISTENT_POLL")) ctx->persistent_poll = (uint32_t)std::min(64, std::max(0, std::atoi(pp)));
  if (const char* a = std::getenv("EG_ATTENTION_SPLIT")) {
    int t = 0, f = 0;
    if (std::sscanf(a, "%d,%d", &t, &f) == 2 && t >= 1 && t <= 64 && f >= 1 && f <= 8) {
      ctx->attention_split_tiles = (uint32_t)t;
      ctx->attention_split_fill = (uint32_t)f;
    }
  }
  if (const char* g = std::getenv("EG_PREFILL_GROUPS")) {
    const int v = std::atoi(g);
    if (v == 1 || v == 2 || v == 4) ctx->prefill_groups = v;
  }
  err = hipMalloc(&ctx->workspace, eg::kWorkspaceBytes);
  if (err != hipSuccess) {
    hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return hip_fail(nullptr, err, "eg_create: workspace");
  }
  ctx->workspace_bytes = eg::kWorkspaceBytes;
  // Counters and state start at zero; this is the only memset and it is never captured.
  err = hipMemset(ctx->workspace, 0, eg::kPartialsOffset);
  if (err == hipSuccess) err = hipDeviceSynchronize();
  if (err != hipSuccess) {
    hipFree(ctx->workspace);
    hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return hip_fail(nullptr, err, "eg_create: workspace init");
  }
  if (eg::noalloc_scratch_init(ctx) != EG_OK) {
    fail(nullptr, EG_ERR_DEVICE, "%s", ctx->error);
    hipFree(ctx->workspace);
    hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return EG_ERR_DEVICE;
  }
  *out_ctx = ctx;
  return EG_OK;
}

int eg_destroy(eg_context* ctx) {
  if (!ctx) return EG_OK;
  hipSetDevice(ctx->device);
  hipStreamSynchronize(ctx->own_stream);
  if (ctx->workspace) hipFree(ctx->workspace);
  hipStreamDestroy(ctx->own_stream);
  delete ctx;
  return EG_OK;
}

int eg_get_stream(eg_context* ctx, void** out_stream) {
  if (!ctx || !out_stream) return fail(ctx, EG_ERR_INVALID, "eg_get_stream: NULL argument");
  *out_stream = reinterpret_cast<void*>(ctx->stream);
  return EG_OK;
}

int eg_set_stream(eg_context* ctx, void* stream) {
  if (!ctx) return fail(nullptr, EG_ERR_INVALID, "eg_set_stream: ctx is NULL");
  if (ctx->capturing) return fail(ctx, EG_ERR_STATE, "eg_set_stream: a graph capture is in progress");
  ctx->stream = stream ? reinterpret_cast<hipStream_t>(stream) : ctx->own_stream;
  return EG_OK;
}

int eg_sync(eg_context* ctx) {
  if (!ctx) return fail(nullptr, EG_ERR_INVALID, "eg_sync: ctx is NULL");
  if (ctx->capturing) return fail(ctx, EG_ERR_STATE, "eg_sync: a graph capture is in progress");
  hipError_t err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess) return hip_fail(ctx, err, "eg_sync");
  return eg::report_sample_failures(ctx, "eg_sync");
}

int eg_buf_alloc(eg_context* ctx, size_t bytes, void** out_ptr) {
  if (!ctx || !out_ptr) return fail(ctx, EG_ERR_INVALID, "eg_buf_alloc: NULL argument");
  *out_ptr = nullptr;
  if (bytes == 0) bytes = 4;  // as the reference's pool.acquire(Math.max(4, ...))
  hipError_t err = hipMalloc(out_ptr, bytes);
  if (err != hipSuccess) return hip_fail(ctx, err, "eg_buf_alloc");
  return EG_OK;
}

int eg_buf_free(eg_context* ctx, void* ptr) {
  if (!ctx) return fail(nullptr, EG_ERR_INVALID, "eg_buf_free: ctx is NULL");
  if (!ptr) return EG_OK;
  hipError_t err = hipFree(ptr);
  if (err != hipSuccess) return hip_fail(ctx, err, "eg_buf_free");
  return EG_OK;
}

int eg_buf_write(eg_context* ctx, void* dst, size_t offset, const void* host_src, size_t bytes) {
  if (!ctx || !dst || (!host_src && bytes))
    return fail(ctx, EG_ERR_INVALID, "eg_buf_write: NULL argument");
  if (bytes == 0) return EG_OK;
  hipError_t err = hipMemcpyAsync(static_cast<uint8_t*>(dst) + offset, host_src, bytes,
                                  hipMemcpyHostToDevice, ctx->stream);
  if (err != hipSuccess) return hip_fail(ctx, err, "eg_buf_write");
  return EG_OK;
}

int eg_buf_read(eg_context* ctx, const void* src, size_t offset, void* host_dst, size_t bytes) {
  if (!ctx || !src || (!host_dst && bytes))
    return fail(ctx, EG_ERR_INVALID, "eg_buf_read: NULL argument");
  if (ctx->capturing) return fail(ctx, EG_ERR_STATE, "eg_buf_read: a graph capture is in progress");
  if (bytes == 0) return EG_OK;
  hipError_t err = hipMemcpyAsync(host_dst, static_cast<const uint8_t*>(src) + offset, bytes,
                                  hipMemcpyDeviceToHost, ctx->stream);
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
  if (err != hipSuccess) return hip_fail(ctx, err, "eg_buf_read");
  return eg::report_sample_failures(ctx, "eg_buf_read");
}

int eg_buf_zero(eg_context* ctx, void* dst, size_t offset, size_t bytes) {
  if (!ctx || !dst) return fail(ctx, EG_ERR_INVALID, "eg_buf_zero: NULL argument");
  if (bytes == 0) return EG_OK;
  size_t blocks = (bytes / 16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 4096) blocks = 4096;
  zero_fill_kernel<<<(unsigned)blocks, 256, 0, ctx->stream>>>(static_cast<uint8_t*>(dst) + offset, bytes);
  return eg::check_launch(ctx, "eg_buf_zero");
}

int eg_test_launch_stamps(eg_context* ctx, uint64_t* buffer, uint32_t launches, uint32_t* recorded) {
  if (!ctx) return fail(nullptr, EG_ERR_INVALID, "test_launch_stamps: ctx is NULL");
  if (ctx->capturing) return fail(ctx, EG_ERR_STATE, "test_launch_stamps: a graph capture is in progress");
  if (!egd::kLaunchStamps && buffer)
    return fail(ctx, EG_ERR_STATE,
                "test_launch_stamps: this library is built without launch stamps; the profiling build "
                "(libenargeia_hip_prof.so, EG_LAUNCH_STAMPS) records them");
  if (recorded) *recorded = ctx->stamp_next;
  ctx->stamps = buffer;
  ctx->stamp_capacity = buffer ? launches : 0u;
  ctx->stamp_next = 0;
  return EG_OK;
}

int eg_graph_begin(eg_context* ctx) {
  if (!ctx) return fail(nullptr, EG_ERR_INVALID, "eg_graph_begin: ctx is NULL");
  if (ctx->capturing) return fail(ctx, EG_ERR_STATE, "eg_graph_begin: capture already in progress");
  if (ctx->stream == nullptr)
    return fail(ctx, EG_ERR_STATE, "eg_graph_begin: cannot capture the null stream");
  hipError_t err = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
  if (err != hipSuccess) return hip_fail(ctx, err, "eg_graph_begin");
  ctx->capturing = true;
  return EG_OK;
}

int eg_graph_end(eg_context* ctx, eg_graph** out_graph) {
  if (!ctx || !out_graph) return fail(ctx, EG_ERR_INVALID, "eg_graph_end: NULL argument");
  if (!ctx->capturing) return fail(ctx, EG_ERR_STATE, "eg_graph_end: no capture in progress");
  *out_graph = nullptr;
  ctx->capturing = false;
  eg_graph* g = new eg_graph();
  hipError_t err = hipStreamEndCapture(ctx->stream, &g->graph);
  if (err != hipSuccess) {
    delete g;
    return hip_fail(ctx, err, "eg_graph_end: hipStreamEndCapture");
  }
  err = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    hipGraphDestroy(g->graph);
    delete g;
    return hip_fail(ctx, err, "eg_graph_end: hipGraphInstantiate");
  }
  *out_graph = g;
  return EG_OK;
}

int eg_graph_launch(eg_context* ctx, eg_graph* graph) {
  if (!ctx || !graph) return fail(ctx, EG_ERR_INVALID, "eg_graph_launch: NULL argument");
  if (ctx->capturing) return fail(ctx, EG_ERR_STATE, "eg_graph_launch: a capture is in progress");
  hipError_t err = hipGraphLaunch(graph->exec, ctx->stream);
  if (err != hipSuccess) return hip_fail(ctx, err, "eg_graph_launch");
  return EG_OK;
}

int eg_graph_destroy(eg_graph* graph) {
  if (!graph) return EG_OK;
  if (graph->exec) hipGraphExecDestroy(graph->exec);
  if (graph->graph) hipGraphDestroy(graph->graph);
  delete graph;
  return EG_OK;
}

}  // extern "C"
