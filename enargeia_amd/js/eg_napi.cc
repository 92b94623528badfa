// Node N-API addon over the C ABI in include/enargeia_hip.h.
//
// This is the thin native layer the reference's TypeScript would bind instead of WebGPU: one
// JS function per C entry point, device pointers as JS numbers (safe integers), uniforms as the
// same ArrayBuffer bytes the reference writes with queue.writeBuffer (matmul_q4.ts:50-64,
// embedding_variants.ts:207-221, argmax.ts:16-18, sample.ts:35-50). A non-zero status becomes
// a thrown RangeError (EG_ERR_RANGE, as kernel.ts:97-107 throws) or Error (everything else)
// carrying eg_last_error's message and the status name as `code`. Nothing here allocates on
// the device except eg_buf_alloc; nothing here launches a kernel except the op calls.
#include <node_api.h>

#include <cstdint>
#include <cstring>
#include <string>
#include <utility>
#include <vector>

#include "enargeia_hip.h"

namespace {

const char* status_name(int st) {
  switch (st) {
    case EG_ERR_INVALID: return "EG_ERR_INVALID";
    case EG_ERR_RANGE: return "EG_ERR_RANGE";
    case EG_ERR_DEVICE: return "EG_ERR_DEVICE";
    case EG_ERR_NOMEM: return "EG_ERR_NOMEM";
    case EG_ERR_STATE: return "EG_ERR_STATE";
    case EG_ERR_FORMAT: return "EG_ERR_FORMAT";
    case EG_ERR_IO: return "EG_ERR_IO";
    case EG_ERR_NOT_FOUND: return "EG_ERR_NOT_FOUND";
    default: return "EG_ERR_UNKNOWN";
  }
}

// Throws for a failed status; returns true when the caller should return early. A malformed
// container throws an Error named EnargeiaError, as the reference's parser does (enargeia.ts:84).
bool throw_status(napi_env env, eg_context* ctx, int st) {
  if (st == EG_OK) return false;
  const char* msg = eg_last_error(ctx);
  if (st == EG_ERR_RANGE) {
    napi_throw_range_error(env, status_name(st), msg);
  } else if (st == EG_ERR_FORMAT) {
    napi_value code, text, err, name;
    napi_create_string_utf8(env, status_name(st), NAPI_AUTO_LENGTH, &code);
    napi_create_string_utf8(env, msg, NAPI_AUTO_LENGTH, &text);
    napi_create_error(env, code, text, &err);
    napi_create_string_utf8(env, "EnargeiaError", NAPI_AUTO_LENGTH, &name);
    napi_set_named_property(env, err, "name", name);
    napi_throw(env, err);
  } else {
    napi_throw_error(env, status_name(st), msg);
  }
  return true;
}

void throw_type(napi_env env, const std::string& what) { napi_throw_type_error(env, "EG_ERR_INVALID", what.c_str()); }

struct DecoderHandle;
struct ContainerHandle {
  eg_container* c;
};

// One type tag per kind of handle.
template <typename T>
const napi_type_tag& tag_of();
template <>
const napi_type_tag& tag_of<eg_context>() {
  static const napi_type_tag t{0x45474354584e4150ull, 0x0000000000000001ull};
  return t;
}
template <>
const napi_type_tag& tag_of<eg_graph>() {
  static const napi_type_tag t{0x45474354584e4150ull, 0x0000000000000002ull};
  return t;
}
template <>
const napi_type_tag& tag_of<DecoderHandle>() {
  static const napi_type_tag t{0x45474354584e4150ull, 0x0000000000000003ull};
  return t;
}

template <>
const napi_type_tag& tag_of<ContainerHandle>() {
  static const napi_type_tag t{0x45474354584e4150ull, 0x0000000000000004ull};
  return t;
}

template <typename T>
napi_value make_handle(napi_env env, T* p, napi_finalize fin) {
  napi_value ext;
  napi_create_external(env, p, fin, nullptr, &ext);
  napi_type_tag_object(env, ext, &tag_of<T>());
  return ext;
}

struct Args {
  napi_env env;
  size_t argc = 12;
  napi_value argv[12];
  bool ok = true;
  const char* fn;

  Args(napi_env e, napi_callback_info info, const char* name, size_t need) : env(e), fn(name) {
    napi_get_cb_info(env, info, &argc, argv, nullptr, nullptr);
    if (argc < need) {
      throw_type(env, std::string(fn) + ": expected " + std::to_string(need) + " arguments, got " +
                          std::to_string(argc));
      ok = false;
    }
  }

  // A context, graph or decoder handle: an External this addon created and type-tagged, so a
  // handle of one kind passed where another is expected is a TypeError, not a crash.
  template <typename T>
  T* handle(size_t i, const char* what) {
    if (!ok) return nullptr;
    napi_valuetype t;
    napi_typeof(env, argv[i], &t);
    void* p = nullptr;
    bool tagged = false;
    if (t == napi_external) napi_check_object_type_tag(env, argv[i], &tag_of<T>(), &tagged);
    if (t != napi_external || !tagged || napi_get_value_external(env, argv[i], &p) != napi_ok) {
      throw_type(env, std::string(fn) + ": argument " + std::to_string(i) + " is not a " + what);
      ok = false;
      return nullptr;
    }
    return static_cast<T*>(p);
  }

  // A device pointer: a non-negative safe integer, or null/undefined for NULL.
  void* ptr(size_t i) {
    if (!ok) return nullptr;
    napi_valuetype t;
    napi_typeof(env, argv[i], &t);
    if (t == napi_null || t == napi_undefined) return nullptr;
    double d = 0;
    if (t != napi_number || napi_get_value_double(env, argv[i], &d) != napi_ok || d < 0 ||
        d > 9007199254740991.0 || d != (double)(int64_t)d) {
      throw_type(env, std::string(fn) + ": argument " + std::to_string(i) + " is not a device pointer");
      ok = false;
      return nullptr;
    }
    return reinterpret_cast<void*>(static_cast<uintptr_t>(d));
  }

  uint64_t u64(size_t i) {
    if (!ok) return 0;
    double d = 0;
    napi_valuetype t;
    napi_typeof(env, argv[i], &t);
    if (t != napi_number || napi_get_value_double(env, argv[i], &d) != napi_ok || d < 0 ||
        d > 9007199254740991.0 || d != (double)(int64_t)d) {
      throw_type(env, std::string(fn) + ": argument " + std::to_string(i) + " is not a non-negative integer");
      ok = false;
      return 0;
    }
    return static_cast<uint64_t>(d);
  }

  int32_t i32(size_t i) {
    if (!ok) return 0;
    int32_t v = 0;
    if (napi_get_value_int32(env, argv[i], &v) != napi_ok) {
      throw_type(env, std::string(fn) + ": argument " + std::to_string(i) + " is not a number");
      ok = false;
    }
    return v;
  }

  // Bytes of an ArrayBuffer, TypedArray or DataView.
  bool bytes(size_t i, void** data, size_t* len) {
    if (!ok) return false;
    bool is = false;
    napi_is_typedarray(env, argv[i], &is);
    if (is) {
      napi_typedarray_type type;
      size_t length, offset;
      napi_value ab;
      void* base;
      napi_get_typedarray_info(env, argv[i], &type, &length, &base, &ab, &offset);
      size_t elem = 1;
      switch (type) {
        case napi_int16_array: case napi_uint16_array: elem = 2; break;
        case napi_int32_array: case napi_uint32_array: case napi_float32_array: elem = 4; break;
        case napi_float64_array: case napi_bigint64_array: case napi_biguint64_array: elem = 8; break;
        default: elem = 1;
      }
      *data = base;  // napi_get_typedarray_info already applies the byte offset
      *len = length * elem;
      return true;
    }
    napi_is_dataview(env, argv[i], &is);
    if (is) {
      napi_value ab;
      size_t offset;
      napi_get_dataview_info(env, argv[i], len, data, &ab, &offset);
      return true;
    }
    napi_is_arraybuffer(env, argv[i], &is);
    if (is) {
      napi_get_arraybuffer_info(env, argv[i], data, len);
      return true;
    }
    throw_type(env, std::string(fn) + ": argument " + std::to_string(i) + " is not an ArrayBuffer or view");
    ok = false;
    return false;
  }

  // A uniform: at least sizeof(T) bytes, copied into a T.
  template <typename T>
  bool uniform(size_t i, T* out) {
    void* data;
    size_t len;
    if (!bytes(i, &data, &len)) return false;
    if (len < sizeof(T)) {
      throw_type(env, std::string(fn) + ": uniform of " + std::to_string(len) + " bytes, expected " +
                          std::to_string(sizeof(T)));
      ok = false;
      return false;
    }
    std::memcpy(out, data, sizeof(T));
    return true;
  }
};

napi_value undefined(napi_env env) {
  napi_value v;
  napi_get_undefined(env, &v);
  return v;
}

napi_value number(napi_env env, double d) {
  napi_value v;
  napi_create_double(env, d, &v);
  return v;
}

// ---- context ---------------------------------------------------------------------------------

void finalize_ctx(napi_env, void*, void*) {
  // Contexts are destroyed explicitly (destroy()); the External only carries the address, so a
  // collected handle leaks nothing the process end does not reclaim.
}

napi_value AbiVersion(napi_env env, napi_callback_info) { return number(env, eg_abi_version()); }

napi_value Create(napi_env env, napi_callback_info info) {
  Args a(env, info, "create", 1);
  int device = a.i32(0);
  if (!a.ok) return nullptr;
  eg_context* ctx = nullptr;
  if (throw_status(env, nullptr, eg_create(device, &ctx))) return nullptr;
  return make_handle(env, ctx, finalize_ctx);
}

napi_value Destroy(napi_env env, napi_callback_info info) {
  Args a(env, info, "destroy", 1);
  auto* ctx = a.handle<eg_context>(0, "context");
  if (!a.ok) return nullptr;
  eg_destroy(ctx);
  return undefined(env);
}

napi_value Sync(napi_env env, napi_callback_info info) {
  Args a(env, info, "sync", 1);
  auto* ctx = a.handle<eg_context>(0, "context");
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_sync(ctx))) return nullptr;
  return undefined(env);
}

napi_value GetStream(napi_env env, napi_callback_info info) {
  Args a(env, info, "getStream", 1);
  auto* ctx = a.handle<eg_context>(0, "context");
  if (!a.ok) return nullptr;
  void* s = nullptr;
  if (throw_status(env, ctx, eg_get_stream(ctx, &s))) return nullptr;
  return number(env, (double)reinterpret_cast<uintptr_t>(s));
}

// ---- buffers ---------------------------------------------------------------------------------

napi_value BufAlloc(napi_env env, napi_callback_info info) {
  Args a(env, info, "bufAlloc", 2);
  auto* ctx = a.handle<eg_context>(0, "context");
  uint64_t bytes = a.u64(1);
  if (!a.ok) return nullptr;
  void* p = nullptr;
  if (throw_status(env, ctx, eg_buf_alloc(ctx, bytes, &p))) return nullptr;
  return number(env, (double)reinterpret_cast<uintptr_t>(p));
}

napi_value BufFree(napi_env env, napi_callback_info info) {
  Args a(env, info, "bufFree", 2);
  auto* ctx = a.handle<eg_context>(0, "context");
  void* p = a.ptr(1);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_buf_free(ctx, p))) return nullptr;
  return undefined(env);
}

// bufWrite(ctx, ptr, offset, data): completes before returning (the JS source may be collected
// or reused as soon as the call returns, so the copy is synchronised here).
napi_value BufWrite(napi_env env, napi_callback_info info) {
  Args a(env, info, "bufWrite", 4);
  auto* ctx = a.handle<eg_context>(0, "context");
  void* p = a.ptr(1);
  uint64_t offset = a.u64(2);
  void* data = nullptr;
  size_t len = 0;
  a.bytes(3, &data, &len);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_buf_write(ctx, p, offset, data, len))) return nullptr;
  if (throw_status(env, ctx, eg_sync(ctx))) return nullptr;
  return undefined(env);
}

// bufRead(ctx, ptr, offset, bytes) -> ArrayBuffer, after all prior work on the stream.
napi_value BufRead(napi_env env, napi_callback_info info) {
  Args a(env, info, "bufRead", 4);
  auto* ctx = a.handle<eg_context>(0, "context");
  void* p = a.ptr(1);
  uint64_t offset = a.u64(2);
  uint64_t bytes = a.u64(3);
  if (!a.ok) return nullptr;
  void* host = nullptr;
  napi_value ab;
  if (napi_create_arraybuffer(env, bytes, &host, &ab) != napi_ok) {
    napi_throw_error(env, "EG_ERR_NOMEM", "bufRead: cannot allocate the host buffer");
    return nullptr;
  }
  if (throw_status(env, ctx, eg_buf_read(ctx, p, offset, host, bytes))) return nullptr;
  return ab;
}

napi_value BufZero(napi_env env, napi_callback_info info) {
  Args a(env, info, "bufZero", 4);
  auto* ctx = a.handle<eg_context>(0, "context");
  void* p = a.ptr(1);
  uint64_t offset = a.u64(2);
  uint64_t bytes = a.u64(3);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_buf_zero(ctx, p, offset, bytes))) return nullptr;
  return undefined(env);
}

// ---- ops -------------------------------------------------------------------------------------

// matmulQ4Decode / matmulQ4Prefill(ctx, x, packed, scales, zeros, bias, out, dims, encoding, bits)
template <int (*FN)(eg_context*, const float*, const uint32_t*, const float*, const uint32_t*, const float*,
                    float*, const eg_matmul_q4_dims*, int, int)>
napi_value Matmul(napi_env env, napi_callback_info info) {
  Args a(env, info, "matmulQ4", 10);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* x = static_cast<const float*>(a.ptr(1));
  auto* packed = static_cast<const uint32_t*>(a.ptr(2));
  auto* scales = static_cast<const float*>(a.ptr(3));
  auto* zeros = static_cast<const uint32_t*>(a.ptr(4));
  auto* bias = static_cast<const float*>(a.ptr(5));
  auto* out = static_cast<float*>(a.ptr(6));
  eg_matmul_q4_dims dims;
  a.uniform(7, &dims);
  int encoding = a.i32(8), bits = a.i32(9);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, FN(ctx, x, packed, scales, zeros, bias, out, &dims, encoding, bits))) return nullptr;
  return undefined(env);
}

// lmHead(ctx, x, packed, scales, zeros, out, dims, encoding, bits)
napi_value LmHead(napi_env env, napi_callback_info info) {
  Args a(env, info, "lmHead", 9);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* x = static_cast<const float*>(a.ptr(1));
  auto* packed = static_cast<const uint32_t*>(a.ptr(2));
  auto* scales = static_cast<const float*>(a.ptr(3));
  auto* zeros = static_cast<const uint32_t*>(a.ptr(4));
  auto* out = static_cast<float*>(a.ptr(5));
  eg_embedding_dims dims;
  a.uniform(6, &dims);
  int encoding = a.i32(7), bits = a.i32(8);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_lm_head(ctx, x, packed, scales, zeros, out, &dims, encoding, bits))) return nullptr;
  return undefined(env);
}

// embedGather(ctx, ids, packed, scales, zeros, out, dims, encoding, bits)
napi_value EmbedGather(napi_env env, napi_callback_info info) {
  Args a(env, info, "embedGather", 9);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* ids = static_cast<const uint32_t*>(a.ptr(1));
  auto* packed = static_cast<const uint32_t*>(a.ptr(2));
  auto* scales = static_cast<const float*>(a.ptr(3));
  auto* zeros = static_cast<const uint32_t*>(a.ptr(4));
  auto* out = static_cast<float*>(a.ptr(5));
  eg_embedding_dims dims;
  a.uniform(6, &dims);
  int encoding = a.i32(7), bits = a.i32(8);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_embed_gather(ctx, ids, packed, scales, zeros, out, &dims, encoding, bits)))
    return nullptr;
  return undefined(env);
}

// lmHeadArgmax(ctx, x, packed, scales, zeros, out|null, result, dims, encoding, bits)
napi_value LmHeadArgmax(napi_env env, napi_callback_info info) {
  Args a(env, info, "lmHeadArgmax", 10);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* x = static_cast<const float*>(a.ptr(1));
  auto* packed = static_cast<const uint32_t*>(a.ptr(2));
  auto* scales = static_cast<const float*>(a.ptr(3));
  auto* zeros = static_cast<const uint32_t*>(a.ptr(4));
  auto* out = static_cast<float*>(a.ptr(5));
  auto* result = static_cast<uint32_t*>(a.ptr(6));
  eg_embedding_dims dims;
  a.uniform(7, &dims);
  int encoding = a.i32(8), bits = a.i32(9);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_lm_head_argmax(ctx, x, packed, scales, zeros, out, result, &dims, encoding, bits)))
    return nullptr;
  return undefined(env);
}

// argmax(ctx, logits, out, dims)
napi_value Argmax(napi_env env, napi_callback_info info) {
  Args a(env, info, "argmax", 4);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* logits = static_cast<const float*>(a.ptr(1));
  auto* out = static_cast<uint32_t*>(a.ptr(2));
  eg_argmax_dims dims;
  a.uniform(3, &dims);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_argmax(ctx, logits, out, &dims))) return nullptr;
  return undefined(env);
}

// sample(ctx, logits, history, out, dims)
napi_value Sample(napi_env env, napi_callback_info info) {
  Args a(env, info, "sample", 5);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* logits = static_cast<float*>(a.ptr(1));
  auto* history = static_cast<const uint32_t*>(a.ptr(2));
  auto* out = static_cast<uint32_t*>(a.ptr(3));
  eg_sample_dims dims;
  a.uniform(4, &dims);
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_sample(ctx, logits, history, out, &dims))) return nullptr;
  return undefined(env);
}

// ---- the decoder --------------------------------------------------------------------------------

// What the External of a decoder carries: the decoder and its context (for error messages).
struct DecoderHandle {
  eg_decoder* dec;
  eg_context* ctx;
};

bool get_prop(napi_env env, napi_value obj, const char* name, napi_value* out) {
  bool has = false;
  if (napi_has_named_property(env, obj, name, &has) != napi_ok || !has) {
    napi_throw_type_error(env, "EG_ERR_INVALID", (std::string("decoderCreate: missing ") + name).c_str());
    return false;
  }
  return napi_get_named_property(env, obj, name, out) == napi_ok;
}

bool get_u32(napi_env env, napi_value obj, const char* name, uint32_t* out) {
  napi_value v;
  if (!get_prop(env, obj, name, &v)) return false;
  if (napi_get_value_uint32(env, v, out) != napi_ok) {
    napi_throw_type_error(env, "EG_ERR_INVALID", (std::string("decoderCreate: ") + name + " is not a number").c_str());
    return false;
  }
  return true;
}

bool get_f32(napi_env env, napi_value obj, const char* name, float* out) {
  napi_value v;
  double d = 0;
  if (!get_prop(env, obj, name, &v)) return false;
  if (napi_get_value_double(env, v, &d) != napi_ok) {
    napi_throw_type_error(env, "EG_ERR_INVALID", (std::string("decoderCreate: ") + name + " is not a number").c_str());
    return false;
  }
  *out = (float)d;
  return true;
}

// A device pointer property: a safe integer, or null/undefined (NULL).
bool get_ptr(napi_env env, napi_value obj, const char* name, const void** out) {
  bool has = false;
  *out = nullptr;
  if (napi_has_named_property(env, obj, name, &has) != napi_ok || !has) return true;
  napi_value v;
  napi_get_named_property(env, obj, name, &v);
  napi_valuetype t;
  napi_typeof(env, v, &t);
  if (t == napi_null || t == napi_undefined) return true;
  double d = 0;
  if (t != napi_number || napi_get_value_double(env, v, &d) != napi_ok || d < 0 || d > 9007199254740991.0 ||
      d != (double)(int64_t)d) {
    napi_throw_type_error(env, "EG_ERR_INVALID", (std::string("decoderCreate: ") + name + " is not a device pointer").c_str());
    return false;
  }
  *out = reinterpret_cast<const void*>(static_cast<uintptr_t>(d));
  return true;
}

bool get_matrix(napi_env env, napi_value obj, const char* name, eg_quant_matrix* m) {
  napi_value v;
  if (!get_prop(env, obj, name, &v)) return false;
  const void *p = nullptr, *s = nullptr, *z = nullptr;
  if (!get_ptr(env, v, "packed", &p) || !get_ptr(env, v, "scales", &s) || !get_ptr(env, v, "zeros", &z)) return false;
  m->packed = static_cast<const uint32_t*>(p);
  m->scales = static_cast<const float*>(s);
  m->zeros = static_cast<const uint32_t*>(z);
  return true;
}

void finalize_decoder(napi_env, void* data, void*) { delete static_cast<DecoderHandle*>(data); }

// decoderCreate(ctx, desc): desc mirrors eg_model_desc with camelCase names and `layer` an array.
napi_value DecoderCreate(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderCreate", 2);
  auto* ctx = a.handle<eg_context>(0, "context");
  if (!a.ok) return nullptr;
  napi_value d = a.argv[1];
  eg_model_desc m{};
  int enc = 0, bits = 0, eenc = 0, ebits = 0;
  uint32_t u = 0;
  const void* final_norm = nullptr;
  if (!get_u32(env, d, "layers", &m.layers) || !get_u32(env, d, "hidden", &m.hidden) ||
      !get_u32(env, d, "heads", &m.heads) || !get_u32(env, d, "kvHeads", &m.kv_heads) ||
      !get_u32(env, d, "headDim", &m.head_dim) || !get_u32(env, d, "intermediate", &m.intermediate) ||
      !get_u32(env, d, "vocab", &m.vocab) || !get_u32(env, d, "maxContext", &m.max_context) ||
      !get_f32(env, d, "rmsEps", &m.rms_eps) || !get_f32(env, d, "ropeTheta", &m.rope_theta) ||
      !get_u32(env, d, "encoding", &u))
    return nullptr;
  enc = (int)u;
  if (!get_u32(env, d, "bits", &u)) return nullptr;
  bits = (int)u;
  if (!get_u32(env, d, "blockSize", &m.block_size) || !get_matrix(env, d, "embedding", &m.embedding) ||
      !get_u32(env, d, "embedEncoding", &u))
    return nullptr;
  eenc = (int)u;
  if (!get_u32(env, d, "embedBits", &u)) return nullptr;
  ebits = (int)u;
  if (!get_u32(env, d, "embedBlockSize", &m.embed_block_size) || !get_ptr(env, d, "finalNorm", &final_norm))
    return nullptr;
  m.encoding = enc;
  m.bits = bits;
  m.embed_encoding = eenc;
  m.embed_bits = ebits;
  m.final_norm = static_cast<const float*>(final_norm);
  napi_value arr;
  if (!get_prop(env, d, "layer", &arr)) return nullptr;
  uint32_t n = 0;
  bool is_array = false;
  napi_is_array(env, arr, &is_array);
  if (!is_array || napi_get_array_length(env, arr, &n) != napi_ok || n != m.layers) {
    napi_throw_type_error(env, "EG_ERR_INVALID", "decoderCreate: layer must be an array of `layers` entries");
    return nullptr;
  }
  std::vector<eg_layer_desc> layers(n);
  for (uint32_t i = 0; i < n; i++) {
    napi_value L;
    napi_get_element(env, arr, i, &L);
    eg_layer_desc& l = layers[i];
    const void *qb = nullptr, *kb = nullptr, *vb = nullptr, *in = nullptr, *pn = nullptr;
    if (!get_matrix(env, L, "q", &l.q) || !get_matrix(env, L, "k", &l.k) || !get_matrix(env, L, "v", &l.v) ||
        !get_matrix(env, L, "o", &l.o) || !get_matrix(env, L, "gate", &l.gate) || !get_matrix(env, L, "up", &l.up) ||
        !get_matrix(env, L, "down", &l.down) || !get_ptr(env, L, "qBias", &qb) || !get_ptr(env, L, "kBias", &kb) ||
        !get_ptr(env, L, "vBias", &vb) || !get_ptr(env, L, "inputNorm", &in) ||
        !get_ptr(env, L, "postAttentionNorm", &pn))
      return nullptr;
    l.q_bias = static_cast<const float*>(qb);
    l.k_bias = static_cast<const float*>(kb);
    l.v_bias = static_cast<const float*>(vb);
    l.input_norm = static_cast<const float*>(in);
    l.post_attention_norm = static_cast<const float*>(pn);
  }
  m.layer = layers.data();
  // optional cacheDType: 'f16' (the default) or 'f32' (SessionOptions.cacheDType, session.ts:44)
  int cache = EG_CACHE_F16;
  bool has_cache = false;
  if (napi_has_named_property(env, d, "cacheDType", &has_cache) == napi_ok && has_cache) {
    napi_value cv;
    char name[8] = {0};
    size_t len = 0;
    napi_get_named_property(env, d, "cacheDType", &cv);
    if (napi_get_value_string_utf8(env, cv, name, sizeof(name), &len) != napi_ok ||
        (std::string(name) != "f16" && std::string(name) != "f32")) {
      napi_throw_type_error(env, "EG_ERR_INVALID", "decoderCreate: cacheDType must be 'f16' or 'f32'");
      return nullptr;
    }
    cache = std::string(name) == "f32" ? EG_CACHE_F32 : EG_CACHE_F16;
  }
  eg_decoder* dec = nullptr;
  if (throw_status(env, ctx, eg_decoder_create_cache(ctx, &m, cache, &dec))) return nullptr;
  return make_handle(env, new DecoderHandle{dec, ctx}, finalize_decoder);
}

napi_value DecoderReset(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderReset", 3);
  auto* h = a.handle<DecoderHandle>(0, "decoder");
  uint64_t position = a.u64(1), token = a.u64(2);
  if (!a.ok) return nullptr;
  if (!h->dec) {
    napi_throw_error(env, "EG_ERR_STATE", "decoderReset: the decoder was destroyed");
    return nullptr;
  }
  if (throw_status(env, h->ctx, eg_decoder_reset(h->dec, (uint32_t)position, (uint32_t)token))) return nullptr;
  return undefined(env);
}

// decoderStep(dec, readToken) -> the new token id (readToken) or undefined
napi_value DecoderStep(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderStep", 2);
  auto* h = a.handle<DecoderHandle>(0, "decoder");
  if (!a.ok) return nullptr;
  bool read = false;
  napi_get_value_bool(env, a.argv[1], &read);
  if (!h->dec) {
    napi_throw_error(env, "EG_ERR_STATE", "decoderStep: the decoder was destroyed");
    return nullptr;
  }
  uint32_t token = 0;
  if (throw_status(env, h->ctx, eg_decoder_step(h->dec, read ? &token : nullptr))) return nullptr;
  return read ? number(env, token) : undefined(env);
}

napi_value DecoderCapture(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderCapture", 1);
  auto* h = a.handle<DecoderHandle>(0, "decoder");
  if (!a.ok) return nullptr;
  if (!h->dec) {
    napi_throw_error(env, "EG_ERR_STATE", "decoderCapture: the decoder was destroyed");
    return nullptr;
  }
  if (throw_status(env, h->ctx, eg_decoder_capture(h->dec))) return nullptr;
  return undefined(env);
}

// A number argument as f32 (sampling parameters, the draw).
bool f32_arg(Args& a, size_t i, float* out) {
  if (!a.ok) return false;
  double d = 0;
  napi_valuetype t;
  napi_typeof(a.env, a.argv[i], &t);
  if (t != napi_number || napi_get_value_double(a.env, a.argv[i], &d) != napi_ok) {
    throw_type(a.env, std::string(a.fn) + ": argument " + std::to_string(i) + " is not a number");
    a.ok = false;
    return false;
  }
  *out = (float)d;
  return true;
}

DecoderHandle* live_decoder(napi_env env, Args& a, const char* fn) {
  auto* h = a.handle<DecoderHandle>(0, "decoder");
  if (!a.ok) return nullptr;
  if (!h->dec) {
    napi_throw_error(env, "EG_ERR_STATE", (std::string(fn) + ": the decoder was destroyed").c_str());
    return nullptr;
  }
  return h;
}

// decoderSetSampling(dec, {temperature, topP, repetitionPenalty}) (DecodeGraph.setSampling)
napi_value DecoderSetSampling(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderSetSampling", 2);
  auto* h = live_decoder(env, a, "decoderSetSampling");
  if (!h) return nullptr;
  eg_sampling_params p{};
  const char* names[3] = {"temperature", "topP", "repetitionPenalty"};
  float* fields[3] = {&p.temperature, &p.top_p, &p.repetition_penalty};
  for (int i = 0; i < 3; i++) {
    napi_value v;
    double d = 0;
    if (napi_get_named_property(env, a.argv[1], names[i], &v) != napi_ok || napi_get_value_double(env, v, &d) != napi_ok) {
      throw_type(env, std::string("decoderSetSampling: params.") + names[i] + " is not a number");
      return nullptr;
    }
    *fields[i] = (float)d;
  }
  if (throw_status(env, h->ctx, eg_decoder_set_sampling(h->dec, &p))) return nullptr;
  return undefined(env);
}

// decoderSeed(dec, seed)
napi_value DecoderSeed(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderSeed", 2);
  auto* h = live_decoder(env, a, "decoderSeed");
  uint64_t seed = a.u64(1);
  if (!h || !a.ok) return nullptr;
  if (throw_status(env, h->ctx, eg_decoder_seed(h->dec, (uint32_t)seed))) return nullptr;
  return undefined(env);
}

// decoderLaunches(dec) -> launches of the next step (eg_decoder_launches)
napi_value DecoderLaunches(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderLaunches", 1);
  auto* h = live_decoder(env, a, "decoderLaunches");
  if (!h || !a.ok) return nullptr;
  uint32_t n = 0;
  if (throw_status(env, h->ctx, eg_decoder_launches(h->dec, &n))) return nullptr;
  napi_value v;
  napi_create_uint32(env, n, &v);
  return v;
}

// decoderSetPosition(dec, position, historyLength, random) (DecodeGraph.setPosition)
napi_value DecoderSetPosition(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderSetPosition", 4);
  auto* h = live_decoder(env, a, "decoderSetPosition");
  uint64_t position = a.u64(1), length = a.u64(2);
  float random = 0.f;
  if (!h || !f32_arg(a, 3, &random)) return nullptr;
  if (throw_status(env, h->ctx, eg_decoder_set_position(h->dec, (uint32_t)position, (uint32_t)length, random)))
    return nullptr;
  return undefined(env);
}

// decoderSetHistory(dec, Uint32Array)
napi_value DecoderSetHistory(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderSetHistory", 2);
  auto* h = live_decoder(env, a, "decoderSetHistory");
  void* data = nullptr;
  size_t len = 0;
  if (!h || !a.bytes(1, &data, &len)) return nullptr;
  if (throw_status(env, h->ctx, eg_decoder_set_history(h->dec, static_cast<const uint32_t*>(data), (uint32_t)(len / 4))))
    return nullptr;
  return undefined(env);
}

// decoderPrefill(dec, position, Uint32Array prompt) -> the first token id
napi_value DecoderPrefill(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderPrefill", 3);
  auto* h = live_decoder(env, a, "decoderPrefill");
  uint64_t position = a.u64(1);
  void* data = nullptr;
  size_t len = 0;
  if (!h || !a.bytes(2, &data, &len)) return nullptr;
  uint32_t token = 0;
  if (throw_status(env, h->ctx, eg_decoder_prefill(h->dec, (uint32_t)position, static_cast<const uint32_t*>(data),
                                                   (uint32_t)(len / 4), &token)))
    return nullptr;
  return number(env, token);
}

// decoderBuffers(dec) -> {kCache, vCache, logits, hidden, token, position, history, sampleParams,
// rng} device pointers
napi_value DecoderBuffers(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderBuffers", 1);
  auto* h = a.handle<DecoderHandle>(0, "decoder");
  if (!a.ok) return nullptr;
  eg_decoder_buffers b{};
  if (!h->dec || throw_status(env, h->ctx, eg_decoder_buffers_get(h->dec, &b))) return nullptr;
  napi_value obj;
  napi_create_object(env, &obj);
  const std::pair<const char*, const void*> fields[] = {{"kCache", b.k_cache}, {"vCache", b.v_cache},
                                                        {"logits", b.logits}, {"hidden", b.hidden},
                                                        {"token", b.token}, {"position", b.position},
                                                        {"history", b.history}, {"sampleParams", b.sample_params},
                                                        {"rng", b.rng}};
  for (const auto& f : fields)
    napi_set_named_property(env, obj, f.first, number(env, (double)reinterpret_cast<uintptr_t>(f.second)));
  return obj;
}

napi_value DecoderDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info, "decoderDestroy", 1);
  auto* h = a.handle<DecoderHandle>(0, "decoder");
  if (!a.ok) return nullptr;
  if (h->dec) eg_decoder_destroy(h->dec);
  h->dec = nullptr;
  return undefined(env);
}

// ---- graphs ----------------------------------------------------------------------------------

napi_value GraphBegin(napi_env env, napi_callback_info info) {
  Args a(env, info, "graphBegin", 1);
  auto* ctx = a.handle<eg_context>(0, "context");
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_graph_begin(ctx))) return nullptr;
  return undefined(env);
}

napi_value GraphEnd(napi_env env, napi_callback_info info) {
  Args a(env, info, "graphEnd", 1);
  auto* ctx = a.handle<eg_context>(0, "context");
  if (!a.ok) return nullptr;
  eg_graph* g = nullptr;
  if (throw_status(env, ctx, eg_graph_end(ctx, &g))) return nullptr;
  return make_handle<eg_graph>(env, g, nullptr);
}

napi_value GraphLaunch(napi_env env, napi_callback_info info) {
  Args a(env, info, "graphLaunch", 2);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* g = a.handle<eg_graph>(1, "graph");
  if (!a.ok) return nullptr;
  if (throw_status(env, ctx, eg_graph_launch(ctx, g))) return nullptr;
  return undefined(env);
}

napi_value GraphDestroy(napi_env env, napi_callback_info info) {
  Args a(env, info, "graphDestroy", 1);
  auto* g = a.handle<eg_graph>(0, "graph");
  if (!a.ok) return nullptr;
  eg_graph_destroy(g);
  return undefined(env);
}

// ---- the .enargeia container -------------------------------------------------------------------

napi_value num(napi_env env, double v) {
  napi_value r;
  napi_create_double(env, v, &r);
  return r;
}
napi_value str(napi_env env, const char* s) {
  napi_value r;
  napi_create_string_utf8(env, s, NAPI_AUTO_LENGTH, &r);
  return r;
}
void set(napi_env env, napi_value obj, const char* name, napi_value v) { napi_set_named_property(env, obj, name, v); }
napi_value range(napi_env env, const uint64_t r[2]) {
  napi_value a;
  napi_create_array_with_length(env, 2, &a);
  napi_set_element(env, a, 0, num(env, (double)r[0]));
  napi_set_element(env, a, 1, num(env, (double)r[1]));
  return a;
}
napi_value ptr_value(napi_env env, const void* p) {
  if (!p) {
    napi_value n;
    napi_get_null(env, &n);
    return n;
  }
  return num(env, (double)reinterpret_cast<uintptr_t>(p));
}

void finalize_container(napi_env, void* data, void*) {
  auto* h = static_cast<ContainerHandle*>(data);
  if (h->c) eg_container_close(h->c);
  delete h;
}

ContainerHandle* open_handle(Args& a, size_t index) {
  auto* h = a.handle<ContainerHandle>(index, "container");
  if (h && !h->c) {
    napi_throw_error(a.env, "EG_ERR_STATE", (std::string(a.fn) + ": the container was closed").c_str());
    return nullptr;
  }
  return h;
}

// containerOpen(path): parses the prefix and header; throws EnargeiaError for a malformed file.
napi_value ContainerOpen(napi_env env, napi_callback_info info) {
  Args a(env, info, "containerOpen", 1);
  if (!a.ok) return nullptr;
  size_t n = 0;
  if (napi_get_value_string_utf8(env, a.argv[0], nullptr, 0, &n) != napi_ok) {
    throw_type(env, "containerOpen: path is not a string");
    return nullptr;
  }
  std::string path(n, '\0');
  napi_get_value_string_utf8(env, a.argv[0], &path[0], n + 1, &n);
  eg_container* c = nullptr;
  if (throw_status(env, nullptr, eg_container_open(nullptr, path.c_str(), &c))) return nullptr;
  return make_handle(env, new ContainerHandle{c}, finalize_container);
}

napi_value ContainerClose(napi_env env, napi_callback_info info) {
  Args a(env, info, "containerClose", 1);
  auto* h = a.handle<ContainerHandle>(0, "container");
  if (!a.ok) return nullptr;
  if (h->c) eg_container_close(h->c);
  h->c = nullptr;
  return undefined(env);
}

// containerHeader(handle): EnargeiaHeader (enargeia.ts:73-82) with `tensors` an array of
// QuantTensorInfo / F32TensorInfo / F16TensorInfo objects in header order.
napi_value ContainerHeader(napi_env env, napi_callback_info info) {
  Args a(env, info, "containerHeader", 1);
  auto* h = open_handle(a, 0);
  if (!a.ok || !h) return nullptr;
  eg_container_header hd;
  if (throw_status(env, nullptr, eg_container_header_get(h->c, &hd))) return nullptr;
  napi_value out, list;
  napi_create_object(env, &out);
  set(env, out, "version", num(env, hd.version));
  set(env, out, "blockSize", num(env, hd.block_size));
  set(env, out, "quantization", str(env, hd.quantization));
  set(env, out, "dataOffset", num(env, (double)hd.data_offset));
  set(env, out, "headerLength", num(env, (double)hd.header_length));
  set(env, out, "fileSize", num(env, (double)hd.file_size));
  napi_create_array_with_length(env, hd.tensor_count, &list);
  static const char* kDtype[] = {"Q4", "Q8", "F32", "F16"};
  for (uint32_t i = 0; i < hd.tensor_count; i++) {
    eg_tensor_info t;
    if (throw_status(env, nullptr, eg_container_tensor(h->c, i, &t))) return nullptr;
    napi_value o, shape;
    napi_create_object(env, &o);
    set(env, o, "name", str(env, t.name));
    set(env, o, "dtype", str(env, kDtype[t.dtype]));
    napi_create_array_with_length(env, t.ndim, &shape);
    for (uint32_t d = 0; d < t.ndim; d++) napi_set_element(env, shape, d, num(env, (double)t.shape[d]));
    set(env, o, "shape", shape);
    if (t.dtype == EG_DTYPE_Q4 || t.dtype == EG_DTYPE_Q8) {
      set(env, o, "bits", num(env, t.bits));
      set(env, o, "blockSize", num(env, t.block_size));
      set(env, o, "packed", range(env, t.packed));
      set(env, o, "scales", range(env, t.scales));
      set(env, o, "zeros", range(env, t.zeros));
      set(env, o, "blocksPerRow", num(env, t.blocks_per_row));
      set(env, o, "totalBlocks", num(env, (double)t.total_blocks));
    } else {
      set(env, o, "data", range(env, t.data));
    }
    napi_set_element(env, list, i, o);
  }
  set(env, out, "tensors", list);
  return out;
}

// containerLoad(ctx, handle, {headDim, maxContext, rmsEps, ropeTheta}): uploads the blob (one
// device allocation; bufFree it when done) and returns {blob, desc} with desc in the shape
// decoderCreate takes.
napi_value ContainerLoad(napi_env env, napi_callback_info info) {
  Args a(env, info, "containerLoad", 3);
  auto* ctx = a.handle<eg_context>(0, "context");
  auto* h = open_handle(a, 1);
  if (!a.ok || !h) return nullptr;
  eg_model_config cfg{};
  napi_value c = a.argv[2];
  if (!get_u32(env, c, "headDim", &cfg.head_dim) || !get_u32(env, c, "maxContext", &cfg.max_context) ||
      !get_f32(env, c, "rmsEps", &cfg.rms_eps) || !get_f32(env, c, "ropeTheta", &cfg.rope_theta))
    return nullptr;
  eg_container_header hd;
  eg_container_header_get(h->c, &hd);
  void* blob = nullptr;
  if (throw_status(env, ctx, eg_container_upload(ctx, h->c, &blob))) return nullptr;
  std::vector<eg_layer_desc> layers(hd.tensor_count + 1);
  eg_model_desc m{};
  const int st = eg_container_model_desc(ctx, h->c, blob, &cfg, &m, layers.data(), (uint32_t)layers.size());
  if (st != EG_OK) {
    eg_buf_free(ctx, blob);
    throw_status(env, ctx, st);
    return nullptr;
  }
  auto matrix = [&](const eg_quant_matrix& q) {
    napi_value o;
    napi_create_object(env, &o);
    set(env, o, "packed", ptr_value(env, q.packed));
    set(env, o, "scales", ptr_value(env, q.scales));
    set(env, o, "zeros", ptr_value(env, q.zeros));
    return o;
  };
  napi_value d, list, out;
  napi_create_object(env, &d);
  set(env, d, "layers", num(env, m.layers));
  set(env, d, "hidden", num(env, m.hidden));
  set(env, d, "heads", num(env, m.heads));
  set(env, d, "kvHeads", num(env, m.kv_heads));
  set(env, d, "headDim", num(env, m.head_dim));
  set(env, d, "intermediate", num(env, m.intermediate));
  set(env, d, "vocab", num(env, m.vocab));
  set(env, d, "maxContext", num(env, m.max_context));
  set(env, d, "rmsEps", num(env, m.rms_eps));
  set(env, d, "ropeTheta", num(env, m.rope_theta));
  set(env, d, "encoding", num(env, m.encoding));
  set(env, d, "bits", num(env, m.bits));
  set(env, d, "blockSize", num(env, m.block_size));
  set(env, d, "embedding", matrix(m.embedding));
  set(env, d, "embedEncoding", num(env, m.embed_encoding));
  set(env, d, "embedBits", num(env, m.embed_bits));
  set(env, d, "embedBlockSize", num(env, m.embed_block_size));
  set(env, d, "finalNorm", ptr_value(env, m.final_norm));
  napi_create_array_with_length(env, m.layers, &list);
  for (uint32_t i = 0; i < m.layers; i++) {
    const eg_layer_desc& L = m.layer[i];
    napi_value o;
    napi_create_object(env, &o);
    set(env, o, "q", matrix(L.q));
    set(env, o, "k", matrix(L.k));
    set(env, o, "v", matrix(L.v));
    set(env, o, "o", matrix(L.o));
    set(env, o, "gate", matrix(L.gate));
    set(env, o, "up", matrix(L.up));
    set(env, o, "down", matrix(L.down));
    set(env, o, "qBias", ptr_value(env, L.q_bias));
    set(env, o, "kBias", ptr_value(env, L.k_bias));
    set(env, o, "vBias", ptr_value(env, L.v_bias));
    set(env, o, "inputNorm", ptr_value(env, L.input_norm));
    set(env, o, "postAttentionNorm", ptr_value(env, L.post_attention_norm));
    napi_set_element(env, list, i, o);
  }
  set(env, d, "layer", list);
  napi_create_object(env, &out);
  set(env, out, "blob", ptr_value(env, blob));
  set(env, out, "desc", d);
  return out;
}

napi_value Init(napi_env env, napi_value exports) {
  const napi_property_descriptor props[] = {
      {"abiVersion", nullptr, AbiVersion, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"create", nullptr, Create, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"destroy", nullptr, Destroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sync", nullptr, Sync, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"getStream", nullptr, GetStream, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"bufAlloc", nullptr, BufAlloc, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"bufFree", nullptr, BufFree, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"bufWrite", nullptr, BufWrite, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"bufRead", nullptr, BufRead, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"bufZero", nullptr, BufZero, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"matmulQ4Decode", nullptr, Matmul<eg_matmul_q4_decode>, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"matmulQ4Prefill", nullptr, Matmul<eg_matmul_q4_prefill>, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lmHead", nullptr, LmHead, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"embedGather", nullptr, EmbedGather, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"lmHeadArgmax", nullptr, LmHeadArgmax, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"argmax", nullptr, Argmax, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"sample", nullptr, Sample, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderCreate", nullptr, DecoderCreate, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderReset", nullptr, DecoderReset, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderStep", nullptr, DecoderStep, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderCapture", nullptr, DecoderCapture, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderBuffers", nullptr, DecoderBuffers, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderSetSampling", nullptr, DecoderSetSampling, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderSeed", nullptr, DecoderSeed, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderLaunches", nullptr, DecoderLaunches, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderSetPosition", nullptr, DecoderSetPosition, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderSetHistory", nullptr, DecoderSetHistory, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderPrefill", nullptr, DecoderPrefill, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"decoderDestroy", nullptr, DecoderDestroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"graphBegin", nullptr, GraphBegin, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"graphEnd", nullptr, GraphEnd, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"graphLaunch", nullptr, GraphLaunch, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"graphDestroy", nullptr, GraphDestroy, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"containerOpen", nullptr, ContainerOpen, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"containerClose", nullptr, ContainerClose, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"containerHeader", nullptr, ContainerHeader, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
      {"containerLoad", nullptr, ContainerLoad, nullptr, nullptr, nullptr, napi_enumerable, nullptr},
  };
  napi_define_properties(env, exports, sizeof(props) / sizeof(props[0]), props);
  return exports;
}

}  // namespace

NAPI_MODULE(NODE_GYP_MODULE_NAME, Init)
