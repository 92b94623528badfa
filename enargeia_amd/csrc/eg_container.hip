// The `.enargeia` container (enargeia.ts:1-50, 112-240): parsed on the host, uploaded as one
// device allocation, and turned into the decoder's model description.
//
// File layout (enargeia.ts:1-18, quantize.py:240-260):
//   "ENARGEIA" | version u32 LE (1) | headerLen u32 LE | header JSON | zeros to 256 | blob
// Every tensor range in the header is relative to the blob and 256-byte aligned. A quantized
// tensor is three ranges (packed codes, f32 scales per block, packed zero-points); F32 and F16
// tensors are one.
//
// MI355X design (not the reference's per-range fetch and ~630 writeBuffer calls,
// weights.ts:299-471): the blob is read once, in large pieces, through two pinned staging
// buffers into ONE device allocation, so a tensor's device address is the allocation plus its
// range - no per-tensor allocations and every range keeps its 256-byte alignment (the GEMV's
// 16-byte vector loads need 16).
#include <cerrno>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "eg_internal.hpp"

namespace {

constexpr char kMagic[8] = {'E', 'N', 'A', 'R', 'G', 'E', 'I', 'A'};
constexpr uint32_t kVersion = 1;
constexpr uint32_t kPrefixBytes = 16;
constexpr uint64_t kMaxHeaderBytes = 64ull * 1024 * 1024;  // enargeia.ts:32
constexpr uint32_t kDefaultBlock = 64;                    // ENARGEIA_BLOCK

// ---- a small JSON reader: objects, arrays, strings, numbers, true / false / null -----------

struct Json {
  enum Kind { kNull, kBool, kNumber, kString, kArray, kObject } kind = kNull;
  bool b = false;
  double num = 0.0;
  std::string str;
  std::vector<Json> items;
  std::vector<std::pair<std::string, Json>> members;  // in document order

  const Json* get(const char* key) const {
    if (kind != kObject) return nullptr;
    for (const auto& m : members)
      if (m.first == key) return &m.second;
    return nullptr;
  }
};

class JsonParser {
 public:
  JsonParser(const char* s, size_t n) : p_(s), end_(s + n) {}

  bool parse(Json& out) {
    skip();
    if (!value(out, 0)) return false;
    skip();
    if (p_ != end_) return fail("unexpected data after the top-level value");
    return true;
  }
  const std::string& error() const { return error_; }

 private:
  const char* p_;
  const char* end_;
  std::string error_;

  bool fail(const char* what) {
    if (error_.empty()) error_ = what;
    return false;
  }
  void skip() {
    while (p_ < end_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) p_++;
  }
  bool literal(const char* word) {
    const size_t n = std::strlen(word);
    if ((size_t)(end_ - p_) < n || std::memcmp(p_, word, n) != 0) return fail("invalid literal");
    p_ += n;
    return true;
  }
  static void utf8(uint32_t cp, std::string& s) {
    if (cp < 0x80) {
      s += (char)cp;
    } else if (cp < 0x800) {
      s += (char)(0xC0 | (cp >> 6));
      s += (char)(0x80 | (cp & 0x3F));
    } else if (cp < 0x10000) {
      s += (char)(0xE0 | (cp >> 12));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    } else {
      s += (char)(0xF0 | (cp >> 18));
      s += (char)(0x80 | ((cp >> 12) & 0x3F));
      s += (char)(0x80 | ((cp >> 6) & 0x3F));
      s += (char)(0x80 | (cp & 0x3F));
    }
  }
  bool hex4(uint32_t& v) {
    if (end_ - p_ < 4) return fail("truncated \\u escape");
    v = 0;
    for (int i = 0; i < 4; i++) {
      const char c = *p_++;
      v <<= 4;
      if (c >= '0' && c <= '9') v |= (uint32_t)(c - '0');
      else if (c >= 'a' && c <= 'f') v |= (uint32_t)(c - 'a' + 10);
      else if (c >= 'A' && c <= 'F') v |= (uint32_t)(c - 'A' + 10);
      else return fail("bad \\u escape");
    }
    return true;
  }
  bool string(std::string& s) {
    p_++;  // opening quote
    while (true) {
      if (p_ >= end_) return fail("unterminated string");
      const char c = *p_++;
      if (c == '"') return true;
      if ((unsigned char)c < 0x20) return fail("control character in a string");
      if (c != '\\') {
        s += c;
        continue;
      }
      if (p_ >= end_) return fail("unterminated escape");
      const char e = *p_++;
      switch (e) {
        case '"': s += '"'; break;
        case '\\': s += '\\'; break;
        case '/': s += '/'; break;
        case 'b': s += '\b'; break;
        case 'f': s += '\f'; break;
        case 'n': s += '\n'; break;
        case 'r': s += '\r'; break;
        case 't': s += '\t'; break;
        case 'u': {
          uint32_t cp;
          if (!hex4(cp)) return false;
          if (cp >= 0xD800 && cp < 0xDC00) {  // surrogate pair
            uint32_t lo;
            if (end_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') return fail("lone surrogate");
            p_ += 2;
            if (!hex4(lo) || lo < 0xDC00 || lo >= 0xE000) return fail("bad surrogate pair");
            cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
          }
          utf8(cp, s);
          break;
        }
        default:
          return fail("bad escape");
      }
    }
  }
  bool number(double& v) {
    const char* start = p_;
    if (p_ < end_ && *p_ == '-') p_++;
    if (p_ >= end_ || !(*p_ >= '0' && *p_ <= '9')) return fail("bad number");
    while (p_ < end_ && ((*p_ >= '0' && *p_ <= '9') || *p_ == '.' || *p_ == 'e' || *p_ == 'E' || *p_ == '+' ||
                         *p_ == '-'))
      p_++;
    const std::string text(start, p_);
    char* stop = nullptr;
    errno = 0;
    v = std::strtod(text.c_str(), &stop);
    if (stop != text.c_str() + text.size() || errno == ERANGE) return fail("bad number");
    return true;
  }
  bool value(Json& out, int depth) {
    if (depth > 64) return fail("nesting too deep");
    skip();
    if (p_ >= end_) return fail("unexpected end of input");
    const char c = *p_;
    if (c == '{') {
      out.kind = Json::kObject;
      p_++;
      skip();
      if (p_ < end_ && *p_ == '}') {
        p_++;
        return true;
      }
      while (true) {
        skip();
        if (p_ >= end_ || *p_ != '"') return fail("expected a string key");
        std::string key;
        if (!string(key)) return false;
        skip();
        if (p_ >= end_ || *p_ != ':') return fail("expected ':'");
        p_++;
        Json v;
        if (!value(v, depth + 1)) return false;
        // A repeated key keeps the last value (JSON.parse semantics).
        bool replaced = false;
        for (auto& m : out.members)
          if (m.first == key) {
            m.second = std::move(v);
            replaced = true;
            break;
          }
        if (!replaced) out.members.emplace_back(std::move(key), std::move(v));
        skip();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == '}') {
          p_++;
          return true;
        }
        return fail("expected ',' or '}'");
      }
    }
    if (c == '[') {
      out.kind = Json::kArray;
      p_++;
      skip();
      if (p_ < end_ && *p_ == ']') {
        p_++;
        return true;
      }
      while (true) {
        Json v;
        if (!value(v, depth + 1)) return false;
        out.items.push_back(std::move(v));
        skip();
        if (p_ < end_ && *p_ == ',') {
          p_++;
          continue;
        }
        if (p_ < end_ && *p_ == ']') {
          p_++;
          return true;
        }
        return fail("expected ',' or ']'");
      }
    }
    if (c == '"') {
      out.kind = Json::kString;
      return string(out.str);
    }
    if (c == 't') {
      out.kind = Json::kBool;
      out.b = true;
      return literal("true");
    }
    if (c == 'f') {
      out.kind = Json::kBool;
      out.b = false;
      return literal("false");
    }
    if (c == 'n') {
      out.kind = Json::kNull;
      return literal("null");
    }
    out.kind = Json::kNumber;
    return number(out.num);
  }
};

// Non-negative integer (JSON numbers are doubles; integers up to 2^53 are exact).
bool as_index(const Json& v, uint64_t& out) {
  if (v.kind != Json::kNumber || !(v.num >= 0.0) || v.num != std::floor(v.num) || v.num > 9007199254740992.0)
    return false;
  out = (uint64_t)v.num;
  return true;
}

// JSON.stringify of a short string, for the reference's error text.
std::string quoted(const std::string& s) {
  std::string r = "\"";
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') {
      r += '\\';
      r += (char)c;
    } else if (c < 0x20) {
      char buf[8];
      std::snprintf(buf, sizeof(buf), "\\u%04x", c);
      r += buf;
    } else {
      r += (char)c;
    }
  }
  return r + "\"";
}

struct Tensor {
  std::string name;
  int dtype = 0;
  int bits = 0;
  std::vector<uint64_t> shape;
  uint32_t block_size = 0, blocks_per_row = 0;
  uint64_t total_blocks = 0;
  uint64_t packed[2] = {0, 0}, scales[2] = {0, 0}, zeros[2] = {0, 0}, data[2] = {0, 0};
};

}  // namespace

struct eg_container {
  std::string path;
  uint32_t version = kVersion, block_size = kDefaultBlock;
  uint64_t header_length = 0, data_offset = 0, file_size = 0, blob_bytes = 0;
  std::string quantization;
  std::vector<Tensor> tensors;  // in header order
  std::map<std::string, size_t> index;
};

namespace {

using eg::fail;

// One byte range of a tensor (enargeia.ts:232-242).
int read_range(eg_context* ctx, const Tensor& t, const char* field, const Json* v, uint64_t out[2]) {
  if (!v || v->kind != Json::kArray || v->items.size() != 2 || !as_index(v->items[0], out[0]) ||
      !as_index(v->items[1], out[1]))
    return fail(ctx, EG_ERR_FORMAT, "%s: offsets.%s is malformed", t.name.c_str(), field);
  if (out[1] < out[0]) return fail(ctx, EG_ERR_FORMAT, "%s: offsets.%s runs backwards", t.name.c_str(), field);
  return EG_OK;
}

int check_size(eg_context* ctx, const Tensor& t, const char* field, const uint64_t r[2], uint64_t expect) {
  if (r[1] - r[0] != expect)
    return fail(ctx, EG_ERR_FORMAT, "%s: %s is %llu bytes, expected %llu", t.name.c_str(), field,
                (unsigned long long)(r[1] - r[0]), (unsigned long long)expect);
  return EG_OK;
}

// One header entry (enargeia.ts:162-230): the same checks in the same order, the same messages.
int parse_tensor(eg_context* ctx, const std::string& name, const Json& v, uint32_t default_block, Tensor& t) {
  t.name = name;
  if (v.kind != Json::kObject) return fail(ctx, EG_ERR_FORMAT, "tensor \"%s\" is not an object", name.c_str());
  const Json* shape = v.get("shape");
  bool shape_ok = shape && shape->kind == Json::kArray;
  if (shape_ok)
    for (const Json& d : shape->items) {
      uint64_t n;
      if (!as_index(d, n) || n == 0) {
        shape_ok = false;
        break;
      }
      t.shape.push_back(n);
    }
  if (!shape_ok) return fail(ctx, EG_ERR_FORMAT, "tensor \"%s\" has a malformed shape", name.c_str());
  const Json* offsets = v.get("offsets");
  if (!offsets || offsets->kind != Json::kObject)
    return fail(ctx, EG_ERR_FORMAT, "tensor \"%s\" has no offsets", name.c_str());
  const Json* dtype = v.get("dtype");
  const std::string dt = dtype && dtype->kind == Json::kString ? dtype->str : std::string();

  if (dt == "F32" || dt == "F16") {
    t.dtype = dt == "F32" ? EG_DTYPE_F32 : EG_DTYPE_F16;
    t.bits = dt == "F32" ? 32 : 16;
    int st = read_range(ctx, t, "data", offsets->get("data"), t.data);
    if (st != EG_OK) return st;
    uint64_t elements = 1;
    for (uint64_t d : t.shape) elements *= d;
    const uint64_t expect = elements * (uint64_t)(t.bits / 8);
    if (t.data[1] - t.data[0] != expect)
      return fail(ctx, EG_ERR_FORMAT, "%s: %s range is %llu bytes, shape needs %llu", name.c_str(), dt.c_str(),
                  (unsigned long long)(t.data[1] - t.data[0]), (unsigned long long)expect);
    return EG_OK;
  }
  if (dt != "Q4" && dt != "Q8") {
    const std::string shown = !dtype ? "undefined" : dtype->kind == Json::kString ? quoted(dtype->str) : "a non-string";
    return fail(ctx, EG_ERR_FORMAT, "tensor \"%s\" has unsupported dtype %s", name.c_str(), shown.c_str());
  }
  t.dtype = dt == "Q4" ? EG_DTYPE_Q4 : EG_DTYPE_Q8;
  t.bits = dt == "Q4" ? 4 : 8;
  const uint64_t per_word = 32 / (uint64_t)t.bits;
  if (t.shape.size() != 2) {
    std::string dims;
    for (size_t i = 0; i < t.shape.size(); i++) dims += (i ? ", " : "") + std::to_string(t.shape[i]);
    return fail(ctx, EG_ERR_FORMAT, "%s: Q4 tensors must be 2-D, got [%s]", name.c_str(), dims.c_str());
  }
  uint64_t block = default_block;
  if (const Json* b = v.get("blockSize"))
    if (b->kind == Json::kNumber) {
      if (!as_index(*b, block) || block == 0 || block > 0xFFFFFFFFull)
        return fail(ctx, EG_ERR_FORMAT, "%s: blockSize is not a positive integer", name.c_str());
    }
  const uint64_t rows = t.shape[0], cols = t.shape[1];
  if (cols % block != 0)
    return fail(ctx, EG_ERR_FORMAT, "%s: reduction axis %llu is not a multiple of block size %llu", name.c_str(),
                (unsigned long long)cols, (unsigned long long)block);
  int st = read_range(ctx, t, "packed", offsets->get("packed"), t.packed);
  if (st == EG_OK) st = read_range(ctx, t, "scales", offsets->get("scales"), t.scales);
  if (st == EG_OK) st = read_range(ctx, t, "zeros", offsets->get("zeros"), t.zeros);
  if (st != EG_OK) return st;
  const uint64_t elements = rows * cols;
  t.block_size = (uint32_t)block;
  t.total_blocks = elements / block;
  t.blocks_per_row = (uint32_t)(cols / block);
  if ((st = check_size(ctx, t, "packed", t.packed, (elements / per_word) * 4)) != EG_OK) return st;
  if ((st = check_size(ctx, t, "scales", t.scales, t.total_blocks * 4)) != EG_OK) return st;
  return check_size(ctx, t, "zeros", t.zeros, ((t.total_blocks + per_word - 1) / per_word) * 4);
}

// Prefix + header (enargeia.ts:96-150), from the file's first bytes.
int parse_header(eg_context* ctx, const std::vector<char>& head, uint64_t file_bytes, eg_container& c) {
  if (head.size() < kPrefixBytes)
    return fail(ctx, EG_ERR_FORMAT, "need at least %u bytes to read the header length", kPrefixBytes);
  if (std::memcmp(head.data(), kMagic, 8) != 0)
    return fail(ctx, EG_ERR_FORMAT, "not a .enargeia file: magic is %s",
                quoted(std::string(head.data(), head.data() + 8)).c_str());
  uint32_t version, header_len;
  std::memcpy(&version, head.data() + 8, 4);
  std::memcpy(&header_len, head.data() + 12, 4);
  if (version != kVersion)
    return fail(ctx, EG_ERR_FORMAT, "unsupported .enargeia version %u, expected %u", version, kVersion);
  if (header_len > kMaxHeaderBytes)
    return fail(ctx, EG_ERR_FORMAT, "header length %u exceeds the %llu byte limit", header_len,
                (unsigned long long)kMaxHeaderBytes);
  const uint64_t total = kPrefixBytes + (uint64_t)header_len;
  if (head.size() < total)
    return fail(ctx, EG_ERR_FORMAT, "header needs %llu bytes, got %llu", (unsigned long long)total,
                (unsigned long long)head.size());
  Json root;
  JsonParser parser(head.data() + kPrefixBytes, header_len);
  if (!parser.parse(root))
    return fail(ctx, EG_ERR_FORMAT, "header is not valid JSON: %s", parser.error().c_str());
  const Json* tensors = root.get("tensors");
  if (!tensors || tensors->kind != Json::kObject) return fail(ctx, EG_ERR_FORMAT, "header has no \"tensors\" object");
  c.block_size = kDefaultBlock;
  if (const Json* b = root.get("blockSize")) {
    uint64_t v;
    if (b->kind != Json::kNull) {
      if (!as_index(*b, v) || v == 0 || v > 0xFFFFFFFFull)
        return fail(ctx, EG_ERR_FORMAT, "header blockSize is not a positive integer");
      c.block_size = (uint32_t)v;
    }
  }
  const Json* q = root.get("quantization");
  c.quantization = q && q->kind == Json::kString ? q->str : "unknown";
  uint64_t end = 0;
  for (const auto& m : tensors->members) {
    Tensor t;
    int st = parse_tensor(ctx, m.first, m.second, c.block_size, t);
    if (st != EG_OK) return st;
    for (const uint64_t* r : {t.packed, t.scales, t.zeros, t.data}) end = std::max(end, r[1]);
    c.index[t.name] = c.tensors.size();
    c.tensors.push_back(std::move(t));
  }
  c.version = version;
  c.header_length = header_len;
  c.data_offset = total + ((256 - total % 256) % 256);  // the blob starts at the next 256-byte boundary
  c.blob_bytes = end;
  c.file_size = c.data_offset + end;
  if (file_bytes < c.file_size)
    return fail(ctx, EG_ERR_FORMAT, "the header's ranges end at byte %llu, past the end of the %llu-byte file",
                (unsigned long long)c.file_size, (unsigned long long)file_bytes);
  return EG_OK;
}

void fill_info(const Tensor& t, eg_tensor_info* out) {
  *out = eg_tensor_info{};
  out->name = t.name.c_str();
  out->dtype = t.dtype;
  out->bits = t.bits;
  out->ndim = (uint32_t)std::min<size_t>(t.shape.size(), EG_MAX_DIMS);
  for (uint32_t i = 0; i < out->ndim; i++) out->shape[i] = t.shape[i];
  out->block_size = t.block_size;
  out->blocks_per_row = t.blocks_per_row;
  out->total_blocks = t.total_blocks;
  for (int i = 0; i < 2; i++) {
    out->packed[i] = t.packed[i];
    out->scales[i] = t.scales[i];
    out->zeros[i] = t.zeros[i];
    out->data[i] = t.data[i];
  }
}

struct File {
  FILE* f = nullptr;
  ~File() {
    if (f) std::fclose(f);
  }
};

}  // namespace

extern "C" {

int eg_container_open(eg_context* ctx, const char* path, eg_container** out) {
  if (!path || !out) return fail(ctx, EG_ERR_INVALID, "container_open: NULL argument");
  *out = nullptr;
  File file;
  file.f = std::fopen(path, "rb");
  if (!file.f) return fail(ctx, EG_ERR_IO, "container_open: cannot open %s: %s", path, std::strerror(errno));
  if (std::fseek(file.f, 0, SEEK_END) != 0) return fail(ctx, EG_ERR_IO, "container_open: cannot seek %s", path);
  const long size = std::ftell(file.f);
  if (size < 0) return fail(ctx, EG_ERR_IO, "container_open: cannot size %s", path);
  std::rewind(file.f);
  // The prefix first, then exactly the header it announces (readEnargeiaHeader, :244-248).
  std::vector<char> head(std::min<uint64_t>((uint64_t)size, kPrefixBytes));
  if (!head.empty() && std::fread(head.data(), 1, head.size(), file.f) != head.size())
    return fail(ctx, EG_ERR_IO, "container_open: short read of %s", path);
  if (head.size() == kPrefixBytes && std::memcmp(head.data(), kMagic, 8) == 0) {
    uint32_t header_len;
    std::memcpy(&header_len, head.data() + 12, 4);
    if (header_len <= kMaxHeaderBytes) {
      const uint64_t want = std::min<uint64_t>((uint64_t)size, kPrefixBytes + (uint64_t)header_len);
      head.resize(want);
      const size_t rest = want - kPrefixBytes;
      if (rest && std::fread(head.data() + kPrefixBytes, 1, rest, file.f) != rest)
        return fail(ctx, EG_ERR_IO, "container_open: short read of %s", path);
    }
  }
  auto c = std::make_unique<eg_container>();
  c->path = path;
  int st = parse_header(ctx, head, (uint64_t)size, *c);
  if (st != EG_OK) return st;
  *out = c.release();
  return EG_OK;
}

int eg_container_close(eg_container* c) {
  delete c;
  return EG_OK;
}

int eg_container_header_get(const eg_container* c, eg_container_header* out) {
  if (!c || !out) return fail(nullptr, EG_ERR_INVALID, "container_header: NULL argument");
  out->version = c->version;
  out->block_size = c->block_size;
  out->tensor_count = (uint32_t)c->tensors.size();
  out->header_length = c->header_length;
  out->data_offset = c->data_offset;
  out->blob_bytes = c->blob_bytes;
  out->file_size = c->file_size;
  out->quantization = c->quantization.c_str();
  return EG_OK;
}

int eg_container_tensor(const eg_container* c, uint32_t index, eg_tensor_info* out) {
  if (!c || !out) return fail(nullptr, EG_ERR_INVALID, "container_tensor: NULL argument");
  if (index >= c->tensors.size())
    return fail(nullptr, EG_ERR_RANGE, "container_tensor: index %u of %zu", index, c->tensors.size());
  fill_info(c->tensors[index], out);
  return EG_OK;
}

int eg_container_find(const eg_container* c, const char* name, eg_tensor_info* out) {
  if (!c || !name || !out) return fail(nullptr, EG_ERR_INVALID, "container_find: NULL argument");
  auto it = c->index.find(name);
  if (it == c->index.end()) return fail(nullptr, EG_ERR_NOT_FOUND, "%s is missing", name);
  fill_info(c->tensors[it->second], out);
  return EG_OK;
}

int eg_container_upload(eg_context* ctx, const eg_container* c, void** out_blob) {
  const char* op = "container_upload";
  if (!ctx) return fail(nullptr, EG_ERR_INVALID, "%s: ctx is NULL", op);
  if (!c || !out_blob) return fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  *out_blob = nullptr;
  if (ctx->capturing) return fail(ctx, EG_ERR_INVALID, "%s: not allowed during graph capture", op);
  File file;
  file.f = std::fopen(c->path.c_str(), "rb");
  if (!file.f) return fail(ctx, EG_ERR_IO, "%s: cannot open %s: %s", op, c->path.c_str(), std::strerror(errno));
  if (std::fseek(file.f, (long)c->data_offset, SEEK_SET) != 0)
    return fail(ctx, EG_ERR_IO, "%s: cannot seek %s", op, c->path.c_str());
  const uint64_t bytes = std::max<uint64_t>(c->blob_bytes, 256);
  void* blob = nullptr;
  hipError_t err = hipMalloc(&blob, bytes);
  if (err != hipSuccess) return eg::hip_fail(ctx, err, op);
  // Two pinned staging buffers: the file read of piece i+1 overlaps the copy of piece i.
  constexpr size_t kPiece = 32u << 20;
  void* stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  for (int i = 0; i < 2 && err == hipSuccess; i++) {
    err = hipHostMalloc(&stage[i], kPiece, hipHostMallocDefault);
    if (err == hipSuccess) err = hipEventCreateWithFlags(&done[i], hipEventDisableTiming);
  }
  int st = EG_OK;
  uint64_t pos = 0;
  for (int i = 0; err == hipSuccess && st == EG_OK && pos < c->blob_bytes; i ^= 1) {
    const size_t n = (size_t)std::min<uint64_t>(kPiece, c->blob_bytes - pos);
    err = hipEventSynchronize(done[i]);  // this staging buffer's previous copy has finished
    if (err != hipSuccess) break;
    if (std::fread(stage[i], 1, n, file.f) != n) {
      st = fail(ctx, EG_ERR_IO, "%s: short read of %s at blob byte %llu", op, c->path.c_str(),
                (unsigned long long)pos);
      break;
    }
    err = hipMemcpyAsync(static_cast<char*>(blob) + pos, stage[i], n, hipMemcpyHostToDevice, ctx->stream);
    if (err == hipSuccess) err = hipEventRecord(done[i], ctx->stream);
    pos += n;
  }
  if (err == hipSuccess) err = hipStreamSynchronize(ctx->stream);
  for (int i = 0; i < 2; i++) {
    if (done[i]) (void)hipEventDestroy(done[i]);
    if (stage[i]) (void)hipHostFree(stage[i]);
  }
  if (err != hipSuccess && st == EG_OK) st = eg::hip_fail(ctx, err, op);
  if (st != EG_OK) {
    (void)hipFree(blob);
    return st;
  }
  *out_blob = blob;
  return EG_OK;
}

// The Qwen2 checkpoint names (weights.ts:47; graph_decode.ts:246-385) over the uploaded blob.
int eg_container_model_desc(eg_context* ctx, const eg_container* c, const void* blob, const eg_model_config* cfg,
                            eg_model_desc* desc, eg_layer_desc* layers, uint32_t layers_capacity) {
  const char* op = "container_model_desc";
  if (!c || !blob || !cfg || !desc) return fail(ctx, EG_ERR_INVALID, "%s: NULL argument", op);
  const char* base = static_cast<const char*>(blob);
  auto find = [&](const std::string& name) -> const Tensor* {
    auto it = c->index.find(name);
    return it == c->index.end() ? nullptr : &c->tensors[it->second];
  };
  auto require = [&](const std::string& name, const Tensor** t) -> int {
    *t = find(name);
    return *t ? EG_OK : fail(ctx, EG_ERR_NOT_FOUND, "%s is missing", name.c_str());
  };
  auto vec = [&](const Tensor* t, uint64_t n, const float** out) -> int {
    if (t->dtype != EG_DTYPE_F32 || t->shape.size() != 1 || t->shape[0] != n)
      return fail(ctx, EG_ERR_FORMAT, "%s: expected an F32 vector of %llu", t->name.c_str(), (unsigned long long)n);
    *out = reinterpret_cast<const float*>(base + t->data[0]);
    return EG_OK;
  };
  auto quant = [&](const Tensor* t, uint64_t rows, uint64_t cols, eg_quant_matrix* m) -> int {
    if (t->dtype != EG_DTYPE_Q4 && t->dtype != EG_DTYPE_Q8)
      return fail(ctx, EG_ERR_FORMAT, "%s: %s is not a quantized tensor this decoder runs", t->name.c_str(),
                  t->dtype == EG_DTYPE_F16 ? "F16" : "F32");
    if (t->shape[0] != rows || t->shape[1] != cols)
      return fail(ctx, EG_ERR_FORMAT, "%s: shape [%llu, %llu], expected [%llu, %llu]", t->name.c_str(),
                  (unsigned long long)t->shape[0], (unsigned long long)t->shape[1], (unsigned long long)rows,
                  (unsigned long long)cols);
    m->packed = reinterpret_cast<const uint32_t*>(base + t->packed[0]);
    m->scales = reinterpret_cast<const float*>(base + t->scales[0]);
    m->zeros = reinterpret_cast<const uint32_t*>(base + t->zeros[0]);
    return EG_OK;
  };

  const Tensor* emb;
  int st = require("model.embed_tokens.weight", &emb);
  if (st != EG_OK) return st;
  if (find("lm_head.weight"))
    return fail(ctx, EG_ERR_FORMAT, "%s: lm_head.weight is present; this decoder runs tied embeddings only", op);
  // the tied table: Q4 / Q8, or F16 / F32 as it is (--embed-dtype f16 / f32; embedding_variants.ts:26-74)
  const bool dense_table = emb->dtype == EG_DTYPE_F16 || emb->dtype == EG_DTYPE_F32;
  if (dense_table && emb->shape.size() != 2)
    return fail(ctx, EG_ERR_FORMAT, "model.embed_tokens.weight: an %s table must be 2-D",
                emb->dtype == EG_DTYPE_F16 ? "F16" : "F32");
  uint32_t n_layers = 0;
  while (find("model.layers." + std::to_string(n_layers) + ".self_attn.q_proj.weight")) n_layers++;
  if (n_layers == 0) return fail(ctx, EG_ERR_NOT_FOUND, "model.layers.0.self_attn.q_proj.weight is missing");
  if (!layers || layers_capacity < n_layers)
    return fail(ctx, EG_ERR_RANGE, "%s: the model has %u layers, room for %u", op, n_layers, layers_capacity);
  if (cfg->head_dim == 0) return fail(ctx, EG_ERR_INVALID, "%s: head_dim is zero", op);

  const uint64_t vocab = emb->shape[0], hidden = emb->shape[1];
  const std::string l0 = "model.layers.0.";
  const Tensor *q0, *k0, *g0;
  if ((st = require(l0 + "self_attn.q_proj.weight", &q0)) != EG_OK) return st;
  if ((st = require(l0 + "self_attn.k_proj.weight", &k0)) != EG_OK) return st;
  if ((st = require(l0 + "mlp.gate_proj.weight", &g0)) != EG_OK) return st;
  if (q0->shape.size() != 2 || k0->shape.size() != 2 || g0->shape.size() != 2)
    return fail(ctx, EG_ERR_FORMAT, "%s: layer 0 projections must be 2-D", op);
  const uint64_t intermediate = g0->shape[0];
  if (q0->shape[0] % cfg->head_dim != 0 || k0->shape[0] % cfg->head_dim != 0)
    return fail(ctx, EG_ERR_FORMAT, "%s: q rows %llu / k rows %llu are not multiples of head_dim %u", op,
                (unsigned long long)q0->shape[0], (unsigned long long)k0->shape[0], cfg->head_dim);
  const uint64_t kvn = k0->shape[0];

  *desc = eg_model_desc{};
  desc->layers = n_layers;
  desc->hidden = (uint32_t)hidden;
  desc->heads = (uint32_t)(q0->shape[0] / cfg->head_dim);
  desc->kv_heads = (uint32_t)(kvn / cfg->head_dim);
  desc->head_dim = cfg->head_dim;
  desc->intermediate = (uint32_t)intermediate;
  desc->vocab = (uint32_t)vocab;
  desc->max_context = cfg->max_context;
  desc->rms_eps = cfg->rms_eps;
  desc->rope_theta = cfg->rope_theta;
  desc->encoding = EG_ENC_OFFSET_ZEROS;  // the container's quantizer is asymmetric (quantize.py:74-103)
  desc->bits = q0->bits;
  desc->block_size = q0->block_size;
  if (dense_table) {
    desc->embedding = eg_quant_matrix{};
    desc->embedding.packed = reinterpret_cast<const uint32_t*>(base + emb->data[0]);
    desc->embed_encoding = EG_ENC_SIGNED;  // not read for an f16 / f32 table
    desc->embed_block_size = (uint32_t)hidden;
  } else {
    if ((st = quant(emb, vocab, hidden, &desc->embedding)) != EG_OK) return st;
    desc->embed_encoding = EG_ENC_OFFSET_ZEROS;
    desc->embed_block_size = emb->block_size;
  }
  desc->embed_bits = emb->bits;
  const Tensor* norm;
  if ((st = require("model.norm.weight", &norm)) != EG_OK) return st;
  if ((st = vec(norm, hidden, &desc->final_norm)) != EG_OK) return st;

  for (uint32_t l = 0; l < n_layers; l++) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    eg_layer_desc& L = layers[l];
    L = eg_layer_desc{};
    struct Proj {
      const char* name;
      eg_quant_matrix* m;
      uint64_t rows, cols;
    } projs[] = {{"self_attn.q_proj", &L.q, hidden, hidden},       {"self_attn.k_proj", &L.k, kvn, hidden},
                 {"self_attn.v_proj", &L.v, kvn, hidden},          {"self_attn.o_proj", &L.o, hidden, hidden},
                 {"mlp.gate_proj", &L.gate, intermediate, hidden}, {"mlp.up_proj", &L.up, intermediate, hidden},
                 {"mlp.down_proj", &L.down, hidden, intermediate}};
    for (const Proj& pr : projs) {
      const Tensor* t;
      if ((st = require(p + pr.name + ".weight", &t)) != EG_OK) return st;
      if (t->bits != desc->bits || t->block_size != desc->block_size)
        return fail(ctx, EG_ERR_FORMAT, "%s: %d-bit blocks of %u, the model's first projection has %d-bit blocks of %u",
                    t->name.c_str(), t->bits, t->block_size, desc->bits, desc->block_size);
      if ((st = quant(t, pr.rows, pr.cols, pr.m)) != EG_OK) return st;
    }
    const char* bias_names[3] = {"self_attn.q_proj.bias", "self_attn.k_proj.bias", "self_attn.v_proj.bias"};
    const float** bias_out[3] = {&L.q_bias, &L.k_bias, &L.v_bias};
    const uint64_t bias_rows[3] = {hidden, kvn, kvn};
    for (int i = 0; i < 3; i++)
      if (const Tensor* b = find(p + bias_names[i]))
        if ((st = vec(b, bias_rows[i], bias_out[i])) != EG_OK) return st;
    const Tensor *n1, *n2;
    if ((st = require(p + "input_layernorm.weight", &n1)) != EG_OK) return st;
    if ((st = require(p + "post_attention_layernorm.weight", &n2)) != EG_OK) return st;
    if ((st = vec(n1, hidden, &L.input_norm)) != EG_OK) return st;
    if ((st = vec(n2, hidden, &L.post_attention_norm)) != EG_OK) return st;
  }
  desc->layer = layers;
  return EG_OK;
}

}  // extern "C"
