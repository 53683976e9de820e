// gguf.hip -- GGUF v3 files held in memory and the upload of a llama-family
// model's tensors to HBM. Host code only.
//
// The reader accepts and rejects what rusticide's GgufFile does
// (crates/rusticide-io/src/gguf/{header.rs,value.rs,file.rs,tensor_info.rs,
// extent.rs,metadata.rs,load.rs}), with the same error kinds, checked in the
// same order: header, metadata (typed values, arrays nested at most 8 deep
// and at most 2^22 array elements in all), the tensor table (at most 4
// dimensions, no element-count overflow, unique names), the alignment key,
// offsets aligned to it, disjoint extents, and a data section that starts
// inside the file. Array values are checked and counted but not kept: the
// model reads scalars and strings only.
//
// The model loader follows DecoderConfig::from_source and
// DecoderWeights::from_source for the llama family
// (crates/rusticide-transformer/src/{hyperparameters.rs,loader.rs},
// crates/rusticide-model/src/weights.rs:40-98,216-239): shapes are checked
// before each allocation, matrices get rh_matrix_load's checks (formats,
// the I2_S trailer) and are uploaded together through pinned staging
// buffers once all are checked; norms are read as f32.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "../../include/rusticide_hip.h"
#include "rh_internal.h"

namespace {

constexpr uint64_t kDefaultAlignment = 32;   // metadata.rs:6
constexpr uint32_t kMaxDimensions = 4;       // tensor_info.rs
constexpr size_t kMaxArrayDepth = 8;         // value.rs:8
constexpr size_t kMaxMetadataElements = size_t{1} << 22;  // value.rs:14
constexpr uint32_t kArray = 9, kString = 8;

// An error with its detail, as the ABI reports it.
struct Err {
  uint32_t kind = RH_GGUF_OK;
  uint64_t value = 0;
  std::string name, other;
};

Err make_err(uint32_t kind, uint64_t value = 0, std::string name = std::string(), std::string other = std::string()) {
  Err e;
  e.kind = kind;
  e.value = value;
  e.name = std::move(name);
  e.other = std::move(other);
  return e;
}

void copy_name(char (&dst)[128], const std::string& src) {
  std::memset(dst, 0, sizeof dst);
  std::memcpy(dst, src.data(), std::min(src.size(), sizeof dst - 1));
}

void report(const Err& e, rh_gguf_error* out) {
  if (!out) return;
  out->kind = e.kind;
  out->value = e.value;
  copy_name(out->name, e.name);
  copy_name(out->other, e.other);
}

// String::from_utf8_lossy: each maximal invalid subsequence becomes U+FFFD.
std::string utf8_lossy(const uint8_t* s, size_t n) {
  std::string out;
  out.reserve(n);
  size_t i = 0;
  while (i < n) {
    const uint8_t b = s[i];
    if (b < 0x80) {
      out.push_back(static_cast<char>(b));
      i++;
      continue;
    }
    size_t need = 0;
    uint8_t lo = 0x80, hi = 0xBF;
    if (b >= 0xC2 && b <= 0xDF) need = 1;
    else if (b == 0xE0) { need = 2; lo = 0xA0; }
    else if ((b >= 0xE1 && b <= 0xEC) || b == 0xEE || b == 0xEF) need = 2;
    else if (b == 0xED) { need = 2; hi = 0x9F; }
    else if (b == 0xF0) { need = 3; lo = 0x90; }
    else if (b >= 0xF1 && b <= 0xF3) need = 3;
    else if (b == 0xF4) { need = 3; hi = 0x8F; }
    size_t k = 1;
    bool ok = need > 0;
    for (; ok && k <= need; k++) {
      if (i + k >= n) { ok = false; break; }
      const uint8_t c = s[i + k];
      if (c < (k == 1 ? lo : 0x80) || c > (k == 1 ? hi : 0xBF)) { ok = false; break; }
    }
    if (ok) {
      out.append(reinterpret_cast<const char*>(s + i), need + 1);
      i += need + 1;
    } else {
      out.append("\xEF\xBF\xBD");
      i += need > 0 ? k : 1;
    }
  }
  return out;
}

// Cursor (cursor.rs): bounds-checked little-endian reads.
struct Cursor {
  const uint8_t* p;
  size_t n, pos = 0;
  bool take(size_t k, const uint8_t** out) {
    if (k > n - pos) return false;
    *out = p + pos;
    pos += k;
    return true;
  }
  bool u32(uint32_t* v) {
    const uint8_t* b;
    if (!take(4, &b)) return false;
    std::memcpy(v, b, 4);
    return true;
  }
  bool u64(uint64_t* v) {
    const uint8_t* b;
    if (!take(8, &b)) return false;
    std::memcpy(v, b, 8);
    return true;
  }
  bool string(std::string* s) {
    uint64_t len;
    const uint8_t* b;
    if (!u64(&len) || !take(len, &b)) return false;
    *s = utf8_lossy(b, len);
    return true;
  }
};

// A metadata value as the model reads it: scalars and strings (arrays keep
// only their type).
struct Value {
  uint32_t type = 0;
  uint64_t u = 0;  // unsigned kinds, and bool
  int64_t i = 0;   // signed kinds
  double f = 0.0;  // float kinds (f32 stored widened, exactly)
  std::string s;
};

struct Budget {
  size_t left = kMaxMetadataElements;
};

bool scalar_size(uint32_t type, size_t* size) {
  static const size_t sizes[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  if (type > 12) return false;
  *size = sizes[type];
  return true;
}

// parse_value_at_depth / parse_array (value.rs:136-186).
bool parse_value(Cursor& c, uint32_t type, size_t depth, Budget& budget, Value* v, Err* err) {
  if (type > 12) {
    *err = make_err(RH_GGUF_INVALID_VALUE_TYPE, type);
    return false;
  }
  if (v) v->type = type;
  if (type == kString) {
    std::string s;
    if (!c.string(&s)) {
      *err = make_err(RH_GGUF_UNEXPECTED_EOF);
      return false;
    }
    if (v) v->s = std::move(s);
    return true;
  }
  if (type == kArray) {
    if (depth + 1 > kMaxArrayDepth) {
      *err = make_err(RH_GGUF_NESTING_TOO_DEEP, kMaxArrayDepth);
      return false;
    }
    uint32_t item;
    uint64_t len;
    if (!c.u32(&item)) {
      *err = make_err(RH_GGUF_UNEXPECTED_EOF);
      return false;
    }
    if (item > 12) {
      *err = make_err(RH_GGUF_INVALID_VALUE_TYPE, item);
      return false;
    }
    if (!c.u64(&len)) {
      *err = make_err(RH_GGUF_UNEXPECTED_EOF);
      return false;
    }
    for (uint64_t k = 0; k < len; k++) {
      if (budget.left == 0) {
        *err = make_err(RH_GGUF_METADATA_TOO_LARGE, kMaxMetadataElements);
        return false;
      }
      budget.left--;
      if (!parse_value(c, item, depth + 1, budget, nullptr, err)) return false;
    }
    return true;
  }
  size_t size = 0;
  scalar_size(type, &size);
  const uint8_t* b;
  if (!c.take(size, &b)) {
    *err = make_err(RH_GGUF_UNEXPECTED_EOF);
    return false;
  }
  if (!v) return true;
  switch (type) {
    case 0: v->u = b[0]; break;
    case 1: v->i = static_cast<int8_t>(b[0]); break;
    case 2: { uint16_t x; std::memcpy(&x, b, 2); v->u = x; break; }
    case 3: { int16_t x; std::memcpy(&x, b, 2); v->i = x; break; }
    case 4: { uint32_t x; std::memcpy(&x, b, 4); v->u = x; break; }
    case 5: { int32_t x; std::memcpy(&x, b, 4); v->i = x; break; }
    case 6: { float x; std::memcpy(&x, b, 4); v->f = x; break; }
    case 7: v->u = b[0] != 0; break;
    case 10: std::memcpy(&v->u, b, 8); break;
    case 11: std::memcpy(&v->i, b, 8); break;
    case 12: std::memcpy(&v->f, b, 8); break;
    default: break;
  }
  return true;
}

struct TensorInfo {
  std::string name;
  std::vector<uint64_t> shape;  // outermost first; [1] for a scalar
  uint32_t type_id = 0;
  uint64_t offset = 0;
};

// Shape::numel (crates/rusticide-core/src/shape.rs:37-45): 0 with any zero
// extent, else the product, UINT64_MAX when it overflows.
uint64_t numel(const std::vector<uint64_t>& shape) {
  for (uint64_t d : shape)
    if (d == 0) return 0;
  uint64_t n = 1;
  for (uint64_t d : shape) {
    if (n > UINT64_MAX / d) return UINT64_MAX;
    n *= d;
  }
  return n;
}

// The block formats the reader knows (quantize/src/format.rs:31-92).
bool block_format(uint32_t type_id, uint64_t* block_size, uint64_t* block_bytes, uint64_t* trailer) {
  switch (type_id) {
    case 2: *block_size = 32; *block_bytes = 18; *trailer = 0; return true;    // Q4_0
    case 6: *block_size = 32; *block_bytes = 22; *trailer = 0; return true;    // Q5_0
    case 8: *block_size = 32; *block_bytes = 34; *trailer = 0; return true;    // Q8_0
    case 12: *block_size = 256; *block_bytes = 144; *trailer = 0; return true; // Q4_K
    case 14: *block_size = 256; *block_bytes = 210; *trailer = 0; return true; // Q6_K
    case 36: *block_size = 128; *block_bytes = 32; *trailer = 32; return true; // I2_S
    default: return false;
  }
}

// byte_len (extent.rs:20-38): F32, F16, or whole blocks plus a trailer.
bool byte_len(const TensorInfo& t, uint64_t* len, Err* err) {
  const uint64_t n = numel(t.shape);
  if (t.type_id == 0 || t.type_id == 1) {
    const uint64_t w = t.type_id == 0 ? 4 : 2;
    if (n > UINT64_MAX / w) {
      *err = make_err(RH_GGUF_CAST_OVERFLOW);
      return false;
    }
    *len = n * w;
    return true;
  }
  uint64_t bs, bb, tr;
  if (!block_format(t.type_id, &bs, &bb, &tr)) {
    *err = make_err(RH_GGUF_UNSUPPORTED_TENSOR_TYPE, t.type_id, t.name);
    return false;
  }
  const uint64_t blocks = n / bs + (n % bs != 0);
  if (blocks > UINT64_MAX / bb || blocks * bb > UINT64_MAX - tr) {
    *err = make_err(RH_GGUF_CAST_OVERFLOW);
    return false;
  }
  *len = blocks * bb + tr;
  return true;
}

}  // namespace

struct rh_gguf {
  // the file: a copy held here, or a read-only mapping of it
  std::vector<uint8_t> owned;
  void* map = nullptr;
  const uint8_t* bytes = nullptr;
  size_t size = 0;
  std::unordered_map<std::string, Value> meta;
  std::vector<TensorInfo> tensors;  // sorted by name
  std::unordered_map<std::string, size_t> index;
  size_t data_start = 0;

  ~rh_gguf() {
    if (map) munmap(map, size);
  }
};

namespace {

// GgufFile::from_bytes (file.rs:39-62).
bool parse_file(rh_gguf* g, Err* err) {
  Cursor c{g->bytes, g->size};
  // Header::parse (header.rs:20-36)
  if (c.n < 24) {
    *err = make_err(RH_GGUF_UNEXPECTED_EOF);
    return false;
  }
  const uint8_t* magic;
  c.take(4, &magic);
  if (std::memcmp(magic, "GGUF", 4) != 0) {
    *err = make_err(RH_GGUF_INVALID_MAGIC);
    return false;
  }
  uint32_t version;
  uint64_t tensor_count, kv_count;
  c.u32(&version);
  if (version != 3) {
    *err = make_err(RH_GGUF_UNSUPPORTED_VERSION, version);
    return false;
  }
  c.u64(&tensor_count);
  c.u64(&kv_count);
  // parse_metadata (file.rs:104-123)
  Budget budget;
  for (uint64_t k = 0; k < kv_count; k++) {
    std::string key;
    uint32_t type;
    if (!c.string(&key) || !c.u32(&type)) {
      *err = make_err(RH_GGUF_UNEXPECTED_EOF);
      return false;
    }
    Value v;
    if (!parse_value(c, type, 0, budget, &v, err)) return false;
    if (!g->meta.emplace(key, std::move(v)).second) {
      *err = make_err(RH_GGUF_DUPLICATE_KEY, 0, key);
      return false;
    }
  }
  // parse_tensor_table (file.rs:125-138), parse_tensor_info (tensor_info.rs:26-62)
  std::unordered_map<std::string, size_t> seen;
  std::vector<TensorInfo> tensors;
  for (uint64_t k = 0; k < tensor_count; k++) {
    TensorInfo t;
    uint32_t dims;
    if (!c.string(&t.name) || !c.u32(&dims)) {
      *err = make_err(RH_GGUF_UNEXPECTED_EOF);
      return false;
    }
    if (dims > kMaxDimensions) {
      *err = make_err(RH_GGUF_TOO_MANY_DIMENSIONS, dims);
      return false;
    }
    for (uint32_t d = 0; d < dims; d++) {
      uint64_t e;
      if (!c.u64(&e)) {
        *err = make_err(RH_GGUF_UNEXPECTED_EOF);
        return false;
      }
      t.shape.push_back(e);
    }
    std::reverse(t.shape.begin(), t.shape.end());
    if (t.shape.empty()) t.shape.push_back(1);
    if (numel(t.shape) == UINT64_MAX) {
      *err = make_err(RH_GGUF_SHAPE_OVERFLOW, 0, t.name);
      return false;
    }
    if (!c.u32(&t.type_id) || !c.u64(&t.offset)) {
      *err = make_err(RH_GGUF_UNEXPECTED_EOF);
      return false;
    }
    if (!seen.emplace(t.name, tensors.size()).second) {
      *err = make_err(RH_GGUF_DUPLICATE_TENSOR, 0, t.name);
      return false;
    }
    tensors.push_back(std::move(t));
  }
  // Metadata::alignment (metadata.rs:105-111)
  uint64_t alignment = kDefaultAlignment;
  auto a = g->meta.find("general.alignment");
  if (a != g->meta.end()) {
    const Value& v = a->second;
    if (v.type != 4 || v.u == 0 || (v.u & (v.u - 1)) != 0) {
      *err = make_err(RH_GGUF_INVALID_ALIGNMENT, v.type == 4 ? v.u : 0);
      return false;
    }
    alignment = v.u;
  }
  // ensure_aligned_offsets (file.rs:140-150)
  for (const TensorInfo& t : tensors)
    if (t.offset % alignment != 0) {
      *err = make_err(RH_GGUF_MISALIGNED_TENSOR, t.offset, t.name);
      return false;
    }
  // ensure_disjoint (extent.rs:40-58): tensors whose length cannot be
  // computed, or that are empty, take no part
  std::vector<std::pair<std::pair<uint64_t, uint64_t>, size_t>> extents;
  for (size_t i = 0; i < tensors.size(); i++) {
    uint64_t len;
    Err ignored;
    if (!byte_len(tensors[i], &len, &ignored) || len == 0) continue;
    if (tensors[i].offset > UINT64_MAX - len) continue;
    extents.push_back({{tensors[i].offset, tensors[i].offset + len}, i});
  }
  // (start, end, name) order, as the tuples sort
  std::sort(extents.begin(), extents.end(), [&](const auto& x, const auto& y) {
    if (x.first != y.first) return x.first < y.first;
    return tensors[x.second].name < tensors[y.second].name;
  });
  for (size_t i = 1; i < extents.size(); i++)
    if (extents[i - 1].first.second > extents[i].first.first) {
      *err = make_err(RH_GGUF_OVERLAPPING_TENSORS, 0, tensors[extents[i - 1].second].name,
                      tensors[extents[i].second].name);
      return false;
    }
  // align_up (file.rs:152-158) and the start inside the file
  const uint64_t pos = c.pos;
  if (pos > UINT64_MAX - (alignment - 1)) {
    *err = make_err(RH_GGUF_CAST_OVERFLOW);
    return false;
  }
  const uint64_t start = (pos + alignment - 1) & ~(alignment - 1);
  if (start > g->size) {
    *err = make_err(RH_GGUF_UNEXPECTED_EOF);
    return false;
  }
  g->data_start = static_cast<size_t>(start);
  std::sort(tensors.begin(), tensors.end(),
            [](const TensorInfo& x, const TensorInfo& y) { return x.name < y.name; });
  for (size_t i = 0; i < tensors.size(); i++) g->index.emplace(tensors[i].name, i);
  g->tensors = std::move(tensors);
  return true;
}

// GgufFile::layout / tensor_bytes (load.rs:56-79).
bool tensor_bytes(const rh_gguf* g, const TensorInfo& t, const uint8_t** data, size_t* len, Err* err) {
  uint64_t n;
  if (!byte_len(t, &n, err)) return false;
  const uint64_t start = g->data_start;
  if (t.offset > UINT64_MAX - start || start + t.offset > UINT64_MAX - n || start + t.offset + n > g->size) {
    *err = make_err(RH_GGUF_UNEXPECTED_EOF);
    return false;
  }
  *data = g->bytes + start + t.offset;
  *len = static_cast<size_t>(n);
  return true;
}

const Value* meta(const rh_gguf* g, const char* key) {
  auto it = g->meta.find(key);
  return it == g->meta.end() ? nullptr : &it->second;
}

// arch_unsigned: u32/u64 or a non-negative i32/i64.
bool as_unsigned(const Value& v, uint64_t* out) {
  switch (v.type) {
    case 4: case 10: *out = v.u; return true;
    case 5: case 11: if (v.i < 0) return false; *out = static_cast<uint64_t>(v.i); return true;
    default: return false;
  }
}

bool as_float(const Value& v, float* out) {
  if (v.type == 6 || v.type == 12) {
    *out = static_cast<float>(v.f);
    return true;
  }
  return false;
}

}  // namespace

struct rh_gguf_model {
  rh_ctx* ctx = nullptr;
  rh_decoder_config config{};
  std::vector<rh_matrix*> matrices;  // owned
  std::vector<rh::PendingUpload> pending;  // checked and allocated, not yet uploaded
  std::vector<std::vector<float>> norms;
  std::vector<rh_decoder_block> blocks;
  rh_decoder_weights weights{};
};

namespace {

rh_status model_fail(rh_ctx* ctx, rh_status st, const std::string& msg) { return rh::set_last_error(ctx, st, msg); }

// check_shape (weights.rs:225-239).
rh_status check_shape(rh_ctx* ctx, const rh_gguf* g, const std::string& name, const std::vector<uint64_t>& want,
                      const TensorInfo** info) {
  auto it = g->index.find(name);
  if (it == g->index.end()) return model_fail(ctx, RH_ERR_MISSING_TENSOR, "missing tensor " + name);
  const TensorInfo& t = g->tensors[it->second];
  if (t.shape != want) return model_fail(ctx, RH_ERR_SHAPE_MISMATCH, "tensor " + name + " has an unexpected shape");
  *info = &t;
  return RH_OK;
}

// Matrix::load (weights.rs:48-98): checked and allocated on the device; the
// bytes go up with every other matrix's once all are checked.
rh_status load_matrix(rh_gguf_model* m, const rh_gguf* g, const std::string& name, size_t rows, size_t cols,
                      const rh_matrix** out) {
  const TensorInfo* t = nullptr;
  rh_status st = check_shape(m->ctx, g, name, {rows, cols}, &t);
  if (st != RH_OK) return st;
  if (cols == 0) return model_fail(m->ctx, RH_ERR_INVALID_CONFIG, "a weight matrix has no columns");
  const uint8_t* data = nullptr;
  size_t len = 0;
  Err err;
  if (!tensor_bytes(g, *t, &data, &len, &err)) return model_fail(m->ctx, RH_ERR_GGUF, "tensor " + name + ": bad extent");
  rh::PendingUpload p;
  st = rh::matrix_prepare(m->ctx, t->type_id, data, len, rows, cols, &p);
  if (st != RH_OK) return st;
  m->matrices.push_back(p.m);
  *out = p.m;
  m->pending.push_back(std::move(p));
  return RH_OK;
}

// load_vector (weights.rs:216-223): F32 or F16 read as f32.
rh_status load_vector(rh_gguf_model* m, const rh_gguf* g, const std::string& name, size_t len, const float** out) {
  const TensorInfo* t = nullptr;
  rh_status st = check_shape(m->ctx, g, name, {len}, &t);
  if (st != RH_OK) return st;
  if (t->type_id != 0 && t->type_id != 1)
    return model_fail(m->ctx, RH_ERR_MISSING_KERNEL, "norm " + name + " is not F32 or F16");
  const uint8_t* data = nullptr;
  size_t bytes = 0;
  Err err;
  if (!tensor_bytes(g, *t, &data, &bytes, &err)) return model_fail(m->ctx, RH_ERR_GGUF, "tensor " + name + ": bad extent");
  std::vector<float> v(len);
  for (size_t i = 0; i < len; i++) {
    if (t->type_id == 0) {
      std::memcpy(&v[i], data + 4 * i, 4);
    } else {
      _Float16 h;
      std::memcpy(&h, data + 2 * i, 2);
      v[i] = static_cast<float>(h);
    }
  }
  m->norms.push_back(std::move(v));
  *out = m->norms.back().data();
  return RH_OK;
}

}  // namespace

extern "C" {

rh_status rh_gguf_parse(const void* bytes, size_t len, rh_gguf** out, rh_gguf_error* err) {
  if (!out || (!bytes && len)) return RH_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  rh_gguf* g = new (std::nothrow) rh_gguf();
  if (!g) return RH_ERR_OUT_OF_MEMORY;
  try {
    g->owned.assign(static_cast<const uint8_t*>(bytes), static_cast<const uint8_t*>(bytes) + len);
    g->bytes = g->owned.data();
    g->size = len;
    Err e;
    if (!parse_file(g, &e)) {
      report(e, err);
      delete g;
      return RH_ERR_GGUF;
    }
  } catch (const std::bad_alloc&) {
    delete g;
    return RH_ERR_OUT_OF_MEMORY;
  }
  report(Err{}, err);
  *out = g;
  return RH_OK;
}

rh_status rh_gguf_open(const char* path, rh_gguf** out, rh_gguf_error* err) {
  if (!path || !out) return RH_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  // non-blocking, so that a pipe without a writer is refused rather than waited on
  const int fd = open(path, O_RDONLY | O_CLOEXEC | O_NONBLOCK);
  if (fd < 0) {
    report(make_err(RH_GGUF_IO, static_cast<uint64_t>(errno), path), err);
    return RH_ERR_GGUF;
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    report(make_err(RH_GGUF_IO, static_cast<uint64_t>(errno), path), err);
    close(fd);
    return RH_ERR_GGUF;
  }
  if (!S_ISREG(st.st_mode)) {  // a directory, device or pipe could be read without end
    report(make_err(RH_GGUF_NOT_A_FILE, 0, path), err);
    close(fd);
    return RH_ERR_GGUF;
  }
  rh_gguf* g = new (std::nothrow) rh_gguf();
  if (!g) {
    close(fd);
    return RH_ERR_OUT_OF_MEMORY;
  }
  g->size = static_cast<size_t>(st.st_size);
  if (g->size) {
    void* p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      report(make_err(RH_GGUF_IO, static_cast<uint64_t>(errno), path), err);
      close(fd);
      delete g;
      return RH_ERR_GGUF;
    }
    g->map = p;
    g->bytes = static_cast<const uint8_t*>(p);
  }
  close(fd);
  try {
    Err e;
    if (!parse_file(g, &e)) {
      report(e, err);
      delete g;
      return RH_ERR_GGUF;
    }
  } catch (const std::bad_alloc&) {
    delete g;
    return RH_ERR_OUT_OF_MEMORY;
  }
  report(Err{}, err);
  *out = g;
  return RH_OK;
}

void rh_gguf_free(rh_gguf* g) { delete g; }

size_t rh_gguf_metadata_count(const rh_gguf* g) { return g ? g->meta.size() : 0; }
size_t rh_gguf_tensor_count(const rh_gguf* g) { return g ? g->tensors.size() : 0; }

rh_status rh_gguf_tensor_at(const rh_gguf* g, size_t index, const char** name, size_t* name_len, uint32_t* type_id,
                            size_t* n_dims, uint64_t shape[4], uint64_t* offset) {
  if (!g || index >= g->tensors.size()) return RH_ERR_INVALID_ARGUMENT;
  const TensorInfo& t = g->tensors[index];
  if (name) *name = t.name.c_str();
  if (name_len) *name_len = t.name.size();
  if (type_id) *type_id = t.type_id;
  if (n_dims) *n_dims = t.shape.size();
  if (shape)
    for (size_t d = 0; d < 4; d++) shape[d] = d < t.shape.size() ? t.shape[d] : 0;
  if (offset) *offset = t.offset;
  return RH_OK;
}

rh_status rh_gguf_tensor_find(const rh_gguf* g, const char* name, size_t* index) {
  if (!g || !name || !index) return RH_ERR_INVALID_ARGUMENT;
  auto it = g->index.find(name);
  if (it == g->index.end()) return RH_ERR_MISSING_TENSOR;
  *index = it->second;
  return RH_OK;
}

rh_status rh_gguf_tensor_data(const rh_gguf* g, const char* name, const uint8_t** data, size_t* len,
                              rh_gguf_error* err) {
  if (!g || !name || !data || !len) return RH_ERR_INVALID_ARGUMENT;
  auto it = g->index.find(name);
  Err e;
  if (it == g->index.end()) {
    report(make_err(RH_GGUF_TENSOR_NOT_FOUND, 0, name), err);
    return RH_ERR_GGUF;
  }
  if (!tensor_bytes(g, g->tensors[it->second], data, len, &e)) {
    report(e, err);
    return RH_ERR_GGUF;
  }
  report(Err{}, err);
  return RH_OK;
}

rh_status rh_gguf_meta_type(const rh_gguf* g, const char* key, uint32_t* value_type) {
  if (!g || !key || !value_type) return RH_ERR_INVALID_ARGUMENT;
  const Value* v = meta(g, key);
  if (!v) return RH_ERR_MISSING_METADATA;
  *value_type = v->type;
  return RH_OK;
}

rh_status rh_gguf_meta_uint(const rh_gguf* g, const char* key, uint64_t* out) {
  if (!g || !key || !out) return RH_ERR_INVALID_ARGUMENT;
  const Value* v = meta(g, key);
  if (!v || !as_unsigned(*v, out)) return RH_ERR_MISSING_METADATA;
  return RH_OK;
}

rh_status rh_gguf_meta_float(const rh_gguf* g, const char* key, float* out) {
  if (!g || !key || !out) return RH_ERR_INVALID_ARGUMENT;
  const Value* v = meta(g, key);
  if (!v || !as_float(*v, out)) return RH_ERR_MISSING_METADATA;
  return RH_OK;
}

rh_status rh_gguf_meta_string(const rh_gguf* g, const char* key, const char** out, size_t* len) {
  if (!g || !key || !out) return RH_ERR_INVALID_ARGUMENT;
  const Value* v = meta(g, key);
  if (!v || v->type != kString) return RH_ERR_MISSING_METADATA;
  *out = v->s.c_str();
  if (len) *len = v->s.size();
  return RH_OK;
}

rh_status rh_gguf_decoder_config(rh_ctx* ctx, const rh_gguf* g, rh_decoder_config* out) {
  if (!g || !out) return RH_ERR_INVALID_ARGUMENT;
  // ModelRegistry (crates/rusticide-model/src/registry.rs:39-55)
  const Value* arch = meta(g, "general.architecture");
  if (!arch || arch->type != kString)
    return model_fail(ctx, RH_ERR_MISSING_METADATA, "missing metadata general.architecture");
  if (arch->s != "llama")
    return model_fail(ctx, RH_ERR_UNKNOWN_ARCHITECTURE, "unknown architecture " + arch->s + "; supported: llama");
  // DecoderConfig::read (hyperparameters.rs:96-120)
  auto required = [&](const char* suffix, size_t* v) -> rh_status {
    const std::string key = std::string("llama.") + suffix;
    const Value* x = meta(g, key.c_str());
    uint64_t u = 0;
    if (!x || !as_unsigned(*x, &u)) return model_fail(ctx, RH_ERR_MISSING_METADATA, "missing metadata " + key);
    *v = static_cast<size_t>(u);
    return RH_OK;
  };
  rh_decoder_config c{};
  rh_status st;
  if ((st = required("embedding_length", &c.embedding_length)) != RH_OK) return st;
  if ((st = required("attention.head_count", &c.head_count)) != RH_OK) return st;
  if ((st = required("block_count", &c.block_count)) != RH_OK) return st;
  if ((st = required("feed_forward_length", &c.feed_forward_length)) != RH_OK) return st;
  c.head_count_kv = c.head_count;
  if (const Value* x = meta(g, "llama.attention.head_count_kv")) {
    uint64_t u;
    if (as_unsigned(*x, &u)) c.head_count_kv = static_cast<size_t>(u);
  }
  c.head_dim = c.head_count ? c.embedding_length / c.head_count : 0;
  if ((st = required("context_length", &c.context_length)) != RH_OK) return st;
  c.rope_freq_base = 10000.0f;
  c.rms_norm_eps = 1e-5f;
  if (const Value* x = meta(g, "llama.rope.freq_base")) as_float(*x, &c.rope_freq_base);
  if (const Value* x = meta(g, "llama.attention.layer_norm_rms_epsilon")) as_float(*x, &c.rms_norm_eps);
  // DecoderConfig::validate (config.rs:61-80), then sizes_fit
  // (hyperparameters.rs:60-67)
  auto ensure = [&](bool ok, const char* reason) -> rh_status {
    return ok ? RH_OK : model_fail(ctx, RH_ERR_INVALID_CONFIG, reason);
  };
  size_t width = 0, kv_dim = 0, projection = 0, square = 0, ffn = 0;
  if ((st = ensure(c.head_count != 0, "head count must be non-zero")) != RH_OK) return st;
  if ((st = ensure(c.head_count_kv != 0 && c.head_count % c.head_count_kv == 0,
                   "kv head count must be non-zero and divide the head count")) != RH_OK)
    return st;
  if ((st = ensure(c.head_dim != 0 && c.head_dim % 2 == 0, "head dimension must be even and non-zero")) != RH_OK)
    return st;
  if ((st = ensure(!__builtin_mul_overflow(c.head_count, c.head_dim, &width) && width == c.embedding_length,
                   "embedding length must be divisible by the head count: it must equal the head count times "
                   "the head dimension")) != RH_OK)
    return st;
  if ((st = ensure(c.block_count != 0 && c.feed_forward_length != 0 && c.context_length != 0,
                   "block count, feed-forward length and context length must be non-zero")) != RH_OK)
    return st;
  const bool fits = !__builtin_mul_overflow(c.head_count_kv, c.head_dim, &kv_dim) &&
                    !__builtin_mul_overflow(kv_dim, c.embedding_length, &projection) &&
                    !__builtin_mul_overflow(c.embedding_length, c.embedding_length, &square) &&
                    !__builtin_mul_overflow(c.embedding_length, c.feed_forward_length, &ffn);
  if ((st = ensure(fits, "model dimensions are too large")) != RH_OK) return st;
  if (const Value* x = meta(g, "llama.rope.dimension_count")) {
    if (x->type != 4 && x->type != 10)
      return model_fail(ctx, RH_ERR_INVALID_CONFIG, "rope dimension count must be an unsigned integer");
    if ((st = ensure(x->u == c.head_dim, "rope dimension count must equal the head dimension")) != RH_OK) return st;
  }
  // vocab_size (hyperparameters.rs:46-58)
  auto it = g->index.find("token_embd.weight");
  if (it == g->index.end()) return model_fail(ctx, RH_ERR_MISSING_TENSOR, "missing tensor token_embd.weight");
  const std::vector<uint64_t>& shape = g->tensors[it->second].shape;
  if (shape.size() != 2 || shape[1] != c.embedding_length || shape[0] == 0)
    return model_fail(ctx, RH_ERR_INVALID_CONFIG, "token_embd.weight must have shape [vocab, embedding length]");
  c.vocab_size = static_cast<size_t>(shape[0]);
  *out = c;
  return RH_OK;
}

rh_status rh_gguf_model_load(rh_ctx* ctx, const rh_gguf* g, rh_gguf_model** out) {
  if (!ctx || !g || !out) return RH_ERR_INVALID_ARGUMENT;
  *out = nullptr;
  rh_gguf_model* m = new (std::nothrow) rh_gguf_model();
  if (!m) return RH_ERR_OUT_OF_MEMORY;
  m->ctx = ctx;
  rh_status st = rh_gguf_decoder_config(ctx, g, &m->config);
  const rh_decoder_config& c = m->config;
  try {
    if (st == RH_OK) {
      m->norms.reserve(2 * c.block_count + 1);  // pointers into it are handed out
      m->blocks.resize(c.block_count);
    }
    const size_t e = c.embedding_length, f = c.feed_forward_length, kv = c.head_count_kv * c.head_dim;
    // load_block (loader.rs:49-92), in its order
    for (size_t l = 0; st == RH_OK && l < c.block_count; l++) {
      rh_decoder_block& b = m->blocks[l];
      auto name = [&](const char* part) { return "blk." + std::to_string(l) + "." + part + ".weight"; };
      if ((st = load_vector(m, g, name("attn_norm"), e, &b.attn_norm)) != RH_OK) break;
      if ((st = load_matrix(m, g, name("attn_q"), e, e, &b.attn_q)) != RH_OK) break;
      if ((st = load_matrix(m, g, name("attn_k"), kv, e, &b.attn_k)) != RH_OK) break;
      if ((st = load_matrix(m, g, name("attn_v"), kv, e, &b.attn_v)) != RH_OK) break;
      for (const char* part : {"attn_q", "attn_k", "attn_v"}) {
        const std::string bias = "blk." + std::to_string(l) + "." + part + ".bias";
        if (g->index.count(bias)) {
          st = model_fail(ctx, RH_ERR_MISSING_KERNEL, "tensor " + bias + ": this decoder adds no attention bias");
          break;
        }
      }
      if (st != RH_OK) break;
      if ((st = load_matrix(m, g, name("attn_output"), e, e, &b.attn_output)) != RH_OK) break;
      if ((st = load_vector(m, g, name("ffn_norm"), e, &b.ffn_norm)) != RH_OK) break;
      if ((st = load_matrix(m, g, name("ffn_gate"), f, e, &b.ffn_gate)) != RH_OK) break;
      if ((st = load_matrix(m, g, name("ffn_up"), f, e, &b.ffn_up)) != RH_OK) break;
      if ((st = load_matrix(m, g, name("ffn_down"), e, f, &b.ffn_down)) != RH_OK) break;
    }
    // DecoderWeights::from_source (loader.rs:19-47): output when present,
    // then token_embd and output_norm
    if (st == RH_OK && g->index.count("output.weight"))
      st = load_matrix(m, g, "output.weight", c.vocab_size, e, &m->weights.output);
    if (st == RH_OK) st = load_matrix(m, g, "token_embd.weight", c.vocab_size, e, &m->weights.token_embd);
    if (st == RH_OK) st = load_vector(m, g, "output_norm.weight", e, &m->weights.output_norm);
    // every tensor checked and allocated: the bytes go up in one pipelined pass
    if (st == RH_OK) st = rh::matrix_upload(ctx, m->pending.data(), m->pending.size());
    m->pending.clear();
    m->pending.shrink_to_fit();
  } catch (const std::bad_alloc&) {
    st = RH_ERR_OUT_OF_MEMORY;
  }
  if (st != RH_OK) {
    rh_gguf_model_free(m);
    return st;
  }
  m->weights.blocks = m->blocks.data();
  *out = m;
  return RH_OK;
}

const rh_decoder_config* rh_gguf_model_config(const rh_gguf_model* m) { return m ? &m->config : nullptr; }

rh_status rh_gguf_model_decoder(rh_gguf_model* m, rh_decoder** out) {
  if (!m || !out) return RH_ERR_INVALID_ARGUMENT;
  return rh_decoder_new(m->ctx, &m->config, &m->weights, out);
}

void rh_gguf_model_free(rh_gguf_model* m) {
  if (!m) return;
  for (rh_matrix* mat : m->matrices) rh_matrix_free(mat);
  delete m;
}

}  // extern "C"
