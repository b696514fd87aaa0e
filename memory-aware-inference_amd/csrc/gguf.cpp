// GGUF model store (include/si_hip_gguf.h).
//
// The container format follows parse_gguf (src/model.rs:1034-1240): magic,
// version 2 or 3, tensor and metadata counts, metadata key/value pairs (13
// value types, arrays nesting), the tensor index, then the tensor data at the
// first multiple of general.alignment (default 32) after the index.  A
// tensor's bytes run from its offset to the next tensor's offset in offset
// order, the last one to the end of the file.  Error messages are the
// reference's.  Files are mapped read-only (GgufModelStore::open,
// model.rs:625-666); nothing is copied until a tensor is uploaded.
#include "si_hip.h"
#include "si_hip_f32.h"
#include "si_hip_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "si_hip_shared.h"
#include "si_hip_status.h"

namespace {

using sihip::clear_error;
using sihip::set_error;

constexpr uint64_t kQ4Bytes = 144, kQ5Bytes = 176, kQ6Bytes = 210;

struct Value {
  uint32_t type = 0;
  uint32_t array_type = 0;
  uint64_t u64 = 0;
  int64_t i64 = 0;
  double f64 = 0.0;
  std::string str;
  std::vector<Value> items;
};

struct Tensor {
  std::string name;
  std::vector<uint64_t> shape;
  uint32_t ggml_type = 0;
  uint64_t offset = 0;
  uint64_t data_start = 0;
  uint64_t data_end = 0;
};

// A parse failure: status and message, raised through the reader.
constexpr int kMaxArrayDepth = 256;

struct ParseError {
  int status;
  std::string message;
};

[[noreturn]] void raise(const std::string &message, int status = SI_HIP_ERR_DIMENSIONS) {
  throw ParseError{status, message};
}

// UTF-8 check with the error position and length core::str::from_utf8
// reports (the reference formats them into its message, model.rs:1190-1193):
// returns true, or false with *valid_up_to = start of the bad sequence and
// *error_len = bytes in its maximal invalid prefix (1-3), 0 when the input
// ends inside the sequence.  Overlong forms, surrogates and values past
// U+10FFFF fail at their second byte.
bool check_utf8(const unsigned char *p, size_t n, size_t *valid_up_to, int *error_len) {
  size_t i = 0;
  while (i < n) {
    const unsigned c = p[i];
    if (c < 0x80) {
      ++i;
      continue;
    }
    const int width = (c >= 0xc2 && c <= 0xdf) ? 2 : (c >= 0xe0 && c <= 0xef) ? 3
                      : (c >= 0xf0 && c <= 0xf4) ? 4 : 0;
    *valid_up_to = i;
    if (width == 0) {
      *error_len = 1;
      return false;
    }
    // the accepted range of the second byte depends on the first
    unsigned lo = 0x80, hi = 0xbf;
    if (c == 0xe0) lo = 0xa0;
    else if (c == 0xed) hi = 0x9f;
    else if (c == 0xf0) lo = 0x90;
    else if (c == 0xf4) hi = 0x8f;
    for (int k = 1; k < width; ++k) {
      if (i + k >= n) {
        *error_len = 0;
        return false;
      }
      const unsigned b = p[i + k];
      if (k == 1 ? (b < lo || b > hi) : (b & 0xc0u) != 0x80u) {
        *error_len = k;
        return false;
      }
    }
    i += width;
  }
  return true;
}

// GgufReader (model.rs:1136-1232): little-endian fields, bounds-checked.
struct Reader {
  const uint8_t *bytes;
  uint64_t len;
  uint64_t offset = 0;

  const uint8_t *take(uint64_t n) {
    if (n > UINT64_MAX - offset) raise("GGUF offset overflows", SI_HIP_ERR_OVERFLOW);
    const uint64_t end = offset + n;
    if (end > len) raise("GGUF header is truncated");
    const uint8_t *p = bytes + offset;
    offset = end;
    return p;
  }
  template <typename T>
  T scalar() {
    T v;
    std::memcpy(&v, take(sizeof(T)), sizeof(T));
    return v;  // the file is little-endian, as is the host
  }
  std::string string() {
    const uint64_t n = scalar<uint64_t>();
    const uint8_t *p = take(n);
    size_t at = 0;
    int bad = 0;
    if (!check_utf8(p, (size_t)n, &at, &bad))
      raise("GGUF string is not UTF-8: " +
            (bad ? "invalid utf-8 sequence of " + std::to_string(bad) + " bytes from index "
                 : std::string("incomplete utf-8 byte sequence from index ")) +
            std::to_string(at));
    return std::string(reinterpret_cast<const char *>(p), (size_t)n);
  }
  Value value(uint32_t type, int depth = 0) {
    // Each nesting level costs 12 bytes of file; the cap bounds the
    // recursion a crafted file could ask for.
    if (depth > kMaxArrayDepth) raise("GGUF metadata arrays nest too deeply");
    Value v;
    v.type = type;
    switch (type) {
      case SI_HIP_GGUF_U8: v.u64 = scalar<uint8_t>(); break;
      case SI_HIP_GGUF_I8: v.i64 = scalar<int8_t>(); break;
      case SI_HIP_GGUF_U16: v.u64 = scalar<uint16_t>(); break;
      case SI_HIP_GGUF_I16: v.i64 = scalar<int16_t>(); break;
      case SI_HIP_GGUF_U32: v.u64 = scalar<uint32_t>(); break;
      case SI_HIP_GGUF_I32: v.i64 = scalar<int32_t>(); break;
      case SI_HIP_GGUF_F32: v.f64 = (double)scalar<float>(); break;
      case SI_HIP_GGUF_BOOL: v.u64 = scalar<uint8_t>() != 0 ? 1u : 0u; break;
      case SI_HIP_GGUF_STRING: v.str = string(); break;
      case SI_HIP_GGUF_ARRAY: {
        v.array_type = scalar<uint32_t>();
        const uint64_t count = scalar<uint64_t>();
        if (count > 0 && v.array_type > SI_HIP_GGUF_F64)
          raise("unsupported GGUF metadata type " + std::to_string(v.array_type));
        // every item takes at least one byte: a count beyond the file is truncation
        if (count > len - offset) raise("GGUF header is truncated");
        v.items.reserve((size_t)count);
        for (uint64_t i = 0; i < count; ++i) v.items.push_back(value(v.array_type, depth + 1));
        break;
      }
      case SI_HIP_GGUF_U64: v.u64 = scalar<uint64_t>(); break;
      case SI_HIP_GGUF_I64: v.i64 = scalar<int64_t>(); break;
      case SI_HIP_GGUF_F64: v.f64 = scalar<double>(); break;
      default: raise("unsupported GGUF metadata type " + std::to_string(type));
    }
    return v;
  }
};

bool checked_mul(uint64_t a, uint64_t b, uint64_t *out) {
  return !__builtin_mul_overflow(a, b, out);
}

}  // namespace

struct si_hip_gguf {
  std::string path;
  void *map = nullptr;  // read-only mapping of the file, or null
  size_t map_len = 0;
  std::vector<uint8_t> owned;  // si_hip_gguf_parse's copy
  const uint8_t *bytes = nullptr;
  uint64_t len = 0;
  uint32_t version = 0;
  uint64_t alignment = 32;
  uint64_t data_base = 0;
  std::map<std::string, Value> metadata;  // byte order, like the reference's BTreeMap
  std::vector<Tensor> tensors;             // index order
  std::map<std::string, uint64_t> by_name;

  ~si_hip_gguf() {
    if (map) munmap(map, map_len);
  }
};

namespace {

// parse_gguf (model.rs:1034-1134) over store->bytes.
void parse(si_hip_gguf *g) {
  Reader r{g->bytes, g->len};
  if (std::memcmp(r.take(4), "GGUF", 4) != 0) raise("GGUF header has invalid magic");
  g->version = r.scalar<uint32_t>();
  if (g->version != 2 && g->version != 3)
    raise("unsupported GGUF version " + std::to_string(g->version));
  const uint64_t tensor_count = r.scalar<uint64_t>();
  const uint64_t metadata_count = r.scalar<uint64_t>();
  for (uint64_t i = 0; i < metadata_count; ++i) {
    std::string key = r.string();
    const uint32_t type = r.scalar<uint32_t>();
    Value v = r.value(type);
    if (!g->metadata.emplace(std::move(key), std::move(v)).second)
      raise("GGUF metadata contains duplicate keys");
  }
  // each tensor record takes at least 24 bytes
  if (tensor_count > (g->len - r.offset) / 24u + 1u) raise("GGUF header is truncated");
  g->tensors.reserve((size_t)tensor_count);
  for (uint64_t i = 0; i < tensor_count; ++i) {
    Tensor t;
    t.name = r.string();
    const uint32_t dims = r.scalar<uint32_t>();
    if (dims > (g->len - r.offset) / 8u) raise("GGUF header is truncated");
    t.shape.reserve(dims);
    for (uint32_t d = 0; d < dims; ++d) t.shape.push_back(r.scalar<uint64_t>());
    t.ggml_type = r.scalar<uint32_t>();
    t.offset = r.scalar<uint64_t>();
    g->tensors.push_back(std::move(t));
  }
  auto al = g->metadata.find("general.alignment");
  g->alignment = 32;
  if (al != g->metadata.end() &&
      (al->second.type == SI_HIP_GGUF_U32 || al->second.type == SI_HIP_GGUF_U64))
    g->alignment = al->second.u64;
  if (g->alignment == 0 || (g->alignment & (g->alignment - 1)) != 0)
    raise("GGUF alignment must be a non-zero power of two");
  const uint64_t rem = r.offset % g->alignment;
  if (rem != 0 && r.offset > UINT64_MAX - (g->alignment - rem))
    raise("packed cache alignment overflows", SI_HIP_ERR_OVERFLOW);
  g->data_base = rem == 0 ? r.offset : r.offset + (g->alignment - rem);

  // tensor ranges: each runs to the next tensor's start in offset order
  // (a stable sort keeps index order between equal offsets)
  std::vector<size_t> order(g->tensors.size());
  for (size_t i = 0; i < order.size(); ++i) order[i] = i;
  std::stable_sort(order.begin(), order.end(), [&](size_t a, size_t b) {
    return g->tensors[a].offset < g->tensors[b].offset;
  });
  for (size_t pos = 0; pos < order.size(); ++pos) {
    Tensor &t = g->tensors[order[pos]];
    if (t.offset > UINT64_MAX - g->data_base)
      raise("GGUF tensor " + t.name + " start overflows", SI_HIP_ERR_OVERFLOW);
    const uint64_t start = g->data_base + t.offset;
    uint64_t end = g->len;
    if (pos + 1 < order.size()) {
      const uint64_t next = g->tensors[order[pos + 1]].offset;
      if (next > UINT64_MAX - g->data_base)
        raise("GGUF tensor " + t.name + " end overflows", SI_HIP_ERR_OVERFLOW);
      end = g->data_base + next;
    }
    if (start > end || end > g->len) raise("GGUF tensor " + t.name + " exceeds file size");
    t.data_start = start;
    t.data_end = end;
  }
  // a name that repeats refers to its last tensor, as the reference's
  // name-keyed map ends up (GgufModelStore::open, model.rs:653-657)
  for (size_t i = 0; i < g->tensors.size(); ++i) g->by_name[g->tensors[i].name] = i;
}

int finish_open(std::unique_ptr<si_hip_gguf> g, si_hip_gguf **out) {
  try {
    parse(g.get());
  } catch (const ParseError &e) {
    return set_error(e.status, "%s", e.message.c_str());
  } catch (const std::bad_alloc &) {
    return set_error(SI_HIP_ERR_OUT_OF_MEMORY, "GGUF index does not fit in host memory");
  }
  *out = g.release();
  return clear_error();
}

void fill(const Value &v, si_hip_gguf_value *out) {
  out->type = v.type;
  out->array_type = v.array_type;
  out->count = v.type == SI_HIP_GGUF_STRING ? v.str.size()
               : v.type == SI_HIP_GGUF_ARRAY ? v.items.size()
                                             : 0u;
  out->u64 = v.u64;
  out->i64 = v.i64;
  out->f64 = v.f64;
  out->str = v.type == SI_HIP_GGUF_STRING ? v.str.c_str() : nullptr;
  out->node = &v;
}

const Tensor *tensor_at(const si_hip_gguf *g, uint64_t index) {
  if (!g) {
    set_error(SI_HIP_ERR_NULL, "GGUF store is null");
    return nullptr;
  }
  if (index >= g->tensors.size()) {
    set_error(SI_HIP_ERR_RANGE, "GGUF tensor index %llu out of range (%zu tensors)",
              (unsigned long long)index, g->tensors.size());
    return nullptr;
  }
  return &g->tensors[(size_t)index];
}

int elements_of(const Tensor &t, uint64_t *out) {
  uint64_t n = 1;
  for (uint64_t d : t.shape)
    if (!checked_mul(n, d, &n))
      return set_error(SI_HIP_ERR_OVERFLOW, "GGUF tensor %s element count overflows",
                       t.name.c_str());
  *out = n;
  return SI_HIP_OK;
}

// GgufTensorInfo::expected_payload_bytes (model.rs:532-573).
int payload_of(const Tensor &t, uint64_t *bytes, int *known) {
  *bytes = 0;
  *known = 0;
  uint64_t n;
  int rc = elements_of(t, &n);
  if (rc) return rc;
  uint64_t per = 0, block = 1;
  const char *label = nullptr;
  switch (t.ggml_type) {
    case 0: per = 4; break;             // F32
    case 1: case 30: per = 2; break;    // F16, BF16
    case SI_HIP_GGML_TYPE_Q4_K: per = kQ4Bytes; block = 256; label = "Q4_K"; break;
    case SI_HIP_GGML_TYPE_Q5_K: per = kQ5Bytes; block = 256; label = "Q5_K"; break;
    case SI_HIP_GGML_TYPE_Q6_K: per = kQ6Bytes; block = 256; label = "Q6_K"; break;
    default: return SI_HIP_OK;
  }
  if (label && n % 256u != 0)
    return set_error(SI_HIP_ERR_DIMENSIONS,
                     "GGUF %s tensor %s has %llu elements; expected a multiple of 256", label,
                     t.name.c_str(), (unsigned long long)n);
  if (!checked_mul(n / block, per, bytes)) {
    // the reference's checked_mul yields None: the size is unknown
    *bytes = 0;
    return SI_HIP_OK;
  }
  *known = 1;
  return SI_HIP_OK;
}

int weight_of(si_hip_context *ctx, const si_hip_gguf *g, uint64_t index, bool mapped,
              si_hip_quant_weight **out) {
  if (!out) return set_error(SI_HIP_ERR_NULL, "output handle pointer is null");
  *out = nullptr;
  const Tensor *t = tensor_at(g, index);
  if (!t) return g ? SI_HIP_ERR_RANGE : SI_HIP_ERR_NULL;
  if (t->ggml_type != SI_HIP_GGML_TYPE_Q4_K && t->ggml_type != SI_HIP_GGML_TYPE_Q5_K &&
      t->ggml_type != SI_HIP_GGML_TYPE_Q6_K)
    return set_error(SI_HIP_ERR_UNSUPPORTED_TYPE, "GGUF tensor %s has type %u; expected 12, 13 or 14",
                     t->name.c_str(), t->ggml_type);
  uint64_t expected;
  int known;
  int rc = payload_of(*t, &expected, &known);
  if (rc) return rc;
  if (!known)
    return set_error(SI_HIP_ERR_OVERFLOW, "GGUF tensor %s has unknown payload size", t->name.c_str());
  const uint64_t have = t->data_end - t->data_start;
  if (have < expected)
    return set_error(SI_HIP_ERR_BYTE_LENGTH, "GGUF tensor %s has %llu bytes; expected at least %llu",
                     t->name.c_str(), (unsigned long long)have, (unsigned long long)expected);
  const uint8_t *p = g->bytes + t->data_start;
  return mapped ? si_hip_bind_quant_weight_mapped(ctx, p, (size_t)expected, t->ggml_type, out)
                : si_hip_upload_quant_weight_private(ctx, p, (size_t)expected, t->ggml_type, out);
}

}  // namespace

extern "C" {

int si_hip_gguf_open(const char *path, si_hip_gguf **out) {
  if (!out) return set_error(SI_HIP_ERR_NULL, "output store pointer is null");
  *out = nullptr;
  if (!path) return set_error(SI_HIP_ERR_NULL, "GGUF path is null");
  auto g = std::make_unique<si_hip_gguf>();
  g->path = path;
  const int fd = open(path, O_RDONLY | O_CLOEXEC);
  // I/O errors read as Rust's io::Error prints them: "<strerror> (os error N)"
  if (fd < 0) {
    const int e = errno;
    return set_error(SI_HIP_ERR_RANGE, "open GGUF model %s: %s (os error %d)", path, strerror(e), e);
  }
  struct stat st;
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    close(fd);
    return set_error(SI_HIP_ERR_RANGE, "%s (os error %d)", strerror(e), e);
  }
  g->len = (uint64_t)st.st_size;
  if (g->len > 0) {
    void *m = mmap(nullptr, (size_t)g->len, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) {
      const int e = errno;
      close(fd);
      return set_error(SI_HIP_ERR_OUT_OF_MEMORY, "%s (os error %d)", strerror(e), e);
    }
    g->map = m;
    g->map_len = (size_t)g->len;
    g->bytes = static_cast<const uint8_t *>(m);
  }
  close(fd);  // the mapping keeps the file
  return finish_open(std::move(g), out);
}

int si_hip_gguf_parse(const uint8_t *bytes, size_t len, si_hip_gguf **out) {
  if (!out) return set_error(SI_HIP_ERR_NULL, "output store pointer is null");
  *out = nullptr;
  if (!bytes && len) return set_error(SI_HIP_ERR_NULL, "GGUF bytes are null");
  auto g = std::make_unique<si_hip_gguf>();
  g->owned.assign(bytes, bytes + len);
  g->bytes = g->owned.data();
  g->len = len;
  return finish_open(std::move(g), out);
}

void si_hip_gguf_close(si_hip_gguf *g) { delete g; }

uint32_t si_hip_gguf_version(const si_hip_gguf *g) { return g ? g->version : 0; }
uint64_t si_hip_gguf_alignment(const si_hip_gguf *g) { return g ? g->alignment : 0; }
uint64_t si_hip_gguf_data_base(const si_hip_gguf *g) { return g ? g->data_base : 0; }
uint64_t si_hip_gguf_file_bytes(const si_hip_gguf *g) { return g ? g->len : 0; }
uint64_t si_hip_gguf_tensor_count(const si_hip_gguf *g) { return g ? g->tensors.size() : 0; }

int si_hip_gguf_tensor_info(const si_hip_gguf *g, uint64_t index, si_hip_gguf_tensor *out) {
  if (!out) return set_error(SI_HIP_ERR_NULL, "output tensor pointer is null");
  const Tensor *t = tensor_at(g, index);
  if (!t) return g ? SI_HIP_ERR_RANGE : SI_HIP_ERR_NULL;
  out->name = t->name.c_str();
  out->n_dims = (uint32_t)t->shape.size();
  out->ggml_type = t->ggml_type;
  out->shape = t->shape.data();
  out->offset = t->offset;
  out->data_start = t->data_start;
  out->data_end = t->data_end;
  return clear_error();
}

int si_hip_gguf_find_tensor(const si_hip_gguf *g, const char *name, uint64_t *out) {
  if (!g || !name || !out) return set_error(SI_HIP_ERR_NULL, "find_tensor argument is null");
  auto it = g->by_name.find(name);
  if (it == g->by_name.end()) return set_error(SI_HIP_ERR_RANGE, "unknown GGUF tensor %s", name);
  *out = it->second;
  return clear_error();
}

int si_hip_gguf_tensor_data(const si_hip_gguf *g, uint64_t index, const uint8_t **data,
                            uint64_t *len) {
  if (!data || !len) return set_error(SI_HIP_ERR_NULL, "tensor_data argument is null");
  const Tensor *t = tensor_at(g, index);
  if (!t) return g ? SI_HIP_ERR_RANGE : SI_HIP_ERR_NULL;
  *data = g->bytes + t->data_start;
  *len = t->data_end - t->data_start;
  return clear_error();
}

int si_hip_gguf_tensor_elements(const si_hip_gguf *g, uint64_t index, uint64_t *out) {
  if (!out) return set_error(SI_HIP_ERR_NULL, "tensor_elements argument is null");
  const Tensor *t = tensor_at(g, index);
  if (!t) return g ? SI_HIP_ERR_RANGE : SI_HIP_ERR_NULL;
  int rc = elements_of(*t, out);
  return rc ? rc : clear_error();
}

int si_hip_gguf_expected_payload_bytes(const si_hip_gguf *g, uint64_t index, uint64_t *bytes,
                                       int *known) {
  if (!bytes || !known) return set_error(SI_HIP_ERR_NULL, "payload argument is null");
  const Tensor *t = tensor_at(g, index);
  if (!t) return g ? SI_HIP_ERR_RANGE : SI_HIP_ERR_NULL;
  int rc = payload_of(*t, bytes, known);
  return rc ? rc : clear_error();
}

uint64_t si_hip_gguf_metadata_count(const si_hip_gguf *g) { return g ? g->metadata.size() : 0; }

int si_hip_gguf_metadata_key(const si_hip_gguf *g, uint64_t index, const char **key) {
  if (!g || !key) return set_error(SI_HIP_ERR_NULL, "metadata_key argument is null");
  if (index >= g->metadata.size())
    return set_error(SI_HIP_ERR_RANGE, "GGUF metadata index %llu out of range",
                     (unsigned long long)index);
  auto it = g->metadata.begin();
  std::advance(it, (long)index);
  *key = it->first.c_str();
  return clear_error();
}

int si_hip_gguf_metadata_get(const si_hip_gguf *g, const char *key, si_hip_gguf_value *out) {
  if (!g || !key || !out) return set_error(SI_HIP_ERR_NULL, "metadata_get argument is null");
  auto it = g->metadata.find(key);
  if (it == g->metadata.end()) return set_error(SI_HIP_ERR_RANGE, "GGUF metadata is missing %s", key);
  fill(it->second, out);
  return clear_error();
}

int si_hip_gguf_value_item(const si_hip_gguf_value *array, uint64_t index, si_hip_gguf_value *out) {
  if (!array || !out || !array->node) return set_error(SI_HIP_ERR_NULL, "value_item argument is null");
  const Value &v = *static_cast<const Value *>(array->node);
  if (v.type != SI_HIP_GGUF_ARRAY) return set_error(SI_HIP_ERR_RANGE, "GGUF value is not an array");
  if (index >= v.items.size())
    return set_error(SI_HIP_ERR_RANGE, "GGUF array index %llu out of range (%zu items)",
                     (unsigned long long)index, v.items.size());
  fill(v.items[(size_t)index], out);
  return clear_error();
}

int si_hip_gguf_upload_tensor(si_hip_context *ctx, const si_hip_gguf *g, uint64_t index,
                              si_hip_quant_weight **out) {
  return weight_of(ctx, g, index, false, out);
}

int si_hip_gguf_bind_tensor_mapped(si_hip_context *ctx, const si_hip_gguf *g, uint64_t index,
                                   si_hip_quant_weight **out) {
  return weight_of(ctx, g, index, true, out);
}

// F32 matvec over rows [row_start, row_start + row_count) of a rank-2 F32
// tensor (f32_matvec_tensor_rows, metal.rs:3074-3110).
int si_hip_gguf_f32_matvec_tensor_rows(si_hip_context *ctx, const si_hip_gguf *g, uint64_t index,
                                       size_t row_start, size_t row_count, const float *x,
                                       size_t x_len, float *y) {
  const Tensor *t = tensor_at(g, index);
  if (!t) return g ? SI_HIP_ERR_RANGE : SI_HIP_ERR_NULL;
  if (t->ggml_type != 0 || t->shape.size() != 2)
    return set_error(SI_HIP_ERR_UNSUPPORTED_TYPE, "F32 matvec requires a rank-2 F32 tensor");
  const uint64_t cols = t->shape[0], rows = t->shape[1];
  if (row_count == 0 || row_start >= rows || row_count > rows - row_start)
    return set_error(SI_HIP_ERR_RANGE, "F32 row range is invalid");
  if (x_len != cols) return set_error(SI_HIP_ERR_DIMENSIONS, "F32 tensor columns or input length is invalid");
  uint64_t row_bytes, start, len, end;
  if (!checked_mul(cols, (uint64_t)sizeof(float), &row_bytes) || !checked_mul(row_count, row_bytes, &len))
    return set_error(SI_HIP_ERR_OVERFLOW, "F32 row byte length overflows");
  if (!checked_mul(row_start, row_bytes, &start) || start > UINT64_MAX - len)
    return set_error(SI_HIP_ERR_OVERFLOW, "F32 row byte range overflows");
  end = start + len;
  if (end > t->data_end - t->data_start)
    return set_error(SI_HIP_ERR_BYTE_LENGTH, "F32 tensor payload is shorter than its shape");
  return si_hip_f32_matvec_bytes(ctx, g->bytes + t->data_start + start, (size_t)len, row_count,
                                 (size_t)cols, x, x_len, y);
}

// One submission of F32 matvecs over several rank-2 F32 tensors with the same
// columns and one input (f32_matvec_many_gguf_tensors, metal.rs:4780-4870).
int si_hip_gguf_f32_matvec_many_tensors(si_hip_context *ctx, const si_hip_gguf *g,
                                        const uint64_t *indices, size_t count, const float *x,
                                        size_t x_len, float *const *outputs) {
  if (!g) return set_error(SI_HIP_ERR_NULL, "GGUF store is null");
  if (count == 0) return set_error(SI_HIP_ERR_EMPTY, "GGUF F32 matvec group requires at least one tensor");
  if (!indices || !outputs) return set_error(SI_HIP_ERR_NULL, "GGUF F32 matvec group argument is null");
  const Tensor *first = tensor_at(g, indices[0]);
  if (!first) return SI_HIP_ERR_RANGE;
  if (first->shape.empty()) return set_error(SI_HIP_ERR_DIMENSIONS, "GGUF F32 matvec tensor is not a matrix");
  const uint64_t cols = first->shape[0];
  if (x_len != cols) return set_error(SI_HIP_ERR_DIMENSIONS, "GGUF F32 matvec group input length is invalid");
  std::vector<const float *> ws(count);
  std::vector<size_t> rows(count);
  for (size_t i = 0; i < count; ++i) {
    const Tensor *t = tensor_at(g, indices[i]);
    if (!t) return SI_HIP_ERR_RANGE;
    if (t->ggml_type != 0 || t->shape.size() != 2 || t->shape[0] != cols)
      return set_error(SI_HIP_ERR_DIMENSIONS, "GGUF F32 matvec group shapes or types differ");
    uint64_t expected;
    if (!checked_mul(t->shape[1], cols, &expected) || !checked_mul(expected, (uint64_t)sizeof(float), &expected))
      return set_error(SI_HIP_ERR_OVERFLOW, "GGUF F32 matvec group byte length overflows");
    if (t->data_end - t->data_start != expected)
      return set_error(SI_HIP_ERR_BYTE_LENGTH, "GGUF F32 matvec group tensor is truncated");
    const uint8_t *p = g->bytes + t->data_start;
    if (reinterpret_cast<uintptr_t>(p) % alignof(float) != 0)
      return set_error(SI_HIP_ERR_BYTE_LENGTH, "F32 matvec bytes are not 4-byte aligned");
    ws[i] = reinterpret_cast<const float *>(p);
    rows[i] = (size_t)t->shape[1];
  }
  return si_hip_f32_matvec_many(ctx, ws.data(), rows.data(), count, (size_t)cols, x, x_len, outputs);
}

// Rows [row_start, row_start + row_count) of a rank-2 tensor of the store:
// F32 through the F32 matvec, Q4_K / Q5_K / Q6_K through the quantized one
// over the mapped bytes, the whole tensor borrowed so that its row ranges
// share one resident HBM copy (gguf_matvec_tensor_rows, metal.rs:5003-5015, with
// q4_k_matvec_tensor_rows / quant_k_matvec_tensor_rows, 4346-4467, and
// gguf_quant_matvec_tensor_rows, 4505-4527: their checks and messages).
int si_hip_gguf_matvec_tensor_rows(si_hip_context *ctx, const si_hip_gguf *g, uint64_t index,
                                   size_t row_start, size_t row_count, const float *x,
                                   size_t x_len, float *y) {
  const Tensor *t = tensor_at(g, index);
  if (!t) return g ? SI_HIP_ERR_RANGE : SI_HIP_ERR_NULL;
  if (t->ggml_type == 0)
    return si_hip_gguf_f32_matvec_tensor_rows(ctx, g, index, row_start, row_count, x, x_len, y);
  return si_hip_gguf_quant_matvec_view_rows(ctx, t->name.c_str(), t->ggml_type, t->shape.data(),
                                            (uint32_t)t->shape.size(), g->bytes + t->data_start,
                                            (size_t)(t->data_end - t->data_start), row_start,
                                            row_count, x, x_len, y);
}

// Several quantized matvecs over one input (gguf_quant_matvec_many_tensors,
// metal.rs:4532-4646): the reference's checks and messages, then the staged
// group path with each tensor's first rows x cols / 256 blocks.
int si_hip_gguf_quant_matvec_many_tensors(si_hip_context *ctx, const si_hip_gguf *g,
                                          const uint64_t *indices, size_t count, const float *x,
                                          size_t x_len, float *const *outputs) {
  if (!g) return set_error(SI_HIP_ERR_NULL, "GGUF store is null");
  if (count == 0) return set_error(SI_HIP_ERR_EMPTY, "quantized matvec group requires at least one tensor");
  if (!indices || !outputs) return set_error(SI_HIP_ERR_NULL, "quantized matvec group argument is null");
  const Tensor *first = tensor_at(g, indices[0]);
  if (!first) return SI_HIP_ERR_RANGE;
  if (first->shape.empty()) return set_error(SI_HIP_ERR_DIMENSIONS, "quantized matvec tensor is not a matrix");
  const uint64_t cols = first->shape[0];
  if (x_len != cols) return set_error(SI_HIP_ERR_DIMENSIONS, "quantized matvec group input length is invalid");
  std::vector<uint32_t> types(count);
  std::vector<const uint8_t *> bytes(count);
  std::vector<size_t> lens(count), rows(count), columns(count);
  for (size_t i = 0; i < count; ++i) {
    const Tensor *t = tensor_at(g, indices[i]);
    if (!t) return SI_HIP_ERR_RANGE;
    const uint32_t ty = t->ggml_type;
    if (t->shape.size() != 2 || t->shape[0] != cols || (ty != 12 && ty != 13 && ty != 14))
      return set_error(SI_HIP_ERR_DIMENSIONS, "quantized matvec group tensor shapes or types differ");
    const uint64_t bb = ty == 12 ? 144u : ty == 13 ? 176u : 210u;
    uint64_t expected;
    if (!checked_mul(t->shape[1], cols / 256, &expected) || !checked_mul(expected, bb, &expected))
      return set_error(SI_HIP_ERR_OVERFLOW, "quantized matvec group byte length overflows");
    if (t->data_end - t->data_start < expected)
      return set_error(SI_HIP_ERR_BYTE_LENGTH, "quantized matvec group tensor is truncated");
    types[i] = ty;
    bytes[i] = g->bytes + t->data_start;
    lens[i] = (size_t)expected;
    rows[i] = (size_t)t->shape[1];
    columns[i] = (size_t)cols;
  }
  return si_hip_gguf_quant_matvec_many_bytes(ctx, types.data(), bytes.data(), lens.data(),
                                             rows.data(), columns.data(), count, x, x_len, outputs);
}

}  // extern "C"
