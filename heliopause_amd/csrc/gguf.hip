// gguf.hip -- GGUF v3 header / metadata / tensor-table reader (host code).
//
// Restates parseGguf (packages/engine/src/gguf.ts:150-215) with its value
// reader and skipper (gguf.ts:265-365), and tensorByteLength / ggmlTypeStorage
// (packages/engine/src/tensor-reader.ts:268-293).  The header is parsed through
// a 1 MiB read buffer; tensor bytes are fetched later with pread, which is
// safe from several threads at once (the HBM loader streams with a pool of
// readers).  No GPU code here.

#include "../../include/hp_gguf.h"

#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cinttypes>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace {

constexpr uint64_t kMaxSafe = 9007199254740991ull;  // Number.MAX_SAFE_INTEGER
constexpr uint64_t kDefaultAlignment = 32;           // gguf.ts:94
constexpr size_t kParseBuffer = 1u << 20;

thread_local std::string g_error;

struct Fail {
  int32_t code;
  std::string msg;
};

struct Node {
  int32_t type = 0;
  double number = 0;
  std::string str;
  int32_t element_type = 0;
  uint64_t length = 0;
  bool truncated = false;
  std::vector<uint64_t> children;
};

struct Tensor {
  std::string name;
  std::vector<uint64_t> dims;
  uint32_t type_id = 0;
  uint64_t offset = 0, data_offset = 0, byte_length = 0;
  bool storage_known = false;
};

struct Storage {
  uint32_t type_id;
  uint32_t block, bytes;
};

// ggmlTypeStorage (tensor-reader.ts:282-293) keyed by ggml type id.
constexpr Storage kStorage[] = {
    {0, 1, 4},      // F32
    {1, 1, 2},      // F16
    {30, 1, 2},     // BF16
    {2, 32, 18},    // Q4_0
    {8, 32, 34},    // Q8_0
    {12, 256, 144}, // Q4_K
    {13, 256, 176}, // Q5_K
    {14, 256, 210}, // Q6_K
    {23, 256, 136}, // IQ4_XS
    {26, 1, 4},     // I32
};

}  // namespace

struct hp_gguf {
  int fd = -1;
  const uint8_t *mem = nullptr;
  uint64_t size = 0;
  uint32_t version = 0;
  uint64_t tensor_count = 0, metadata_count = 0, data_start = 0, alignment = kDefaultAlignment;
  std::vector<Node> nodes;
  std::vector<std::string> keys;
  std::vector<uint64_t> key_node;
  std::unordered_map<std::string, size_t> key_index;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> tensor_index;

  ~hp_gguf() {
    if (fd >= 0) ::close(fd);
  }

  // Bytes available at [off, off + n); false past the end.
  bool read_at(uint64_t off, void *dst, uint64_t n) const {
    if (off > size || n > size - off) return false;
    if (mem) {
      std::memcpy(dst, mem + off, n);
      return true;
    }
    auto *p = static_cast<uint8_t *>(dst);
    while (n > 0) {
      const size_t want = n > (1ull << 30) ? (size_t)(1ull << 30) : (size_t)n;
      const ssize_t got = ::pread(fd, p, want, (off_t)off);
      if (got < 0 && errno == EINTR) continue;
      if (got <= 0) return false;
      p += got;
      off += (uint64_t)got;
      n -= (uint64_t)got;
    }
    return true;
  }
};

namespace {

// GgufCursor (gguf.ts:380-462) over a buffered window of the source.
class Cursor {
 public:
  explicit Cursor(const hp_gguf &g) : g_(g) {}
  uint64_t offset = 0;

  void bytes(void *dst, uint64_t n) {
    if (offset > g_.size || n > g_.size - offset) throw Fail{HP_ERR_FORMAT, "Unexpected EOF at offset " + std::to_string(offset)};
    if (g_.mem) {
      std::memcpy(dst, g_.mem + offset, n);
    } else {
      auto *p = static_cast<uint8_t *>(dst);
      uint64_t off = offset, left = n;
      while (left > 0) {
        if (off < buf_off_ || off >= buf_off_ + buf_.size()) fill(off);
        const uint64_t in = buf_off_ + buf_.size() - off;
        const uint64_t take = in < left ? in : left;
        std::memcpy(p, buf_.data() + (off - buf_off_), take);
        p += take;
        off += take;
        left -= take;
      }
    }
    offset += n;
  }
  template <typename T>
  T scalar() {
    T v;
    bytes(&v, sizeof(T));  // GGUF is little-endian, as is the host
    return v;
  }
  uint64_t safe_u64(const std::string &label) {
    const uint64_t v = scalar<uint64_t>();
    if (v > kMaxSafe) throw Fail{HP_ERR_FORMAT, label + " exceeds JavaScript safe integer range: " + std::to_string(v)};
    return v;
  }
  std::string string() {
    const uint64_t n = safe_u64("string length");
    if (offset > g_.size || n > g_.size - offset) throw Fail{HP_ERR_FORMAT, "Unexpected EOF at offset " + std::to_string(offset)};
    std::string s((size_t)n, '\0');
    bytes(&s[0], n);
    return s;
  }
  void skip(uint64_t n) { offset += n; }  // no bounds check, as GgufCursor.skipBytes

 private:
  void fill(uint64_t off) {
    const uint64_t n = g_.size - off < kParseBuffer ? g_.size - off : kParseBuffer;
    buf_.resize((size_t)n);
    if (!g_.read_at(off, buf_.data(), n)) throw Fail{HP_ERR_IO, "read failed at offset " + std::to_string(off)};
    buf_off_ = off;
  }
  const hp_gguf &g_;
  std::vector<uint8_t> buf_;
  uint64_t buf_off_ = 0;
};

class Parser {
 public:
  Parser(hp_gguf &g, Cursor &c) : g_(g), c_(c) {}

  // readMetadataValue (gguf.ts:265-300); returns a node id.
  uint64_t value(uint32_t type, uint64_t max_sample) {
    if (type == HP_GGUF_ARRAY && depth_ >= kMaxDepth) throw Fail{HP_ERR_FORMAT, "GGUF arrays nested too deeply"};
    Node n;
    n.type = (int32_t)type;
    switch (type) {
      case HP_GGUF_UINT8: n.number = c_.scalar<uint8_t>(); break;
      case HP_GGUF_INT8: n.number = c_.scalar<int8_t>(); break;
      case HP_GGUF_UINT16: n.number = c_.scalar<uint16_t>(); break;
      case HP_GGUF_INT16: n.number = c_.scalar<int16_t>(); break;
      case HP_GGUF_UINT32: n.number = c_.scalar<uint32_t>(); break;
      case HP_GGUF_INT32: n.number = c_.scalar<int32_t>(); break;
      case HP_GGUF_FLOAT32: n.number = c_.scalar<float>(); break;
      case HP_GGUF_BOOL: n.number = c_.scalar<uint8_t>() != 0 ? 1.0 : 0.0; break;
      case HP_GGUF_STRING: n.str = c_.string(); break;
      case HP_GGUF_ARRAY: {
        depth_++;
        const uint64_t id = array(max_sample);
        depth_--;
        return id;
      }
      case HP_GGUF_UINT64: n.number = (double)c_.safe_u64("uint64 metadata value"); break;
      case HP_GGUF_INT64: {
        const int64_t v = c_.scalar<int64_t>();
        if (v > (int64_t)kMaxSafe || v < -(int64_t)kMaxSafe)
          throw Fail{HP_ERR_FORMAT, "int64 metadata value exceeds JavaScript safe integer range: " + std::to_string(v)};
        n.number = (double)v;
        break;
      }
      case HP_GGUF_FLOAT64: n.number = c_.scalar<double>(); break;
      default: throw Fail{HP_ERR_FORMAT, "Unsupported GGUF metadata type id: " + std::to_string(type)};
    }
    g_.nodes.push_back(std::move(n));
    return g_.nodes.size() - 1;
  }

  // readArraySummary (gguf.ts:302-326).
  uint64_t array(uint64_t max_sample) {
    const uint32_t elem = c_.scalar<uint32_t>();
    const uint64_t length = c_.safe_u64("array length");
    const uint64_t keep = length < max_sample ? length : max_sample;
    std::vector<uint64_t> children;
    children.reserve((size_t)(keep < (1u << 20) ? keep : (1u << 20)));
    for (uint64_t i = 0; i < keep; i++) children.push_back(value(elem, max_sample));
    skip_n(elem, length - keep);
    Node n;
    n.type = HP_GGUF_ARRAY;
    n.element_type = (int32_t)elem;
    n.length = length;
    n.truncated = length > keep;
    n.children = std::move(children);
    g_.nodes.push_back(std::move(n));
    return g_.nodes.size() - 1;
  }

  // skipMetadataValue (gguf.ts:328-365).
  void skip(uint32_t type) {
    switch (type) {
      case HP_GGUF_UINT8: case HP_GGUF_INT8: case HP_GGUF_BOOL: c_.skip(1); return;
      case HP_GGUF_UINT16: case HP_GGUF_INT16: c_.skip(2); return;
      case HP_GGUF_UINT32: case HP_GGUF_INT32: case HP_GGUF_FLOAT32: c_.skip(4); return;
      case HP_GGUF_STRING: c_.skip(c_.safe_u64("string length")); return;
      case HP_GGUF_ARRAY: {
        if (depth_ >= kMaxDepth) throw Fail{HP_ERR_FORMAT, "GGUF arrays nested too deeply"};
        const uint32_t elem = c_.scalar<uint32_t>();
        const uint64_t length = c_.safe_u64("array length");
        depth_++;
        skip_n(elem, length);
        depth_--;
        return;
      }
      case HP_GGUF_UINT64: case HP_GGUF_INT64: case HP_GGUF_FLOAT64: c_.skip(8); return;
      default: throw Fail{HP_ERR_FORMAT, "Unsupported GGUF metadata type id: " + std::to_string(type)};
    }
  }

 private:
  // `count` skipMetadataValue calls.  Fixed-size elements move the cursor
  // by count * size at once: those skips read nothing, so no error can
  // occur between them and the result is the same.  Strings and arrays read
  // a length each, so their loop ends at the end of the file at the latest.
  void skip_n(uint32_t type, uint64_t count) {
    const uint64_t size = fixed_size(type);
    if (size != 0) {
      c_.skip(count * size);  // count <= 2^53 - 1, size <= 8: no overflow
      return;
    }
    for (uint64_t i = 0; i < count; i++) skip(type);
  }

  static uint64_t fixed_size(uint32_t type) {
    switch (type) {
      case HP_GGUF_UINT8: case HP_GGUF_INT8: case HP_GGUF_BOOL: return 1;
      case HP_GGUF_UINT16: case HP_GGUF_INT16: return 2;
      case HP_GGUF_UINT32: case HP_GGUF_INT32: case HP_GGUF_FLOAT32: return 4;
      case HP_GGUF_UINT64: case HP_GGUF_INT64: case HP_GGUF_FLOAT64: return 8;
      default: return 0;
    }
  }

  // Nesting bound (the TS parser is bounded by the JS stack instead); real
  // files nest at most one level.
  static constexpr int kMaxDepth = 64;
  hp_gguf &g_;
  Cursor &c_;
  int depth_ = 0;
};

bool is_number_type(int32_t t) {
  return t == HP_GGUF_UINT8 || t == HP_GGUF_INT8 || t == HP_GGUF_UINT16 || t == HP_GGUF_INT16 || t == HP_GGUF_UINT32 ||
         t == HP_GGUF_INT32 || t == HP_GGUF_FLOAT32 || t == HP_GGUF_UINT64 || t == HP_GGUF_INT64 || t == HP_GGUF_FLOAT64;
}

// tensorByteLength (tensor-reader.ts:268-280): elements / block * typeSize.
void size_tensor(Tensor &t) {
  t.storage_known = false;
  t.byte_length = 0;
  for (const Storage &s : kStorage) {
    if (s.type_id != t.type_id) continue;
    uint64_t elements = 1;
    for (uint64_t d : t.dims)
      if (__builtin_mul_overflow(elements, d, &elements)) return;
    if (elements % s.block != 0) return;
    uint64_t bytes;
    if (__builtin_mul_overflow(elements / s.block, (uint64_t)s.bytes, &bytes)) return;
    t.byte_length = bytes;
    t.storage_known = true;
    return;
  }
}

// parseGguf (gguf.ts:150-215).
void parse(hp_gguf &g, uint64_t max_sample, const std::unordered_set<std::string> &complete) {
  Cursor c(g);
  Parser p(g, c);
  char magic[4];
  c.bytes(magic, 4);
  if (std::memcmp(magic, "GGUF", 4) != 0) {
    // String.fromCharCode of the bytes (gguf.ts:389), written as UTF-8
    std::string got;
    for (char ch : magic) {
      const unsigned char u = (unsigned char)ch;
      if (u < 0x80) {
        got += (char)u;
      } else {
        got += (char)(0xC0 | (u >> 6));
        got += (char)(0x80 | (u & 0x3F));
      }
    }
    throw Fail{HP_ERR_FORMAT, "Invalid GGUF magic: expected GGUF, got " + got};
  }
  g.version = c.scalar<uint32_t>();
  g.tensor_count = c.safe_u64("tensor count");
  g.metadata_count = c.safe_u64("metadata count");
  for (uint64_t i = 0; i < g.metadata_count; i++) {
    std::string key = c.string();
    const uint32_t type = c.scalar<uint32_t>();
    const uint64_t node = p.value(type, complete.count(key) ? kMaxSafe : max_sample);
    auto it = g.key_index.find(key);
    if (it != g.key_index.end()) {
      g.key_node[it->second] = node;  // JS object: first position, last value
    } else {
      g.key_index.emplace(key, g.keys.size());
      g.keys.push_back(std::move(key));
      g.key_node.push_back(node);
    }
  }
  for (uint64_t i = 0; i < g.tensor_count; i++) {
    Tensor t;
    t.name = c.string();
    const uint32_t nd = c.scalar<uint32_t>();
    for (uint32_t d = 0; d < nd; d++) t.dims.push_back(c.safe_u64("dimension for " + t.name));
    t.type_id = c.scalar<uint32_t>();
    t.offset = c.scalar<uint64_t>();
    g.tensor_index[t.name] = g.tensors.size();  // Map: the last wins
    g.tensors.push_back(std::move(t));
  }
  // getMetadataNumber(metadata, "general.alignment") ?? 32
  auto it = g.key_index.find("general.alignment");
  if (it != g.key_index.end()) {
    const Node &n = g.nodes[g.key_node[it->second]];
    if (is_number_type(n.type)) {
      // BigInt() of a fraction, or a remainder by 0n, throws in the TS parser
      if (!(n.number >= 1 && n.number <= 4294967296.0) || n.number != (double)(uint64_t)n.number)
        throw Fail{HP_ERR_FORMAT, "general.alignment must be a positive integer"};
      g.alignment = (uint64_t)n.number;
    }
  }
  const uint64_t rem = c.offset % g.alignment;
  g.data_start = rem == 0 ? c.offset : c.offset + g.alignment - rem;
  for (Tensor &t : g.tensors) {
    t.data_offset = g.data_start + t.offset;
    size_tensor(t);
  }
}

int32_t open_common(hp_gguf *g, uint64_t max_sample, const char *const *keys, size_t nkeys, hp_gguf_t **out) {
  std::unordered_set<std::string> complete;
  for (size_t i = 0; i < nkeys; i++)
    if (keys && keys[i]) complete.insert(keys[i]);
  try {
    parse(*g, max_sample, complete);
  } catch (const Fail &f) {
    g_error = f.msg;
    delete g;
    return f.code;
  } catch (const std::bad_alloc &) {
    g_error = "out of host memory while parsing GGUF";
    delete g;
    return HP_ERR_FORMAT;
  }
  *out = g;
  g_error.clear();
  return 0;
}

void fill_value(const hp_gguf &g, uint64_t id, hp_gguf_value_t *v) {
  const Node &n = g.nodes[id];
  std::memset(v, 0, sizeof *v);
  v->type = n.type;
  v->number = n.number;
  if (n.type == HP_GGUF_STRING) {
    v->string = n.str.c_str();
    v->string_length = n.str.size();
  }
  if (n.type == HP_GGUF_ARRAY) {
    v->element_type = n.element_type;
    v->length = n.length;
    v->sample_count = n.children.size();
    v->truncated = n.truncated ? 1 : 0;
  }
  v->node = id;
}

int32_t arg_error(const char *msg) {
  g_error = msg;
  return 18;  // HP_ERR_ARG
}

}  // namespace

extern "C" {

int32_t hp_gguf_open(const char *path, uint64_t max_array_sample, const char *const *complete_array_keys,
                     size_t complete_key_count, hp_gguf_t **out) {
  if (!path || !out) return arg_error("null pointer");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    g_error = std::string("cannot open ") + path + ": " + std::strerror(errno);
    return HP_ERR_IO;
  }
  struct stat sb;
  if (::fstat(fd, &sb) != 0) {
    g_error = std::string("cannot stat ") + path + ": " + std::strerror(errno);
    ::close(fd);
    return HP_ERR_IO;
  }
  auto *g = new hp_gguf;
  g->fd = fd;
  g->size = (uint64_t)sb.st_size;
  return open_common(g, max_array_sample, complete_array_keys, complete_key_count, out);
}

int32_t hp_gguf_open_memory(const uint8_t *data, size_t size, uint64_t max_array_sample,
                            const char *const *complete_array_keys, size_t complete_key_count, hp_gguf_t **out) {
  if ((!data && size) || !out) return arg_error("null pointer");
  *out = nullptr;
  static const uint8_t empty = 0;
  auto *g = new hp_gguf;
  g->mem = data ? data : &empty;
  g->size = size;
  return open_common(g, max_array_sample, complete_array_keys, complete_key_count, out);
}

void hp_gguf_close(hp_gguf_t *g) { delete g; }

const char *hp_gguf_last_error(void) { return g_error.c_str(); }

int32_t hp_gguf_header(const hp_gguf_t *g, uint32_t *version, uint64_t *tensor_count, uint64_t *metadata_count,
                       uint64_t *data_start, uint64_t *alignment, uint64_t *file_size) {
  if (!g) return arg_error("null pointer");
  if (version) *version = g->version;
  if (tensor_count) *tensor_count = g->tensor_count;
  if (metadata_count) *metadata_count = g->metadata_count;
  if (data_start) *data_start = g->data_start;
  if (alignment) *alignment = g->alignment;
  if (file_size) *file_size = g->size;
  return 0;
}

uint64_t hp_gguf_metadata_count(const hp_gguf_t *g) { return g ? g->keys.size() : 0; }

int32_t hp_gguf_metadata_entry(const hp_gguf_t *g, uint64_t index, const char **key, uint64_t *key_length,
                               hp_gguf_value_t *value) {
  if (!g || !value) return arg_error("null pointer");
  if (index >= g->keys.size()) return arg_error("metadata index out of range");
  if (key) *key = g->keys[index].c_str();
  if (key_length) *key_length = g->keys[index].size();
  fill_value(*g, g->key_node[index], value);
  return 0;
}

int32_t hp_gguf_metadata_find(const hp_gguf_t *g, const char *key, hp_gguf_value_t *value) {
  if (!g || !key || !value) return arg_error("null pointer");
  auto it = g->key_index.find(key);
  if (it == g->key_index.end()) return arg_error("metadata key not found");
  fill_value(*g, g->key_node[it->second], value);
  return 0;
}

int32_t hp_gguf_array_element(const hp_gguf_t *g, uint64_t node, uint64_t index, hp_gguf_value_t *value) {
  if (!g || !value) return arg_error("null pointer");
  if (node >= g->nodes.size() || g->nodes[node].type != HP_GGUF_ARRAY) return arg_error("not an array value");
  const Node &n = g->nodes[node];
  if (index >= n.children.size()) return arg_error("array element out of range");
  fill_value(*g, n.children[index], value);
  return 0;
}

int32_t hp_gguf_tensor_info(const hp_gguf_t *g, uint64_t index, hp_gguf_tensor_t *out) {
  if (!g || !out) return arg_error("null pointer");
  if (index >= g->tensors.size()) return arg_error("tensor index out of range");
  const Tensor &t = g->tensors[index];
  out->name = t.name.c_str();
  out->name_length = t.name.size();
  out->n_dims = (uint32_t)t.dims.size();
  out->dims = t.dims.data();
  out->type_id = t.type_id;
  out->offset = t.offset;
  out->data_offset = t.data_offset;
  out->byte_length = t.byte_length;
  out->storage_known = t.storage_known ? 1 : 0;
  return 0;
}

int64_t hp_gguf_find_tensor(const hp_gguf_t *g, const char *name) {
  if (!g || !name) return -1;
  auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : (int64_t)it->second;
}

const char *hp_gguf_type_name(uint32_t type_id) {
  // ggmlTypeNames (gguf.ts:112-148)
  switch (type_id) {
    case 0: return "F32";
    case 1: return "F16";
    case 2: return "Q4_0";
    case 3: return "Q4_1";
    case 6: return "Q5_0";
    case 7: return "Q5_1";
    case 8: return "Q8_0";
    case 9: return "Q8_1";
    case 10: return "Q2_K";
    case 11: return "Q3_K";
    case 12: return "Q4_K";
    case 13: return "Q5_K";
    case 14: return "Q6_K";
    case 15: return "Q8_K";
    case 16: return "IQ2_XXS";
    case 17: return "IQ2_XS";
    case 18: return "IQ3_XXS";
    case 19: return "IQ1_S";
    case 20: return "IQ4_NL";
    case 21: return "IQ3_S";
    case 22: return "IQ2_S";
    case 23: return "IQ4_XS";
    case 24: return "I8";
    case 25: return "I16";
    case 26: return "I32";
    case 27: return "I64";
    case 28: return "F64";
    case 29: return "IQ1_M";
    case 30: return "BF16";
    case 34: return "TQ1_0";
    case 35: return "TQ2_0";
    case 39: return "MXFP4";
    case 40: return "NVFP4";
    case 41: return "Q1_0";
    default: break;
  }
  static thread_local char buf[32];
  std::snprintf(buf, sizeof buf, "UNKNOWN_%" PRIu32, type_id);
  return buf;
}

int32_t hp_gguf_read(const hp_gguf_t *g, uint64_t offset, void *dst, uint64_t length) {
  if (!g || (!dst && length)) return arg_error("null pointer");
  if (!g->read_at(offset, dst, length)) {
    g_error = "read of " + std::to_string(length) + " bytes at offset " + std::to_string(offset) + " failed";
    return HP_ERR_IO;
  }
  return 0;
}

}  // extern "C"
