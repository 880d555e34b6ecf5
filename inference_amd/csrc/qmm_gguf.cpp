// GGUF container reader and resident loader (host side of libqmm.so).
//
// Parses the llama.cpp single-file container (spec v2/v3: little-endian
// header, typed metadata key/value table, tensor-info table, aligned data
// section) and uploads its Q8_0 / Q4_K / Q6_K tensors straight into device
// QTensors -- no dequantize -> requantize round trip -- with the llama.cpp
// q/k row order undone on the quantized rows themselves (a row of k-quant
// blocks is one output row, so the un-permute is an exact row gather).
//
// Behaviour follows the reference reader (crates/llm/mlx-llm/src/gguf/reader.rs:
// magic and version checks :211-223, metadata table :227-233, tensor infos with
// the ne order reversed to [out, in] :236-257, general.alignment default 32
// :260-265, data section at the first aligned offset :268-278, value types
// :466-498, bounds-checked tensor slices :311-328) and the engine's GGUF load
// (crates/llm/candle-llm/src/gguf.rs: remap_key :293-318, unpermute_qk
// :333-356). Type sizes: crates/llm/mlx-llm/src/gguf/dequant.rs:86-153.
#include "qmm.h"

#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

// Sets the calling thread's qmm_last_error() message (qmm_host.cpp; not exported).
int qmm_internal_fail(int code, const char* msg);

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint64_t kDefaultAlignment = 32;
constexpr uint64_t kMaxItems = 1ull << 20;  // cap for counts read from the file

enum : int {
  T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
  T_STRING = 8, T_ARRAY = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return qmm_internal_fail(code, buf);
}

// (elements, bytes) per block of a GGML type tag; false for unknown tags.
bool type_block(int tag, uint64_t* be, uint64_t* bb) {
  static const struct {
    int tag;
    uint64_t be, bb;
  } table[] = {
      {0, 1, 4},     {1, 1, 2},     {30, 1, 2},     // F32, F16, BF16
      {2, 32, 18},   {3, 32, 20},   {6, 32, 22},    // Q4_0, Q4_1, Q5_0
      {7, 32, 24},   {8, 32, 34},                   // Q5_1, Q8_0
      {10, 256, 84}, {11, 256, 110}, {12, 256, 144}, {13, 256, 176}, {14, 256, 210},  // Q2_K..Q6_K
      {16, 256, 66}, {17, 256, 74},  {18, 256, 98},  {19, 256, 50},  {20, 32, 18},    // IQ2_XXS..IQ4_NL
      {21, 256, 110}, {22, 256, 82}, {23, 256, 136}, {29, 256, 56},                   // IQ3_S..IQ1_M
  };
  for (const auto& t : table)
    if (t.tag == tag) {
      *be = t.be;
      *bb = t.bb;
      return true;
    }
  return false;
}

struct Meta {
  std::string key;
  int type = 0;       // value type (T_ARRAY for arrays)
  int elem = 0;       // element type of an array
  uint64_t count = 0; // array length (1 for scalars)
  size_t at = 0;      // file offset of the value (arrays: of the first element)
  std::vector<size_t> str_at;  // string arrays: offset of each element's length field
};

struct Tensor {
  std::string name;
  int ndims = 0;
  int64_t shape[4] = {0, 0, 0, 0};  // torch order ([out, in] for a linear weight)
  int type = 0;
  uint64_t offset = 0;
  uint64_t elems = 0;
};

// Forward-only little-endian reader with bounds checks.
struct Cursor {
  const uint8_t* p;
  size_t n, pos = 0;
  bool take(size_t k, const uint8_t** out) {
    if (k > n - pos) return false;
    *out = p + pos;
    pos += k;
    return true;
  }
  template <class T>
  bool get(T* v) {
    const uint8_t* b;
    if (!take(sizeof(T), &b)) return false;
    memcpy(v, b, sizeof(T));
    return true;
  }
  bool str(std::string* s) {
    uint64_t len;
    const uint8_t* b;
    if (!get(&len) || len > n - pos || !take((size_t)len, &b)) return false;
    s->assign(reinterpret_cast<const char*>(b), (size_t)len);
    return true;
  }
  bool skip_str() {
    uint64_t len;
    const uint8_t* b;
    return get(&len) && len <= n - pos && take((size_t)len, &b);
  }
};

size_t scalar_size(int t) {
  switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
    default: return 0;
  }
}

}  // namespace

struct qmm_gguf {
  const uint8_t* data = nullptr;
  size_t size = 0;
  void* map = nullptr;       // mmap'd file
  std::vector<uint8_t> own;  // in-memory image
  int version = 0;
  uint64_t alignment = kDefaultAlignment;
  size_t data_start = 0;
  std::vector<Meta> meta;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> meta_index, tensor_index;
};

namespace {

int parse(qmm_gguf* g) {
  Cursor c{g->data, g->size};
  uint32_t magic = 0, version = 0;
  uint64_t ntensors = 0, nmeta = 0;
  if (!c.get(&magic)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file");
  if (magic != kMagic) return fail(QMM_ERR_INVALID, "gguf: bad magic 0x%08x (expected 0x%08x)", magic, kMagic);
  if (!c.get(&version)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file");
  if (version < 2 || version > 3)
    return fail(QMM_ERR_UNSUPPORTED, "gguf version %u (only v2/v3 are supported)", version);
  g->version = (int)version;
  if (!c.get(&ntensors) || !c.get(&nmeta)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file");
  if (ntensors > kMaxItems || nmeta > kMaxItems)
    return fail(QMM_ERR_INVALID, "gguf: %llu tensors / %llu metadata entries exceed the %llu cap",
                (unsigned long long)ntensors, (unsigned long long)nmeta, (unsigned long long)kMaxItems);
  g->meta.reserve((size_t)nmeta);
  for (uint64_t i = 0; i < nmeta; ++i) {
    Meta m;
    uint32_t vt;
    if (!c.str(&m.key) || !c.get(&vt)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in metadata");
    m.type = (int)vt;
    m.count = 1;
    if (vt == T_ARRAY) {
      uint32_t et;
      uint64_t len;
      if (!c.get(&et) || !c.get(&len)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in metadata");
      if (et == T_ARRAY) return fail(QMM_ERR_UNSUPPORTED, "gguf: nested metadata arrays");
      m.elem = (int)et;
      m.count = len;
      m.at = c.pos;
      if (et == T_STRING) {
        if (len > (c.n - c.pos) / 8) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in metadata");
        m.str_at.reserve((size_t)len);
        for (uint64_t k = 0; k < len; ++k) {
          m.str_at.push_back(c.pos);
          if (!c.skip_str()) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in metadata");
        }
      } else {
        const size_t es = scalar_size((int)et);
        if (es == 0) return fail(QMM_ERR_INVALID, "gguf: unknown metadata value type %u", et);
        const uint8_t* b;
        if (len > (c.n - c.pos) / es || !c.take((size_t)(len * es), &b))
          return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in metadata");
      }
    } else if (vt == T_STRING) {
      m.at = c.pos;
      if (!c.skip_str()) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in metadata");
    } else {
      const size_t es = scalar_size((int)vt);
      if (es == 0) return fail(QMM_ERR_INVALID, "gguf: unknown metadata value type %u", vt);
      m.at = c.pos;
      const uint8_t* b;
      if (!c.take(es, &b)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in metadata");
    }
    g->meta_index[m.key] = g->meta.size();  // a repeated key keeps its last value
    g->meta.push_back(std::move(m));
  }
  g->tensors.reserve((size_t)ntensors);
  for (uint64_t i = 0; i < ntensors; ++i) {
    Tensor t;
    uint32_t nd, ty;
    if (!c.str(&t.name) || !c.get(&nd)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in tensor infos");
    if (nd == 0 || nd > 4) return fail(QMM_ERR_INVALID, "gguf: tensor \"%s\" has %u dims (expected 1..=4)", t.name.c_str(), nd);
    t.ndims = (int)nd;
    uint64_t ne[4];
    for (uint32_t d = 0; d < nd; ++d)
      if (!c.get(&ne[d])) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in tensor infos");
    t.elems = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      t.shape[d] = (int64_t)ne[nd - 1 - d];  // ne is fastest-axis first
      if (ne[d] != 0 && t.elems > UINT64_MAX / ne[d]) return fail(QMM_ERR_INVALID, "gguf: tensor \"%s\" too large", t.name.c_str());
      t.elems *= ne[d];
    }
    if (!c.get(&ty) || !c.get(&t.offset)) return fail(QMM_ERR_INVALID, "gguf: unexpected end of file in tensor infos");
    t.type = (int)ty;
    g->tensor_index[t.name] = g->tensors.size();
    g->tensors.push_back(std::move(t));
  }
  auto it = g->meta_index.find("general.alignment");
  if (it != g->meta_index.end()) {
    uint64_t a = 0;
    if (qmm_gguf_meta_u64(g, (int64_t)it->second, -1, &a) == QMM_OK) g->alignment = a;
    // a non-integer general.alignment keeps the default (as_u64 gives none)
  }
  if (g->alignment == 0) g->alignment = 1;
  // data start = end of the tensor infos rounded up to the alignment, without
  // wrapping: a rounding that would pass 2^64 (a huge general.alignment)
  // lands past the end of any file
  const uint64_t end = c.pos, rem = end % g->alignment;
  const uint64_t pad = rem ? g->alignment - rem : 0;
  const bool wraps = pad > UINT64_MAX - end;
  const uint64_t start = wraps ? UINT64_MAX : end + pad;
  if (!g->tensors.empty() && start > g->size) return fail(QMM_ERR_INVALID, "gguf: data section starts past end of file");
  g->data_start = (size_t)(start > g->size ? g->size : start);
  return QMM_OK;
}

int finish_open(qmm_gguf* g, qmm_gguf** out) {
  const int rc = parse(g);
  if (rc != QMM_OK) {
    qmm_gguf_close(g);
    return rc;
  }
  *out = g;
  return QMM_OK;
}

// Scalar element `elem` of metadata entry m (elem < 0: the scalar itself): type and offset.
int meta_elem(const qmm_gguf* g, int64_t i, int64_t elem, int* type, size_t* at) {
  if (!g || i < 0 || (uint64_t)i >= g->meta.size()) return fail(QMM_ERR_INVALID, "gguf: metadata index out of range");
  const Meta& m = g->meta[(size_t)i];
  if (m.type == T_ARRAY) {
    if (elem < 0 || (uint64_t)elem >= m.count) return fail(QMM_ERR_INVALID, "gguf: array element out of range");
    *type = m.elem;
    *at = m.elem == T_STRING ? m.str_at[(size_t)elem] : m.at + (size_t)elem * scalar_size(m.elem);
  } else {
    if (elem >= 0) return fail(QMM_ERR_INVALID, "gguf: metadata \"%s\" is not an array", m.key.c_str());
    *type = m.type;
    *at = m.at;
  }
  return QMM_OK;
}

template <class T>
T rd(const qmm_gguf* g, size_t at) {
  T v;
  memcpy(&v, g->data + at, sizeof(T));
  return v;
}

}  // namespace

extern "C" {

int qmm_gguf_open(const char* path, qmm_gguf** out) {
  if (!path || !out) return fail(QMM_ERR_INVALID, "null pointer");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(QMM_ERR_INVALID, "gguf: open %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return fail(QMM_ERR_INVALID, "gguf: stat %s: %s", path, strerror(errno));
  }
  qmm_gguf* g = new qmm_gguf();
  g->size = (size_t)st.st_size;
  if (g->size > 0) {
    void* p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
      close(fd);
      delete g;
      return fail(QMM_ERR_INVALID, "gguf: mmap %s: %s", path, strerror(errno));
    }
    g->map = p;
    g->data = static_cast<const uint8_t*>(p);
  }
  close(fd);
  return finish_open(g, out);
}

int qmm_gguf_open_memory(const void* bytes, size_t len, qmm_gguf** out) {
  if (!out || (!bytes && len)) return fail(QMM_ERR_INVALID, "null pointer");
  *out = nullptr;
  qmm_gguf* g = new qmm_gguf();
  g->own.assign(static_cast<const uint8_t*>(bytes), static_cast<const uint8_t*>(bytes) + len);
  g->data = g->own.data();
  g->size = len;
  return finish_open(g, out);
}

void qmm_gguf_close(qmm_gguf* g) {
  if (!g) return;
  if (g->map) munmap(g->map, g->size);
  delete g;
}

int qmm_gguf_version(const qmm_gguf* g) { return g ? g->version : 0; }
uint64_t qmm_gguf_alignment(const qmm_gguf* g) { return g ? g->alignment : 0; }
int64_t qmm_gguf_tensor_count(const qmm_gguf* g) { return g ? (int64_t)g->tensors.size() : -1; }
int64_t qmm_gguf_metadata_count(const qmm_gguf* g) { return g ? (int64_t)g->meta.size() : -1; }

int64_t qmm_gguf_find_tensor(const qmm_gguf* g, const char* name) {
  if (!g || !name) return -1;
  auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : (int64_t)it->second;
}

int qmm_gguf_tensor_info(const qmm_gguf* g, int64_t i, const char** name, int* ndims, int64_t* shape, int* ggml_type,
                         uint64_t* offset) {
  if (!g || i < 0 || (uint64_t)i >= g->tensors.size()) return fail(QMM_ERR_INVALID, "gguf: tensor index out of range");
  const Tensor& t = g->tensors[(size_t)i];
  if (name) *name = t.name.c_str();
  if (ndims) *ndims = t.ndims;
  if (shape)
    for (int d = 0; d < 4; ++d) shape[d] = d < t.ndims ? t.shape[d] : 0;
  if (ggml_type) *ggml_type = t.type;
  if (offset) *offset = t.offset;
  return QMM_OK;
}

int qmm_gguf_type_size(int ggml_type, uint64_t* block_elems, uint64_t* block_bytes) {
  uint64_t be, bb;
  if (!type_block(ggml_type, &be, &bb)) return fail(QMM_ERR_UNSUPPORTED, "GGUF type tag %d", ggml_type);
  if (block_elems) *block_elems = be;
  if (block_bytes) *block_bytes = bb;
  return QMM_OK;
}

int qmm_gguf_tensor_data(const qmm_gguf* g, int64_t i, const void** data, size_t* bytes) {
  if (!g || i < 0 || (uint64_t)i >= g->tensors.size()) return fail(QMM_ERR_INVALID, "gguf: tensor index out of range");
  const Tensor& t = g->tensors[(size_t)i];
  uint64_t be, bb;
  if (!type_block(t.type, &be, &bb)) return fail(QMM_ERR_UNSUPPORTED, "GGUF type tag %d", t.type);
  if (t.elems % be) return fail(QMM_ERR_INVALID, "gguf: %llu elements not a multiple of %llu for type %d",
                                (unsigned long long)t.elems, (unsigned long long)be, t.type);
  const uint64_t n = t.elems / be * bb;
  const uint64_t start = (uint64_t)g->data_start + t.offset;
  if (start < t.offset || start > g->size || n > g->size - start)
    return fail(QMM_ERR_INVALID, "gguf: tensor \"%s\" data [%llu..%llu] out of range (file %zu bytes)", t.name.c_str(),
                (unsigned long long)start, (unsigned long long)(start + n), g->size);
  if (data) *data = g->data + start;
  if (bytes) *bytes = (size_t)n;
  return QMM_OK;
}

int64_t qmm_gguf_meta_find(const qmm_gguf* g, const char* key) {
  if (!g || !key) return -1;
  auto it = g->meta_index.find(key);
  return it == g->meta_index.end() ? -1 : (int64_t)it->second;
}

int qmm_gguf_meta_info(const qmm_gguf* g, int64_t i, const char** key, int* type, int* elem_type, uint64_t* count) {
  if (!g || i < 0 || (uint64_t)i >= g->meta.size()) return fail(QMM_ERR_INVALID, "gguf: metadata index out of range");
  const Meta& m = g->meta[(size_t)i];
  if (key) *key = m.key.c_str();
  if (type) *type = m.type;
  if (elem_type) *elem_type = m.type == T_ARRAY ? m.elem : m.type;
  if (count) *count = m.count;
  return QMM_OK;
}

int qmm_gguf_meta_u64(const qmm_gguf* g, int64_t i, int64_t elem, uint64_t* v) {
  int t;
  size_t at;
  if (int rc = meta_elem(g, i, elem, &t, &at); rc != QMM_OK) return rc;
  int64_t s = 0;
  switch (t) {
    case T_U8: *v = rd<uint8_t>(g, at); return QMM_OK;
    case T_U16: *v = rd<uint16_t>(g, at); return QMM_OK;
    case T_U32: *v = rd<uint32_t>(g, at); return QMM_OK;
    case T_U64: *v = rd<uint64_t>(g, at); return QMM_OK;
    case T_BOOL: *v = rd<uint8_t>(g, at) != 0; return QMM_OK;
    case T_I8: s = rd<int8_t>(g, at); break;
    case T_I16: s = rd<int16_t>(g, at); break;
    case T_I32: s = rd<int32_t>(g, at); break;
    case T_I64: s = rd<int64_t>(g, at); break;
    default: return fail(QMM_ERR_INVALID, "gguf: metadata value of type %d is not an unsigned integer", t);
  }
  if (s < 0) return fail(QMM_ERR_INVALID, "gguf: negative metadata value is not an unsigned integer");
  *v = (uint64_t)s;
  return QMM_OK;
}

int qmm_gguf_meta_i64(const qmm_gguf* g, int64_t i, int64_t elem, int64_t* v) {
  int t;
  size_t at;
  if (int rc = meta_elem(g, i, elem, &t, &at); rc != QMM_OK) return rc;
  switch (t) {
    case T_U8: *v = rd<uint8_t>(g, at); return QMM_OK;
    case T_U16: *v = rd<uint16_t>(g, at); return QMM_OK;
    case T_U32: *v = rd<uint32_t>(g, at); return QMM_OK;
    case T_U64: *v = (int64_t)rd<uint64_t>(g, at); return QMM_OK;
    case T_I8: *v = rd<int8_t>(g, at); return QMM_OK;
    case T_I16: *v = rd<int16_t>(g, at); return QMM_OK;
    case T_I32: *v = rd<int32_t>(g, at); return QMM_OK;
    case T_I64: *v = rd<int64_t>(g, at); return QMM_OK;
    default: return fail(QMM_ERR_INVALID, "gguf: metadata value of type %d is not an integer", t);
  }
}

int qmm_gguf_meta_f64(const qmm_gguf* g, int64_t i, int64_t elem, double* v) {
  int t;
  size_t at;
  if (int rc = meta_elem(g, i, elem, &t, &at); rc != QMM_OK) return rc;
  if (t == T_F32) {
    *v = rd<float>(g, at);
    return QMM_OK;
  }
  if (t == T_F64) {
    *v = rd<double>(g, at);
    return QMM_OK;
  }
  return fail(QMM_ERR_INVALID, "gguf: metadata value of type %d is not a float", t);
}

int qmm_gguf_meta_string(const qmm_gguf* g, int64_t i, int64_t elem, const char** s, uint64_t* len) {
  int t;
  size_t at;
  if (int rc = meta_elem(g, i, elem, &t, &at); rc != QMM_OK) return rc;
  if (t != T_STRING) return fail(QMM_ERR_INVALID, "gguf: metadata value of type %d is not a string", t);
  const uint64_t n = rd<uint64_t>(g, at);
  if (s) *s = reinterpret_cast<const char*>(g->data + at + 8);
  if (len) *len = n;
  return QMM_OK;
}

// Device QTensor from a 2-D Q8_0 / Q4_K / Q6_K tensor; unpermute_heads > 0
// undoes llama.cpp's per-head q/k row order: torch row r = k * (hd / 2) + j of
// a head comes from GGUF row 2 * j + k (candle-llm gguf.rs:333-356).
int qmm_gguf_load_qtensor(const qmm_gguf* g, int64_t i, int unpermute_heads, void* stream, qmm_qtensor** out) {
  if (!out) return fail(QMM_ERR_INVALID, "null pointer");
  *out = nullptr;
  const void* src;
  size_t bytes;
  if (int rc = qmm_gguf_tensor_data(g, i, &src, &bytes); rc != QMM_OK) return rc;
  const Tensor& t = g->tensors[(size_t)i];
  int dtype;
  switch (t.type) {
    case 8: dtype = QMM_Q8_0; break;
    case 12: dtype = QMM_Q4K; break;
    case 14: dtype = QMM_Q6K; break;
    default: return fail(QMM_ERR_UNSUPPORTED, "gguf: tensor \"%s\" has type %d (resident loads take Q8_0, Q4_K, Q6_K)",
                         t.name.c_str(), t.type);
  }
  if (t.ndims != 2) return fail(QMM_ERR_UNSUPPORTED, "gguf: tensor \"%s\" is %d-D (resident loads take 2-D weights)",
                                t.name.c_str(), t.ndims);
  const int64_t n = t.shape[0], k = t.shape[1];
  if (n < 1 || k < 1) return fail(QMM_ERR_INVALID, "gguf: tensor \"%s\" has an empty dimension (%lld x %lld)",
                                  t.name.c_str(), (long long)n, (long long)k);
  if (unpermute_heads <= 0) return qmm_qtensor_from_ggml(dtype, n, k, src, 0, stream, out);
  if (n % unpermute_heads) return fail(QMM_ERR_INVALID, "gguf: q/k permute: out %lld not divisible by n_head %d",
                                       (long long)n, unpermute_heads);
  const int64_t hd = n / unpermute_heads;
  if (hd % 2) return fail(QMM_ERR_INVALID, "gguf: q/k permute: odd head_dim %lld", (long long)hd);
  const size_t row = bytes / (size_t)n, half = (size_t)hd / 2;
  std::vector<uint8_t> buf(bytes);
  const uint8_t* s8 = static_cast<const uint8_t*>(src);
  for (int64_t h = 0; h < unpermute_heads; ++h)
    for (int64_t r = 0; r < hd; ++r) {
      const size_t kk = (size_t)r / half, j = (size_t)r % half;
      memcpy(buf.data() + (size_t)(h * hd + r) * row, s8 + (size_t)(h * hd + 2 * j + kk) * row, row);
    }
  return qmm_qtensor_from_ggml(dtype, n, k, buf.data(), 0, stream, out);
}

}  // extern "C"
