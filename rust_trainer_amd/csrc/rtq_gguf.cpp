// rtq_gguf.cpp — GGUF v3 container reader and writer of librtq.so (C ABI in include/rtq.h).
//
// Replaces the container half of rie-core's gguf module that Rust_Trainer calls
// (GgufFile::open / from_bytes, get_str / get_f32, tensor + tensor_data: src/rie.rs:159-166,
// 370-384; GgufWriter::new / kv / tensor / to_bytes: src/rie.rs:349-363) and serves the synthetic
// model builder (SyntheticSpec, src/main.rs:648-677, examples/bench_train.rs:28-32, tests/engine.rs:27-31).
//
// Layout (public GGUF v3 specification, little-endian):
//   u32 magic "GGUF", u32 version, u64 tensor_count, u64 kv_count;
//   kv_count x { gguf_string key, u32 value_type, value };
//   tensor_count x { gguf_string name, u32 n_dims, u64 ne[n_dims], u32 ggml_type, u64 offset };
//   padding to general.alignment (default 32); tensor data, each tensor at data_start + offset
//   (offset a multiple of the alignment).
//   gguf_string = u64 length + bytes (no terminator); value types: u8 0, i8 1, u16 2, i16 3, u32 4,
//   i32 5, f32 6, bool 7, string 8, array 9 (u32 element type, u64 count, elements), u64 10,
//   i64 11, f64 12.
// The reader maps the file (or borrows the caller's bytes) and checks every length and offset
// against the image; malformed images fail with RTQ_ERR_INVALID and a message.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <algorithm>
#include <string>
#include <unordered_map>
#include <vector>

#include "rtq.h"

// the runtime's error reporting (rtq_runtime.cpp)
rtq_status rtq_fail(rtq_status s, const char* fmt, ...);

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
enum : int { T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 };

int scalar_size(int t) {
  switch (t) {
    case T_U8: case T_I8: case T_BOOL: return 1;
    case T_U16: case T_I16: return 2;
    case T_U32: case T_I32: case T_F32: return 4;
    case T_U64: case T_I64: case T_F64: return 8;
  }
  return 0;
}

// bytes of n elements of a ggml type (block types: n a multiple of the block), 0 if unknown
uint64_t ggml_nbytes(int type, uint64_t n) {
  struct S { int type; uint32_t elems, bytes; };
  static const S sizes[] = {{0, 1, 4},     {1, 1, 2},     {2, 32, 18},    {3, 32, 20},   {6, 32, 22},
                            {7, 32, 24},   {8, 32, 34},   {9, 32, 36},    {10, 256, 84}, {11, 256, 110},
                            {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {24, 1, 1},
                            {25, 1, 2},    {26, 1, 4},    {27, 1, 8},     {28, 1, 8},    {30, 1, 2}};
  for (const S& s : sizes)
    if (s.type == type) return n % s.elems ? 0 : n / s.elems * s.bytes;
  return 0;
}

struct Kv {
  std::string key;
  int type = 0, elem = -1;
  uint64_t count = 1;
  const uint8_t* data = nullptr;  // scalar / string bytes / first array element in the image
};

struct Tensor {
  std::string name;
  int type = 0, n_dims = 0;
  int64_t ne[4] = {1, 1, 1, 1};
  uint64_t offset = 0, nbytes = 0;
  const uint8_t* data = nullptr;
};

struct Reader {
  const uint8_t* p;
  size_t n, at = 0;
  bool ok = true;
  bool need(size_t k) {
    if (!ok || k > n - at) ok = false;
    return ok;
  }
  template <class T>
  T get() {
    T v{};
    if (need(sizeof(T))) {
      memcpy(&v, p + at, sizeof(T));
      at += sizeof(T);
    }
    return v;
  }
  bool str(std::string* s, const uint8_t** where = nullptr) {
    const uint64_t len = get<uint64_t>();
    if (!need(len)) return false;
    if (where) *where = p + at;
    if (s) s->assign(reinterpret_cast<const char*>(p + at), len);
    at += len;
    return true;
  }
  // skips one value of type t (count elements of an array's element type)
  bool skip(int t) {
    if (t == T_STR) return str(nullptr);
    const int sz = scalar_size(t);
    if (!sz) return ok = false;
    return need(sz) && (at += sz, true);
  }
};

}  // namespace

struct rtq_gguf {
  const uint8_t* base = nullptr;
  size_t size = 0;
  void* map = nullptr;  // mmap'd image (rtq_gguf_open), else the caller's bytes
  uint32_t version = 0, alignment = 32;
  std::vector<Kv> kvs;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, int64_t> kv_index, tensor_index;
};

namespace {

rtq_status parse(rtq_gguf* g) {
  Reader r{g->base, g->size};
  if (r.get<uint32_t>() != kMagic || !r.ok) return rtq_fail(RTQ_ERR_INVALID, "not a GGUF image (magic)");
  g->version = r.get<uint32_t>();
  if (g->version < 2 || g->version > 3) return rtq_fail(RTQ_ERR_INVALID, "GGUF version %u not supported", g->version);
  const uint64_t nt = r.get<uint64_t>(), nk = r.get<uint64_t>();
  if (!r.ok || nt > (1u << 24) || nk > (1u << 24)) return rtq_fail(RTQ_ERR_INVALID, "GGUF header truncated or too large");
  g->kvs.resize(nk);
  for (uint64_t i = 0; i < nk; i++) {
    Kv& kv = g->kvs[i];
    if (!r.str(&kv.key)) return rtq_fail(RTQ_ERR_INVALID, "GGUF key %llu truncated", (unsigned long long)i);
    kv.type = (int)r.get<uint32_t>();
    if (kv.type == T_ARR) {
      kv.elem = (int)r.get<uint32_t>();
      kv.count = r.get<uint64_t>();
      if (kv.elem == T_ARR || (kv.elem != T_STR && !scalar_size(kv.elem)))
        return rtq_fail(RTQ_ERR_INVALID, "GGUF key %s: bad array element type %d", kv.key.c_str(), kv.elem);
      kv.data = g->base + r.at;
      if (kv.elem == T_STR) {
        for (uint64_t j = 0; j < kv.count && r.ok; j++) r.str(nullptr);
      } else if (!r.need(kv.count * (uint64_t)scalar_size(kv.elem)) || kv.count > (1ull << 40)) {
        return rtq_fail(RTQ_ERR_INVALID, "GGUF key %s: array truncated", kv.key.c_str());
      } else {
        r.at += kv.count * scalar_size(kv.elem);
      }
    } else if (kv.type == T_STR) {
      r.str(nullptr, &kv.data);
      kv.count = kv.data ? (uint64_t)(g->base + r.at - kv.data) : 0;
    } else {
      kv.data = g->base + r.at;
      if (!r.skip(kv.type)) return rtq_fail(RTQ_ERR_INVALID, "GGUF key %s: bad value type %d", kv.key.c_str(), kv.type);
    }
    if (!r.ok) return rtq_fail(RTQ_ERR_INVALID, "GGUF key %s: value truncated", kv.key.c_str());
    g->kv_index[kv.key] = (int64_t)i;
  }
  auto al = g->kv_index.find("general.alignment");
  if (al != g->kv_index.end()) {
    const Kv& kv = g->kvs[al->second];
    if (kv.type != T_U32) return rtq_fail(RTQ_ERR_INVALID, "general.alignment is not a u32");
    memcpy(&g->alignment, kv.data, 4);
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1)))
      return rtq_fail(RTQ_ERR_INVALID, "general.alignment %u is not a power of two", g->alignment);
  }
  g->tensors.resize(nt);
  for (uint64_t i = 0; i < nt; i++) {
    Tensor& t = g->tensors[i];
    if (!r.str(&t.name)) return rtq_fail(RTQ_ERR_INVALID, "GGUF tensor %llu name truncated", (unsigned long long)i);
    t.n_dims = (int)r.get<uint32_t>();
    if (t.n_dims < 1 || t.n_dims > 4) return rtq_fail(RTQ_ERR_INVALID, "tensor %s: %d dims", t.name.c_str(), t.n_dims);
    uint64_t n = 1;
    for (int d = 0; d < t.n_dims; d++) {
      const uint64_t e = r.get<uint64_t>();
      if (e == 0 || e > (1ull << 40) || n > (1ull << 62) / e)
        return rtq_fail(RTQ_ERR_INVALID, "tensor %s: bad dimension", t.name.c_str());
      t.ne[d] = (int64_t)e;
      n *= e;
    }
    t.type = (int)r.get<uint32_t>();
    t.offset = r.get<uint64_t>();
    if (!r.ok) return rtq_fail(RTQ_ERR_INVALID, "tensor %s: info truncated", t.name.c_str());
    t.nbytes = ggml_nbytes(t.type, n);
    if (t.offset % g->alignment) return rtq_fail(RTQ_ERR_INVALID, "tensor %s: unaligned offset", t.name.c_str());
    g->tensor_index[t.name] = (int64_t)i;
  }
  const uint64_t data_start = (r.at + g->alignment - 1) / g->alignment * g->alignment;
  for (Tensor& t : g->tensors) {
    if (data_start > g->size || t.offset > g->size - data_start || t.nbytes > g->size - data_start - t.offset)
      return rtq_fail(RTQ_ERR_INVALID, "tensor %s: data past the end of the image", t.name.c_str());
    t.data = g->base + data_start + t.offset;
  }
  return RTQ_OK;
}

rtq_status finish_open(rtq_gguf* g, rtq_gguf** out) {
  const rtq_status s = parse(g);
  if (s != RTQ_OK) {
    rtq_gguf_close(g);
    return s;
  }
  *out = g;
  return RTQ_OK;
}

const Kv* find_kv(const rtq_gguf* g, const char* key) {
  if (!g || !key) return nullptr;
  auto it = g->kv_index.find(key);
  return it == g->kv_index.end() ? nullptr : &g->kvs[it->second];
}

}  // namespace

extern "C" {

rtq_status rtq_gguf_open(const char* path, rtq_gguf** out) {
  if (!path || !out) return rtq_fail(RTQ_ERR_INVALID, "null path/out");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return rtq_fail(RTQ_ERR_INVALID, "cannot open %s", path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size <= 0) {
    close(fd);
    return rtq_fail(RTQ_ERR_INVALID, "cannot stat %s (or empty)", path);
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m == MAP_FAILED) return rtq_fail(RTQ_ERR_INVALID, "cannot map %s", path);
  rtq_gguf* g = new rtq_gguf();
  g->map = m;
  g->base = static_cast<const uint8_t*>(m);
  g->size = (size_t)st.st_size;
  return finish_open(g, out);
}

rtq_status rtq_gguf_from_bytes(const void* data, size_t nbytes, rtq_gguf** out) {
  if (!data || !out) return rtq_fail(RTQ_ERR_INVALID, "null data/out");
  *out = nullptr;
  rtq_gguf* g = new rtq_gguf();
  g->base = static_cast<const uint8_t*>(data);
  g->size = nbytes;
  return finish_open(g, out);
}

void rtq_gguf_close(rtq_gguf* g) {
  if (!g) return;
  if (g->map) munmap(g->map, g->size);
  delete g;
}

uint32_t rtq_gguf_version(const rtq_gguf* g) { return g ? g->version : 0; }
int64_t rtq_gguf_kv_count(const rtq_gguf* g) { return g ? (int64_t)g->kvs.size() : 0; }
int64_t rtq_gguf_tensor_count(const rtq_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }

int64_t rtq_gguf_find_kv(const rtq_gguf* g, const char* key) {
  const Kv* kv = find_kv(g, key);
  return kv ? (int64_t)(kv - g->kvs.data()) : -1;
}

rtq_status rtq_gguf_kv(const rtq_gguf* g, int64_t i, const char** key, int* type, int* elem_type, uint64_t* count,
                       const void** data) {
  if (!g || i < 0 || i >= (int64_t)g->kvs.size()) return rtq_fail(RTQ_ERR_INVALID, "kv index out of range");
  const Kv& kv = g->kvs[i];
  if (key) *key = kv.key.c_str();
  if (type) *type = kv.type;
  if (elem_type) *elem_type = kv.elem;
  if (count) *count = kv.count;
  if (data) *data = kv.data;
  return RTQ_OK;
}

rtq_status rtq_gguf_get_str(const rtq_gguf* g, const char* key, const char** s, uint64_t* len) {
  const Kv* kv = find_kv(g, key);
  if (!kv || kv->type != T_STR) return rtq_fail(RTQ_ERR_INVALID, "no string key %s", key ? key : "(null)");
  if (s) *s = reinterpret_cast<const char*>(kv->data);
  if (len) *len = kv->count;
  return RTQ_OK;
}

rtq_status rtq_gguf_get_f64(const rtq_gguf* g, const char* key, double* v) {
  const Kv* kv = find_kv(g, key);
  if (!kv || !v) return rtq_fail(RTQ_ERR_INVALID, "no key %s", key ? key : "(null)");
  const uint8_t* d = kv->data;
  switch (kv->type) {
    case T_U8: case T_BOOL: *v = d[0]; break;
    case T_I8: *v = (int8_t)d[0]; break;
    case T_U16: { uint16_t x; memcpy(&x, d, 2); *v = x; break; }
    case T_I16: { int16_t x; memcpy(&x, d, 2); *v = x; break; }
    case T_U32: { uint32_t x; memcpy(&x, d, 4); *v = x; break; }
    case T_I32: { int32_t x; memcpy(&x, d, 4); *v = x; break; }
    case T_F32: { float x; memcpy(&x, d, 4); *v = x; break; }
    case T_U64: { uint64_t x; memcpy(&x, d, 8); *v = (double)x; break; }
    case T_I64: { int64_t x; memcpy(&x, d, 8); *v = (double)x; break; }
    case T_F64: memcpy(v, d, 8); break;
    default: return rtq_fail(RTQ_ERR_INVALID, "key %s is not a number", key);
  }
  return RTQ_OK;
}

int64_t rtq_gguf_find_tensor(const rtq_gguf* g, const char* name) {
  if (!g || !name) return -1;
  auto it = g->tensor_index.find(name);
  return it == g->tensor_index.end() ? -1 : it->second;
}

rtq_status rtq_gguf_tensor(const rtq_gguf* g, int64_t i, const char** name, int* type, int* n_dims, int64_t ne[4],
                           const void** data, size_t* nbytes) {
  if (!g || i < 0 || i >= (int64_t)g->tensors.size()) return rtq_fail(RTQ_ERR_INVALID, "tensor index out of range");
  const Tensor& t = g->tensors[i];
  if (name) *name = t.name.c_str();
  if (type) *type = t.type;
  if (n_dims) *n_dims = t.n_dims;
  if (ne) memcpy(ne, t.ne, sizeof(t.ne));
  if (data) *data = t.data;
  if (nbytes) *nbytes = (size_t)t.nbytes;
  return RTQ_OK;
}

rtq_status rtq_weight_from_gguf(rtq_ctx* c, const rtq_gguf* g, const char* name, rtq_weight** out) {
  const int64_t i = rtq_gguf_find_tensor(g, name);
  if (i < 0) return rtq_fail(RTQ_ERR_INVALID, "no tensor %s", name ? name : "(null)");
  const Tensor& t = g->tensors[i];
  if (t.nbytes == 0) return rtq_fail(RTQ_ERR_UNSUPPORTED, "tensor %s: ggml type %d has no known size", name, t.type);
  int64_t rows = 1;
  for (int d = 1; d < t.n_dims; d++) rows *= t.ne[d];
  return rtq_weight_create(c, t.type, t.data, (size_t)t.nbytes, rows, t.ne[0], out);
}

}  // extern "C"

// ------------------------------------------------------------------ writer
struct rtq_gguf_writer {
  struct WKv {
    std::string key;
    int type, elem;
    uint64_t count;
    std::vector<uint8_t> bytes;  // value encoding after the type tag(s)
  };
  struct WTensor {
    std::string name;
    int type, n_dims;
    int64_t ne[4];
    std::vector<uint8_t> data;
  };
  std::vector<WKv> kvs;
  std::vector<WTensor> tensors;
  std::vector<uint8_t> image;
  uint32_t alignment = 32;
};

namespace {

void put_u32(std::vector<uint8_t>& b, uint32_t v) { b.insert(b.end(), (uint8_t*)&v, (uint8_t*)&v + 4); }
void put_u64(std::vector<uint8_t>& b, uint64_t v) { b.insert(b.end(), (uint8_t*)&v, (uint8_t*)&v + 8); }
void put_str(std::vector<uint8_t>& b, const char* s, uint64_t len) {
  put_u64(b, len);
  b.insert(b.end(), (const uint8_t*)s, (const uint8_t*)s + len);
}

}  // namespace

extern "C" {

rtq_status rtq_gguf_writer_create(rtq_gguf_writer** out) {
  if (!out) return rtq_fail(RTQ_ERR_INVALID, "null out");
  *out = new rtq_gguf_writer();
  return RTQ_OK;
}

void rtq_gguf_writer_destroy(rtq_gguf_writer* w) { delete w; }

// type: a scalar type with count 1 and data -> the value; T_STR (8) with data -> count bytes;
// T_ARR (9) of elem_type with count elements at data (string arrays: data is const char* const*,
// each NUL-terminated)
rtq_status rtq_gguf_writer_kv(rtq_gguf_writer* w, const char* key, int type, int elem_type, uint64_t count,
                              const void* data) {
  if (!w || !key || (!data && count)) return rtq_fail(RTQ_ERR_INVALID, "null writer/key/data");
  rtq_gguf_writer::WKv kv{key, type, elem_type, count, {}};
  if (type == T_STR) {
    kv.bytes.assign((const uint8_t*)data, (const uint8_t*)data + count);
  } else if (type == T_ARR) {
    if (elem_type == T_STR) {
      const char* const* s = static_cast<const char* const*>(data);
      for (uint64_t i = 0; i < count; i++) put_str(kv.bytes, s[i], strlen(s[i]));
    } else if (scalar_size(elem_type)) {
      kv.bytes.assign((const uint8_t*)data, (const uint8_t*)data + count * scalar_size(elem_type));
    } else {
      return rtq_fail(RTQ_ERR_INVALID, "key %s: bad array element type %d", key, elem_type);
    }
  } else if (scalar_size(type) && count == 1) {
    kv.bytes.assign((const uint8_t*)data, (const uint8_t*)data + scalar_size(type));
    if (!strcmp(key, "general.alignment")) {
      if (type != T_U32) return rtq_fail(RTQ_ERR_INVALID, "general.alignment must be a u32");
      memcpy(&w->alignment, data, 4);
      if (w->alignment == 0 || (w->alignment & (w->alignment - 1)))
        return rtq_fail(RTQ_ERR_INVALID, "general.alignment %u is not a power of two", w->alignment);
    }
  } else {
    return rtq_fail(RTQ_ERR_INVALID, "key %s: bad value type %d", key, type);
  }
  w->kvs.push_back(std::move(kv));
  return RTQ_OK;
}

rtq_status rtq_gguf_writer_tensor(rtq_gguf_writer* w, const char* name, int type, int n_dims, const int64_t* ne,
                                  const void* data, size_t nbytes) {
  if (!w || !name || !ne || (!data && nbytes)) return rtq_fail(RTQ_ERR_INVALID, "null writer/name/ne/data");
  if (n_dims < 1 || n_dims > 4) return rtq_fail(RTQ_ERR_INVALID, "tensor %s: %d dims", name, n_dims);
  rtq_gguf_writer::WTensor t{name, type, n_dims, {1, 1, 1, 1}, {}};
  uint64_t n = 1;
  for (int d = 0; d < n_dims; d++) {
    if (ne[d] <= 0) return rtq_fail(RTQ_ERR_INVALID, "tensor %s: bad dimension", name);
    t.ne[d] = ne[d];
    n *= (uint64_t)ne[d];
  }
  const uint64_t want = ggml_nbytes(type, n);
  if (want == 0 || want != nbytes)
    return rtq_fail(RTQ_ERR_INVALID, "tensor %s: %zu bytes for %llu elements of type %d", name, nbytes,
                    (unsigned long long)n, type);
  t.data.assign((const uint8_t*)data, (const uint8_t*)data + nbytes);
  w->tensors.push_back(std::move(t));
  return RTQ_OK;
}

}  // extern "C"

namespace {

// the header and tensor directory, padded to the alignment; offs[i] = tensor i's data offset,
// returns the size of the data section
uint64_t writer_header(const rtq_gguf_writer* w, std::vector<uint8_t>& b, std::vector<uint64_t>& offs) {
  b.clear();
  put_u32(b, kMagic);
  put_u32(b, 3);
  put_u64(b, w->tensors.size());
  put_u64(b, w->kvs.size());
  for (const auto& kv : w->kvs) {
    put_str(b, kv.key.data(), kv.key.size());
    put_u32(b, (uint32_t)kv.type);
    if (kv.type == T_ARR) {
      put_u32(b, (uint32_t)kv.elem);
      put_u64(b, kv.count);
    } else if (kv.type == T_STR) {
      put_u64(b, kv.bytes.size());
    }
    b.insert(b.end(), kv.bytes.begin(), kv.bytes.end());
  }
  const uint64_t al = w->alignment;
  uint64_t off = 0;
  offs.clear();
  for (const auto& t : w->tensors) {
    put_str(b, t.name.data(), t.name.size());
    put_u32(b, (uint32_t)t.n_dims);
    for (int d = 0; d < t.n_dims; d++) put_u64(b, (uint64_t)t.ne[d]);
    put_u32(b, (uint32_t)t.type);
    put_u64(b, off);
    offs.push_back(off);
    off = (off + t.data.size() + al - 1) / al * al;
  }
  b.resize((b.size() + al - 1) / al * al, 0);
  return off;
}

}  // namespace

extern "C" {

// the serialised image (GgufWriter::to_bytes), owned by the writer until the next call or destroy
rtq_status rtq_gguf_writer_bytes(rtq_gguf_writer* w, const void** data, size_t* nbytes) {
  if (!w || !data || !nbytes) return rtq_fail(RTQ_ERR_INVALID, "null writer/out");
  std::vector<uint8_t>& b = w->image;
  std::vector<uint64_t> offs;
  const uint64_t data_bytes = writer_header(w, b, offs);
  const size_t data_start = b.size();
  b.resize(data_start + data_bytes, 0);
  for (size_t i = 0; i < w->tensors.size(); i++)
    memcpy(b.data() + data_start + offs[i], w->tensors[i].data.data(), w->tensors[i].data.size());
  *data = b.data();
  *nbytes = b.size();
  return RTQ_OK;
}

// streams the image to path.tmp, then renames it to path (write_gguf_adapter, src/rie.rs:359-362)
rtq_status rtq_gguf_writer_write(rtq_gguf_writer* w, const char* path) {
  if (!w || !path) return rtq_fail(RTQ_ERR_INVALID, "null writer/path");
  std::vector<uint8_t> head;
  std::vector<uint64_t> offs;
  const uint64_t data_bytes = writer_header(w, head, offs);
  const std::string tmp = std::string(path) + ".tmp";
  FILE* f = fopen(tmp.c_str(), "wb");
  if (!f) return rtq_fail(RTQ_ERR_INVALID, "cannot create %s", tmp.c_str());
  bool ok = fwrite(head.data(), 1, head.size(), f) == head.size();
  static const uint8_t zeros[256] = {};
  uint64_t at = 0;
  auto pad_to = [&](uint64_t end) {
    while (ok && at < end) {
      const size_t k = (size_t)std::min<uint64_t>(end - at, sizeof zeros);
      ok = fwrite(zeros, 1, k, f) == k;
      at += k;
    }
  };
  for (size_t i = 0; ok && i < w->tensors.size(); i++) {
    pad_to(offs[i]);
    const auto& d = w->tensors[i].data;
    ok = ok && fwrite(d.data(), 1, d.size(), f) == d.size();
    at += d.size();
  }
  pad_to(data_bytes);
  ok = (fclose(f) == 0) && ok;
  if (!ok || rename(tmp.c_str(), path) != 0) {
    remove(tmp.c_str());
    return rtq_fail(RTQ_ERR_INVALID, "cannot write %s", path);
  }
  return RTQ_OK;
}

}  // extern "C"
