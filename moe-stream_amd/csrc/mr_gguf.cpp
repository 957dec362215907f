// mr_gguf.cpp -- GGUF container reader and layer preload for the C ABI (host code).
//
// Parsing follows GgufReader::open (gguf/reader.rs:259-358): little-endian header
// (magic "GGUF", version 2 or 3, tensor count, metadata count, both <= 1e6), the
// metadata key/value list (value types 0..12, arrays of up to 1e7 elements), the
// tensor index (name, n_dims, dims in GGUF order, ggml type, offset relative to the
// data section), then the data section at the header end rounded up to
// general.alignment (default 32). Tensor types outside GgmlQuantType::from_u32
// (reader.rs:63-83) make the open fail, as there. The file is memory-mapped; tensor
// bytes are views into the mapping.
//
// mr_gguf_layer_create does the per-layer part of the reference's preload
// (engine.rs:606-652 router gates, bias and dummy-expert detection; 1079-1255 expert
// tensors; layer.rs:1130-1135 names): stacked ffn_*_exps tensors are uploaded in their
// native bytes (expert e at e * bytes_per_expert, expert_slice_data, reader.rs:394-444),
// vectors as f32.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <memory>
#include <string>
#include <unordered_map>
#include <vector>

#include "mr_internal.h"

namespace {

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"
constexpr uint64_t kMaxMeta = 1000000, kMaxTensors = 1000000, kMaxArray = 10000000;

enum : uint32_t {
  T_U8 = 0, T_I8 = 1, T_U16 = 2, T_I16 = 3, T_U32 = 4, T_I32 = 5, T_F32 = 6, T_BOOL = 7,
  T_STR = 8, T_ARR = 9, T_U64 = 10, T_I64 = 11, T_F64 = 12
};

struct Meta {
  uint32_t type = 0;
  uint64_t u = 0;    // unsigned / bool
  int64_t i = 0;     // signed
  double f = 0.0;    // float
  uint64_t s_off = 0, s_len = 0;  // string: bytes in the mapping
  uint32_t elem = 0;              // array element type
  std::vector<Meta> arr;
};

struct Tensor {
  std::string name;
  std::vector<uint64_t> dims;  // GGUF order
  uint32_t type = 0;
  uint64_t offset = 0;         // absolute
  uint64_t n_elements = 0;
};

// GgmlQuantType::from_u32 (reader.rs:63-83)
bool known_type(uint32_t t) {
  switch (t) {
    case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 9: case 10: case 11: case 12:
    case 13: case 14: case 15: case 30: case 39:
      return true;
    default:
      return false;
  }
}
// element_size / block_info (reader.rs:88-112): bytes and elements per block; false: no
// size (Q8_K has neither, as in the reference)
bool type_block(uint32_t t, uint64_t& bytes, uint64_t& elems) {
  elems = 1;
  switch (t) {
    case 0: bytes = 4; return true;
    case 1: case 30: bytes = 2; return true;
    case 10: bytes = 84, elems = 256; return true;
    case 11: bytes = 110, elems = 256; return true;
    case 12: bytes = 144, elems = 256; return true;
    case 13: bytes = 176, elems = 256; return true;
    case 14: bytes = 210, elems = 256; return true;
    case 2: bytes = 18, elems = 32; return true;
    case 3: bytes = 20, elems = 32; return true;
    case 6: bytes = 22, elems = 32; return true;
    case 7: bytes = 24, elems = 32; return true;
    case 8: bytes = 34, elems = 32; return true;
    case 9: bytes = 36, elems = 32; return true;
    case 39: bytes = 17, elems = 32; return true;
    default: return false;
  }
}
// raw_size (reader.rs:114-127): ceil(n / block_elems) * block_bytes
bool raw_size(uint32_t t, uint64_t n, uint64_t& out) {
  uint64_t b, e;
  if (!type_block(t, b, e)) return false;
  out = (n + e - 1) / e * b;
  return true;
}

struct Cursor {
  const uint8_t* p;
  uint64_t size, pos = 0;
  std::string err;
  bool need(uint64_t n, const char* what) {
    if (n > size - pos) {
      if (err.empty()) err = std::string("unexpected end of file reading ") + what;
      return false;
    }
    return true;
  }
  bool u8(uint8_t& v) { if (!need(1, "u8")) return false; v = p[pos++]; return true; }
  bool u16(uint16_t& v) { if (!need(2, "u16")) return false; memcpy(&v, p + pos, 2); pos += 2; return true; }
  bool u32(uint32_t& v) { if (!need(4, "u32")) return false; memcpy(&v, p + pos, 4); pos += 4; return true; }
  bool u64(uint64_t& v) { if (!need(8, "u64")) return false; memcpy(&v, p + pos, 8); pos += 8; return true; }
  // gguf string: u64 length, then the bytes
  bool str(uint64_t& off, uint64_t& len) {
    if (!u64(len)) return false;
    if (!need(len, "string")) return false;
    off = pos, pos += len;
    return true;
  }
  bool value(uint32_t type, Meta& m, int depth) {
    m.type = type;
    switch (type) {
      case T_U8: { uint8_t v; if (!u8(v)) return false; m.u = v; return true; }
      case T_I8: { uint8_t v; if (!u8(v)) return false; m.i = (int8_t)v; return true; }
      case T_U16: { uint16_t v; if (!u16(v)) return false; m.u = v; return true; }
      case T_I16: { uint16_t v; if (!u16(v)) return false; m.i = (int16_t)v; return true; }
      case T_U32: { uint32_t v; if (!u32(v)) return false; m.u = v; return true; }
      case T_I32: { uint32_t v; if (!u32(v)) return false; m.i = (int32_t)v; return true; }
      case T_F32: { uint32_t v; if (!u32(v)) return false; float f; memcpy(&f, &v, 4); m.f = f; return true; }
      case T_BOOL: { uint8_t v; if (!u8(v)) return false; m.u = v != 0; return true; }
      case T_STR: return str(m.s_off, m.s_len);
      case T_U64: return u64(m.u);
      case T_I64: { uint64_t v; if (!u64(v)) return false; m.i = (int64_t)v; return true; }
      case T_F64: { uint64_t v; if (!u64(v)) return false; memcpy(&m.f, &v, 8); return true; }
      case T_ARR: {
        uint64_t n;
        if (!u32(m.elem) || !u64(n)) return false;
        if (n > kMaxArray) return fail("array element count " + std::to_string(n) + " exceeds maximum 10000000");
        if (depth > 8) return fail("arrays nested too deeply");
        m.arr.resize(n);
        for (uint64_t k = 0; k < n; ++k)
          if (!value(m.elem, m.arr[k], depth + 1)) return false;
        return true;
      }
      default:
        return fail("unknown metadata type " + std::to_string(type));
    }
  }
  bool fail(const std::string& m) {
    if (err.empty()) err = m;
    return false;
  }
};

}  // namespace

struct mr_gguf {
  int fd = -1;
  const uint8_t* map = nullptr;
  uint64_t size = 0;
  std::unordered_map<std::string, Meta> meta;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> index;
  ~mr_gguf() {
    if (map) munmap(const_cast<uint8_t*>(map), size);
    if (fd >= 0) close(fd);
  }
  const Tensor* find(const char* name) const {
    auto it = index.find(name);
    return it == index.end() ? nullptr : &tensors[it->second];
  }
  const Meta* get(const char* key) const {
    auto it = meta.find(key);
    return it == meta.end() ? nullptr : &it->second;
  }
  std::string s(const Meta& m) const { return std::string(reinterpret_cast<const char*>(map + m.s_off), m.s_len); }
};

namespace {

int gerr(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return mr::set_error(nullptr, code, buf);
}

// MetadataValue::as_u32 (reader.rs:170-179)
bool as_u32(const Meta& m, uint32_t& v) {
  switch (m.type) {
    case T_U8: case T_U16: case T_U32: case T_U64: v = (uint32_t)m.u; return true;
    case T_I32: v = (uint32_t)m.i; return true;
    default: return false;
  }
}
// as_u64 (reader.rs:181-187)
bool as_u64(const Meta& m, uint64_t& v) {
  if (m.type == T_U64 || m.type == T_U32) { v = m.u; return true; }
  return false;
}

float half_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, f = h & 0x3FFu;
  uint32_t bits;
  if (e == 0) {
    if (f == 0) {
      bits = s;
    } else {  // subnormal: normalise
      int k = -1;
      uint32_t m = f;
      do { m <<= 1, ++k; } while (!(m & 0x400u));
      bits = s | ((uint32_t)(127 - 15 - k) << 23) | ((m & 0x3FFu) << 13);
    }
  } else if (e == 31) {
    bits = s | 0x7F800000u | (f << 13);
  } else {
    bits = s | ((e + 112u) << 23) | (f << 13);
  }
  float out;
  memcpy(&out, &bits, 4);
  return out;
}

// A vector tensor (F32 / F16 / BF16) as f32 on the host (load_weight -> dequantize_tensor).
int read_f32(const mr_gguf* g, const Tensor& t, std::vector<float>& out) {
  uint64_t nb;
  if (!raw_size(t.type, t.n_elements, nb)) return gerr(MR_E_UNSUPPORTED, "tensor %s: type %u has no size", t.name.c_str(), t.type);
  if (t.offset > g->size || nb > g->size - t.offset)
    return gerr(MR_E_INVAL, "tensor %s: data [%llu, +%llu) exceeds the file size %llu", t.name.c_str(),
                (unsigned long long)t.offset, (unsigned long long)nb, (unsigned long long)g->size);
  const uint8_t* p = g->map + t.offset;
  out.resize(t.n_elements);
  if (t.type == 0) {
    memcpy(out.data(), p, t.n_elements * 4);
  } else if (t.type == 1) {
    for (uint64_t i = 0; i < t.n_elements; ++i) {
      uint16_t h;
      memcpy(&h, p + 2 * i, 2);
      out[i] = half_to_f32(h);
    }
  } else if (t.type == 30) {
    for (uint64_t i = 0; i < t.n_elements; ++i) {
      uint16_t h;
      memcpy(&h, p + 2 * i, 2);
      const uint32_t bits = (uint32_t)h << 16;
      memcpy(&out[i], &bits, 4);
    }
  } else {
    return gerr(MR_E_UNSUPPORTED, "tensor %s: ggml type %u is not F32, F16 or BF16", t.name.c_str(), t.type);
  }
  return MR_OK;
}

}  // namespace

extern "C" {

int mr_gguf_open(const char* path, mr_gguf** out) {
  if (!out) return gerr(MR_E_INVAL, "mr_gguf_open: out pointer is NULL");
  *out = nullptr;
  if (!path) return gerr(MR_E_INVAL, "mr_gguf_open: path is NULL");
  std::unique_ptr<mr_gguf> g(new mr_gguf);
  g->fd = open(path, O_RDONLY | O_CLOEXEC);
  if (g->fd < 0) return gerr(MR_E_INVAL, "cannot open %s: %s", path, strerror(errno));
  struct stat st;
  if (fstat(g->fd, &st) != 0) return gerr(MR_E_INVAL, "cannot stat %s: %s", path, strerror(errno));
  g->size = (uint64_t)st.st_size;
  if (g->size == 0) return gerr(MR_E_INVAL, "%s: empty file", path);
  void* m = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
  if (m == MAP_FAILED) return gerr(MR_E_INVAL, "cannot map %s: %s", path, strerror(errno));
  g->map = static_cast<const uint8_t*>(m);

  Cursor c{g->map, g->size};
  uint32_t magic = 0, version = 0;
  uint64_t n_tensors = 0, n_meta = 0;
  if (!c.u32(magic)) return gerr(MR_E_INVAL, "%s: %s", path, c.err.c_str());
  if (magic != kMagic) return gerr(MR_E_INVAL, "%s: invalid GGUF magic 0x%08X", path, magic);
  if (!c.u32(version) || !c.u64(n_tensors) || !c.u64(n_meta)) return gerr(MR_E_INVAL, "%s: %s", path, c.err.c_str());
  if (version < 2 || version > 3) return gerr(MR_E_UNSUPPORTED, "%s: unsupported GGUF version %u", path, version);
  if (n_meta > kMaxMeta)
    return gerr(MR_E_INVAL, "%s: metadata count %llu exceeds maximum 1000000", path, (unsigned long long)n_meta);
  if (n_tensors > kMaxTensors)
    return gerr(MR_E_INVAL, "%s: tensor count %llu exceeds maximum 1000000", path, (unsigned long long)n_tensors);
  for (uint64_t k = 0; k < n_meta; ++k) {
    uint64_t ko, kl;
    uint32_t type;
    Meta v;
    if (!c.str(ko, kl) || !c.u32(type) || !c.value(type, v, 0)) return gerr(MR_E_INVAL, "%s: %s", path, c.err.c_str());
    g->meta[std::string(reinterpret_cast<const char*>(g->map + ko), kl)] = std::move(v);
  }
  std::vector<uint64_t> rel;
  g->tensors.resize(n_tensors);
  rel.resize(n_tensors);
  for (uint64_t k = 0; k < n_tensors; ++k) {
    Tensor& t = g->tensors[k];
    uint64_t no, nl;
    uint32_t nd;
    if (!c.str(no, nl) || !c.u32(nd)) return gerr(MR_E_INVAL, "%s: %s", path, c.err.c_str());
    t.name.assign(reinterpret_cast<const char*>(g->map + no), nl);
    if (nd > 8) return gerr(MR_E_INVAL, "%s: tensor %s has %u dims", path, t.name.c_str(), nd);
    t.dims.resize(nd);
    t.n_elements = 1;
    for (uint32_t d = 0; d < nd; ++d) {
      if (!c.u64(t.dims[d])) return gerr(MR_E_INVAL, "%s: %s", path, c.err.c_str());
      if (t.dims[d] != 0 && t.n_elements > UINT64_MAX / t.dims[d])
        return gerr(MR_E_INVAL, "%s: tensor %s element count overflows", path, t.name.c_str());
      t.n_elements *= t.dims[d];
    }
    if (!c.u32(t.type) || !c.u64(rel[k])) return gerr(MR_E_INVAL, "%s: %s", path, c.err.c_str());
    if (!known_type(t.type)) return gerr(MR_E_UNSUPPORTED, "%s: tensor %s: unsupported quant type %u", path, t.name.c_str(), t.type);
  }
  uint64_t align = 32;
  if (const Meta* a = g->get("general.alignment")) {
    uint64_t v;
    if (as_u64(*a, v) && v > 0) align = v;
  }
  const uint64_t data_start = (c.pos + align - 1) / align * align;
  for (uint64_t k = 0; k < n_tensors; ++k) {
    Tensor& t = g->tensors[k];
    if (rel[k] > UINT64_MAX - data_start) return gerr(MR_E_INVAL, "%s: tensor %s offset overflows", path, t.name.c_str());
    t.offset = data_start + rel[k];
    g->index[t.name] = k;
  }
  *out = g.release();
  return MR_OK;
}

void mr_gguf_close(mr_gguf* g) { delete g; }

uint64_t mr_gguf_n_tensors(const mr_gguf* g) { return g ? g->tensors.size() : 0; }

const char* mr_gguf_tensor_name(const mr_gguf* g, uint64_t i) {
  return (g && i < g->tensors.size()) ? g->tensors[i].name.c_str() : nullptr;
}

int mr_gguf_tensor_info(const mr_gguf* g, const char* name, mr_gguf_tensor* out) {
  if (!g || !name || !out) return gerr(MR_E_INVAL, "mr_gguf_tensor_info: NULL argument");
  const Tensor* t = g->find(name);
  if (!t) return gerr(MR_E_INVAL, "tensor not found: %s", name);
  if (t->dims.size() > 4) return gerr(MR_E_UNSUPPORTED, "tensor %s has %zu dims (at most 4 reported)", name, t->dims.size());
  memset(out, 0, sizeof(*out));
  out->ggml_type = t->type;
  out->n_dims = (uint32_t)t->dims.size();
  for (size_t d = 0; d < t->dims.size(); ++d) out->dims[d] = t->dims[d];
  out->data_offset = t->offset;
  uint64_t nb = 0;
  out->nbytes = raw_size(t->type, t->n_elements, nb) ? nb : 0;
  return MR_OK;
}

int mr_gguf_tensor_data(const mr_gguf* g, const char* name, const void** data, uint64_t* nbytes) {
  if (!g || !name || !data || !nbytes) return gerr(MR_E_INVAL, "mr_gguf_tensor_data: NULL argument");
  const Tensor* t = g->find(name);
  if (!t) return gerr(MR_E_INVAL, "tensor not found: %s", name);
  uint64_t nb;
  if (!raw_size(t->type, t->n_elements, nb)) return gerr(MR_E_UNSUPPORTED, "tensor %s: type %u has no size", name, t->type);
  if (t->offset > g->size || nb > g->size - t->offset)
    return gerr(MR_E_INVAL, "data out of bounds: offset %llu + size %llu exceeds file size %llu",
                (unsigned long long)t->offset, (unsigned long long)nb, (unsigned long long)g->size);
  *data = g->map + t->offset;
  *nbytes = nb;
  return MR_OK;
}

int mr_gguf_meta_u32(const mr_gguf* g, const char* key, uint32_t* out) {
  if (!g || !key || !out) return gerr(MR_E_INVAL, "mr_gguf_meta_u32: NULL argument");
  const Meta* m = g->get(key);
  if (!m) return gerr(MR_E_INVAL, "metadata key not found: %s", key);
  if (!as_u32(*m, *out)) return gerr(MR_E_INVAL, "metadata %s (type %u) is not an unsigned integer", key, m->type);
  return MR_OK;
}

int mr_gguf_meta_f32(const mr_gguf* g, const char* key, float* out) {
  if (!g || !key || !out) return gerr(MR_E_INVAL, "mr_gguf_meta_f32: NULL argument");
  const Meta* m = g->get(key);
  if (!m) return gerr(MR_E_INVAL, "metadata key not found: %s", key);
  if (m->type != T_F32 && m->type != T_F64) return gerr(MR_E_INVAL, "metadata %s (type %u) is not a float", key, m->type);
  *out = (float)m->f;  // as_f32 (reader.rs:189-195)
  return MR_OK;
}

int mr_gguf_meta_str(const mr_gguf* g, const char* key, const char** str, uint64_t* len) {
  if (!g || !key || !str || !len) return gerr(MR_E_INVAL, "mr_gguf_meta_str: NULL argument");
  const Meta* m = g->get(key);
  if (!m) return gerr(MR_E_INVAL, "metadata key not found: %s", key);
  if (m->type != T_STR) return gerr(MR_E_INVAL, "metadata %s (type %u) is not a string", key, m->type);
  *str = reinterpret_cast<const char*>(g->map + m->s_off);
  *len = m->s_len;
  return MR_OK;
}

int mr_gguf_meta_u32_array(const mr_gguf* g, const char* key, uint32_t* out, uint64_t cap, uint64_t* n) {
  if (!g || !key || !n) return gerr(MR_E_INVAL, "mr_gguf_meta_u32_array: NULL argument");
  const Meta* m = g->get(key);
  if (!m) return gerr(MR_E_INVAL, "metadata key not found: %s", key);
  if (m->type != T_ARR) return gerr(MR_E_INVAL, "metadata %s (type %u) is not an array", key, m->type);
  *n = m->arr.size();
  for (uint64_t k = 0; k < m->arr.size(); ++k) {
    uint32_t v;
    if (!as_u32(m->arr[k], v)) return gerr(MR_E_INVAL, "metadata %s[%llu] is not an unsigned integer", key, (unsigned long long)k);
    if (out && k < cap) out[k] = v;
  }
  return MR_OK;
}

int mr_gguf_upload_experts(mr_ctx* ctx, const mr_gguf* g, const char* name, mr_pack** out) {
  if (!ctx) return gerr(MR_E_INVAL, "context is NULL");
  if (!g || !name || !out) return mr::set_error(ctx, MR_E_INVAL, "mr_gguf_upload_experts: NULL argument");
  const Tensor* t = g->find(name);
  if (!t) return mr::set_error(ctx, MR_E_INVAL, (std::string("tensor not found: ") + name).c_str());
  // stacked [E, out, in] = GGUF dims [in, out, E] (pt_shape, reader.rs:145-148)
  if (t->dims.size() != 3)
    return mr::set_error(ctx, MR_E_INVAL, (std::string("expert tensor ") + name + " is not 3-dimensional").c_str());
  const void* data;
  uint64_t nb;
  int rc = mr_gguf_tensor_data(g, name, &data, &nb);
  if (rc) return mr::set_error(ctx, rc, mr_last_error(nullptr));
  const uint64_t in = t->dims[0], outf = t->dims[1], E = t->dims[2];
  if (in > UINT32_MAX || outf > UINT32_MAX || E > UINT32_MAX)
    return mr::set_error(ctx, MR_E_INVAL, "expert tensor dimensions exceed 32 bits");
  return mr_pack_upload(ctx, (int)t->type, data, nb, (uint32_t)E, (uint32_t)outf, (uint32_t)in, nullptr, out);
}

}  // extern "C"

// ---- layer preload ----------------------------------------------------------------------
namespace {

std::string blk(uint32_t l, const char* suffix) { return "blk." + std::to_string(l) + "." + suffix; }

// Device copy of a host f32 vector, recorded as owned by the layer under construction.
int upload_vec(mr_ctx* ctx, const std::vector<float>& v, std::vector<void*>& owned, float** out) {
  void* d = nullptr;
  int rc = mr_dev_alloc(ctx, v.size() * 4 + 64, &d);
  if (rc) return rc;
  owned.push_back(d);
  rc = mr_upload(ctx, d, v.data(), v.size() * 4);
  if (rc) return rc;
  *out = static_cast<float*>(d);
  return MR_OK;
}

}  // namespace

extern "C" int mr_gguf_layer_create(mr_ctx* ctx, const mr_gguf* g, uint32_t l, const mr_gguf_layer_opts* opts,
                                    mr_layer** out, const float** norm_w, float* eps) {
  if (!ctx) return gerr(MR_E_INVAL, "context is NULL");
  if (!g || !out) return mr::set_error(ctx, MR_E_INVAL, "mr_gguf_layer_create: NULL argument");
  *out = nullptr;
  if (norm_w) *norm_w = nullptr;
  std::string arch = "qwen2moe";  // config.rs:253-257 default
  {
    const char* s;
    uint64_t n;
    if (mr_gguf_meta_str(g, "general.architecture", &s, &n) == MR_OK) arch.assign(s, n);
  }
  const bool oai = arch == "gpt-oss";
  std::vector<mr_pack*> packs;
  std::vector<void*> owned;
  auto cleanup = [&](int rc) {
    for (mr_pack* p : packs) mr_pack_destroy(p);
    for (void* d : owned) (void)mr_dev_free(ctx, d);
    return rc;
  };
  mr_layer_desc d{};
  mr_pack *gate = nullptr, *up = nullptr, *down = nullptr;
  int rc;
  if ((rc = mr_gguf_upload_experts(ctx, g, blk(l, "ffn_gate_exps.weight").c_str(), &gate))) return cleanup(rc);
  packs.push_back(gate);
  if ((rc = mr_gguf_upload_experts(ctx, g, blk(l, "ffn_up_exps.weight").c_str(), &up))) return cleanup(rc);
  packs.push_back(up);
  if ((rc = mr_gguf_upload_experts(ctx, g, blk(l, "ffn_down_exps.weight").c_str(), &down))) return cleanup(rc);
  packs.push_back(down);
  d.gate = gate, d.up = up, d.down = down;

  // router (engine.rs:606-626) and dummy experts: rows whose elements all equal the first
  // within 1e-6 get -inf (engine.rs:628-652)
  const Tensor* rt = g->find(blk(l, "ffn_gate_inp.weight").c_str());
  if (!rt) return cleanup(mr::set_error(ctx, MR_E_INVAL, ("tensor not found: " + blk(l, "ffn_gate_inp.weight")).c_str()));
  std::vector<float> rw;
  if ((rc = read_f32(g, *rt, rw))) return cleanup(mr::set_error(ctx, rc, mr_last_error(nullptr)));
  const uint64_t H = rt->dims.empty() ? 0 : rt->dims[0];
  const uint64_t E = H ? rw.size() / H : 0;
  if (rt->dims.size() != 2 || E == 0) return cleanup(mr::set_error(ctx, MR_E_INVAL, "router weight is not [E, H]"));
  float* dev = nullptr;
  if ((rc = upload_vec(ctx, rw, owned, &dev))) return cleanup(rc);
  d.router_w = dev;
  std::vector<float> mask(E, 0.f);
  bool any_dummy = false;
  for (uint64_t e = 0; e < E; ++e) {
    const float first = rw[e * H];
    bool uniform = true;
    for (uint64_t i = 0; i < H && uniform; ++i) uniform = std::fabs(rw[e * H + i] - first) < 1e-6f;
    if (uniform) mask[e] = -INFINITY, any_dummy = true;
  }
  if (any_dummy) {
    if ((rc = upload_vec(ctx, mask, owned, &dev))) return cleanup(rc);
    d.dummy_mask = dev;
  }
  // optional vectors: router bias, expert biases (GPT-OSS), shared-expert gate row
  struct Opt { const char* name; const float** dst; };
  const Opt opt_vecs[] = {{"ffn_gate_inp.bias", &d.router_b}, {"ffn_gate_exps.bias", &d.gate_bias},
                          {"ffn_up_exps.bias", &d.up_bias}, {"ffn_down_exps.bias", &d.down_bias},
                          {"ffn_gate_inp_shexp.weight", &d.sh_gate_inp}};
  for (const Opt& o : opt_vecs) {
    const Tensor* t = g->find(blk(l, o.name).c_str());
    if (!t) continue;
    std::vector<float> v;
    if ((rc = read_f32(g, *t, v))) return cleanup(mr::set_error(ctx, rc, mr_last_error(nullptr)));
    if ((rc = upload_vec(ctx, v, owned, &dev))) return cleanup(rc);
    *o.dst = dev;
  }
  // shared expert (layer.rs:1898-1953): [Ish, H] / [H, Ish] matrices, uploaded as one-expert packs
  if (g->find(blk(l, "ffn_gate_shexp.weight").c_str())) {
    const char* names[3] = {"ffn_gate_shexp.weight", "ffn_up_shexp.weight", "ffn_down_shexp.weight"};
    const mr_pack** dst[3] = {&d.sh_gate, &d.sh_up, &d.sh_down};
    for (int k = 0; k < 3; ++k) {
      const std::string n = blk(l, names[k]);
      const Tensor* t = g->find(n.c_str());
      if (!t || t->dims.size() != 2) return cleanup(mr::set_error(ctx, MR_E_INVAL, ("shared expert tensor missing or not 2-D: " + n).c_str()));
      const void* data;
      uint64_t nb;
      if ((rc = mr_gguf_tensor_data(g, n.c_str(), &data, &nb))) return cleanup(mr::set_error(ctx, rc, mr_last_error(nullptr)));
      mr_pack* p = nullptr;
      if ((rc = mr_pack_upload(ctx, (int)t->type, data, nb, 1, (uint32_t)t->dims[1], (uint32_t)t->dims[0], nullptr, &p)))
        return cleanup(rc);
      packs.push_back(p);
      *dst[k] = p;
    }
  }
  // routing and activation (config.rs:287, 364; layer.rs:1027, 873-874)
  uint32_t top_k = opts ? opts->top_k : 0;
  if (!top_k && mr_gguf_meta_u32(g, (arch + ".expert_used_count").c_str(), &top_k) != MR_OK) top_k = 8;
  d.top_k = top_k;
  if (opts && opts->route_flags >= 0) {
    d.route_flags = (uint32_t)opts->route_flags;
  } else if (oai) {
    d.route_flags = MR_ROUTE_SOFTMAX_AFTER_TOPK;
  } else {
    const char* s;
    uint64_t n;
    std::string name;
    if (mr_gguf_meta_str(g, "general.name", &s, &n) == MR_OK) name.assign(s, n);
    const bool norm = name.find("Qwen1.5") == std::string::npos && name.find("Qwen2") == std::string::npos;
    d.route_flags = norm ? MR_ROUTE_NORM_TOPK : 0u;
  }
  d.act = (opts && opts->act >= 0) ? (uint32_t)opts->act : (oai ? MR_ACT_SWIGLU_OAI : MR_ACT_SILU);
  d.alpha = (opts && opts->alpha > 0.f) ? opts->alpha : 1.702f;
  d.limit = (opts && opts->limit > 0.f) ? opts->limit : 7.0f;

  // post-attention norm (layer.rs:463) and eps (config.rs:293) for mr_moe_forward_residual
  float* nw = nullptr;
  if (const Tensor* t = g->find(blk(l, "post_attention_norm.weight").c_str())) {
    std::vector<float> v;
    if ((rc = read_f32(g, *t, v))) return cleanup(mr::set_error(ctx, rc, mr_last_error(nullptr)));
    if ((rc = upload_vec(ctx, v, owned, &nw))) return cleanup(rc);
  }
  if (eps) {
    float e = 1e-6f;
    if (mr_gguf_meta_f32(g, (arch + ".attention.layer_norm_rms_epsilon").c_str(), &e) != MR_OK) e = 1e-6f;
    *eps = e;
  }
  mr_layer* L = nullptr;
  if ((rc = mr_layer_create(ctx, &d, &L))) return cleanup(rc);
  mr::layer_adopt(L, packs.data(), packs.size(), owned.data(), owned.size());
  L->norm_w = nw;  // owned by the layer: the previous layer may prefetch it
  if (norm_w) *norm_w = nw;
  *out = L;
  return MR_OK;
}
