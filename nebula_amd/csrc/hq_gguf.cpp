// hq_gguf.cpp — GGUF container loader (C ABI in include/hq_qgemm.h): a read-only memory map of
// the file, its header, typed key-value metadata and tensor directory, and the import of the
// quantized tensors this library runs: TQ1_0 blocks (device repack into the ternary tile
// layout) and GGML Q4_K blocks (host conversion into int4 codes, fp16 scales and fp32 biases
// with groups of 32).
//
// Replaces hydrogen::ModelLoader / parse_gguf (hydrogen/include/tensor_loader.hpp:14-53,
// hydrogen/include/gguf_parser.hpp:33-145, hydrogen/src/model/tensor_loader.cpp) for this
// path. The parse keeps the reference's rules: magic "GGUF", versions 2 and 3 only, 64-bit
// counts, every metadata value type (arrays of any element type, nested), at most 4 tensor
// dimensions, general.alignment (default 32, 0 read as 32) for the start of the tensor data,
// a tensor's bytes from its element count and its type's block traits, and a null data
// pointer for a tensor that extends past the end of the file. Where the reference throws, the
// ABI returns HQ_ERR_FORMAT (malformed or unsupported file) with the reason in hq_last_error.
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

#include "hq_internal.hpp"
#include "hq_layout.hpp"
#include "hq_qgemm.h"

namespace {

// Metadata value types (gguf_parser.hpp:17-31).
enum : uint32_t {
  kU8 = 0, kI8 = 1, kU16 = 2, kI16 = 3, kU32 = 4, kI32 = 5, kF32 = 6, kBool = 7, kString = 8, kArray = 9,
  kU64 = 10, kI64 = 11, kF64 = 12
};

struct Value {
  uint32_t type = 0;
  uint64_t u = 0;  // unsigned and bool values
  int64_t i = 0;   // signed values
  double f = 0.0;  // float values
  std::string s;
  uint32_t arr_type = 0;
  uint64_t arr_count = 0;
};

struct Reader {
  const uint8_t* p;
  size_t size, cur = 0;
  std::string err;
  bool need(size_t n) {
    if (!err.empty()) return false;
    if (n > size - cur) {
      char b[96];
      std::snprintf(b, sizeof b, "unexpected end of the GGUF data at offset %zu", cur);
      err = b;
      return false;
    }
    return true;
  }
  template <class T>
  T pod() {
    T v{};
    if (need(sizeof(T))) {
      std::memcpy(&v, p + cur, sizeof(T));
      cur += sizeof(T);
    }
    return v;
  }
  std::string str() {
    const uint64_t n = pod<uint64_t>();
    if (!need(n)) return {};
    std::string s(reinterpret_cast<const char*>(p + cur), (size_t)n);
    cur += (size_t)n;
    return s;
  }
  // One value of type t into v (arrays: element type and count kept, elements parsed and dropped).
  void value(uint32_t t, Value& v, int depth = 0) {
    v.type = t;
    switch (t) {
      case kU8: v.u = pod<uint8_t>(); v.i = (int64_t)v.u; break;
      case kI8: v.i = pod<int8_t>(); v.u = (uint64_t)v.i; break;
      case kU16: v.u = pod<uint16_t>(); v.i = (int64_t)v.u; break;
      case kI16: v.i = pod<int16_t>(); v.u = (uint64_t)v.i; break;
      case kU32: v.u = pod<uint32_t>(); v.i = (int64_t)v.u; break;
      case kI32: v.i = pod<int32_t>(); v.u = (uint64_t)v.i; break;
      case kF32: v.f = pod<float>(); break;
      case kBool: v.u = pod<uint8_t>() != 0; break;
      case kString: v.s = str(); break;
      case kU64: v.u = pod<uint64_t>(); v.i = (int64_t)v.u; break;
      case kI64: v.i = pod<int64_t>(); v.u = (uint64_t)v.i; break;
      case kF64: v.f = pod<double>(); break;
      case kArray: {
        if (depth > 8) {
          err = "GGUF arrays nested more than 8 deep";
          return;
        }
        v.arr_type = pod<uint32_t>();
        v.arr_count = pod<uint64_t>();
        Value e;
        for (uint64_t k = 0; k < v.arr_count && err.empty(); ++k) value(v.arr_type, e, depth + 1);
        break;
      }
      default: {
        char b[64];
        std::snprintf(b, sizeof b, "unknown GGUF value type %u", t);
        err = b;
      }
    }
  }
};

// Block traits of a tensor type (gguf_parser.hpp:108-139): elements per block, bytes per block.
void type_traits(uint32_t type, uint64_t& bs, uint64_t& bb) {
  switch (type) {
    case 0: bs = 1; bb = 4; return;      // F32
    case 1: bs = 1; bb = 2; return;      // F16
    case 30: bs = 1; bb = 2; return;     // BF16
    case 24: bs = 1; bb = 1; return;     // I8
    case 25: bs = 1; bb = 2; return;     // I16
    case 26: bs = 1; bb = 4; return;     // I32
    case 27: bs = 1; bb = 8; return;     // I64
    case 28: bs = 1; bb = 8; return;     // F64
    case 2: bs = 32; bb = 18; return;    // Q4_0
    case 3: bs = 32; bb = 20; return;    // Q4_1
    case 6: bs = 32; bb = 22; return;    // Q5_0
    case 7: bs = 32; bb = 24; return;    // Q5_1
    case 8: bs = 32; bb = 34; return;    // Q8_0
    case 9: bs = 32; bb = 40; return;    // Q8_1
    case 10: bs = 256; bb = 84; return;  // Q2_K
    case 11: bs = 256; bb = 110; return; // Q3_K
    case 12: bs = 256; bb = 144; return; // Q4_K
    case 13: bs = 256; bb = 176; return; // Q5_K
    case 14: bs = 256; bb = 210; return; // Q6_K
    case 15: bs = 256; bb = 292; return; // Q8_K
    case 20: bs = 32; bb = 18; return;   // IQ4_NL
    case 34: bs = 256; bb = 56; return;  // TQ1_0 (the PrismML block)
    case 35: bs = 256; bb = 70; return;  // TQ2_0
    case 142: bs = 256; bb = 70; return; // PQ2_0
    case 143: bs = 256; bb = 56; return; // PrismML TQ1_0
    default: bs = 1; bb = 1; return;     // unlisted types: one byte per element, as the reference
  }
}

struct Tensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t shape[4] = {0, 0, 0, 0};
  uint32_t type = 0;
  uint64_t offset = 0, abs_offset = 0, size_bytes = 0;
  const uint8_t* data = nullptr;
};

}  // namespace

struct hq_gguf {
  void* map = nullptr;  // mmap of a file (null when parsing caller memory)
  size_t map_bytes = 0;
  const uint8_t* base = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint64_t tensor_count = 0, kv_count = 0, alignment = 32, header_bytes = 0, data_offset = 0, total_tensor_bytes = 0;
  std::unordered_map<std::string, Value> meta;
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> by_name;
};

namespace {

hq_status parse(hq_gguf* g) {
  if (!g->base || g->size < 24) return hq_set_error(HQ_ERR_FORMAT, "invalid or truncated GGUF data (%zu bytes < 24)", g->size);
  Reader r{g->base, g->size};
  if (r.pod<uint32_t>() != 0x46554747u) return hq_set_error(HQ_ERR_FORMAT, "invalid GGUF magic (expected 'GGUF')");
  g->version = r.pod<uint32_t>();
  if (g->version < 2 || g->version > 3) return hq_set_error(HQ_ERR_FORMAT, "unsupported GGUF version %u", g->version);
  g->tensor_count = r.pod<uint64_t>();
  g->kv_count = r.pod<uint64_t>();
  // Every key needs at least 12 bytes and every tensor info 24: counts beyond the data are malformed.
  if (g->kv_count > g->size / 12 || g->tensor_count > g->size / 24)
    return hq_set_error(HQ_ERR_FORMAT, "GGUF counts (%llu keys, %llu tensors) exceed the data",
                        (unsigned long long)g->kv_count, (unsigned long long)g->tensor_count);
  for (uint64_t i = 0; i < g->kv_count && r.err.empty(); ++i) {
    std::string key = r.str();
    const uint32_t t = r.pod<uint32_t>();
    Value v;
    r.value(t, v);
    if (r.err.empty()) g->meta[std::move(key)] = std::move(v);
  }
  if (!r.err.empty()) return hq_set_error(HQ_ERR_FORMAT, "%s", r.err.c_str());
  auto al = g->meta.find("general.alignment");
  g->alignment = al != g->meta.end() && al->second.type != kString && al->second.type != kArray ? al->second.u : 32u;
  if (g->alignment == 0) g->alignment = 32;
  g->tensors.reserve((size_t)g->tensor_count);
  for (uint64_t i = 0; i < g->tensor_count && r.err.empty(); ++i) {
    Tensor t;
    t.name = r.str();
    t.n_dims = r.pod<uint32_t>();
    if (r.err.empty() && t.n_dims > 4)
      return hq_set_error(HQ_ERR_FORMAT, "tensor %s has %u dimensions (at most 4)", t.name.c_str(), t.n_dims);
    for (uint32_t d = 0; d < t.n_dims; ++d) t.shape[d] = r.pod<uint64_t>();
    t.type = r.pod<uint32_t>();
    t.offset = r.pod<uint64_t>();
    uint64_t elems = t.n_dims ? 1 : 0;
    for (uint32_t d = 0; d < t.n_dims; ++d) elems *= t.shape[d];
    uint64_t bs = 1, bb = 1;
    type_traits(t.type, bs, bb);
    t.size_bytes = elems / bs * bb;
    g->tensors.push_back(std::move(t));
  }
  if (!r.err.empty()) return hq_set_error(HQ_ERR_FORMAT, "%s", r.err.c_str());
  g->header_bytes = r.cur;
  g->data_offset = (r.cur + g->alignment - 1) / g->alignment * g->alignment;
  uint64_t extent = 0;
  for (size_t i = 0; i < g->tensors.size(); ++i) {
    Tensor& t = g->tensors[i];
    t.abs_offset = g->data_offset + t.offset;
    const bool inside = t.abs_offset >= g->data_offset && t.abs_offset <= g->size && t.size_bytes <= g->size - t.abs_offset;
    t.data = inside ? g->base + t.abs_offset : nullptr;
    g->by_name[t.name] = i;
    if (t.offset + t.size_bytes > extent) extent = t.offset + t.size_bytes;
  }
  g->total_tensor_bytes = extent;
  return HQ_OK;
}

void fill_info(const Tensor& t, hq_gguf_tensor_info* o) {
  o->name = t.name.c_str();
  o->n_dims = t.n_dims;
  for (int d = 0; d < 4; ++d) o->shape[d] = t.shape[d];
  o->type = t.type;
  o->offset = t.offset;
  o->absolute_offset = t.abs_offset;
  o->size_bytes = t.size_bytes;
  o->data = t.data;
}

const Tensor* find(const hq_gguf* g, const char* name) {
  auto it = g->by_name.find(name);
  return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

// A 2-D tensor of K inputs (shape[0]) and N output rows (shape[1]) of the given block type.
hq_status check_matrix(const hq_gguf* g, const char* name, bool (*type_ok)(uint32_t), const char* what,
                       const Tensor** out) {
  if (!g || !name) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  const Tensor* t = find(g, name);
  if (!t) return hq_set_error(HQ_ERR_NOT_FOUND, "no tensor named %s", name);
  if (!type_ok(t->type)) return hq_set_error(HQ_ERR_UNSUPPORTED, "tensor %s has type %u, not %s", name, t->type, what);
  if (t->n_dims != 2 || t->shape[0] == 0 || t->shape[1] == 0 || t->shape[0] > 0xFFFFFFFFu || t->shape[1] > 0xFFFFFFFFu)
    return hq_set_error(HQ_ERR_SHAPE, "tensor %s is not a 2-D [K, N] matrix", name);
  if (t->shape[0] % 256) return hq_set_error(HQ_ERR_SHAPE, "tensor %s: K=%llu must be a multiple of 256", name,
                                             (unsigned long long)t->shape[0]);
  if (!t->data) return hq_set_error(HQ_ERR_FORMAT, "tensor %s extends past the end of the file", name);
  *out = t;
  return HQ_OK;
}

bool is_tq1_0(uint32_t type) { return type == 34u || type == 143u; }
bool is_q4_k(uint32_t type) { return type == 12u; }

// ---- GGML Q4_K (the published block_q4_K): per 256 weights, fp16 d and dmin, 12 bytes of
// 6-bit sub-block scales and mins, 128 bytes of 4-bit codes. Sub-block j (32 weights) has scale
// d * sc_j and min dmin * m_j, weight = d * sc_j * q - dmin * m_j; codes of weights 64 c + l
// and 64 c + 32 + l (l < 32) are the low and high nibble of byte 32 c + l.
constexpr uint32_t kQ4kBytes = 144;
inline void q4k_scale_min(uint32_t j, const uint8_t* s, uint32_t& sc, uint32_t& m) {
  if (j < 4) {
    sc = s[j] & 63u;
    m = s[j + 4] & 63u;
  } else {
    sc = (s[j + 4] & 15u) | ((s[j - 4] >> 6) << 4);
    m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}
inline float h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31u, m = h & 1023u;
  uint32_t b;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f;  // m * 2^-24, exact
    std::memcpy(&b, &v, 4);
    b |= sign;
  } else if (e == 31) {
    b = sign | 0x7F800000u | (m << 13);
  } else {
    b = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  std::memcpy(&f, &b, 4);
  return f;
}
inline uint16_t f2h(float f) {  // round to nearest even
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, a = x & 0x7FFFFFFFu;
  if (a >= 0x7F800000u) return (uint16_t)(sign | (a > 0x7F800000u ? 0x7E00u : 0x7C00u));
  if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
  if (a < 0x38800000u) {
    if (a <= 0x33000000u) return (uint16_t)sign;
    const uint32_t e = a >> 23, mm = (a & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
    uint32_t q = mm >> sh;
    const uint32_t rem = mm & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
  }
  uint32_t q = (((a >> 23) - 112u) << 10) | ((a >> 13) & 0x3FFu);
  const uint32_t rem = a & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
  return (uint16_t)(sign | q);
}

}  // namespace

extern "C" {

hq_status hq_gguf_parse(const void* data, size_t bytes, hq_gguf** out) {
  if (!out) return hq_set_error(HQ_ERR_INVALID_ARG, "out is null");
  *out = nullptr;
  if (!data) return hq_set_error(HQ_ERR_INVALID_ARG, "data is null");
  hq_gguf* g = new hq_gguf();
  g->base = static_cast<const uint8_t*>(data);
  g->size = bytes;
  const hq_status st = parse(g);
  if (st != HQ_OK) {
    delete g;
    return st;
  }
  *out = g;
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_open(const char* path, hq_gguf** out) {
  if (!out || !path) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  *out = nullptr;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) return hq_set_error(HQ_ERR_IO, "cannot open %s: %s", path, std::strerror(errno));
  struct stat st {};
  if (fstat(fd, &st) != 0) {
    const int e = errno;
    ::close(fd);
    return hq_set_error(HQ_ERR_IO, "cannot stat %s: %s", path, std::strerror(e));
  }
  const size_t bytes = (size_t)st.st_size;
  void* map = bytes ? mmap(nullptr, bytes, PROT_READ, MAP_PRIVATE, fd, 0) : nullptr;
  const int e = errno;
  ::close(fd);
  if (bytes && map == MAP_FAILED) return hq_set_error(HQ_ERR_IO, "cannot map %s: %s", path, std::strerror(e));
  if (bytes) (void)madvise(map, bytes, MADV_SEQUENTIAL);
  hq_gguf* g = new hq_gguf();
  g->map = bytes ? map : nullptr;
  g->map_bytes = bytes;
  g->base = static_cast<const uint8_t*>(g->map);
  g->size = bytes;
  const hq_status s = parse(g);
  if (s != HQ_OK) {
    hq_gguf_close(g);
    return s;
  }
  *out = g;
  return hq_set_error(HQ_OK, "");
}

void hq_gguf_close(hq_gguf* g) {
  if (!g) return;
  if (g->map) munmap(g->map, g->map_bytes);
  delete g;
}

hq_status hq_gguf_header(const hq_gguf* g, hq_gguf_header_info* out) {
  if (!g || !out) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  out->version = g->version;
  out->tensor_count = g->tensor_count;
  out->kv_count = g->kv_count;
  out->alignment = g->alignment;
  out->header_bytes = g->header_bytes;
  out->tensor_data_offset = g->data_offset;
  out->total_tensor_bytes = g->total_tensor_bytes;
  out->file_bytes = g->size;
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_tensor_at(const hq_gguf* g, uint64_t index, hq_gguf_tensor_info* out) {
  if (!g || !out) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  if (index >= g->tensors.size())
    return hq_set_error(HQ_ERR_NOT_FOUND, "tensor index %llu >= %zu", (unsigned long long)index, g->tensors.size());
  fill_info(g->tensors[(size_t)index], out);
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_find_tensor(const hq_gguf* g, const char* name, hq_gguf_tensor_info* out) {
  if (!g || !name || !out) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  const Tensor* t = find(g, name);
  if (!t) return hq_set_error(HQ_ERR_NOT_FOUND, "no tensor named %s", name);
  fill_info(*t, out);
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_get_int(const hq_gguf* g, const char* key, int64_t* out) {
  if (!g || !key || !out) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  auto it = g->meta.find(key);
  if (it == g->meta.end()) return hq_set_error(HQ_ERR_NOT_FOUND, "no metadata key %s", key);
  const Value& v = it->second;
  if (v.type == kString || v.type == kArray || v.type == kF32 || v.type == kF64)
    return hq_set_error(HQ_ERR_INVALID_ARG, "metadata %s is not an integer (type %u)", key, v.type);
  *out = v.type == kBool ? (int64_t)v.u : v.i;
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_get_float(const hq_gguf* g, const char* key, double* out) {
  if (!g || !key || !out) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  auto it = g->meta.find(key);
  if (it == g->meta.end()) return hq_set_error(HQ_ERR_NOT_FOUND, "no metadata key %s", key);
  if (it->second.type != kF32 && it->second.type != kF64)
    return hq_set_error(HQ_ERR_INVALID_ARG, "metadata %s is not a float (type %u)", key, it->second.type);
  *out = it->second.f;
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_get_string(const hq_gguf* g, const char* key, char* buf, size_t buf_len, size_t* len) {
  if (!g || !key) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  auto it = g->meta.find(key);
  if (it == g->meta.end()) return hq_set_error(HQ_ERR_NOT_FOUND, "no metadata key %s", key);
  if (it->second.type != kString) return hq_set_error(HQ_ERR_INVALID_ARG, "metadata %s is not a string", key);
  const std::string& s = it->second.s;
  if (len) *len = s.size();
  if (buf && buf_len) {
    const size_t n = s.size() < buf_len - 1 ? s.size() : buf_len - 1;
    std::memcpy(buf, s.data(), n);
    buf[n] = 0;
  }
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_get_array(const hq_gguf* g, const char* key, uint32_t* elem_type, uint64_t* count) {
  if (!g || !key || !elem_type || !count) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  auto it = g->meta.find(key);
  if (it == g->meta.end()) return hq_set_error(HQ_ERR_NOT_FOUND, "no metadata key %s", key);
  if (it->second.type != kArray) return hq_set_error(HQ_ERR_INVALID_ARG, "metadata %s is not an array", key);
  *elem_type = it->second.arr_type;
  *count = it->second.arr_count;
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_load_tq1_0(const hq_gguf* g, const char* name, void* d_staging, size_t staging_bytes,
                             uint32_t* d_packed, uint16_t* d_scales, uint32_t* K, uint32_t* N, hq_stream stream) {
  const Tensor* t = nullptr;
  hq_status st = check_matrix(g, name, is_tq1_0, "TQ1_0 (type 34 or 143)", &t);
  if (st != HQ_OK) return st;
  if (!d_staging || !d_packed || !d_scales || !K || !N) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  if (staging_bytes < t->size_bytes)
    return hq_set_error(HQ_ERR_WORKSPACE, "staging buffer of %zu bytes < the tensor's %llu", staging_bytes,
                        (unsigned long long)t->size_bytes);
  const uint32_t k = (uint32_t)t->shape[0], n = (uint32_t)t->shape[1];
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const hipError_t e = hipMemcpyAsync(d_staging, t->data, t->size_bytes, hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return hq_set_error(HQ_ERR_DEVICE, "hipMemcpyAsync: %s", hipGetErrorString(e));
  st = hq_repack_tq1_0_device(d_staging, k, n, d_packed, d_scales, stream);
  if (st != HQ_OK) return st;
  *K = k;
  *N = n;
  return hq_set_error(HQ_OK, "");
}

hq_status hq_convert_q4_k(const void* blocks, uint32_t K, uint32_t N, uint32_t* codes_linear, uint16_t* scales,
                          float* bias) {
  if (!blocks || !codes_linear || !scales || !bias) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  if (K == 0 || N == 0 || K % 256) return hq_set_error(HQ_ERR_SHAPE, "K=%u must be a positive multiple of 256, N=%u > 0", K, N);
  const uint32_t nb = K / 256;
  const uint8_t* src = static_cast<const uint8_t*>(blocks);
  auto work = [=](uint32_t n0, uint32_t n1) {
    for (uint32_t n = n0; n < n1; ++n)
      for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t* p = src + ((size_t)n * nb + b) * kQ4kBytes;
        const float d = h2f((uint16_t)(p[0] | (p[1] << 8))), dmin = h2f((uint16_t)(p[2] | (p[3] << 8)));
        const uint8_t* sm = p + 4;
        const uint8_t* qs = p + 16;
        for (uint32_t j = 0; j < 8; ++j) {  // sub-block j: weights 256 b + 32 j .. + 31
          uint32_t sc, m;
          q4k_scale_min(j, sm, sc, m);
          const size_t row = (size_t)b * 8 + j;  // group of 32
          scales[row * N + n] = f2h(d * (float)sc);
          bias[row * N + n] = -(dmin * (float)m);
          const uint8_t* q = qs + 32 * (j / 2);
          const uint32_t shift = (j & 1) ? 4u : 0u;
          for (uint32_t w = 0; w < 4; ++w) {  // four linear words of 8 codes
            uint32_t lin = 0;
            for (uint32_t i = 0; i < 8; ++i) lin |= (uint32_t)((q[8 * w + i] >> shift) & 15u) << (4 * i);
            codes_linear[((size_t)b * 32 + j * 4 + w) * N + n] = lin;
          }
        }
      }
  };
  unsigned nt = std::thread::hardware_concurrency();
  nt = nt == 0 ? 1 : (nt > 16 ? 16 : nt);
  if ((uint64_t)N * K < (1u << 20) || nt == 1) {
    work(0, N);
  } else {
    std::vector<std::thread> th;
    const uint32_t chunk = (N + nt - 1) / nt;
    for (unsigned i = 0; i < nt; ++i) {
      const uint32_t a = i * chunk, z = a + chunk < N ? a + chunk : N;
      if (a < z) th.emplace_back(work, a, z);
    }
    for (auto& x : th) x.join();
  }
  return hq_set_error(HQ_OK, "");
}

hq_status hq_gguf_convert_q4_k(const hq_gguf* g, const char* name, uint32_t* codes_linear, uint16_t* scales,
                               float* bias, uint32_t* K, uint32_t* N) {
  const Tensor* t = nullptr;
  hq_status st = check_matrix(g, name, is_q4_k, "Q4_K (type 12)", &t);
  if (st != HQ_OK) return st;
  if (!K || !N) return hq_set_error(HQ_ERR_INVALID_ARG, "null pointer");
  st = hq_convert_q4_k(t->data, (uint32_t)t->shape[0], (uint32_t)t->shape[1], codes_linear, scales, bias);
  if (st != HQ_OK) return st;
  *K = (uint32_t)t->shape[0];
  *N = (uint32_t)t->shape[1];
  return HQ_OK;
}

}  // extern "C"
