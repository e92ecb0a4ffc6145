// vdx_gguf.cpp -- GGUF model-file reader for the lm_head's inputs
// (TVdxGGUFReader, src/VindexLLM.GGUFReader.pas): the file is memory-mapped
// read-only and its header, metadata and tensor directory are parsed so the
// caller can find `token_embd.weight` (the tied lm_head, Model.Gemma3.pas:
// 180-198), `output_norm.weight` (:174) and the model dimensions, and hand the
// tensor bytes, still in their GGUF layout, to vdx_lmhead.
//
// File layout (GGUF v2/v3, little endian), as the reader parses it
// (GGUFReader.pas:605-745): magic "GGUF" (0x46554747), u32 version (>= 2),
// u64 tensor count, u64 metadata count; metadata entries (string key, u32
// value type, value; strings are u64 length + bytes, arrays u32 element type
// + u64 length + elements); tensor infos (string name, u32 n_dims, n_dims x
// u64 dims, u32 GGML type, u64 offset relative to the data section); the data
// section starts at the next multiple of general.alignment (default 32).
// Tensor byte sizes follow VdxGGMLTensorBytes (GGUFReader.pas:264-318).
//
// Every read is bounds-checked against the mapping; a malformed file is an
// error, never a fault.  Messages start with the reference's error codes
// (GGUFReader.pas:24-30: GG01 parse, GG02 magic, GG03 version, GG04 metadata
// key, GG05 tensor; VirtualFile.pas:27-32: VF02 open, VF03 map, VF06 empty).
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <strings.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "vdx_sampler.h"

namespace {

struct Meta {
  uint32_t type = 0;       // GGUF value type
  uint64_t u = 0;          // unsigned / bool
  int64_t i = 0;           // signed
  double f = 0.0;          // float
  std::string s;           // string
  uint32_t arr_type = 0;   // arrays: element type and count (elements not kept)
  uint64_t arr_len = 0;
};

struct Tensor {
  std::string name;
  uint32_t n_dims = 0;
  uint64_t dims[4] = {1, 1, 1, 1};
  uint32_t type = 0;
  uint64_t offset = 0;
};

// bytes of `elements` values of GGML type `t` (0 when the type is not sized)
uint64_t ggml_bytes(uint32_t t, uint64_t elements) {
  switch (t) {
    case 2: return elements / 32 * 18;    // Q4_0
    case 3: return elements / 32 * 20;    // Q4_1
    case 8: return elements / 32 * 34;    // Q8_0
    case 12: return elements / 256 * 144; // Q4_K
    case 13: return elements / 256 * 176; // Q5_K
    case 14: return elements / 256 * 210; // Q6_K
    case 0: case 26: return elements * 4; // F32, I32
    case 1: case 25: case 30: return elements * 2;  // F16, I16, BF16
    case 24: return elements;             // I8
    case 27: case 28: return elements * 8;  // I64, F64
    default: return 0;
  }
}

}  // namespace

struct vdx_gguf {
  int fd = -1;
  const uint8_t *base = nullptr;
  size_t size = 0;
  uint32_t version = 0;
  uint32_t alignment = 32;
  uint64_t data_start = 0;
  uint64_t meta_count = 0;                // as the header states
  std::unordered_map<std::string, Meta> meta;
  std::vector<std::string> keys;          // distinct keys, file order
  std::vector<Tensor> tensors;
  std::unordered_map<std::string, size_t> by_name;
  std::string err;

  // ---- bounds-checked cursor ----
  size_t cur = 0;
  bool fail = false;
  bool need(uint64_t n) {
    if (fail || n > size || cur > size - n) {
      if (!fail) err = "GG01: gguf: truncated file (read past the end at byte " + std::to_string(cur) + ")";
      fail = true;
      return false;
    }
    return true;
  }
  template <typename T> T rd() {
    T v{};
    if (need(sizeof(T))) {
      memcpy(&v, base + cur, sizeof(T));
      cur += sizeof(T);
    }
    return v;
  }
  std::string rd_str() {
    const uint64_t n = rd<uint64_t>();
    if (!need(n)) return std::string();
    std::string s((const char *)base + cur, (size_t)n);
    cur += n;
    return s;
  }
  bool skip_value(uint32_t t, int depth);
  bool read_value(uint32_t t, Meta &m);
  bool parse();
};

static const uint64_t kScalarBytes[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};

bool vdx_gguf::skip_value(uint32_t t, int depth) {
  if (t > 12 || depth > 4) {
    err = "GG01: gguf: unknown metadata value type " + std::to_string(t);
    fail = true;
    return false;
  }
  if (t == 8) {  // string
    rd_str();
  } else if (t == 9) {  // array
    const uint32_t et = rd<uint32_t>();
    const uint64_t n = rd<uint64_t>();
    if (et <= 12 && et != 8 && et != 9) {
      if (n > size) { err = "GG01: gguf: bad array length"; fail = true; return false; }
      if (need(n * kScalarBytes[et])) cur += (size_t)(n * kScalarBytes[et]);
    } else {
      for (uint64_t k = 0; k < n && !fail; ++k) skip_value(et, depth + 1);
    }
  } else if (need(kScalarBytes[t])) {
    cur += kScalarBytes[t];
  }
  return !fail;
}

bool vdx_gguf::read_value(uint32_t t, Meta &m) {
  m.type = t;
  switch (t) {
    case 0: m.u = rd<uint8_t>(); break;
    case 1: m.i = rd<int8_t>(); break;
    case 2: m.u = rd<uint16_t>(); break;
    case 3: m.i = rd<int16_t>(); break;
    case 4: m.u = rd<uint32_t>(); break;
    case 5: m.i = rd<int32_t>(); break;
    case 6: m.f = rd<float>(); break;
    case 7: m.u = rd<uint8_t>() ? 1u : 0u; break;
    case 8: m.s = rd_str(); break;
    case 9: {
      const size_t at = cur;
      m.arr_type = rd<uint32_t>();
      m.arr_len = rd<uint64_t>();
      cur = at;
      skip_value(9, 0);
      break;
    }
    case 10: m.u = rd<uint64_t>(); break;
    case 11: m.i = rd<int64_t>(); break;
    case 12: m.f = rd<double>(); break;
    default:
      err = "GG01: gguf: unknown metadata value type " + std::to_string(t);
      fail = true;
  }
  if (t == 1 || t == 3 || t == 5 || t == 11) m.u = (uint64_t)m.i;
  if (t == 0 || t == 2 || t == 4 || t == 10 || t == 7) m.i = (int64_t)m.u;
  return !fail;
}

bool vdx_gguf::parse() {
  cur = 0;
  if (rd<uint32_t>() != 0x46554747u) {
    if (!fail) err = "GG02: gguf: bad magic (not a GGUF file)";
    return false;
  }
  version = rd<uint32_t>();
  if (!fail && version < 2) {
    err = "GG03: gguf: unsupported version " + std::to_string(version) + " (need >= 2)";
    return false;
  }
  const uint64_t nt = rd<uint64_t>(), nm = rd<uint64_t>();
  if (fail) return false;
  meta_count = nm;
  if (nt > size / 8 || nm > size / 8) {
    err = "GG01: gguf: implausible tensor or metadata count";
    return false;
  }
  for (uint64_t k = 0; k < nm && !fail; ++k) {
    std::string key = rd_str();
    const uint32_t t = rd<uint32_t>();
    Meta m;
    if (!read_value(t, m)) break;
    // the override is read as an unsigned value; any other type reads as 0
    // and so as the default (GGUFReader.pas:657-663)
    if (strcasecmp(key.c_str(), "general.alignment") == 0) {
      const bool unsigned_type = t == 0 || t == 2 || t == 4 || t == 10;
      alignment = unsigned_type ? (uint32_t)m.u : 0u;
      if (alignment == 0) alignment = 32;
    }
    auto it = meta.find(key);
    if (it == meta.end()) {
      keys.push_back(key);
      meta.emplace(std::move(key), std::move(m));
    } else {
      it->second = std::move(m);  // a repeated key keeps the last value
    }
  }
  if (fail) return false;
  tensors.reserve((size_t)nt);
  for (uint64_t k = 0; k < nt && !fail; ++k) {
    Tensor t;
    t.name = rd_str();
    t.n_dims = rd<uint32_t>();
    if (!fail && (t.n_dims == 0 || t.n_dims > 4)) {
      err = "GG01: gguf: tensor '" + t.name + "' has " + std::to_string(t.n_dims) + " dimensions";
      fail = true;
      break;
    }
    for (uint32_t d = 0; d < t.n_dims; ++d) t.dims[d] = rd<uint64_t>();
    t.type = rd<uint32_t>();
    t.offset = rd<uint64_t>();
    by_name[t.name] = tensors.size();
    tensors.push_back(std::move(t));
  }
  if (fail) return false;
  data_start = ((uint64_t)cur + alignment - 1) / alignment * alignment;
  if (data_start > size) {
    err = "GG01: gguf: data section starts past the end of the file";
    return false;
  }
  return true;
}

static thread_local std::string g_gguf_err;

extern "C" {

int vdx_gguf_open(vdx_gguf **out, const char *path) {
  if (!out || !path) return VDX_E_INVALID_ARG;
  *out = nullptr;
  vdx_gguf *g = new vdx_gguf();
  g->fd = ::open(path, O_RDONLY);
  struct stat st {};
  if (g->fd < 0 || fstat(g->fd, &st) != 0 || st.st_size <= 0) {
    // error codes of the reference's file layer (VirtualFile.pas:27-32)
    g_gguf_err = (g->fd >= 0 && st.st_size == 0 ? std::string("VF06: gguf: empty file ")
                                                : std::string("VF02: gguf: cannot open ")) + path;
    vdx_gguf_close(g);
    return VDX_E_INVALID_ARG;
  }
  g->size = (size_t)st.st_size;
  void *p = mmap(nullptr, g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
  if (p == MAP_FAILED) {
    g_gguf_err = std::string("VF03: gguf: cannot map ") + path;
    g->base = nullptr;
    vdx_gguf_close(g);
    return VDX_E_NO_MEMORY;
  }
  g->base = (const uint8_t *)p;
  if (!g->parse()) {
    g_gguf_err = g->err;
    vdx_gguf_close(g);
    return VDX_E_INVALID_ARG;
  }
  g_gguf_err.clear();
  *out = g;
  return VDX_OK;
}

void vdx_gguf_close(vdx_gguf *g) {
  if (!g) return;
  if (g->base) munmap((void *)g->base, g->size);
  if (g->fd >= 0) ::close(g->fd);
  delete g;
}

const char *vdx_gguf_last_error(const vdx_gguf *g) { return g ? g->err.c_str() : g_gguf_err.c_str(); }

int vdx_gguf_get_info(const vdx_gguf *g, vdx_gguf_info *out) {
  if (!g || !out) return VDX_E_INVALID_ARG;
  out->version = g->version;
  out->alignment = g->alignment;
  out->tensor_count = g->tensors.size();
  out->metadata_count = g->meta_count;
  out->file_size = g->size;
  out->data_offset = g->data_start;
  return VDX_OK;
}

static int copy_out(const std::string &s, char *buf, int32_t cap) {
  const size_t k = s.size() < (size_t)(cap - 1) ? s.size() : (size_t)(cap - 1);
  memcpy(buf, s.data(), k);
  buf[k] = '\0';
  return (int)s.size();
}

int vdx_gguf_tensor_name(const vdx_gguf *g, int64_t index, char *buf, int32_t cap) {
  if (!g || index < 0 || index >= (int64_t)g->tensors.size() || !buf || cap <= 0) return VDX_E_INVALID_ARG;
  return copy_out(g->tensors[(size_t)index].name, buf, cap);
}

int vdx_gguf_meta_key(const vdx_gguf *g, int64_t index, char *buf, int32_t cap) {
  if (!g || index < 0 || index >= (int64_t)g->keys.size() || !buf || cap <= 0) return VDX_E_INVALID_ARG;
  return copy_out(g->keys[(size_t)index], buf, cap);
}

int vdx_gguf_meta_type(const vdx_gguf *g, const char *key) {
  if (!g || !key) return VDX_E_INVALID_ARG;
  auto it = g->meta.find(key);
  return it == g->meta.end() ? VDX_E_INVALID_ARG : (int)it->second.type;
}

int vdx_gguf_find_tensor(vdx_gguf *g, const char *name, vdx_gguf_tensor *out) {
  if (!g || !name || !out) return VDX_E_INVALID_ARG;
  auto it = g->by_name.find(name);
  if (it == g->by_name.end()) {
    g->err = std::string("GG05: gguf: tensor '") + name + "' not found";
    return VDX_E_INVALID_ARG;
  }
  const Tensor &t = g->tensors[it->second];
  // element count and byte size must not wrap (the caller trusts the dims)
  uint64_t elements = 1;
  bool wrap = false;
  for (uint32_t d = 0; d < t.n_dims; ++d) wrap |= __builtin_mul_overflow(elements, t.dims[d], &elements);
  wrap |= elements > (UINT64_MAX >> 4);
  const uint64_t nb = wrap ? 0 : ggml_bytes(t.type, elements);
  out->type = (int32_t)t.type;
  out->n_dims = (int32_t)t.n_dims;
  for (int d = 0; d < 4; ++d) out->dims[d] = t.dims[d];
  out->nbytes = nb;
  out->file_offset = g->data_start + t.offset;
  out->data = nullptr;
  if (wrap || t.offset > g->size - g->data_start || nb > g->size - g->data_start - t.offset) {
    g->err = std::string("GG05: gguf: tensor '") + name + "' extends past the end of the file";
    return VDX_E_UNSUPPORTED;
  }
  out->data = g->base + g->data_start + t.offset;
  return VDX_OK;
}

int vdx_gguf_meta_int(vdx_gguf *g, const char *key, int64_t *out) {
  if (!g || !key || !out) return VDX_E_INVALID_ARG;
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type == 6 || it->second.type == 8 || it->second.type == 9 ||
      it->second.type == 12) {
    g->err = std::string("GG04: gguf: no integer metadata '") + key + "'";
    return VDX_E_INVALID_ARG;
  }
  *out = it->second.i;
  return VDX_OK;
}

int vdx_gguf_meta_float(vdx_gguf *g, const char *key, double *out) {
  if (!g || !key || !out) return VDX_E_INVALID_ARG;
  auto it = g->meta.find(key);
  if (it == g->meta.end() || (it->second.type != 6 && it->second.type != 12)) {
    g->err = std::string("GG04: gguf: no float metadata '") + key + "'";
    return VDX_E_INVALID_ARG;
  }
  *out = it->second.f;
  return VDX_OK;
}

int vdx_gguf_meta_string(vdx_gguf *g, const char *key, char *buf, int32_t cap) {
  if (!g || !key || !buf || cap <= 0) return VDX_E_INVALID_ARG;
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type != 8) {
    g->err = std::string("GG04: gguf: no string metadata '") + key + "'";
    return VDX_E_INVALID_ARG;
  }
  return copy_out(it->second.s, buf, cap);
}

int vdx_gguf_meta_array(vdx_gguf *g, const char *key, int32_t *elem_type, int64_t *length) {
  if (!g || !key || !elem_type || !length) return VDX_E_INVALID_ARG;
  auto it = g->meta.find(key);
  if (it == g->meta.end() || it->second.type != 9) {
    g->err = std::string("GG04: gguf: no array metadata '") + key + "'";
    return VDX_E_INVALID_ARG;
  }
  *elem_type = (int32_t)it->second.arr_type;
  *length = (int64_t)it->second.arr_len;
  return VDX_OK;
}

}  // extern "C"
