// Read-only GGUF v2/v3 parser for the expert tensors (engine/src/gguf.rs,
// engine/src/model.rs:28-104): the file is memory-mapped, the metadata
// key-value section is walked (values skipped by type), the tensor infos
// are read, and the data section starts at the next 32-byte boundary.  Tensor
// data is handed out as host pointers into the mapping; the caller uploads
// what it needs to the device.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>
#include <string>
#include <vector>

#include "dsmoe.h"

namespace dsm_gguf {
int fail(int code, const std::string& msg);  // dsmoe_host.cpp: sets dsmoe_last_error
}

struct dsmoe_gguf {
  const uint8_t* map = nullptr;
  size_t size = 0;
  uint64_t data_offset = 0;
  size_t kv_start = 0;
  uint64_t n_kv = 0;
  struct Tensor {
    std::string name;
    int32_t type;
    std::vector<uint64_t> dims;
    uint64_t offset;
    uint64_t bytes;
  };
  std::vector<Tensor> tensors;
};

namespace {

using dsm_gguf::fail;

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF", little-endian

// Bytes of n elements of GGUF type `t` (model.rs:54-85), or 0 for a type the
// engine does not know.
// The products are checked: a count whose byte size does not fit 64 bits
// gives UINT64_MAX, which no file can hold.
uint64_t type_bytes(int32_t t, uint64_t n) {
  uint64_t per = 0, blk = 1;
  switch (t) {
    case DSMOE_GGUF_F32: per = 4; break;
    case DSMOE_GGUF_F16: per = 2; break;
    case DSMOE_GGUF_Q8_0: per = 34; blk = 32; break;
    case DSMOE_GGUF_Q2_K: per = 84; blk = 256; break;
    case DSMOE_GGUF_Q4_K: per = 144; blk = 256; break;
    case DSMOE_GGUF_IQ2_XXS: per = 66; blk = 256; break;
    case DSMOE_GGUF_I32: per = 4; break;
    default: return 0;
  }
  const uint64_t blocks = n / blk + (n % blk != 0);
  uint64_t bytes = 0;
  if (__builtin_mul_overflow(blocks, per, &bytes)) return UINT64_MAX;
  return bytes;
}
bool known_type(uint32_t t) { return t == 0 || t == 1 || t == 8 || t == 10 || t == 12 || t == 16 || t == 26; }

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
  const uint8_t* p;
  size_t n, at = 0;
  bool ok = true;
  bool need(size_t k) {
    if (!ok || k > n - at) ok = false;
    return ok;
  }
  uint32_t u32() {
    uint32_t v = 0;
    if (need(4)) { memcpy(&v, p + at, 4); at += 4; }
    return v;
  }
  uint64_t u64() {
    uint64_t v = 0;
    if (need(8)) { memcpy(&v, p + at, 8); at += 8; }
    return v;
  }
  std::string str() {
    const uint64_t len = u64();
    if (!need(len)) return std::string();
    std::string s((const char*)p + at, (size_t)len);
    at += len;
    return s;
  }
  void skip(size_t k) {
    if (need(k)) at += k;
  }
};

// Skips one metadata value of type `vt` (gguf.rs:202-260); false on an
// unknown type.
bool skip_value(Cursor& c, uint32_t vt, int depth = 0) {
  switch (vt) {
    case 0: case 1: case 7: c.skip(1); return c.ok;
    case 2: case 3: c.skip(2); return c.ok;
    case 4: case 5: case 6: c.skip(4); return c.ok;
    case 10: case 11: case 12: c.skip(8); return c.ok;
    case 8: { const uint64_t len = c.u64(); c.skip(len); return c.ok; }
    case 9: {
      if (depth > 4) return false;
      const uint32_t et = c.u32();
      const uint64_t count = c.u64();
      for (uint64_t i = 0; i < count && c.ok; i++)
        if (!skip_value(c, et, depth + 1)) return false;
      return c.ok;
    }
    default: return false;
  }
}

void fill(const dsmoe_gguf* g, const dsmoe_gguf::Tensor& t, dsmoe_gguf_tensor* out) {
  out->name = t.name.c_str();
  out->type = t.type;
  out->n_dims = (int32_t)t.dims.size();
  for (int i = 0; i < 4; i++) out->dims[i] = i < (int)t.dims.size() ? t.dims[i] : 1;
  out->offset = t.offset;
  out->bytes = t.bytes;
  out->data = g->map + g->data_offset + t.offset;
}

}  // namespace

extern "C" {

int dsmoe_gguf_open(const char* path, dsmoe_gguf** out) {
  if (!path || !out) return fail(DSMOE_ERR_INVALID, "gguf_open: null pointer");
  *out = nullptr;
  const int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(DSMOE_ERR_INVALID, std::string("gguf_open: cannot open ") + path);
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    return fail(DSMOE_ERR_INVALID, "gguf_open: not a GGUF file (shorter than its header)");
  }
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m == MAP_FAILED) return fail(DSMOE_ERR_INVALID, "gguf_open: mmap failed");
  dsmoe_gguf* g = new dsmoe_gguf();
  g->map = (const uint8_t*)m;
  g->size = (size_t)st.st_size;
  auto bad = [&](const std::string& msg) {
    dsmoe_gguf_close(g);
    return fail(DSMOE_ERR_INVALID, "gguf_open: " + msg);
  };
  Cursor c{g->map, g->size};
  const uint32_t magic = c.u32();
  if (magic != kMagic) {
    char buf[64];
    snprintf(buf, sizeof buf, "not a GGUF file (bad magic %08x)", magic);
    return bad(buf);
  }
  const uint32_t version = c.u32();
  if (version < 2 || version > 3) return bad("unsupported GGUF version " + std::to_string(version));
  const uint64_t n_tensors = c.u64();
  g->n_kv = c.u64();
  g->kv_start = c.at;
  for (uint64_t i = 0; i < g->n_kv && c.ok; i++) {
    (void)c.str();
    const uint32_t vt = c.u32();
    if (!skip_value(c, vt)) return bad(c.ok ? "unknown GGUF metadata type " + std::to_string(vt) : "truncated metadata");
  }
  if (!c.ok || n_tensors > (g->size - c.at) / 24) return bad("truncated metadata or tensor count past the file");
  g->tensors.reserve((size_t)n_tensors);
  for (uint64_t i = 0; i < n_tensors; i++) {
    dsmoe_gguf::Tensor t;
    t.name = c.str();
    const uint32_t nd = c.u32();
    if (!c.ok || nd > 4) return bad(c.ok ? "tensor '" + t.name + "' has more than 4 dims" : "truncated tensor info");
    uint64_t n = 1;
    bool wrap = false;
    for (uint32_t k = 0; k < nd; k++) {
      t.dims.push_back(c.u64());
      wrap |= __builtin_mul_overflow(n, t.dims.back(), &n);
    }
    const uint32_t ty = c.u32();
    t.offset = c.u64();
    if (!c.ok) return bad("truncated tensor info");
    if (!known_type(ty)) return bad("unknown tensor type " + std::to_string(ty) + " for '" + t.name + "'");
    if (wrap) return bad("tensor '" + t.name + "' has an element count beyond 64 bits");
    t.type = (int32_t)ty;
    t.bytes = type_bytes(t.type, n);
    g->tensors.push_back(std::move(t));
  }
  g->data_offset = ((uint64_t)c.at + 31) & ~(uint64_t)31;
  // data_offset + offset + bytes <= size, written so that nothing can wrap
  for (const auto& t : g->tensors)
    if (g->data_offset > g->size || t.offset > g->size - g->data_offset ||
        t.bytes > g->size - g->data_offset - t.offset)
      return bad("tensor '" + t.name + "' extends past the end of the file");
  *out = g;
  return DSMOE_OK;
}

int dsmoe_gguf_close(dsmoe_gguf* g) {
  if (!g) return DSMOE_OK;
  if (g->map) munmap((void*)g->map, g->size);
  delete g;
  return DSMOE_OK;
}

int64_t dsmoe_gguf_tensor_count(const dsmoe_gguf* g) { return g ? (int64_t)g->tensors.size() : 0; }

uint64_t dsmoe_gguf_data_offset(const dsmoe_gguf* g) { return g ? g->data_offset : 0; }

int dsmoe_gguf_tensor_at(const dsmoe_gguf* g, int64_t i, dsmoe_gguf_tensor* out) {
  if (!g || !out) return fail(DSMOE_ERR_INVALID, "gguf_tensor_at: null pointer");
  if (i < 0 || i >= (int64_t)g->tensors.size()) return fail(DSMOE_ERR_INVALID, "gguf_tensor_at: index out of range");
  fill(g, g->tensors[(size_t)i], out);
  return DSMOE_OK;
}

int dsmoe_gguf_find(const dsmoe_gguf* g, const char* name, dsmoe_gguf_tensor* out) {
  if (!g || !name || !out) return fail(DSMOE_ERR_INVALID, "gguf_find: null pointer");
  for (const auto& t : g->tensors)
    if (t.name == name) {
      fill(g, t, out);
      return DSMOE_OK;
    }
  return fail(DSMOE_ERR_NOT_FOUND, std::string("gguf_find: no tensor '") + name + "'");
}

int dsmoe_gguf_kv_u32(const dsmoe_gguf* g, const char* key, uint32_t* out) {
  if (!g || !key || !out) return fail(DSMOE_ERR_INVALID, "gguf_kv_u32: null pointer");
  Cursor c{g->map, g->size, g->kv_start};
  for (uint64_t i = 0; i < g->n_kv; i++) {
    const std::string k = c.str();
    const uint32_t vt = c.u32();
    if (k == key && vt == 4) {
      *out = c.u32();
      return DSMOE_OK;
    }
    if (!skip_value(c, vt)) break;
  }
  return fail(DSMOE_ERR_NOT_FOUND, std::string("gguf_kv_u32: no u32 key '") + key + "'");
}

int dsmoe_gguf_kv_i32_array(const dsmoe_gguf* g, const char* key, int32_t* out, int64_t cap, int64_t* count) {
  if (!g || !key || !count) return fail(DSMOE_ERR_INVALID, "gguf_kv_i32_array: null pointer");
  Cursor c{g->map, g->size, g->kv_start};
  for (uint64_t i = 0; i < g->n_kv; i++) {
    const std::string k = c.str();
    const uint32_t vt = c.u32();
    if (k == key && vt == 9) {
      const uint32_t et = c.u32();
      const uint64_t n = c.u64();
      if (!c.ok || et != 5) break;  // not an i32 array
      *count = (int64_t)n;
      for (uint64_t j = 0; j < n && c.ok; j++) {
        const uint32_t v = c.u32();
        if (out && (int64_t)j < cap) out[j] = (int32_t)v;
      }
      return c.ok ? DSMOE_OK : fail(DSMOE_ERR_INVALID, "gguf_kv_i32_array: truncated array");
    }
    if (!skip_value(c, vt)) break;
  }
  *count = 0;
  return fail(DSMOE_ERR_NOT_FOUND, std::string("gguf_kv_i32_array: no i32 array key '") + key + "'");
}

int dsmoe_gguf_moe_layer(const dsmoe_gguf* g, int32_t layer, dsmoe_gguf_tensor* out, int32_t* present) {
  if (!g || !out || !present) return fail(DSMOE_ERR_INVALID, "gguf_moe_layer: null pointer");
  // engine.rs:175-187 names (the correction bias under llama.cpp's name)
  static const char* names[DSMOE_GGUF_MOE_TENSORS] = {
      "ffn_gate_inp.weight",   "exp_probs_b.bias",      "ffn_gate_exps.weight",  "ffn_up_exps.weight",
      "ffn_down_exps.weight",  "ffn_gate_shexp.weight", "ffn_up_shexp.weight",   "ffn_down_shexp.weight",
      "ffn_gate_tid2eid.weight", "ffn_norm.weight"};
  *present = 0;
  for (int i = 0; i < DSMOE_GGUF_MOE_TENSORS; i++) {
    const std::string n = "blk." + std::to_string(layer) + "." + names[i];
    memset(&out[i], 0, sizeof out[i]);
    for (const auto& t : g->tensors)
      if (t.name == n) {
        fill(g, t, &out[i]);
        *present |= 1 << i;
        break;
      }
  }
  return DSMOE_OK;
}

}  // extern "C"
