// lle_model_load_gguf: GGUF v2/v3 parse + upload.
//
// Follows the reference reader (internal/gguf/reader.go): magic 0x46554747, version 2..3,
// u64 counts (:228-240); typed KV values, getters type-switch strictly (:293-342); tensor infos
// {name, u32 n_dims, u64 dims, u32 type, u64 offset}; data section at the next 32-byte
// boundary after the tensor table, `general.alignment` ignored (:266-269);
// ByteSize = nel / blockSize * typeSize (:196-204). Metadata keys and tensor names follow
// LoadBertModel (internal/embed/bert.go:98-104,151-208). The file is memory-mapped for the
// duration of the upload only.
#include <errno.h>
#include <fcntl.h>
#include <stdint.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <map>
#include <string>
#include <vector>

#include "lle_internal.h"

namespace lle {
namespace {

struct Cursor {
  const uint8_t* p;
  const uint8_t* end;
  bool ok = true;
  bool need(size_t n) {
    if (!ok || (size_t)(end - p) < n) ok = false;
    return ok;
  }
  template <class T>
  T get() {
    T v{};
    if (need(sizeof(T))) {
      memcpy(&v, p, sizeof(T));
      p += sizeof(T);
    }
    return v;
  }
  std::string str() {
    uint64_t n = get<uint64_t>();
    if (!need(n)) return std::string();
    std::string s((const char*)p, (size_t)n);
    p += n;
    return s;
  }
};

struct KV {
  uint32_t type = 0;
  uint32_t u32 = 0;
  float f32 = 0.f;
  std::string str;
};

struct TInfo {
  std::vector<uint64_t> dims;
  uint32_t type = 0;
  uint64_t offset = 0;
};

// BlockSize / TypeSize of the reference GGMLType (reader.go:106-194).
bool block_geometry(uint32_t t, uint64_t* bs, uint64_t* ts) {
  static const std::map<uint32_t, std::pair<uint64_t, uint64_t>> g = {
      {0, {1, 4}},    {1, {1, 2}},     {2, {32, 18}},   {3, {32, 20}},   {6, {32, 22}},   {7, {32, 24}},
      {8, {32, 34}},  {9, {32, 36}},   {10, {256, 84}}, {11, {256, 110}}, {12, {256, 144}}, {13, {256, 176}},
      {14, {256, 210}}, {15, {256, 292}}, {24, {1, 1}},  {25, {1, 2}},    {26, {1, 4}},    {27, {1, 8}}};
  auto it = g.find(t);
  if (it == g.end()) return false;
  *bs = it->second.first;
  *ts = it->second.second;
  return true;
}

// Skip (or keep) one typed value (readValue, reader.go:420-456). Arrays of arrays recurse; a
// nesting deeper than kMaxDepth is rejected (each level costs only 12 bytes of file, so a small
// crafted file could otherwise exhaust the stack).
constexpr int kMaxDepth = 16;
bool read_value(Cursor& c, uint32_t t, KV* kv, int depth = 0) {
  switch (t) {
    case 0: case 1: case 7: c.get<uint8_t>(); break;
    case 2: case 3: c.get<uint16_t>(); break;
    case 4: {
      uint32_t v = c.get<uint32_t>();
      if (kv) kv->u32 = v;
      break;
    }
    case 5: c.get<uint32_t>(); break;
    case 6: {
      float v = c.get<float>();
      if (kv) kv->f32 = v;
      break;
    }
    case 8: {
      std::string s = c.str();
      if (kv) kv->str = s;
      break;
    }
    case 9: {
      if (depth >= kMaxDepth) return false;
      uint32_t et = c.get<uint32_t>();
      uint64_t n = c.get<uint64_t>();
      for (uint64_t i = 0; i < n && c.ok; i++)
        if (!read_value(c, et, nullptr, depth + 1)) return false;
      break;
    }
    case 10: case 11: case 12: c.get<uint64_t>(); break;
    default: return false;
  }
  return c.ok;
}

}  // namespace
}  // namespace lle

using namespace lle;

extern "C" int32_t lle_model_load_gguf(const char* path, lle_model** out) {
  if (!path || !out) return fail(LLE_EINVAL, "null argument");
  int fd = open(path, O_RDONLY);
  if (fd < 0) return fail(LLE_EIO, std::string("gguf: open ") + path + ": " + strerror(errno));
  struct stat st;
  if (fstat(fd, &st) != 0) {
    close(fd);
    return fail(LLE_EIO, "gguf: stat failed");
  }
  const size_t size = (size_t)st.st_size;
  // an empty file maps nothing and fails the magic check like any other short file
  static const uint8_t kEmpty[1] = {0};
  void* map = size ? mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0) : (void*)kEmpty;
  close(fd);
  if (map == MAP_FAILED) return fail(LLE_EIO, "gguf: mmap failed");
  struct Unmap {
    void* p;
    size_t n;
    ~Unmap() {
      if (n) munmap(p, n);
    }
  } unmap{map, size};

  Cursor c{(const uint8_t*)map, (const uint8_t*)map + size};
  const uint32_t magic = c.get<uint32_t>();
  if (!c.ok || magic != 0x46554747u) {
    char b[96];
    snprintf(b, sizeof(b), "gguf: invalid magic: 0x%08x (expected 0x%08x)", magic, 0x46554747u);
    return fail(LLE_EIO, b);
  }
  const uint32_t version = c.get<uint32_t>();
  if (version < 2 || version > 3) return fail(LLE_EIO, "gguf: unsupported version: " + std::to_string(version));
  const uint64_t n_t = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
  if (!c.ok) return fail(LLE_EIO, "gguf: reading header: truncated");
  std::map<std::string, KV> kvs;
  for (uint64_t i = 0; i < n_kv; i++) {
    KV kv;
    std::string key = c.str();
    kv.type = c.get<uint32_t>();
    if (!c.ok || !read_value(c, kv.type, &kv)) return fail(LLE_EIO, "gguf: reading KV pair " + std::to_string(i));
    kvs.emplace(key, kv);  // first occurrence wins, as GetKV's linear scan does
  }
  std::map<std::string, TInfo> tensors;
  for (uint64_t i = 0; i < n_t; i++) {
    TInfo ti;
    std::string name = c.str();
    const uint32_t nd = c.get<uint32_t>();
    if (!c.ok || nd > 8) return fail(LLE_EIO, "gguf: reading tensor " + std::to_string(i));
    for (uint32_t d = 0; d < nd; d++) ti.dims.push_back(c.get<uint64_t>());
    ti.type = c.get<uint32_t>();
    ti.offset = c.get<uint64_t>();
    if (!c.ok) return fail(LLE_EIO, "gguf: reading tensor " + std::to_string(i));
    tensors.emplace(name, ti);
  }
  const uint64_t pos = (uint64_t)(c.p - (const uint8_t*)map);
  const uint64_t data_off = (pos + 31) & ~(uint64_t)31;

  auto u32 = [&](const char* k) -> uint32_t {
    auto it = kvs.find(k);
    return (it != kvs.end() && it->second.type == 4) ? it->second.u32 : 0u;
  };
  auto f32 = [&](const char* k) -> float {
    auto it = kvs.find(k);
    return (it != kvs.end() && it->second.type == 6) ? it->second.f32 : 0.f;
  };
  lle_model_desc d;
  memset(&d, 0, sizeof(d));
  d.n_layer = (int32_t)u32("nomic-bert.block_count");
  d.d_model = (int32_t)u32("nomic-bert.embedding_length");
  d.d_ff = (int32_t)u32("nomic-bert.feed_forward_length");
  d.n_head = (int32_t)u32("nomic-bert.attention.head_count");
  d.max_seq = (int32_t)u32("nomic-bert.context_length");
  const float eps = f32("nomic-bert.attention.layer_norm_epsilon");
  const float base = f32("nomic-bert.rope.freq_base");
  memcpy(&d.ln_eps_bits, &eps, 4);
  memcpy(&d.rope_base_bits, &base, 4);
  if (d.n_layer == 0 || d.d_model == 0) return fail(LLE_EINVAL, "embed: missing model params in GGUF metadata");
  if (d.n_layer < 0 || d.n_layer > 4096) return fail(LLE_EINVAL, "embed: implausible block_count");

  // The first failing tensor (in LoadBertModel's order) decides the error: a missing name is
  // ENOTFOUND (loadTensor's "tensor %q not found", bert.go:132-136); dims whose element count,
  // row count or byte size overflow, or data outside the file (the reference's mmap slice
  // would panic, bert.go:137-139), are EIO.
  std::string missing;
  int missing_code = LLE_OK;
  auto tensor = [&](const std::string& name) -> lle_tensor {
    lle_tensor t;
    memset(&t, 0, sizeof(t));
    auto bad = [&](int code, const std::string& msg) {
      if (missing_code == LLE_OK) {
        missing_code = code;
        missing = msg;
      }
      return t;
    };
    auto it = tensors.find(name);
    if (it == tensors.end()) return bad(LLE_ENOTFOUND, "tensor \"" + name + "\" not found");
    const TInfo& ti = it->second;
    // NumElements / ByteSize (reader.go:185-204) in checked arithmetic
    uint64_t nel = 1;
    for (uint64_t x : ti.dims)
      if (__builtin_mul_overflow(nel, x, &nel)) return bad(LLE_EIO, "gguf: tensor " + name + ": element count overflows");
    uint64_t bs = 0, ts = 0, bytes = 0;
    if (block_geometry(ti.type, &bs, &ts) && __builtin_mul_overflow(nel / bs, ts, &bytes))
      return bad(LLE_EIO, "gguf: tensor " + name + ": byte size overflows");
    uint64_t off = 0;
    if (__builtin_add_overflow(data_off, ti.offset, &off) || off > size || bytes > size - off)
      return bad(LLE_EIO, "gguf: tensor " + name + ": data past end of file");
    uint64_t ne1 = 1;
    for (size_t k = 1; k < ti.dims.size(); k++) ne1 *= ti.dims[k];  // <= nel: cannot overflow
    const uint64_t ne0 = ti.dims.empty() ? 0 : ti.dims[0];
    if (ne0 > (uint64_t)INT32_MAX || ne1 > (uint64_t)INT32_MAX)
      return bad(LLE_EIO, "gguf: tensor " + name + ": a dimension above 2^31-1");
    t.type = (int32_t)ti.type;
    t.ne0 = (int64_t)ne0;
    t.ne1 = (int64_t)ne1;
    t.data = (const uint8_t*)map + off;
    t.nbytes = (int64_t)bytes;
    return t;
  };
  d.token_embd = tensor("token_embd.weight");
  d.token_types = tensor("token_types.weight");
  d.embd_norm_w = tensor("token_embd_norm.weight");
  d.embd_norm_b = tensor("token_embd_norm.bias");
  const int nl = d.n_layer;
  std::vector<lle_tensor> qkv(nl), o(nl), anw(nl), anb(nl), up(nl), gate(nl), down(nl), onw(nl), onb(nl);
  for (int l = 0; l < nl; l++) {
    const std::string p = "blk." + std::to_string(l) + ".";
    qkv[l] = tensor(p + "attn_qkv.weight");
    o[l] = tensor(p + "attn_output.weight");
    up[l] = tensor(p + "ffn_up.weight");
    gate[l] = tensor(p + "ffn_gate.weight");
    down[l] = tensor(p + "ffn_down.weight");
    anw[l] = tensor(p + "attn_output_norm.weight");
    anb[l] = tensor(p + "attn_output_norm.bias");
    onw[l] = tensor(p + "layer_output_norm.weight");
    onb[l] = tensor(p + "layer_output_norm.bias");
  }
  if (missing_code != LLE_OK) return fail(missing_code, missing);
  d.qkv = qkv.data();
  d.out = o.data();
  d.attn_norm_w = anw.data();
  d.attn_norm_b = anb.data();
  d.up = up.data();
  d.gate = gate.data();
  d.down = down.data();
  d.out_norm_w = onw.data();
  d.out_norm_b = onb.data();
  return lle_model_create(&d, out);
}
