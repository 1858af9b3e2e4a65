// hy3x_gguf.hip -- the MoE tensors of one layer straight from a hy3 GGUF file
// (host code).
//
// GGUF as the reference reads it (hy3.c:63-79 value types, :193-232 tensor
// sizes, :238-292 metadata and tensor directory): magic "GGUF", version,
// n_tensors, n_kv (u64), key/value pairs, tensor infos (name, n_dims,
// dims[u64], ggml type, offset relative to the data section), and the data
// section at the end of the directory rounded up to general.alignment (32 by
// default). Type 8 is hy3's own Q8_0 (36-byte blocks). The file is mapped
// read-only and every read is bounds-checked: a malformed file yields an
// error, never a read past the mapping.
//
// Tensor names are the converter's (hy3_convert.c:960-1035) as hy3.c binds
// them for a MoE layer (hy3.c:740-787).
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <string>
#include <unordered_map>

#include "../../include/hy3x_moe.h"

namespace {

struct TensorInfo {
  uint32_t type = 0;
  uint32_t ndim = 0;
  uint64_t dim[4] = {0, 0, 0, 0};
  uint64_t elements = 0, offset = 0, bytes = 0;
};

struct Gguf {
  const uint8_t *map = nullptr;
  size_t size = 0;
  uint64_t data_pos = 0;
  std::unordered_map<std::string, TensorInfo> tensors;
  std::string err;
  ~Gguf() {
    if (map) munmap((void *)map, size);
  }
  const uint8_t *data(const TensorInfo &t) const { return map + data_pos + t.offset; }
};

struct Cursor {
  const uint8_t *p;
  size_t n, pos = 0;
  bool ok = true;
  bool take(void *dst, size_t k) {
    if (!ok || k > n - pos) return ok = false;
    memcpy(dst, p + pos, k);
    pos += k;
    return true;
  }
  bool skip(uint64_t k) {
    if (!ok || k > n - pos) return ok = false;
    pos += (size_t)k;
    return true;
  }
  uint32_t u32() {
    uint32_t v = 0;
    take(&v, 4);
    return v;
  }
  uint64_t u64() {
    uint64_t v = 0;
    take(&v, 8);
    return v;
  }
  bool str(std::string *out) {
    const uint64_t len = u64();
    if (!ok || len > n - pos) return ok = false;
    if (out) out->assign((const char *)p + pos, (size_t)len);
    pos += (size_t)len;
    return true;
  }
};

// Bytes per block and elements per block of a ggml type (hy3.c:193-223); 0
// for types this library has no use for.
void type_size(uint32_t type, uint64_t *be, uint64_t *bb) {
  switch (type) {
    case 0: *be = 1, *bb = 4; return;     // F32
    case 1: *be = 1, *bb = 2; return;     // F16
    case 8: *be = 32, *bb = 36; return;   // hy3 Q8_0
    case 12: *be = 256, *bb = 144; return;  // Q4_K
    default: *be = 0, *bb = 0; return;
  }
}

// Skip one metadata value of `type` (hy3.c:150-181), arrays nested at most 2 deep.
bool skip_value(Cursor &c, uint32_t type, int depth) {
  switch (type) {
    case 0: case 1: case 7: return c.skip(1);
    case 2: case 3: return c.skip(2);
    case 4: case 5: case 6: return c.skip(4);
    case 10: case 11: case 12: return c.skip(8);
    case 8: return c.str(nullptr);
    case 9: {
      if (depth > 1) return c.ok = false;
      const uint32_t et = c.u32();
      const uint64_t count = c.u64();
      if (!c.ok) return false;
      for (uint64_t i = 0; i < count; i++)
        if (!skip_value(c, et, depth + 1)) return false;
      return true;
    }
    default: return c.ok = false;
  }
}

bool open_gguf(const char *path, Gguf &g) {
  const int fd = open(path, O_RDONLY);
  if (fd < 0) {
    g.err = std::string("cannot open ") + path + ": " + strerror(errno);
    return false;
  }
  struct stat st;
  if (fstat(fd, &st) != 0 || st.st_size < 24) {
    close(fd);
    g.err = std::string(path) + ": not a GGUF file (too small)";
    return false;
  }
  void *m = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (m == MAP_FAILED) {
    g.err = std::string("cannot map ") + path;
    return false;
  }
  g.map = (const uint8_t *)m;
  g.size = (size_t)st.st_size;
  Cursor c{g.map, g.size};
  if (c.u32() != 0x46554747u) {  // "GGUF"
    g.err = std::string(path) + ": bad magic";
    return false;
  }
  const uint32_t version = c.u32();
  if (version < 2 || version > 3) {
    g.err = std::string(path) + ": unsupported GGUF version " + std::to_string(version);
    return false;
  }
  const uint64_t n_tensors = c.u64(), n_kv = c.u64();
  if (!c.ok || n_tensors > (1u << 24) || n_kv > (1u << 24)) {
    g.err = std::string(path) + ": implausible tensor / key counts";
    return false;
  }
  uint64_t align = 32;
  for (uint64_t i = 0; i < n_kv && c.ok; i++) {
    std::string key;
    c.str(&key);
    const uint32_t type = c.u32();
    if (c.ok && key == "general.alignment" && type == 4) {
      Cursor t = c;
      const uint32_t a = t.u32();
      if (t.ok && a != 0) align = a;
    }
    skip_value(c, type, 0);
  }
  for (uint64_t i = 0; i < n_tensors && c.ok; i++) {
    std::string name;
    TensorInfo t;
    c.str(&name);
    t.ndim = c.u32();
    if (t.ndim > 4) c.ok = false;
    t.elements = 1;
    for (uint32_t d = 0; d < t.ndim && c.ok; d++) {
      t.dim[d] = c.u64();
      t.elements *= t.dim[d];
    }
    t.type = c.u32();
    t.offset = c.u64();
    uint64_t be, bb;
    type_size(t.type, &be, &bb);
    t.bytes = be ? t.elements / be * bb : 0;
    if (c.ok) g.tensors[name] = t;
  }
  if (!c.ok) {
    g.err = std::string(path) + ": truncated or malformed GGUF header";
    return false;
  }
  g.data_pos = (c.pos + align - 1) / align * align;
  for (const auto &kv : g.tensors) {
    const TensorInfo &t = kv.second;
    if (t.bytes && (t.offset > g.size || g.data_pos + t.offset + t.bytes > g.size)) {
      g.err = std::string(path) + ": tensor " + kv.first + " extends past the end of the file";
      return false;
    }
  }
  return true;
}

// One tensor of the layer, checked for presence, type and shape. rows: the
// first dimension (the reference's t->dim[0], HF [out, in] order).
const TensorInfo *need(const Gguf &g, const std::string &name, uint32_t type, uint64_t elements,
                       uint64_t rows, std::string &err) {
  auto it = g.tensors.find(name);
  if (it == g.tensors.end()) {
    err = "tensor " + name + " not found";
    return nullptr;
  }
  const TensorInfo &t = it->second;
  if (t.type != type || t.elements != elements || (rows && t.dim[0] != rows)) {
    err = "tensor " + name + ": type " + std::to_string(t.type) + ", " +
          std::to_string(t.elements) + " elements, dim0 " + std::to_string(t.dim[0]) +
          "; expected type " + std::to_string(type) + ", " + std::to_string(elements) +
          (rows ? ", dim0 " + std::to_string(rows) : std::string());
    return nullptr;
  }
  return &t;
}

std::string layer_name(int il, const char *what) {
  return "blk." + std::to_string(il) + "." + what;
}

std::string expert_name(int il, const char *kind, int e) {  // hy3_convert.c:1013-1018
  return "blk." + std::to_string(il) + ".ffn_" + kind + "_exps." + std::to_string(e) + "." +
         kind + "_proj.weight";
}

struct LayerTensors {
  const TensorInfo *norm, *router, *bias, *exp[192][3], *sh[3];
  int shared_type;
};

// Everything hy3.c binds for a MoE layer (hy3.c:740-787, plus ffn_norm).
bool find_layer(const Gguf &g, int il, LayerTensors &lt, std::string &err) {
  constexpr uint64_t D = HY3X_D_MODEL, F = HY3X_D_FF, E = HY3X_N_EXPERT;
  if (!(lt.norm = need(g, layer_name(il, "ffn_norm.weight"), 0, D, 0, err))) return false;
  if (!(lt.router = need(g, layer_name(il, "ffn_gate_inp.weight"), 0, E * D, E, err))) return false;
  lt.bias = nullptr;
  if (g.tensors.count(layer_name(il, "ffn_gate_exps_b.bias")) &&
      !(lt.bias = need(g, layer_name(il, "ffn_gate_exps_b.bias"), 0, E, 0, err)))
    return false;
  const char *kinds[3] = {"gate", "up", "down"};
  for (int e = 0; e < (int)E; e++)
    for (int m = 0; m < 3; m++)
      if (!(lt.exp[e][m] = need(g, expert_name(il, kinds[m], e), 12, F * D, m == 2 ? D : F, err)))
        return false;
  const std::string shn[3] = {layer_name(il, "ffn_gate_shexp.weight"),
                              layer_name(il, "ffn_up_shexp.weight"),
                              layer_name(il, "ffn_down_shexp.weight")};
  auto it = g.tensors.find(shn[0]);
  lt.shared_type = it == g.tensors.end() ? 12 : (int)it->second.type;
  if (lt.shared_type != 8 && lt.shared_type != 12) {
    err = "tensor " + shn[0] + ": shared expert type " + std::to_string(lt.shared_type) +
          " (expected 8, hy3's Q8_0, or 12, Q4_K)";
    return false;
  }
  for (int m = 0; m < 3; m++)
    if (!(lt.sh[m] = need(g, shn[m], (uint32_t)lt.shared_type, F * D, m == 2 ? D : F, err)))
      return false;
  return true;
}

}  // namespace

namespace hy3x {
int set_error(int code, const char *msg);  // hy3x_layer.hip: the message hy3x_last_error() returns
}  // namespace hy3x

namespace {
int gguf_fail(int code, const std::string &msg) { return hy3x::set_error(code, msg.c_str()); }
}  // namespace

extern "C" {

int hy3x_gguf_check_layer(const char *path, int layer_index, int *shared_type) {
  if (!path || layer_index < 0) return gguf_fail(HY3X_E_ARG, "bad argument");
  Gguf g;
  if (!open_gguf(path, g)) return gguf_fail(HY3X_E_ARG, g.err);
  LayerTensors lt;
  std::string err;
  if (!find_layer(g, layer_index, lt, err)) return gguf_fail(HY3X_E_ARG, std::string(path) + ": " + err);
  if (shared_type) *shared_type = lt.shared_type;
  return HY3X_OK;
}

int hy3x_layer_load_gguf(hy3x_layer *layer, const char *path, int layer_index) {
  if (!layer || !path || layer_index < 0) return gguf_fail(HY3X_E_ARG, "bad argument");
  Gguf g;
  if (!open_gguf(path, g)) return gguf_fail(HY3X_E_ARG, g.err);
  LayerTensors lt;
  std::string err;
  if (!find_layer(g, layer_index, lt, err)) return gguf_fail(HY3X_E_ARG, std::string(path) + ": " + err);
  int rc = hy3x_layer_set_router(layer, (const float *)g.data(*lt.norm),
                                 (const float *)g.data(*lt.router),
                                 lt.bias ? (const float *)g.data(*lt.bias) : nullptr);
  for (int e = 0; e < HY3X_N_EXPERT && rc == HY3X_OK; e++)
    rc = hy3x_layer_set_expert_q4k(layer, e, g.data(*lt.exp[e][0]), g.data(*lt.exp[e][1]),
                                   g.data(*lt.exp[e][2]), 0);
  if (rc == HY3X_OK) {
    if (lt.shared_type == 8)
      rc = hy3x_layer_set_shared_q8_0(layer, g.data(*lt.sh[0]), g.data(*lt.sh[1]),
                                      g.data(*lt.sh[2]), 0);
    else
      rc = hy3x_layer_set_expert_q4k(layer, HY3X_N_EXPERT, g.data(*lt.sh[0]), g.data(*lt.sh[1]),
                                     g.data(*lt.sh[2]), 0);
  }
  return rc;
}

}  // extern "C"
