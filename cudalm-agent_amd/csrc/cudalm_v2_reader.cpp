// `.cudalm` v2 container reader with repack-at-load (include/cudalm_v2.h).
//
// Reference behaviour followed (file:line in the reference tree):
//   container rules          src/runtime/weight_loader_v2.cpp:48-240
//   layout constants         include/cudalm/weight_format_v2.h:31-100
//   config blob field order  include/cudalm/weight_format_v2.h:129-193
//   config validity          include/cudalm/qwen35_config.h:55-116
//   per-layer tensor sets    src/runtime/weight_loader_v2.cpp:263-376
//   upload at load           src/runtime/weight_loader_v2.cpp:416-500
//
// The reference reads the whole file into a heap vector; here the file is
// mapped read-only, so a 400 MB checkpoint costs no copy before the
// per-projection repack, and tensor views point straight into the mapping.

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <set>
#include <string>
#include <utility>
#include <vector>

#include "cudalm_v2.h"
#include "cudalm_w4a16.h"

struct cudalm_v2_file {
  void* map = nullptr;
  size_t map_bytes = 0;
  const uint8_t* base = nullptr;
  uint64_t payload_offset = 0;
  uint64_t payload_size = 0;
  cudalm_v2_config cfg{};
  std::vector<std::pair<std::string, std::string>> meta;
  struct Entry {
    std::string name;
    cudalm_v2_tensor t;
  };
  std::vector<Entry> tensors;
};

namespace {

constexpr char kMagic[8] = {'C', 'U', 'D', 'L', 'M', 'W', '0', '2'};
constexpr uint32_t kVersion = 2;
constexpr size_t kHeaderBytes = 88;
constexpr size_t kConfigBytes = 88;
constexpr size_t kConfigReserved = 84;
constexpr uint64_t kPayloadAlign = 16;
constexpr size_t kMaxNameLen = 255;
constexpr int64_t kMaxDim = 100000000;
constexpr uint32_t kMaxTensors = 100000;
constexpr uint32_t kMaxMeta = 256;
constexpr size_t kMaxMetaValue = 4096;
constexpr size_t kEntryTail = 1 + 1 + 2 + 8 * 8 + 8 + 8 + 1 + 1;  // after the name

template <typename T>
T rd(const uint8_t* p) {
  T v;
  std::memcpy(&v, p, sizeof(T));
  return v;
}

void set_err(char* err, size_t n, const char* fmt, ...) {
  if (!err || n == 0) return;
  va_list ap;
  va_start(ap, fmt);
  std::vsnprintf(err, n, fmt, ap);
  va_end(ap);
}

size_t dtype_bytes(int d) {
  switch (d) {
    case CUDALM_V2_DTYPE_FP16: return 2;
    case CUDALM_V2_DTYPE_INT4_PACKED: return 1;
    case CUDALM_V2_DTYPE_FP16_SCALE: return 2;
    case CUDALM_V2_DTYPE_FP32: return 4;
    case CUDALM_V2_DTYPE_BF16: return 2;
    default: return 0;
  }
}

bool name_ok(const uint8_t* s, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const uint8_t c = s[i];
    const bool ok = (c >= '0' && c <= '9') || (c >= 'A' && c <= 'Z') || (c >= 'a' && c <= 'z') ||
                    c == '.' || c == '_' || c == '-';
    if (!ok) return false;
  }
  return true;
}

cudalm_v2_config parse_config(const uint8_t* p) {
  cudalm_v2_config c{};
  int32_t* ints[] = {&c.hidden_size,       &c.num_hidden_layers,   &c.intermediate_size,
                     &c.vocab_size,        &c.n_heads,             &c.n_kv_heads,
                     &c.head_dim,          &c.lin_num_k_heads,     &c.lin_num_v_heads,
                     &c.lin_key_head_dim,  &c.lin_value_head_dim,  &c.lin_conv_kernel_dim,
                     &c.full_attention_interval, &c.group_size,    &c.max_seq_len};
  for (int k = 0; k < 15; ++k) *ints[k] = rd<int32_t>(p + 4 * k);
  c.eps = rd<float>(p + 60);
  c.rope_theta = rd<float>(p + 64);
  c.partial_rotary_factor = rd<float>(p + 68);
  for (int k = 0; k < 3; ++k) c.mrope_section[k] = rd<int32_t>(p + 72 + 4 * k);
  return c;
}

int rotary_dim(const cudalm_v2_config& c) {
  return static_cast<int>(static_cast<float>(c.head_dim) * c.partial_rotary_factor + 0.5f);
}
int q_proj_out(const cudalm_v2_config& c) { return c.n_heads * c.head_dim * 2; }
int kv_proj_out(const cudalm_v2_config& c) { return c.n_kv_heads * c.head_dim; }
int o_proj_in(const cudalm_v2_config& c) { return c.n_heads * c.head_dim; }
int lin_value_dim(const cudalm_v2_config& c) { return c.lin_num_v_heads * c.lin_value_head_dim; }
int lin_conv_dim(const cudalm_v2_config& c) {
  return 2 * c.lin_num_k_heads * c.lin_key_head_dim + lin_value_dim(c);
}
bool is_full_attention(const cudalm_v2_config& c, int i) {
  return c.num_hidden_layers > 0 && i >= 0 && i < c.num_hidden_layers &&
         c.full_attention_interval > 0 && (i + 1) % c.full_attention_interval == 0;
}

bool config_valid(const cudalm_v2_config& c) {
  if (c.hidden_size <= 0 || c.num_hidden_layers <= 0 || c.intermediate_size <= 0) return false;
  if (c.n_heads <= 0 || c.n_kv_heads <= 0 || c.head_dim <= 0) return false;
  if (c.n_heads % c.n_kv_heads != 0) return false;
  if (c.lin_num_k_heads <= 0 || c.lin_num_v_heads <= 0) return false;
  if (c.lin_num_v_heads % c.lin_num_k_heads != 0) return false;
  if (c.lin_key_head_dim <= 0 || c.lin_value_head_dim <= 0) return false;
  if (c.lin_conv_kernel_dim < 2 || c.full_attention_interval < 2) return false;
  if (c.group_size <= 0 || c.max_seq_len <= 0) return false;
  if (!(c.eps > 0.0f) || !(c.rope_theta > 0.0f)) return false;
  const int rd2 = rotary_dim(c);
  if (rd2 <= 0 || rd2 > c.head_dim || rd2 % 2 != 0) return false;
  if (c.mrope_section[0] + c.mrope_section[1] + c.mrope_section[2] != rd2 / 2) return false;
  if (c.hidden_size % c.group_size != 0 || o_proj_in(c) % c.group_size != 0 ||
      c.intermediate_size % c.group_size != 0 || lin_value_dim(c) % c.group_size != 0)
    return false;
  return true;
}

// Parse and validate the mapped bytes into f; "" on success, else the reason.
std::string parse(const uint8_t* p, uint64_t n, cudalm_v2_file* f) {
  if (n < kHeaderBytes) return "file too small for v2 header";
  if (std::memcmp(p, kMagic, 8) != 0) return "bad magic (not CUDLMW02)";
  if (rd<uint32_t>(p + 8) != kVersion) return "unsupported version " + std::to_string(rd<uint32_t>(p + 8));
  if (rd<uint32_t>(p + 12) != 0) return "reserved flags must be 0";
  const uint32_t num_tensors = rd<uint32_t>(p + 16);
  const uint16_t num_meta = rd<uint16_t>(p + 20);
  if (rd<uint16_t>(p + 22) != 0) return "reserved pad must be 0";
  uint64_t sec[4][2];
  for (int s = 0; s < 4; ++s) {
    sec[s][0] = rd<uint64_t>(p + 24 + 16 * s);
    sec[s][1] = rd<uint64_t>(p + 32 + 16 * s);
  }
  auto within = [n](uint64_t off, uint64_t size) { return off <= n && size <= n - off; };
  if (num_tensors > kMaxTensors) return "num_tensors exceeds limit";
  if (num_meta > kMaxMeta) return "num_metadata exceeds limit";
  if (sec[0][1] != kConfigBytes) return "config_size must be 88";
  const char* names[4] = {"config section", "metadata section", "tensor table", "payload"};
  for (int s = 0; s < 4; ++s)
    if (!within(sec[s][0], sec[s][1])) return std::string(names[s]) + " out of bounds";
  if (sec[3][0] % kPayloadAlign != 0) return "payload_offset must be 16B-aligned";
  for (int a = 0; a < 4; ++a)
    for (int b = a + 1; b < 4; ++b)
      if (sec[a][0] < sec[b][0] + sec[b][1] && sec[b][0] < sec[a][0] + sec[a][1])
        return "sections overlap";

  const uint8_t* cblob = p + sec[0][0];
  f->cfg = parse_config(cblob);
  if (rd<uint32_t>(cblob + kConfigReserved) != 0) return "config blob reserved word must be 0";
  if (!config_valid(f->cfg)) return "Qwen35Config blob failed validation";

  {  // metadata
    uint64_t pos = sec[1][0];
    const uint64_t end = sec[1][0] + sec[1][1];
    for (uint32_t k = 0; k < num_meta; ++k) {
      if (pos + 1 > end) return "metadata: key_len out of bounds";
      const size_t klen = p[pos];
      pos += 1;
      if (pos + klen + 2 > end) return "metadata: key/value_len out of bounds";
      std::string key(reinterpret_cast<const char*>(p + pos), klen);
      pos += klen;
      const size_t vlen = rd<uint16_t>(p + pos);
      pos += 2;
      if (vlen > kMaxMetaValue) return "metadata: value too long for key '" + key + "'";
      if (pos + vlen > end) return "metadata: value out of bounds for '" + key + "'";
      f->meta.emplace_back(std::move(key), std::string(reinterpret_cast<const char*>(p + pos), vlen));
      pos += vlen;
    }
    if (pos != end) return "metadata: trailing bytes";
  }

  {  // tensor table
    std::set<std::string> seen;
    uint64_t pos = sec[2][0];
    const uint64_t end = sec[2][0] + sec[2][1];
    const uint64_t poff = sec[3][0], psize = sec[3][1];
    for (uint32_t k = 0; k < num_tensors; ++k) {
      if (pos + 1 > end) return "tensor table: name_len out of bounds";
      const size_t nlen = p[pos];
      pos += 1;
      if (nlen == 0 || nlen > kMaxNameLen) return "tensor table: bad name_len";
      if (pos + nlen + kEntryTail > end) return "tensor table: entry out of bounds";
      cudalm_v2_file::Entry e;
      e.name.assign(reinterpret_cast<const char*>(p + pos), nlen);
      if (!name_ok(p + pos, nlen)) return "tensor table: bad name charset in '" + e.name + "'";
      pos += nlen;
      if (!seen.insert(e.name).second) return "duplicate tensor name '" + e.name + "'";
      cudalm_v2_tensor& t = e.t;
      t.dtype = p[pos];
      if (dtype_bytes(t.dtype) == 0) return "bad dtype in tensor '" + e.name + "'";
      t.ndim = p[pos + 1];
      if (t.ndim < 1 || t.ndim > 8) return "bad ndim in tensor '" + e.name + "'";
      if (rd<uint16_t>(p + pos + 2) != 0) return "tensor '" + e.name + "': reserved pad must be 0";
      pos += 4;
      for (int d = 0; d < 8; ++d) {
        const int64_t dv = rd<int64_t>(p + pos + 8 * d);
        if (d < t.ndim) {
          if (dv <= 0 || dv > kMaxDim) return "bad dim in tensor '" + e.name + "'";
        } else if (dv != 0) {
          return "tensor '" + e.name + "': unused dim must be 0";
        }
        t.dims[d] = d < t.ndim ? dv : 0;
      }
      pos += 64;
      t.offset = rd<uint64_t>(p + pos);
      t.byte_size = rd<uint64_t>(p + pos + 8);
      t.align = p[pos + 16];
      if (p[pos + 17] != 0) return "tensor '" + e.name + "': reserved pad must be 0";
      pos += 18;
      if (!(t.align == 1 || t.align == 2 || t.align == 4 || t.align == 8 || t.align == 16))
        return "tensor '" + e.name + "': bad align";
      if (t.offset > psize || t.byte_size > psize - t.offset)
        return "tensor '" + e.name + "' out of payload bounds";
      if ((poff + t.offset) % static_cast<uint64_t>(t.align) != 0)
        return "tensor '" + e.name + "' not " + std::to_string(t.align) + "B-aligned";
      // byte_size must equal numel * element bytes; numel is recomputed
      // with overflow detection (a product that wraps cannot match a size
      // that fits in the payload)
      unsigned __int128 exact = 1;
      for (int d = 0; d < t.ndim; ++d) exact *= static_cast<unsigned __int128>(t.dims[d]);
      exact *= dtype_bytes(t.dtype);
      if (exact != static_cast<unsigned __int128>(t.byte_size))
        return "tensor '" + e.name + "': byte_size != expected for dtype/shape";
      t.host = p + poff + t.offset;
      f->tensors.push_back(std::move(e));
    }
    if (pos != end) return "tensor table: trailing bytes";
  }
  for (auto& e : f->tensors) e.t.name = e.name.c_str();
  return "";
}

const cudalm_v2_tensor* find_tensor(const cudalm_v2_file* f, const std::string& name) {
  for (const auto& e : f->tensors)
    if (e.name == name) return &e.t;
  return nullptr;
}

std::string expect(const cudalm_v2_file* f, const std::string& name, int dtype,
                   std::vector<int64_t> dims) {
  const cudalm_v2_tensor* t = find_tensor(f, name);
  if (!t) return "missing tensor '" + name + "'";
  if (t->dtype != dtype) return "dtype mismatch for '" + name + "'";
  if (static_cast<size_t>(t->ndim) != dims.size()) return "shape mismatch for '" + name + "'";
  for (size_t d = 0; d < dims.size(); ++d)
    if (t->dims[d] != dims[d]) return "shape mismatch for '" + name + "'";
  return "";
}

std::string validate_layer(const cudalm_v2_file* f, int li) {
  const cudalm_v2_config& c = f->cfg;
  if (li < 0 || li >= c.num_hidden_layers) return "layer_idx out of range";
  const std::string L = "layers." + std::to_string(li) + ".";
  const int H = c.hidden_size, G = c.group_size;
  const int I4 = CUDALM_V2_DTYPE_INT4_PACKED, SC = CUDALM_V2_DTYPE_FP16_SCALE,
            BF = CUDALM_V2_DTYPE_BF16, F32 = CUDALM_V2_DTYPE_FP32;
  struct Req {
    std::string name;
    int dtype;
    std::vector<int64_t> dims;
  };
  std::vector<Req> req = {
      {"input_layernorm.weight", BF, {H}},
      {"post_attention_layernorm.weight", BF, {H}},
      {"mlp.gate_proj.weight", I4, {c.intermediate_size, H / 2}},
      {"mlp.up_proj.weight", I4, {c.intermediate_size, H / 2}},
      {"mlp.gate_proj.scale", SC, {c.intermediate_size, H / G}},
      {"mlp.up_proj.scale", SC, {c.intermediate_size, H / G}},
      {"mlp.down_proj.weight", I4, {H, c.intermediate_size / 2}},
      {"mlp.down_proj.scale", SC, {H, c.intermediate_size / G}},
  };
  auto proj = [&](const char* base, int n, int k) {
    req.push_back({std::string(base) + ".weight", I4, {n, k / 2}});
    req.push_back({std::string(base) + ".scale", SC, {n, k / G}});
  };
  if (is_full_attention(c, li)) {
    proj("self_attn.q_proj", q_proj_out(c), H);
    proj("self_attn.k_proj", kv_proj_out(c), H);
    proj("self_attn.v_proj", kv_proj_out(c), H);
    proj("self_attn.o_proj", H, o_proj_in(c));
    req.push_back({"self_attn.q_norm.weight", BF, {c.head_dim}});
    req.push_back({"self_attn.k_norm.weight", BF, {c.head_dim}});
  } else {
    proj("linear_attn.in_proj_qkv", lin_conv_dim(c), H);
    proj("linear_attn.in_proj_z", lin_value_dim(c), H);
    proj("linear_attn.in_proj_b", c.lin_num_v_heads, H);
    proj("linear_attn.in_proj_a", c.lin_num_v_heads, H);
    proj("linear_attn.out_proj", H, lin_value_dim(c));
    req.push_back({"linear_attn.conv1d.weight", BF, {lin_conv_dim(c), 1, c.lin_conv_kernel_dim}});
    req.push_back({"linear_attn.dt_bias", BF, {c.lin_num_v_heads}});
    req.push_back({"linear_attn.A_log", F32, {c.lin_num_v_heads}});
    req.push_back({"linear_attn.norm.weight", F32, {c.lin_value_head_dim}});
  }
  for (const auto& r : req) {
    const std::string e = expect(f, L + r.name, r.dtype, r.dims);
    if (!e.empty()) return e;
  }
  return "";
}

}  // namespace

extern "C" {

int cudalm_v2_open(const char* path, cudalm_v2_file** out, char* err, size_t errlen) {
  if (!out) return CUDALM_W4A16_ENULL;
  *out = nullptr;
  if (!path) return CUDALM_W4A16_ENULL;
  const int fd = ::open(path, O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    set_err(err, errlen, "cannot open %s", path);
    return CUDALM_V2_EIO;
  }
  struct stat st;
  if (::fstat(fd, &st) != 0 || st.st_size < 0) {
    ::close(fd);
    set_err(err, errlen, "cannot stat %s", path);
    return CUDALM_V2_EIO;
  }
  auto* f = new cudalm_v2_file;
  f->map_bytes = static_cast<size_t>(st.st_size);
  if (f->map_bytes > 0) {
    f->map = ::mmap(nullptr, f->map_bytes, PROT_READ, MAP_PRIVATE, fd, 0);
    if (f->map == MAP_FAILED) {
      ::close(fd);
      delete f;
      set_err(err, errlen, "cannot map %s", path);
      return CUDALM_V2_EIO;
    }
    f->base = static_cast<const uint8_t*>(f->map);
  }
  ::close(fd);
  static const uint8_t empty[1] = {0};
  const std::string why = parse(f->base ? f->base : empty, f->map_bytes, f);
  if (!why.empty()) {
    set_err(err, errlen, "%s", why.c_str());
    cudalm_v2_close(f);
    return CUDALM_V2_EFORMAT;
  }
  f->payload_offset = rd<uint64_t>(f->base + 72);
  f->payload_size = rd<uint64_t>(f->base + 80);
  *out = f;
  return CUDALM_W4A16_OK;
}

void cudalm_v2_close(cudalm_v2_file* f) {
  if (!f) return;
  if (f->map && f->map != MAP_FAILED) ::munmap(f->map, f->map_bytes);
  delete f;
}

int cudalm_v2_num_tensors(const cudalm_v2_file* f) {
  return f ? static_cast<int>(f->tensors.size()) : CUDALM_W4A16_ENULL;
}

int cudalm_v2_tensor_at(const cudalm_v2_file* f, int index, cudalm_v2_tensor* out) {
  if (!f || !out) return CUDALM_W4A16_ENULL;
  if (index < 0 || static_cast<size_t>(index) >= f->tensors.size()) return CUDALM_W4A16_ERANGE;
  *out = f->tensors[index].t;
  return CUDALM_W4A16_OK;
}

int cudalm_v2_find(const cudalm_v2_file* f, const char* name, cudalm_v2_tensor* out) {
  if (!f || !name || !out) return CUDALM_W4A16_ENULL;
  const cudalm_v2_tensor* t = find_tensor(f, name);
  if (!t) return CUDALM_V2_ENOTFOUND;
  *out = *t;
  return CUDALM_W4A16_OK;
}

const char* cudalm_v2_meta(const cudalm_v2_file* f, const char* key) {
  if (!f || !key) return nullptr;
  for (const auto& kv : f->meta)
    if (kv.first == key) return kv.second.c_str();
  return nullptr;
}

int cudalm_v2_get_config(const cudalm_v2_file* f, cudalm_v2_config* out) {
  if (!f || !out) return CUDALM_W4A16_ENULL;
  *out = f->cfg;
  return CUDALM_W4A16_OK;
}

int cudalm_v2_validate_layer(const cudalm_v2_file* f, int layer_idx, char* err, size_t errlen) {
  if (!f) return CUDALM_W4A16_ENULL;
  const std::string why = validate_layer(f, layer_idx);
  if (why.empty()) return CUDALM_W4A16_OK;
  set_err(err, errlen, "%s", why.c_str());
  return CUDALM_V2_ENOTFOUND;
}

int cudalm_v2_w4a16_shape(const cudalm_v2_file* f, const char* prefix, int* N, int* K) {
  if (!f || !prefix || !N || !K) return CUDALM_W4A16_ENULL;
  const cudalm_v2_tensor* w = find_tensor(f, std::string(prefix) + ".weight");
  const cudalm_v2_tensor* s = find_tensor(f, std::string(prefix) + ".scale");
  if (!w || !s || w->dtype != CUDALM_V2_DTYPE_INT4_PACKED || w->ndim != 2 ||
      s->dtype != CUDALM_V2_DTYPE_FP16_SCALE || s->ndim != 2)
    return CUDALM_V2_ENOTFOUND;
  const int64_t n = w->dims[0], k = 2 * w->dims[1];
  if (k % CUDALM_W4A16_GROUP != 0 || s->dims[0] != n || s->dims[1] != k / CUDALM_W4A16_GROUP ||
      n > (1 << 30) || k > (1 << 24))
    return CUDALM_V2_ENOTFOUND;
  *N = static_cast<int>(n);
  *K = static_cast<int>(k);
  return CUDALM_W4A16_OK;
}

int cudalm_v2_upload_w4a16_packed(const cudalm_v2_file* f, const char* prefix, void* packed_dev,
                                  size_t bytes, hipStream_t stream) {
  int N = 0, K = 0;
  if (!packed_dev) return CUDALM_W4A16_ENULL;
  if (int rc = cudalm_v2_w4a16_shape(f, prefix, &N, &K)) return rc;
  const size_t need = cudalm_w4a16_packed_bytes(N, K);
  if (bytes < need) return CUDALM_W4A16_ERANGE;
  if ((reinterpret_cast<uintptr_t>(packed_dev) & 15) != 0) return CUDALM_W4A16_EALIGN;
  const cudalm_v2_tensor* w = find_tensor(f, std::string(prefix) + ".weight");
  const cudalm_v2_tensor* s = find_tensor(f, std::string(prefix) + ".scale");
  // scales may sit at any 2-byte offset of the mapping; the host repack
  // reads them through an aligned copy when they are not
  std::vector<uint16_t> scale_copy;
  const uint16_t* sp = static_cast<const uint16_t*>(s->host);
  if ((reinterpret_cast<uintptr_t>(sp) & 1) != 0) {
    scale_copy.resize(s->byte_size / 2);
    std::memcpy(scale_copy.data(), s->host, s->byte_size);
    sp = scale_copy.data();
  }
  std::vector<uint8_t> staging(need);
  if (int rc = cudalm_w4a16_repack_host(static_cast<const uint8_t*>(w->host), sp, staging.data(),
                                        N, K))
    return rc;
  if (hipMemcpyAsync(packed_dev, staging.data(), need, hipMemcpyHostToDevice, stream) !=
          hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return CUDALM_W4A16_ELAUNCH;
  return CUDALM_W4A16_OK;
}

int cudalm_v2_upload(const cudalm_v2_file* f, const char* name, void* dst_dev, size_t dst_bytes,
                     hipStream_t stream) {
  if (!f || !name || !dst_dev) return CUDALM_W4A16_ENULL;
  const cudalm_v2_tensor* t = find_tensor(f, name);
  if (!t) return CUDALM_V2_ENOTFOUND;
  if (dst_bytes < t->byte_size) return CUDALM_W4A16_ERANGE;
  if (t->byte_size == 0) return CUDALM_W4A16_OK;
  if (hipMemcpyAsync(dst_dev, t->host, t->byte_size, hipMemcpyHostToDevice, stream) !=
          hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return CUDALM_W4A16_ELAUNCH;
  return CUDALM_W4A16_OK;
}

}  // extern "C"
