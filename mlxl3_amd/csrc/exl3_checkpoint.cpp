// EXL3 checkpoint loading: safetensors header inspection and the loaders that
// upload one projection or one SwitchGLU expert bank to the current device.
//
//   exl3_checkpoint_open   checkpoint::inspect      native/src/checkpoint.rs:197-330
//                          checkpoint::read_header  native/src/checkpoint.rs:38-93
//   exl3_checkpoint_read   TensorInfo::read_bytes   native/src/checkpoint.rs:113-125
//   exl3_linear_load       Exl3Linear::from_checkpoint (tensor names, legacy
//                          su/sv names, codebook flags, K from the trellis)
//                          native/src/linear.rs:454-575
//   exl3_moe_load          Exl3SwitchGlu::from_checkpoint_names
//                          native/src/moe.rs:629-800
//   exl3_moe_load_gemma    Exl3SwitchGlu::from_gemma_checkpoint (GELU)
//                          native/src/moe.rs:663-680
//
// The inspection validates every header before any weight is read (same
// checks and messages as the reference); payloads are read on request with
// pread() on descriptors opened at inspection, so a shard replaced on disk
// afterwards cannot pair old offsets with new bytes.  Loaded handles own one
// device allocation holding all of their weights.
#include <dirent.h>
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <new>
#include <string>
#include <vector>

#include "../../include/exl3_hip.h"
#include "exl3_json.hpp"
#include "exl3_launch.hpp"

using exl3::fail;

namespace {

struct Tensor {
  std::string dtype;
  std::vector<uint64_t> shape;
  uint64_t start = 0, end = 0;  // data_offsets, relative to the payload
  uint64_t payload = 0;         // 8 + header length
  int shard = -1;               // index into exl3_checkpoint::shards
};

struct Shard {
  std::string path;
  std::string file_name;
  int fd = -1;
};

std::string strprintf(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
std::string strprintf(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  return buf;
}

// An error message plus its status code, carried out of nested helpers.
struct Error {
  int code = EXL3_OK;
  std::string msg;
  explicit operator bool() const { return code != EXL3_OK; }
};
Error err(int code, std::string msg) { return Error{code, std::move(msg)}; }
Error invalid(std::string msg) { return err(EXL3_EINVAL, std::move(msg)); }
int raise(const Error& e) { return fail(e.code, "%s", e.msg.c_str()); }

// safetensors element sizes (checkpoint.rs:28-36).
bool dtype_size(const std::string& d, uint64_t& size) {
  static const std::pair<const char*, uint64_t> kSizes[] = {
      {"BOOL", 1}, {"U8", 1},  {"I8", 1},   {"F8_E4M3", 1}, {"F8_E5M2", 1}, {"U16", 2},
      {"I16", 2},  {"F16", 2}, {"BF16", 2}, {"U32", 4},     {"I32", 4},     {"F32", 4},
      {"U64", 8},  {"I64", 8}, {"F64", 8}};
  for (auto& s : kSizes)
    if (d == s.first) {
      size = s.second;
      return true;
    }
  return false;
}

// Checked product of the dimensions times the element size
// (contracts.rs:1816-1820).
bool tensor_bytes(const std::vector<uint64_t>& shape, uint64_t item, uint64_t& out) {
  uint64_t n = item;
  for (uint64_t d : shape) {
    if (d != 0 && n > UINT64_MAX / d) return false;
    n *= d;
  }
  out = n;
  return true;
}

bool read_full(int fd, void* dst, size_t bytes, uint64_t offset) {
  char* p = (char*)dst;
  while (bytes > 0) {
    ssize_t r = pread(fd, p, bytes, (off_t)offset);
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    p += r;
    bytes -= (size_t)r;
    offset += (uint64_t)r;
  }
  return true;
}

bool as_u64(const exl3::json::Value& v, uint64_t& out) {
  if (!v.is_number() || !v.is_uint) return false;
  out = v.u;
  return true;
}

bool as_shape(const exl3::json::Value& v, std::vector<uint64_t>& out) {
  if (!v.is_array()) return false;
  out.clear();
  for (auto& d : v.arr) {
    uint64_t n;
    if (!as_u64(d, n)) return false;
    out.push_back(n);
  }
  return true;
}

bool read_text_file(const std::string& path, std::string& out, Error& e) {
  int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) {
    e = invalid(strprintf("%s: %s", path.c_str(), strerror(errno)));
    return false;
  }
  struct stat st;
  bool ok = fstat(fd, &st) == 0;
  if (ok) {
    out.resize((size_t)st.st_size);
    ok = read_full(fd, &out[0], out.size(), 0);
  }
  close(fd);
  if (!ok) e = invalid(strprintf("%s: read failed", path.c_str()));
  return ok;
}

bool read_json_file(const std::string& path, exl3::json::Value& v, Error& e) {
  std::string text;
  if (!read_text_file(path, text, e)) return false;
  std::string why;
  if (!exl3::json::parse(text.data(), text.size(), v, why)) {
    e = invalid(strprintf("invalid JSON in %s: %s", path.c_str(), why.c_str()));
    return false;
  }
  return true;
}

bool starts_with(const std::string& s, const char* p) { return s.rfind(p, 0) == 0; }
bool ends_with(const std::string& s, const char* p) {
  size_t n = strlen(p);
  return s.size() >= n && s.compare(s.size() - n, n, p) == 0;
}

}  // namespace

struct exl3_checkpoint {
  std::string path;
  std::string model_type;
  double bits = NAN;
  uint64_t size_bytes = 0;
  std::vector<std::string> modules;
  std::map<std::string, Tensor> tensors;
  std::vector<const std::string*> names;  // tensors' keys in sorted order
  std::vector<Shard> shards;

  ~exl3_checkpoint() {
    for (auto& s : shards)
      if (s.fd >= 0) close(s.fd);
  }
};

namespace {

// read_header, checkpoint.rs:38-93: one shard's tensors, validated so that the
// tensors tile the payload exactly (no gaps, no overlaps, nothing unclaimed).
Error read_header(exl3_checkpoint& c, const std::string& path, const std::string& file_name,
                  std::map<std::string, Tensor>& out) {
  int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
  if (fd < 0) return invalid(strprintf("opening %s: %s", path.c_str(), strerror(errno)));
  c.shards.push_back(Shard{path, file_name, fd});
  int shard = (int)c.shards.size() - 1;
  struct stat st;
  if (fstat(fd, &st) != 0) return invalid(strprintf("opening %s: %s", path.c_str(), strerror(errno)));
  uint64_t file_len = (uint64_t)st.st_size;
  unsigned char len_bytes[8];
  if (file_len < 8 || !read_full(fd, len_bytes, 8, 0))
    return invalid("missing safetensors header length");
  uint64_t header_len = 0;
  for (int i = 7; i >= 0; --i) header_len = (header_len << 8) | len_bytes[i];
  if (header_len > 100000000ull || header_len > file_len - 8)
    return invalid("invalid safetensors header length");
  std::string header((size_t)header_len, '\0');
  if (header_len && !read_full(fd, &header[0], header.size(), 8))
    return invalid(strprintf("reading %s: truncated header", path.c_str()));
  exl3::json::Value root;
  std::string why;
  if (!exl3::json::parse(header.data(), header.size(), root, why))
    return invalid("invalid safetensors header JSON: " + why);
  if (!root.is_object()) return invalid("invalid safetensors header JSON: expected an object");
  // Last value of a repeated key wins, entries in key order (a sorted map).
  std::map<std::string, const exl3::json::Value*> entries;
  for (auto& kv : root.obj) entries[kv.first] = &kv.second;
  auto meta = entries.find("__metadata__");
  if (meta != entries.end()) {
    const exl3::json::Value& m = *meta->second;
    bool ok = m.is_object();
    if (ok)
      for (auto& kv : m.obj) ok = ok && kv.second.is_string();
    if (!ok) return invalid("invalid safetensors metadata");
    entries.erase(meta);
  }
  const uint64_t payload_offset = header_len + 8;
  const uint64_t payload = file_len - payload_offset;
  std::vector<std::pair<uint64_t, uint64_t>> ranges;
  for (auto& kv : entries) {
    const std::string& name = kv.first;
    const exl3::json::Value& v = *kv.second;
    Tensor t;
    const exl3::json::Value* dtype = v.find("dtype");
    const exl3::json::Value* shape = v.find("shape");
    const exl3::json::Value* offs = v.find("data_offsets");
    if (!v.is_object() || !dtype || !dtype->is_string() || !shape || !as_shape(*shape, t.shape) ||
        !offs || !offs->is_array() || offs->arr.size() != 2 || !as_u64(offs->arr[0], t.start) ||
        !as_u64(offs->arr[1], t.end))
      return invalid("invalid tensor " + name);
    t.dtype = dtype->str;
    uint64_t item, bytes;
    if (!dtype_size(t.dtype, item)) return invalid("unsupported safetensors dtype " + t.dtype);
    if (!tensor_bytes(t.shape, item, bytes)) return invalid("tensor size overflow");
    // valid_data_range, contracts.rs:1829-1831
    if (!(t.end >= t.start && t.end <= payload && t.end - t.start == bytes))
      return invalid("invalid data range for tensor " + name);
    t.payload = payload_offset;
    t.shard = shard;
    ranges.emplace_back(t.start, t.end);
    out[name] = std::move(t);
  }
  std::sort(ranges.begin(), ranges.end());
  uint64_t end = 0;
  for (auto& r : ranges) {
    if (r.first != end) return invalid("safetensors payload has gaps or overlapping tensors");
    end = r.second;
  }
  if (end != payload) return invalid("unclaimed safetensors payload");
  return Error{};
}

// Validation of the exl3 modules named by tensor_storage and of the shard index
// (checkpoint.rs:247-330).
Error check_storage(exl3_checkpoint& c, const exl3::json::Value& storage) {
  std::map<std::string, const exl3::json::Value*> entries;
  for (auto& kv : storage.obj) entries[kv.first] = &kv.second;
  for (auto& kv : entries) {
    const std::string& prefix = kv.first;
    const exl3::json::Value& meta = *kv.second;
    if (!meta.is_object()) return invalid("invalid tensor_storage entry " + prefix);
    if (const exl3::json::Value* stored = meta.find("stored_tensors")) {
      if (!stored->is_object()) return invalid("invalid stored_tensors");
      std::map<std::string, const exl3::json::Value*> specs;
      for (auto& s : stored->obj) specs[s.first] = &s.second;
      for (auto& s : specs) {
        const std::string& name = s.first;
        std::vector<uint64_t> shape;
        const exl3::json::Value* sh = s.second->find("shape");
        if (!sh || !as_shape(*sh, shape)) return invalid("invalid stored tensor shape");
        auto it = c.tensors.find(name);
        if (it == c.tensors.end() && c.model_type == "lfm2_moe" &&
            starts_with(name, "model.layers.") && ends_with(name, ".feed_forward.gate.expert_bias")) {
          std::string alias = name;
          alias.replace(alias.size() - strlen(".gate.expert_bias"), strlen(".gate.expert_bias"),
                        ".expert_bias");
          it = c.tensors.find(alias);
        }
        if (it == c.tensors.end()) return invalid("missing tensor " + name);
        if (it->second.shape != shape) return invalid("invalid shape for tensor " + name);
      }
    }
    const exl3::json::Value* fmt = meta.find("quant_format");
    if (!fmt || !fmt->string_equals("exl3")) continue;
    auto t = c.tensors.find(prefix + ".trellis");
    if (t == c.tensors.end()) return invalid("missing trellis " + prefix);
    const Tensor& tr = t->second;
    bool ok = (tr.dtype == "U16" || tr.dtype == "I16") && tr.shape.size() == 3;
    for (uint64_t d : tr.shape) ok = ok && d > 0;
    ok = ok && tr.shape[2] % 16 == 0 && tr.shape[2] <= 128;
    if (!ok) return invalid("invalid EXL3 trellis " + prefix);
    const char* names[2][2] = {{"suh", "su"}, {"svh", "sv"}};
    for (int axis = 0; axis < 2; ++axis) {
      auto s = c.tensors.find(prefix + "." + names[axis][0]);
      if (s == c.tensors.end()) s = c.tensors.find(prefix + "." + names[axis][1]);
      if (s == c.tensors.end()) return invalid("missing scale " + prefix + "." + names[axis][0]);
      if (tr.shape[axis] > UINT64_MAX / 16) return invalid("scale length overflow");
      if (s->second.shape != std::vector<uint64_t>{tr.shape[axis] * 16})
        return invalid("invalid scale shape " + prefix + "." + names[axis][0]);
      const std::string& d = s->second.dtype;
      if (d != "F16" && d != "BF16" && d != "F32")
        return invalid("invalid scale dtype " + prefix + "." + names[axis][0]);
    }
    c.modules.push_back(prefix);
  }
  if (c.modules.empty()) return invalid("checkpoint contains no EXL3 modules");
  std::sort(c.modules.begin(), c.modules.end());
  std::string index = c.path + "/model.safetensors.index.json";
  struct stat st;
  if (stat(index.c_str(), &st) == 0) {
    exl3::json::Value v;
    Error e;
    if (!read_json_file(index, v, e)) return e;
    const exl3::json::Value* map = v.find("weight_map");
    if (!map || !map->is_object()) return invalid("invalid shard index");
    for (auto& kv : map->obj) {
      if (!kv.second.is_string()) return invalid("invalid shard name");
      const std::string& shard = kv.second.str;
      if (shard.empty() || shard.find('/') != std::string::npos || shard == "." || shard == "..")
        return invalid("invalid shard path");
      auto it = c.tensors.find(kv.first);
      if (it == c.tensors.end()) return invalid("missing indexed tensor " + kv.first);
      if (c.shards[it->second.shard].file_name != shard)
        return invalid("tensor " + kv.first + " is in the wrong shard");
    }
  }
  return Error{};
}

Error inspect(exl3_checkpoint& c, const char* dir) {
  char* real = realpath(dir, nullptr);
  if (!real) return invalid(strprintf("model directory %s: %s", dir, strerror(errno)));
  c.path = real;
  free(real);
  exl3::json::Value config, quant;
  Error e;
  if (!read_json_file(c.path + "/config.json", config, e)) return e;
  if (!config.is_object()) return invalid("model config must be an object");
  if (!read_json_file(c.path + "/quantization_config.json", quant, e)) return e;
  const exl3::json::Value* method = quant.find("quant_method");
  if (!method || !method->string_equals("exl3")) return invalid("expected quant_method='exl3'");
  const exl3::json::Value* storage = quant.find("tensor_storage");
  if (!storage || !storage->is_object()) return invalid("invalid EXL3 tensor_storage");
  const exl3::json::Value* mt = config.find("model_type");
  c.model_type = mt && mt->is_string() ? mt->str : "unknown";
  const exl3::json::Value* bits = quant.find("bits");
  c.bits = bits && bits->is_number() ? bits->num : NAN;

  DIR* d = opendir(c.path.c_str());
  if (!d) return invalid(strprintf("%s: %s", c.path.c_str(), strerror(errno)));
  std::vector<std::string> files;
  while (dirent* ent = readdir(d)) {
    std::string name = ent->d_name;
    if (name == "." || name == "..") continue;
    files.push_back(name);
  }
  closedir(d);
  std::sort(files.begin(), files.end());
  bool tokenizer = false;
  for (const std::string& name : files) {
    std::string path = c.path + "/" + name;
    struct stat st, lst;
    // Regular files after following links; the size is that of the entry
    // itself (a link counts its own length), as DirEntry::metadata reports.
    if (stat(path.c_str(), &st) != 0 || !S_ISREG(st.st_mode)) continue;
    if (lstat(path.c_str(), &lst) != 0) continue;
    if (c.size_bytes > UINT64_MAX - (uint64_t)lst.st_size) return invalid("checkpoint size overflow");
    c.size_bytes += (uint64_t)lst.st_size;
    tokenizer |= starts_with(name, "tokenizer") || ends_with(name, ".model") || name == "vocab.json";
    bool sidecar = c.model_type == "qwen4_exp" && (name == "ngram_embedding.safetensors" ||
                                                   name == "mtp_hyper_connection_mixer_patch.safetensors");
    if ((starts_with(name, "model") || sidecar) && ends_with(name, ".safetensors")) {
      std::map<std::string, Tensor> shard;
      if (Error he = read_header(c, path, name, shard)) return he;
      for (auto& kv : shard) {
        if (!c.tensors.emplace(kv.first, kv.second).second)
          return invalid("duplicate tensor " + kv.first);
      }
    }
  }
  if (c.tensors.empty()) return invalid("checkpoint has no safetensors weights");
  if (!tokenizer) return invalid("missing tokenizer files; download the complete checkpoint");
  if (Error se = check_storage(c, *storage)) return se;
  c.names.reserve(c.tensors.size());
  for (auto& kv : c.tensors) c.names.push_back(&kv.first);
  return Error{};
}

const Tensor* lookup(const exl3_checkpoint* c, const std::string& name) {
  auto it = c->tensors.find(name);
  return it == c->tensors.end() ? nullptr : &it->second;
}

uint64_t nbytes(const Tensor& t) { return t.end - t.start; }

// TensorInfo::source + read_bytes (checkpoint.rs:96-125).
Error read_tensor(const exl3_checkpoint* c, const Tensor& t, void* dst) {
  const Shard& s = c->shards[t.shard];
  uint64_t abs_end = t.payload + t.end;
  struct stat st;
  if (fstat(s.fd, &st) != 0 || (uint64_t)st.st_size < abs_end)
    return invalid("checkpoint was truncated after inspection");
  if (!read_full(s.fd, dst, nbytes(t), t.payload + t.start))
    return err(EXL3_EDEVICE, strprintf("reading %s failed", s.path.c_str()));
  return Error{};
}

// checkpoint_dtype, linear.rs:346-358: the tensor types a model may hold.
Error model_dtype(const Tensor& t, const std::string& name) {
  static const char* kOk[] = {"F16", "BF16", "F32", "U16", "I16", "U32", "I32", "BOOL"};
  for (const char* d : kOk)
    if (t.dtype == d) return Error{};
  return invalid("unsupported model tensor dtype " + t.dtype + " (" + name + ")");
}

// IEEE binary32 -> binary16, round to nearest even (overflow to infinity,
// gradual underflow, NaN kept quiet with its sign).
uint16_t f32_to_f16(uint32_t x) {
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
  if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // >= 65520 (and inf)
  if (ax >= 0x38800000u) {                                   // normal f16
    uint32_t h = (ax - 0x38000000u) >> 13;
    uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  int exp = (int)(ax >> 23);
  if (exp < 102) return (uint16_t)sign;  // below 2^-25 (and f32 subnormals): zero
  uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
  int shift = 126 - exp;  // 14..24: f16 subnormal units of 2^-24
  uint32_t m = mant >> shift;
  uint32_t rem = mant & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (m & 1u))) ++m;
  return (uint16_t)(sign | m);
}

// Converts a float tensor's payload to f16 (MLX astype(Float16)).
Error to_f16(const std::string& dtype, const std::string& name, const std::vector<char>& raw,
             uint16_t* out, size_t count) {
  if (dtype == "F16") {
    memcpy(out, raw.data(), count * 2);
  } else if (dtype == "BF16") {
    for (size_t i = 0; i < count; ++i) {
      uint16_t b;
      memcpy(&b, raw.data() + 2 * i, 2);
      out[i] = f32_to_f16((uint32_t)b << 16);
    }
  } else if (dtype == "F32") {
    for (size_t i = 0; i < count; ++i) {
      uint32_t w;
      memcpy(&w, raw.data() + 4 * i, 4);
      out[i] = f32_to_f16(w);
    }
  } else {
    return err(EXL3_EUNSUPPORTED, "cannot convert " + dtype + " tensor " + name + " to F16");
  }
  return Error{};
}

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

// One device allocation for a handle's weights, filled from host images.
struct Upload {
  std::vector<std::pair<const void*, size_t>> parts;
  std::vector<size_t> offsets;
  size_t total = 0;
  size_t add(const void* src, size_t bytes) {
    size_t off = total;
    parts.emplace_back(src, bytes);
    offsets.push_back(off);
    total = align256(off + bytes);
    return off;
  }
  Error run(char*& dev) {
    dev = nullptr;
    hipError_t e = hipMalloc((void**)&dev, std::max<size_t>(total, 256));
    if (e != hipSuccess)
      return err(EXL3_EDEVICE, strprintf("hipMalloc of %zu bytes: %s", total, hipGetErrorString(e)));
    for (size_t i = 0; i < parts.size(); ++i) {
      if (!parts[i].second) continue;
      e = hipMemcpy(dev + offsets[i], parts[i].first, parts[i].second, hipMemcpyHostToDevice);
      if (e != hipSuccess) {
        (void)hipFree(dev);
        dev = nullptr;
        return err(EXL3_EDEVICE, strprintf("hipMemcpy: %s", hipGetErrorString(e)));
      }
    }
    return Error{};
  }
};

std::string scale_key(const exl3_checkpoint* c, const std::string& base, const char* primary,
                      const char* legacy) {
  std::string key = base + "." + primary;
  return lookup(c, key) ? key : base + "." + legacy;
}

int codebook_of(const exl3_checkpoint* c, const std::string& prefix) {
  if (lookup(c, prefix + ".mul1")) return EXL3_CB_MUL1;
  if (lookup(c, prefix + ".mcg")) return EXL3_CB_MCG;
  return EXL3_CB_3INST;
}

Error load_linear(const exl3_checkpoint* c, const std::string& prefix, exl3_linear** out) {
  // Tensors resolve in the reference's order: trellis, bias, then the scales.
  const std::string tname = prefix + ".trellis";
  const Tensor* tr = lookup(c, tname);
  if (!tr) return invalid("missing tensor " + tname);
  if (Error e = model_dtype(*tr, tname)) return e;
  for (uint64_t d : tr->shape)
    if (d > INT32_MAX) return invalid("tensor " + tname + " dimension exceeds i32");
  const int cb = codebook_of(c, prefix);
  const std::string bname = prefix + ".bias";
  const Tensor* bias = lookup(c, bname);
  if (bias) {
    if (Error e = model_dtype(*bias, bname)) return e;
  }
  if (tr->shape.empty()) return invalid("trellis must have dimensions");
  const uint64_t k = tr->shape.back() / 16;
  const std::string sname = scale_key(c, prefix, "suh", "su");
  const std::string vname = scale_key(c, prefix, "svh", "sv");
  const Tensor* suh = lookup(c, sname);
  if (!suh) return invalid("missing tensor " + sname);
  if (Error e = model_dtype(*suh, sname)) return e;
  const Tensor* svh = lookup(c, vname);
  if (!svh) return invalid("missing tensor " + vname);
  if (Error e = model_dtype(*svh, vname)) return e;
  // Exl3Linear::new, linear.rs:577-607.
  if (k < 1 || k > 8) return invalid(strprintf("K must be in 1..=8, got %llu", (unsigned long long)k));
  bool shape_ok = tr->shape.size() == 3 && tr->shape[2] == 16 * k;
  for (uint64_t d : tr->shape) shape_ok = shape_ok && d > 0;
  if (!shape_ok) return invalid("invalid trellis shape");
  const uint64_t rows = tr->shape[0] * 16, cols = tr->shape[1] * 16;
  if (rows > INT32_MAX || cols > INT32_MAX) return invalid("row overflow");
  if (rows % 128 || cols % 128)
    return invalid("public EXL3 projections require 128-aligned dimensions");
  if (suh->shape != std::vector<uint64_t>{rows} || svh->shape != std::vector<uint64_t>{cols})
    return invalid("EXL3 scales have wrong dimensions");
  if (bias && bias->shape != std::vector<uint64_t>{cols})
    return invalid("EXL3 bias has wrong dimensions");
  if (tr->dtype != "U16" && tr->dtype != "I16")
    return invalid("EXL3 trellis must contain 16-bit integers");

  std::vector<char> trellis, raw;
  std::vector<uint16_t> s16(rows), v16(cols), b16(bias ? cols : 0);
  try {
    trellis.resize(nbytes(*tr));
  } catch (const std::bad_alloc&) {
    return err(EXL3_ENOMEM, "not enough memory for tensor " + tname);
  }
  if (Error e = read_tensor(c, *tr, trellis.data())) return e;
  struct Scale {
    const Tensor* t;
    const std::string* name;
    uint16_t* dst;
    size_t n;
  } scales[3] = {{suh, &sname, s16.data(), rows}, {svh, &vname, v16.data(), cols},
                 {bias, &bname, b16.data(), cols}};
  for (auto& s : scales) {
    if (!s.t) continue;
    raw.resize(nbytes(*s.t));
    if (Error e = read_tensor(c, *s.t, raw.data())) return e;
    if (Error e = to_f16(s.t->dtype, *s.name, raw, s.dst, s.n)) return e;
  }
  Upload up;
  size_t o_tr = up.add(trellis.data(), trellis.size());
  size_t o_s = up.add(s16.data(), rows * 2);
  size_t o_v = up.add(v16.data(), cols * 2);
  size_t o_b = bias ? up.add(b16.data(), cols * 2) : 0;
  char* dev;
  if (Error e = up.run(dev)) return e;
  exl3_linear* h = nullptr;
  int st = exl3_linear_create((const uint16_t*)(dev + o_tr), (int)rows, (int)cols, (int)k, cb,
                              (const uint16_t*)(dev + o_s), (const uint16_t*)(dev + o_v),
                              bias ? (const uint16_t*)(dev + o_b) : nullptr, &h);
  if (st != EXL3_OK) {
    (void)hipFree(dev);
    return err(st, exl3_last_error());
  }
  exl3::adopt_device_memory(h, dev);
  *out = h;
  return Error{};
}

// Exl3SwitchGlu::from_checkpoint_names, moe.rs:681-800.  The bank is assembled
// on the host: gate trellises of experts 0..E-1 then up trellises concatenated
// along the output-tile axis, down trellises likewise; scales stacked per
// expert ([E][2][in], [E][2][H], [E][H], [E][in]).
// logical_hidden > 0: a GELU bank (from_gemma_checkpoint, moe.rs:663-680).
Error load_moe(const exl3_checkpoint* c, const std::string& prefix, int experts, int top_k,
               const char* const proj[3], int logical_hidden, exl3_moe** out) {
  if (!(experts > 0 && top_k > 0 && top_k <= experts &&
        (uint64_t)experts <= c->tensors.size() / 3))
    return invalid("invalid expert count or incomplete expert bank");
  std::vector<std::string> names[3];
  for (int p = 0; p < 3; ++p)
    for (int e = 0; e < experts; ++e) names[p].push_back(strprintf("%s.%d.%s", prefix.c_str(), e, proj[p]));
  int64_t k = -1;
  int cb = -1;
  for (int p = 0; p < 3; ++p)
    for (const std::string& name : names[p]) {
      const Tensor* t = lookup(c, name + ".trellis");
      if (!t) return invalid("missing expert trellis " + name);
      if (t->dtype != "I16" && t->dtype != "U16")
        return invalid(name + ": expert trellis must contain 16-bit integers");
      if (t->shape.empty()) return invalid("empty expert trellis");
      int64_t bits = (int64_t)(t->shape.back() / 16);
      if (k >= 0 && k != bits) return invalid("mixed expert bit widths");
      k = bits;
      int mode = codebook_of(c, name);
      if (cb >= 0 && cb != mode) return invalid("mixed expert codebooks");
      cb = mode;
    }
  // Shapes every expert must share; the concatenated bank then has the
  // layout new_with_activation checks (moe.rs:849-875).
  const Tensor* g0 = lookup(c, names[0][0] + ".trellis");
  if (g0->shape.size() != 3) return invalid("SwitchGLU trellis/scales disagree");
  const uint64_t in = g0->shape[0] * 16, hidden = g0->shape[1] * 16, packed = g0->shape[2];
  if (in > INT32_MAX || hidden > INT32_MAX || (uint64_t)experts * hidden > INT32_MAX ||
      (uint64_t)experts * in > INT32_MAX || k < 1 || k > 8 || k == 7 || in % 128 || hidden % 128 ||
      packed != (uint64_t)(16 * k))
    return invalid("invalid or overflowing SwitchGLU dimensions");
  const std::vector<uint64_t> gu_shape{in / 16, hidden / 16, packed};
  const std::vector<uint64_t> dn_shape{hidden / 16, in / 16, packed};
  const char* kinds[2][2] = {{"suh", "su"}, {"svh", "sv"}};
  for (int p = 0; p < 3; ++p)
    for (const std::string& name : names[p]) {
      const Tensor* t = lookup(c, name + ".trellis");
      if (t->shape != (p < 2 ? gu_shape : dn_shape)) return invalid("SwitchGLU trellis/scales disagree");
      for (int s = 0; s < 2; ++s) {
        std::string key = scale_key(c, name, kinds[s][0], kinds[s][1]);
        const Tensor* st = lookup(c, key);
        if (!st) return invalid("missing tensor " + key);
        if (Error e = model_dtype(*st, key)) return e;
        uint64_t want = (p < 2) == (s == 0) ? in : hidden;
        if (st->shape != std::vector<uint64_t>{want}) return invalid("SwitchGLU trellis/scales disagree");
        // The expert kernels read the scales as f16 (the reference reads them
        // at their stored type); only f16 banks load.
        if (st->dtype != "F16")
          return err(EXL3_EUNSUPPORTED,
                     "SwitchGLU scale " + key + " is " + st->dtype + "; this build loads F16 banks");
      }
    }
  const size_t E = (size_t)experts;
  const size_t tile_words = (size_t)packed;  // u16 per 16x16 tile
  const size_t gu_row = 2 * E * (hidden / 16) * tile_words;  // u16 per input tile row
  const size_t dn_row = E * (in / 16) * tile_words;
  std::vector<uint16_t> gu, dn, gu_suh, gu_svh, dn_suh, dn_svh;
  std::vector<char> raw;
  try {
    gu.resize((in / 16) * gu_row);
    dn.resize((hidden / 16) * dn_row);
    gu_suh.resize(E * 2 * in);
    gu_svh.resize(E * 2 * hidden);
    dn_suh.resize(E * hidden);
    dn_svh.resize(E * in);
  } catch (const std::bad_alloc&) {
    return err(EXL3_ENOMEM, "not enough host memory for the expert bank");
  }
  for (int p = 0; p < 3; ++p)
    for (size_t e = 0; e < E; ++e) {
      const std::string& name = names[p][e];
      const Tensor* t = lookup(c, name + ".trellis");
      raw.resize(nbytes(*t));
      if (Error er = read_tensor(c, *t, raw.data())) return er;
      const uint64_t rows = t->shape[0], cols = t->shape[1];
      const size_t run = cols * tile_words;  // u16 of one tile row of this expert
      uint16_t* dst = p < 2 ? gu.data() : dn.data();
      const size_t stride = p < 2 ? gu_row : dn_row;
      const size_t col0 = (p == 1 ? E + e : e) * run;
      for (uint64_t r = 0; r < rows; ++r)
        memcpy(dst + r * stride + col0, raw.data() + r * run * 2, run * 2);
      for (int s = 0; s < 2; ++s) {
        const Tensor* st = lookup(c, scale_key(c, name, kinds[s][0], kinds[s][1]));
        raw.resize(nbytes(*st));
        if (Error er = read_tensor(c, *st, raw.data())) return er;
        uint16_t* sdst;
        if (p < 2)
          sdst = s == 0 ? gu_suh.data() + (e * 2 + p) * in : gu_svh.data() + (e * 2 + p) * hidden;
        else
          sdst = s == 0 ? dn_suh.data() + e * hidden : dn_svh.data() + e * in;
        memcpy(sdst, raw.data(), raw.size());
      }
    }
  Upload up;
  size_t o[6];
  o[0] = up.add(gu.data(), gu.size() * 2);
  o[1] = up.add(gu_suh.data(), gu_suh.size() * 2);
  o[2] = up.add(gu_svh.data(), gu_svh.size() * 2);
  o[3] = up.add(dn.data(), dn.size() * 2);
  o[4] = up.add(dn_suh.data(), dn_suh.size() * 2);
  o[5] = up.add(dn_svh.data(), dn_svh.size() * 2);
  char* dev;
  if (Error er = up.run(dev)) return er;
  exl3_moe* h = nullptr;
  auto P = [&](int i) { return (const uint16_t*)(dev + o[i]); };
  int st = logical_hidden > 0
               ? exl3_moe_create_gelu(P(0), P(1), P(2), P(3), P(4), P(5), (int)in, (int)hidden,
                                      experts, top_k, (int)k, cb, logical_hidden, &h)
               : exl3_moe_create(P(0), P(1), P(2), P(3), P(4), P(5), (int)in, (int)hidden,
                                 experts, top_k, (int)k, cb, &h);
  if (st != EXL3_OK) {
    (void)hipFree(dev);
    return err(st, exl3_last_error());
  }
  exl3::adopt_device_memory(h, dev);
  *out = h;
  return Error{};
}

}  // namespace

extern "C" {

int exl3_checkpoint_open(const char* dir, exl3_checkpoint** out) {
  if (!out) return fail(EXL3_EINVAL, "null output handle pointer");
  *out = nullptr;
  if (!dir) return fail(EXL3_EINVAL, "null model directory");
  exl3_checkpoint* c = new (std::nothrow) exl3_checkpoint;
  if (!c) return fail(EXL3_ENOMEM, "out of host memory");
  Error e;
  try {
    e = inspect(*c, dir);
  } catch (const std::bad_alloc&) {
    e = err(EXL3_ENOMEM, "out of host memory");
  }
  if (e) {
    delete c;
    return raise(e);
  }
  *out = c;
  return EXL3_OK;
}

void exl3_checkpoint_close(exl3_checkpoint* c) { delete c; }

const char* exl3_checkpoint_path(const exl3_checkpoint* c) { return c ? c->path.c_str() : ""; }

const char* exl3_checkpoint_model_type(const exl3_checkpoint* c) {
  return c ? c->model_type.c_str() : "";
}

double exl3_checkpoint_bits(const exl3_checkpoint* c) { return c ? c->bits : NAN; }

uint64_t exl3_checkpoint_size_bytes(const exl3_checkpoint* c) { return c ? c->size_bytes : 0; }

int32_t exl3_checkpoint_module_count(const exl3_checkpoint* c) {
  return c ? (int32_t)c->modules.size() : 0;
}

const char* exl3_checkpoint_module(const exl3_checkpoint* c, int32_t i) {
  if (!c || i < 0 || (size_t)i >= c->modules.size()) return nullptr;
  return c->modules[(size_t)i].c_str();
}

int64_t exl3_checkpoint_tensor_count(const exl3_checkpoint* c) {
  return c ? (int64_t)c->names.size() : 0;
}

const char* exl3_checkpoint_tensor_name(const exl3_checkpoint* c, int64_t i) {
  if (!c || i < 0 || (size_t)i >= c->names.size()) return nullptr;
  return c->names[(size_t)i]->c_str();
}

int exl3_checkpoint_tensor(const exl3_checkpoint* c, const char* name, exl3_tensor_info* info) {
  if (!c || !name || !info) return fail(EXL3_EINVAL, "null checkpoint argument");
  const Tensor* t = lookup(c, name);
  if (!t) return fail(EXL3_EINVAL, "missing tensor %s", name);
  if (t->shape.size() > 8) return fail(EXL3_EUNSUPPORTED, "tensor %s has more than 8 dimensions", name);
  memset(info, 0, sizeof *info);
  snprintf(info->dtype, sizeof info->dtype, "%s", t->dtype.c_str());
  info->ndim = (int32_t)t->shape.size();
  for (size_t i = 0; i < t->shape.size(); ++i) info->shape[i] = (int64_t)t->shape[i];
  info->offset = t->payload + t->start;
  info->bytes = nbytes(*t);
  info->shard = c->shards[t->shard].path.c_str();
  return EXL3_OK;
}

int exl3_checkpoint_read(const exl3_checkpoint* c, const char* name, void* dst, size_t bytes) {
  if (!c || !name) return fail(EXL3_EINVAL, "null checkpoint argument");
  const Tensor* t = lookup(c, name);
  if (!t) return fail(EXL3_EINVAL, "missing tensor %s", name);
  if (bytes != nbytes(*t))
    return fail(EXL3_EINVAL, "tensor %s has %llu bytes, buffer has %zu", name,
                (unsigned long long)nbytes(*t), bytes);
  if (bytes && !dst) return fail(EXL3_EINVAL, "null destination");
  if (Error e = read_tensor(c, *t, dst)) return raise(e);
  return EXL3_OK;
}

int exl3_checkpoint_read_f16(const exl3_checkpoint* c, const char* name, uint16_t* dst,
                             size_t count) {
  if (!c || !name) return fail(EXL3_EINVAL, "null checkpoint argument");
  const Tensor* t = lookup(c, name);
  if (!t) return fail(EXL3_EINVAL, "missing tensor %s", name);
  uint64_t n = 1;
  for (uint64_t d : t->shape) n *= d;  // bounded: the payload size was checked
  if (count != n)
    return fail(EXL3_EINVAL, "tensor %s has %llu elements, buffer has %zu", name,
                (unsigned long long)n, count);
  if (count && !dst) return fail(EXL3_EINVAL, "null destination");
  Error e;
  try {
    std::vector<char> raw(nbytes(*t));
    e = read_tensor(c, *t, raw.data());
    if (!e) e = to_f16(t->dtype, name, raw, dst, count);
  } catch (const std::bad_alloc&) {
    e = err(EXL3_ENOMEM, "out of host memory");
  }
  return e ? raise(e) : EXL3_OK;
}

int exl3_linear_load(const exl3_checkpoint* c, const char* prefix, exl3_linear** out) {
  if (!out) return fail(EXL3_EINVAL, "null output handle pointer");
  *out = nullptr;
  if (!c || !prefix) return fail(EXL3_EINVAL, "null checkpoint argument");
  Error e;
  try {
    e = load_linear(c, prefix, out);
  } catch (const std::bad_alloc&) {
    e = err(EXL3_ENOMEM, "out of host memory");
  }
  return e ? raise(e) : EXL3_OK;
}

int exl3_moe_load(const exl3_checkpoint* c, const char* prefix, int32_t experts, int32_t top_k,
                  const char* gate, const char* up, const char* down, exl3_moe** out) {
  if (!out) return fail(EXL3_EINVAL, "null output handle pointer");
  *out = nullptr;
  if (!c || !prefix) return fail(EXL3_EINVAL, "null checkpoint argument");
  const char* proj[3] = {gate ? gate : "gate_proj", up ? up : "up_proj", down ? down : "down_proj"};
  Error e;
  try {
    e = load_moe(c, prefix, experts, top_k, proj, 0, out);
  } catch (const std::bad_alloc&) {
    e = err(EXL3_ENOMEM, "out of host memory");
  }
  return e ? raise(e) : EXL3_OK;
}

int exl3_moe_load_gemma(const exl3_checkpoint* c, const char* prefix, int32_t experts,
                        int32_t top_k, int32_t logical_hidden, exl3_moe** out) {
  if (!out) return fail(EXL3_EINVAL, "null output handle pointer");
  *out = nullptr;
  if (!c || !prefix) return fail(EXL3_EINVAL, "null checkpoint argument");
  if (logical_hidden <= 0) return fail(EXL3_EINVAL, "invalid logical GLU width");
  const char* proj[3] = {"gate_proj", "up_proj", "down_proj"};
  Error e;
  try {
    e = load_moe(c, prefix, experts, top_k, proj, logical_hidden, out);
  } catch (const std::bad_alloc&) {
    e = err(EXL3_ENOMEM, "out of host memory");
  }
  return e ? raise(e) : EXL3_OK;
}

}  // extern "C"
