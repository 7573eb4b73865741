// exl3_codec: the reference engine's `codec` JSON-lines protocol
// (codec_loop, native/src/main.rs:286-1360; request fields CodecRequest
// main.rs:78-270) served by this library, so the reference's harnesses that
// drive `mlxl3-rs codec` (e.g. docs/native-coverage/baselines/exl3/
// check-metal-tiles.py.txt) can drive the HIP build instead.
//
// One request per input line, one response per output line:
// {"data": ...} or {"error": "..."}.  Operations:
//   pack, permutation                 host (codec.rs:73-100, :126-138)
//   unpack, metal-decode              GPU tile decode (exl3_decode_tiles)
//   metal-pack                        GPU tile pack (exl3_pack_tiles)
//   codebook                          GPU codewords (exl3_codewords)
//   metal-qmv                         GPU inner QMV (exl3_qmv_inner)
//   metal-swiglu                      GPU SwiGLU (exl3_swiglu)
//   metal-prepare128, -prepare-view   GPU input prologue (exl3_prepare128), the
//                                     latter on strided f16/f32 views
//   mlx-linear, mlx-group             GPU Exl3Linear / Exl3Group forward
//   mlx-switch                        GPU Exl3SwitchGlu forward (bank in the request)
//   mlx-checkpoint-switch/-group      the same on projections of a checkpoint
//   mlx-swiglu-prepare, mlx-expert-reduce   the SwitchGLU glue steps
//   mlx-expert                        GPU mapped expert QMV (exl3_expert_mapped)
//   metal-checkpoint-linear, metal-exl3-linear, metal-checkpoint-expert,
//   metal-checkpoint-group            checkpoint projections, dense experts and
//                                     projection bundles under the direct-Metal
//                                     path's geometry and input checks
// Any other op answers "unknown or unavailable codec operation <op>", as a
// reference build without the feature does.  The GPU is initialised on the
// first request that needs it.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <iostream>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/exl3_hip.h"
#include "exl3_json.hpp"

namespace {

using exl3::json::Value;

struct Failure {
  std::string msg;
};
[[noreturn]] void bail(const std::string& msg) { throw Failure{msg}; }

// ---- request (CodecRequest: serde defaults, unknown fields ignored) ---------
struct Request {
  std::string op;
  uint64_t k = 4;  // default_k, main.rs:273-275
  uint64_t mode = 0;
  uint64_t cols = 0;
  uint64_t key_heads = 0, top_k = 0;
  std::vector<uint16_t> data, x, suh, svh, beta, down_data, down_suh, down_svh;
  std::vector<uint32_t> selected;
  std::vector<float> state, x_f32;
  bool has_x_f32 = false;
  // MatrixLayout (tensor_layout.rs:6-10) of x and of the scales, when given
  struct Layout {
    bool given = false;
    uint32_t shape[2] = {0, 0};
    int64_t strides[2] = {0, 0};
    int64_t offset = 0;
  } x_layout, scale_layout;
  std::vector<uint64_t> widths;
  std::string path, prefix;
  std::vector<std::string> prefixes;
  uint64_t projections_per_route = 0, projection_stride_tiles = 0;
  bool return_raw = false;
};

std::vector<uint32_t> u32_array(const Value* v, const char* field) {
  std::vector<uint32_t> out;
  if (!v) return out;
  if (!v->is_array()) bail(std::string("invalid codec request: ") + field + " must be an array");
  for (const Value& e : v->arr) {
    if (!e.is_number() || !e.is_uint || e.u > 0xFFFFFFFFull)
      bail(std::string("invalid codec request: ") + field + " must hold u32 values");
    out.push_back((uint32_t)e.u);
  }
  return out;
}

uint64_t uint_field(const Value* v, const char* field, uint64_t dflt, uint64_t max);

int64_t i64_value(const Value& e, const char* field) {
  if (e.is_number() && e.is_uint && e.u <= (uint64_t)INT64_MAX) return (int64_t)e.u;
  if (e.is_number() && !e.is_uint && e.num < 0 && e.num >= -9.2233720368547758e18 &&
      e.num == (double)(int64_t)e.num)
    return (int64_t)e.num;
  bail(std::string("invalid codec request: ") + field + " must hold i64 values");
}

Request::Layout layout_field(const Value* v, const char* field) {
  Request::Layout l;
  if (!v || v->kind == exl3::json::Kind::Null) return l;
  const Value* shape = v->find("shape");
  const Value* strides = v->find("strides");
  const Value* offset = v->find("offset");
  if (!v->is_object() || !shape || !shape->is_array() || shape->arr.size() != 2 || !strides ||
      !strides->is_array() || strides->arr.size() != 2 || !offset)
    bail(std::string("invalid codec request: ") + field + " must be a matrix layout");
  for (int i = 0; i < 2; ++i) {
    l.shape[i] = (uint32_t)uint_field(&shape->arr[i], field, 0, UINT32_MAX);
    l.strides[i] = i64_value(strides->arr[i], field);
  }
  l.offset = i64_value(*offset, field);
  l.given = true;
  return l;
}

// MatrixLayout::fits (tensor_layout.rs:67-85): both extrema of the view inside
// `elements`; an empty view may start one element past the end.
bool layout_fits(const Request::Layout& l, uint64_t elements) {
  if (elements > (uint64_t)INT64_MAX) return false;
  const __int128 limit = (__int128)elements;
  if (l.offset < 0 || l.offset > limit) return false;
  if (l.shape[0] == 0 || l.shape[1] == 0) return true;
  __int128 first = l.offset, last = l.offset;
  for (int i = 0; i < 2; ++i) {
    const __int128 reach = (__int128)(l.shape[i] - 1) * l.strides[i];
    first += reach < 0 ? reach : 0;
    last += reach > 0 ? reach : 0;
  }
  return first >= 0 && last < limit;
}

std::string string_field(const Value* v, const char* field) {
  if (!v) return "";
  if (!v->is_string()) bail(std::string("invalid codec request: ") + field + " must be a string");
  return v->str;
}

std::vector<uint16_t> u16_array(const Value* v, const char* field) {
  std::vector<uint16_t> out;
  if (!v) return out;
  if (!v->is_array()) bail(std::string("invalid codec request: ") + field + " must be an array");
  out.reserve(v->arr.size());
  for (const Value& e : v->arr) {
    if (!e.is_number() || !e.is_uint || e.u > 0xFFFF)
      bail(std::string("invalid codec request: ") + field + " must hold u16 values");
    out.push_back((uint16_t)e.u);
  }
  return out;
}

uint64_t uint_field(const Value* v, const char* field, uint64_t dflt, uint64_t max) {
  if (!v) return dflt;
  if (!v->is_number() || !v->is_uint || v->u > max)
    bail(std::string("invalid codec request: ") + field + " must be an unsigned integer");
  return v->u;
}

Request parse_request(const std::string& line) {
  Value v;
  std::string why;
  if (!exl3::json::parse(line.data(), line.size(), v, why)) bail("invalid codec request: " + why);
  if (!v.is_object()) bail("invalid codec request: expected an object");
  Request r;
  const Value* op = v.find("op");
  if (!op || !op->is_string()) bail("invalid codec request: missing field `op`");
  r.op = op->str;
  r.k = uint_field(v.find("k"), "k", 4, UINT64_MAX);
  r.mode = uint_field(v.find("mode"), "mode", 0, UINT32_MAX);
  r.cols = uint_field(v.find("cols"), "cols", 0, UINT64_MAX);
  r.data = u16_array(v.find("data"), "data");
  r.x = u16_array(v.find("x"), "x");
  r.suh = u16_array(v.find("suh"), "suh");
  r.svh = u16_array(v.find("svh"), "svh");
  if (const Value* w = v.find("widths")) {
    if (!w->is_array()) bail("invalid codec request: widths must be an array");
    for (const Value& e : w->arr) r.widths.push_back(uint_field(&e, "widths", 0, UINT64_MAX));
  }
  r.key_heads = uint_field(v.find("key_heads"), "key_heads", 0, UINT64_MAX);
  r.top_k = uint_field(v.find("top_k"), "top_k", 0, UINT64_MAX);
  r.selected = u32_array(v.find("selected"), "selected");
  if (const Value* xf = v.find("x_f32"); xf && xf->kind != exl3::json::Kind::Null) {
    if (!xf->is_array()) bail("invalid codec request: x_f32 must be an array");
    r.has_x_f32 = true;
    for (const Value& e : xf->arr) {
      if (!e.is_number()) bail("invalid codec request: x_f32 must hold numbers");
      r.x_f32.push_back((float)e.num);
    }
  }
  r.x_layout = layout_field(v.find("x_layout"), "x_layout");
  r.scale_layout = layout_field(v.find("scale_layout"), "scale_layout");
  if (const Value* st = v.find("state")) {
    if (!st->is_array()) bail("invalid codec request: state must be an array");
    for (const Value& e : st->arr) {
      if (!e.is_number()) bail("invalid codec request: state must hold numbers");
      r.state.push_back((float)e.num);
    }
  }
  r.beta = u16_array(v.find("beta"), "beta");
  r.down_data = u16_array(v.find("down_data"), "down_data");
  r.down_suh = u16_array(v.find("down_suh"), "down_suh");
  r.down_svh = u16_array(v.find("down_svh"), "down_svh");
  r.path = string_field(v.find("path"), "path");
  r.prefix = string_field(v.find("prefix"), "prefix");
  r.projections_per_route =
      uint_field(v.find("projections_per_route"), "projections_per_route", 0, UINT64_MAX);
  r.projection_stride_tiles =
      uint_field(v.find("projection_stride_tiles"), "projection_stride_tiles", 0, UINT64_MAX);
  if (const Value* rr = v.find("return_raw")) {
    if (rr->kind != exl3::json::Kind::Bool)
      bail("invalid codec request: return_raw must be a boolean");
    r.return_raw = rr->b;
  }
  if (const Value* ps = v.find("prefixes")) {
    if (!ps->is_array()) bail("invalid codec request: prefixes must be an array");
    for (const Value& e : ps->arr) r.prefixes.push_back(string_field(&e, "prefixes"));
  }
  return r;
}

// ---- JSON output ------------------------------------------------------------
std::string json_string(const std::string& s) {
  std::string o = "\"";
  for (unsigned char c : s) {
    if (c == '"' || c == '\\') {
      o += '\\';
      o += (char)c;
    } else if (c < 0x20) {
      char buf[8];
      snprintf(buf, sizeof buf, "\\u%04x", c);
      o += buf;
    } else {
      o += (char)c;
    }
  }
  return o + "\"";
}
template <typename T>
std::string json_list(const std::vector<T>& v) {
  std::string o = "[";
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) o += ',';
    o += std::to_string(v[i]);
  }
  return o + "]";
}

// f32 values as JSON numbers that read back to the same f32 (9 significant
// digits); non-finite values as null, as serde_json writes them
std::string json_f32_list(const std::vector<float>& v) {
  std::string o = "[";
  char buf[32];
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) o += ',';
    if (std::isfinite(v[i])) {
      snprintf(buf, sizeof buf, "%.9g", (double)v[i]);
      o += buf;
    } else {
      o += "null";
    }
  }
  return o + "]";
}

// ---- host codec (the on-disk format) -----------------------------------------
void check_k(uint64_t k) {
  if (k < 1 || k > 8) bail("K must be in 1..=8, got " + std::to_string(k));
}

// pack, codec.rs:73-100: output word `logical` of a tile (stored at
// logical ^ 1) gathers 16 stream bits, most significant first; stream bit sb
// of span logical/k is bit k-1-sb%k of state span*16 + sb/k.
std::vector<uint16_t> pack(const std::vector<uint16_t>& states, int k) {
  std::vector<uint16_t> out(states.size() / 256 * 16 * k);
  for (size_t t = 0; t < states.size() / 256; ++t) {
    const uint16_t* in = &states[t * 256];
    uint16_t* o = &out[t * 16 * k];
    for (int logical = 0; logical < 16 * k; ++logical) {
      uint32_t word = 0;
      const int span = logical / k;
      for (int bit = 0; bit < 16; ++bit) {
        const int sb = (logical % k) * 16 + bit;
        word = (word << 1) | ((in[span * 16 + sb / k] >> (k - 1 - sb % k)) & 1u);
      }
      o[logical ^ 1] = (uint16_t)word;
    }
  }
  return out;
}

// permutation, codec.rs:126-138: stored index 8*lane + 4*cg + ri holds tile
// element (row {r0, r0+1, r0+8, r0+9}[ri], column lane/4 + 8*cg), r0 = 2*(lane%4).
std::vector<uint64_t> permutation() {
  std::vector<uint64_t> p(256);
  for (int lane = 0; lane < 32; ++lane) {
    const int r0 = 2 * (lane % 4), c = lane / 4;
    const int rows[4] = {r0, r0 + 1, r0 + 8, r0 + 9};
    for (int cg = 0; cg < 2; ++cg)
      for (int ri = 0; ri < 4; ++ri) p[lane * 8 + cg * 4 + ri] = rows[ri] * 16 + c + 8 * cg;
  }
  return p;
}

// ---- device plumbing -----------------------------------------------------------
void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) bail(std::string(what) + ": " + hipGetErrorString(e));
}
void lib_check(int rc) {
  if (rc != EXL3_OK) bail(exl3_last_error());
}

struct DeviceBuffer {
  void* p = nullptr;
  size_t bytes = 0;
  explicit DeviceBuffer(size_t n) : bytes(n) {
    hip_check(hipMalloc(&p, n ? n : 16), "hipMalloc");
  }
  template <typename T>
  DeviceBuffer(const std::vector<T>& v) : DeviceBuffer(v.size() * sizeof(T)) {
    if (!v.empty()) hip_check(hipMemcpy(p, v.data(), bytes, hipMemcpyHostToDevice), "hipMemcpy");
  }
  ~DeviceBuffer() { (void)hipFree(p); }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  template <typename T>
  std::vector<T> read(size_t n) const {
    std::vector<T> v(n);
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    if (n) hip_check(hipMemcpy(v.data(), p, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
    return v;
  }
  template <typename T>
  T* as() const {
    return (T*)p;
  }
};

// workspaces come from *_workspace_bytes (multiples of 256 bytes)
void zero_workspace(DeviceBuffer& ws) {
  lib_check(exl3_workspace_init(ws.p, ws.bytes / 4 * 4, nullptr));
}

// states and values of whole tiles (gpu.rs:1498-1521 / metal-decode)
void decode(const std::vector<uint16_t>& packed, int k, int cb, std::vector<uint16_t>* states,
            std::vector<uint16_t>* values) {
  const int64_t tiles = (int64_t)(packed.size() / (16 * k));
  DeviceBuffer in(packed), st(tiles * 256 * 2), val(tiles * 256 * 2);
  lib_check(exl3_decode_tiles(in.as<uint16_t>(), tiles, k, cb, states ? st.as<uint16_t>() : nullptr,
                              val.as<uint16_t>(), nullptr));
  if (states) *states = st.read<uint16_t>(tiles * 256);
  if (values) *values = val.read<uint16_t>(tiles * 256);
}

// switch_glu_route_rows / switch_glu_layout (contracts.rs:4-44)
int64_t route_rows(const std::vector<uint32_t>& ids, uint64_t experts, uint64_t top_k) {
  if (experts == 0 || experts > INT32_MAX || top_k == 0 || top_k > experts || ids.empty() ||
      ids.size() > (size_t)INT32_MAX / 2 || ids.size() % top_k)
    return -1;
  for (uint32_t id : ids)
    if (id >= experts) return -1;
  return (int64_t)(ids.size() / top_k);
}
bool glu_layout_ok(uint64_t experts, uint64_t top_k, uint64_t input, uint64_t hidden, uint64_t k) {
  return experts > 0 && experts <= INT32_MAX && top_k > 0 && top_k <= experts && input > 0 &&
         input <= INT32_MAX && hidden > 0 && hidden <= INT32_MAX && input % 128 == 0 &&
         hidden % 128 == 0 && k >= 1 && k <= 8 && k != 7 &&
         experts * hidden <= INT32_MAX && experts * input <= INT32_MAX;
}
// Array::from_bytes's check (array.rs:884-888) for each tensor of a request
void expect_len(size_t got, uint64_t want) {
  if (got != want) bail("tensor byte count does not match shape and dtype");
}

struct MoeGuard {
  exl3_moe* h = nullptr;
  ~MoeGuard() { exl3_moe_destroy(h); }
};
struct CheckpointGuard {
  exl3_checkpoint* c = nullptr;
  ~CheckpointGuard() { exl3_checkpoint_close(c); }
};

// y[rows][in] of a SwitchGLU handle on f16 x, u32 routes and f16 scores
std::vector<uint16_t> moe_run(exl3_moe* h, const std::vector<uint16_t>& xv,
                              const std::vector<uint32_t>& sel, const std::vector<uint16_t>& sc,
                              int64_t rows) {
  DeviceBuffer x(xv), s(sel), b(sc), y(xv.size() * 2);
  const size_t wb = exl3_moe_workspace_bytes(h, rows);
  if (wb == 0) bail("MoE slot overflow");
  DeviceBuffer ws(wb);
  lib_check(exl3_moe_forward(h, x.p, EXL3_F16, rows, s.as<uint32_t>(), b.p, EXL3_F16, y.p, ws.p,
                             wb, nullptr));
  return y.read<uint16_t>(xv.size());
}

// CodecRequest::input_view (main.rs:261-270) with TensorStorage::matrix
// (gpu/view.rs:30-41): the x_layout view of x (f16 bits) or of x_f32 (f32,
// rounded to f16 as the preparation kernels cast it), gathered row-major.
// Views of more than 2^32 - 1 elements (a zero stride lets a view exceed its
// storage) fail with `too_large` before anything is gathered.
std::vector<uint16_t> gather_view(const Request& r, uint32_t* rows, uint32_t* cols,
                                  const char* too_large) {
  if (!r.x_layout.given) bail("missing input matrix layout");
  if (r.has_x_f32 && !r.x.empty()) bail("conflicting input buffer dtypes");
  if (!layout_fits(r.x_layout, r.has_x_f32 ? r.x_f32.size() : r.x.size()))
    bail("matrix view outside initialized storage");
  const Request::Layout& l = r.x_layout;
  *rows = l.shape[0];
  *cols = l.shape[1];
  if ((uint64_t)l.shape[0] * l.shape[1] > UINT32_MAX) bail(too_large);
  std::vector<uint16_t> out((size_t)l.shape[0] * l.shape[1]);
  for (uint64_t i = 0; i < l.shape[0]; ++i)
    for (uint64_t j = 0; j < l.shape[1]; ++j) {
      const int64_t e = l.offset + (int64_t)i * l.strides[0] + (int64_t)j * l.strides[1];
      out[i * l.shape[1] + j] = r.has_x_f32 ? __builtin_bit_cast(uint16_t, (_Float16)r.x_f32[e])
                                            : r.x[e];
    }
  return out;
}

// The direct-Metal projection path's geometry, FlashProjection::load /
// load_exl3 (gpu/projection.rs:134-205): its split policy decides which
// projections it accepts, so the checks run before anything is uploaded.
struct FlashGeometry {
  uint32_t input = 0, output = 0, splits = 1;
  int k = 0, cb = 0;
  bool generic = false;
};

// flash_support::reference_splits (flash_support.rs:815-823)
uint32_t reference_splits(uint32_t input_tiles, uint32_t output_tiles) {
  uint32_t s = 1;
  while ((uint64_t)output_tiles * s < 8192 && (uint64_t)input_tiles / ((uint64_t)s * 2) >= 128)
    s *= 2;
  return s;
}
// contracts::exl3_projection_splits (contracts.rs:1995-2011); 0 for None
uint32_t exl3_projection_splits(uint32_t input, uint32_t output) {
  if (input == 0 || output == 0 || input % 128 || output % 128) return 0;
  const uint32_t it = input / 16, ot = output / 16;
  const uint32_t target = ot <= 64 ? std::max(ot / 2, 32u) : std::min(std::max(ot, 32u), 256u);
  uint32_t s = 1;
  while (it / s / 2 >= target) s *= 2;
  return s;
}
// contracts::exl3_projection_extents / projection_extents
// (contracts.rs:2014-2027, :2082-2101) for a batch of `batch` rows
bool flash_extents(const FlashGeometry& g, uint64_t batch) {
  if (batch == 0) return false;
  if (g.generic) {
    if (!exl3_projection_splits(g.input, g.output)) return false;
    if (g.splits == 0 || (g.splits & (g.splits - 1)) || g.splits > g.input / 128) return false;
  } else if (g.input > INT32_MAX || g.output > INT32_MAX || g.input % 128 || g.output % 128 ||
             (g.splits != 1 && g.splits != 2)) {
    return false;
  }
  const uint64_t count = batch * g.output;
  return batch * g.input <= UINT32_MAX && count <= UINT32_MAX && count * g.splits <= UINT32_MAX;
}

FlashGeometry flash_geometry(const exl3_checkpoint* c, const std::string& name, bool exl3_loader) {
  const bool flash_ckpt = std::strcmp(exl3_checkpoint_model_type(c), "qwen4_exp") == 0;
  if (!exl3_loader && !flash_ckpt) bail("requires a Flash reference checkpoint");
  FlashGeometry g;
  g.generic = exl3_loader && !flash_ckpt;
  exl3_tensor_info t;
  if (exl3_checkpoint_tensor(c, (name + ".trellis").c_str(), &t) != EXL3_OK)
    bail("missing projection trellis");
  if (t.ndim != 3) bail("invalid trellis rank");
  if ((std::strcmp(t.dtype, "I16") != 0 && std::strcmp(t.dtype, "U16") != 0) || t.shape[2] % 16)
    bail("invalid packed trellis");
  if (t.shape[0] > UINT32_MAX / 16) bail("input width overflow");
  if (t.shape[1] > UINT32_MAX / 16) bail("output width overflow");
  g.input = (uint32_t)(t.shape[0] * 16);
  g.output = (uint32_t)(t.shape[1] * 16);
  const int64_t k = t.shape[2] / 16;
  // contracts::qmv_words (contracts.rs:1875-1886), as a u32 word count
  if (g.input == 0 || g.output == 0 || k < 1 || k > 8 ||
      (uint64_t)t.shape[0] * t.shape[1] * 16 * k > UINT32_MAX)
    bail("invalid packed geometry or index overflow");
  g.k = (int)k;
  exl3_tensor_info m;
  g.cb = exl3_checkpoint_tensor(c, (name + ".mul1").c_str(), &m) == EXL3_OK  ? 2
         : exl3_checkpoint_tensor(c, (name + ".mcg").c_str(), &m) == EXL3_OK ? 1
                                                                             : 0;
  const bool mtp_hidden = !g.generic && name == "mtp.fc_hidden";
  if (mtp_hidden && (g.input != 2560 || g.output != 2560 || g.k == 7))
    bail("unsupported MTP hidden projection");
  if (mtp_hidden) {
    g.splits = 2;
  } else if (g.k == 7) {
    g.splits = 1;
  } else if (g.generic) {
    g.splits = exl3_projection_splits(g.input, g.output);
    if (!g.splits) bail("invalid EXL3 dimensions");
  } else {
    g.splits = reference_splits(g.input / 16, g.output / 16);
  }
  if (!flash_extents(g, 1)) bail("unsupported projection geometry/split count");
  return g;
}

struct LinearGuard {
  exl3_linear* h = nullptr;
  ~LinearGuard() { exl3_linear_destroy(h); }
};

// y[rows][out] (f16) of one loaded projection on f16 rows
std::vector<uint16_t> linear_run(const exl3_linear* h, const std::vector<uint16_t>& xv,
                                 int64_t rows) {
  const int64_t out = exl3_linear_out_features(h);
  DeviceBuffer x(xv), y((size_t)rows * out * 2);
  const size_t wb = exl3_linear_workspace_bytes(h, rows);
  DeviceBuffer ws(wb);
  zero_workspace(ws);
  lib_check(exl3_linear_forward(h, x.p, EXL3_F16, rows, y.p, EXL3_F16, ws.p, wb, nullptr));
  return y.read<uint16_t>((size_t)rows * out);
}

// {"grouped": .., "outputs": [..]} of loaded projections on one f16 row: one
// exl3_group_forward launch for a compatible bundle of at most 8 projections
// (Exl3Group::forward), else each projection's own forward.  The two can
// differ in the last bit where the group's wider output changes the split-K
// order, so both bundle ops take the same route for the same bundle.
std::string group_outputs(const std::vector<exl3_linear*>& parts, bool grouped,
                          const std::vector<uint16_t>& xv) {
  const bool one_launch = grouped && parts.size() <= 8;
  DeviceBuffer x(xv);
  std::vector<std::unique_ptr<DeviceBuffer>> ys;
  std::vector<void*> yp;
  for (auto* h : parts) {
    ys.emplace_back(new DeviceBuffer((size_t)exl3_linear_out_features(h) * 2));
    yp.push_back(ys.back()->p);
  }
  if (one_launch) {
    const size_t wb = exl3_group_workspace_bytes(parts.data(), (int)parts.size(), 1);
    DeviceBuffer ws(wb);
    zero_workspace(ws);
    lib_check(exl3_group_forward(parts.data(), (int)parts.size(), x.p, EXL3_F16, 1, yp.data(),
                                 ws.p, wb, nullptr));
  } else {
    for (size_t i = 0; i < parts.size(); ++i) {
      const size_t wb = exl3_linear_workspace_bytes(parts[i], 1);
      DeviceBuffer ws(wb);
      zero_workspace(ws);
      lib_check(exl3_linear_forward(parts[i], x.p, EXL3_F16, 1, yp[i], EXL3_F16, ws.p, wb,
                                    nullptr));
    }
  }
  std::string out = std::string("{\"grouped\":") + (grouped ? "true" : "false") + ",\"outputs\":[";
  for (size_t i = 0; i < ys.size(); ++i) {
    if (i) out += ',';
    out += json_list(ys[i]->read<uint16_t>(exl3_linear_out_features(parts[i])));
  }
  return out + "]}";
}

// ---- operations ------------------------------------------------------------
std::string run(const Request& r) {
  if (r.mode > 2) bail("invalid EXL3 codebook " + std::to_string(r.mode));
  const int cb = (int)r.mode;
  if (r.op == "pack") {
    check_k(r.k);
    if (r.data.size() % 256) bail("encoded length must be a multiple of 256");
    return json_list(pack(r.data, (int)r.k));
  }
  if (r.op == "unpack") {
    check_k(r.k);
    if (r.data.size() % (16 * r.k)) bail("packed length is not a whole tile");
    std::vector<uint16_t> states;
    if (!r.data.empty()) decode(r.data, (int)r.k, cb, &states, nullptr);
    return json_list(states);
  }
  if (r.op == "codebook") {
    std::vector<uint16_t> values;
    if (!r.data.empty()) {
      DeviceBuffer in(r.data), out(r.data.size() * 2);
      lib_check(exl3_codewords(in.as<uint16_t>(), (int64_t)r.data.size(), cb, out.as<uint16_t>(),
                               nullptr));
      values = out.read<uint16_t>(r.data.size());
    }
    return json_list(values);
  }
  if (r.op == "permutation") return json_list(permutation());
  if (r.op == "metal-decode") {
    check_k(r.k);
    if (r.data.size() % (16 * r.k)) bail("expected whole packed tiles");
    std::vector<uint16_t> states, values;
    if (!r.data.empty()) decode(r.data, (int)r.k, cb, &states, &values);
    return "{\"states\":" + json_list(states) + ",\"values\":" + json_list(values) + "}";
  }
  if (r.op == "metal-qmv") {
    check_k(r.k);
    const uint64_t rows = r.x.size(), cols = r.cols;
    if (!(rows > 0 && cols > 0 && rows % 16 == 0 && cols % 16 == 0))
      bail("expected positive 16-aligned dimensions");
    if (rows > INT32_MAX || cols > INT32_MAX || r.data.size() != rows / 16 * (cols / 16) * 16 * r.k)
      bail("invalid trellis size or Metal index overflow");
    DeviceBuffer packed(r.data), x(r.x), y(cols * 2);
    const size_t wb = exl3_qmv_inner_workspace_bytes((int)rows, (int)cols);
    DeviceBuffer ws(wb);
    lib_check(exl3_qmv_inner(packed.as<uint16_t>(), (int)rows, (int)cols, (int)r.k, cb,
                             x.as<uint16_t>(), y.as<uint16_t>(), ws.p, wb, nullptr));
    return json_list(y.read<uint16_t>(cols));
  }
  if (r.op == "metal-swiglu") {
    if (r.x.empty() || r.x.size() != r.data.size()) bail("invalid SwiGLU input extents");
    DeviceBuffer g(r.x), u(r.data), o(r.x.size() * 2);
    lib_check(exl3_swiglu(g.as<uint16_t>(), u.as<uint16_t>(), o.as<uint16_t>(),
                          (int64_t)r.x.size(), nullptr));
    return json_list(o.read<uint16_t>(r.x.size()));
  }
  if (r.op == "metal-pack") {  // main.rs:1343, gpu.rs:1470-1495
    check_k(r.k);
    if (r.data.size() % 256) bail("expected whole 256-state tiles");
    if (r.data.empty()) return "[]";
    const int64_t tiles = (int64_t)(r.data.size() / 256);
    DeviceBuffer st(r.data), out((size_t)tiles * 16 * r.k * 2);
    lib_check(exl3_pack_tiles(st.as<uint16_t>(), tiles, (int)r.k, out.as<uint16_t>(), nullptr));
    return json_list(out.read<uint16_t>((size_t)tiles * 16 * r.k));
  }
  if (r.op == "metal-prepare-view") {  // main.rs:1294-1302, gpu/view.rs:181-195, :257-272
    uint32_t rows = 0, cols = 0;
    if (!r.x_layout.given) bail("missing input matrix layout");
    if (r.has_x_f32 && !r.x.empty()) bail("conflicting input buffer dtypes");
    if (!layout_fits(r.x_layout, r.has_x_f32 ? r.x_f32.size() : r.x.size()))
      bail("matrix view outside initialized storage");
    if (!r.scale_layout.given) bail("missing scale matrix layout");
    if (!layout_fits(r.scale_layout, r.data.size())) bail("matrix view outside initialized storage");
    const Request::Layout& sl = r.scale_layout;
    if (r.x_layout.shape[0] != sl.shape[0] || r.x_layout.shape[1] != sl.shape[1])
      bail("invalid H128 view shape or scale dtype");
    const std::vector<uint16_t> xs = gather_view(r, &rows, &cols, "H128 view size overflow");
    const uint64_t n = (uint64_t)rows * cols;
    if (cols == 0 || cols % 128) bail("H128 view width must be positive and 128-aligned");
    if (n == 0) return "[]";
    std::vector<uint16_t> ss(n);
    for (uint64_t i = 0; i < rows; ++i)
      for (uint64_t j = 0; j < cols; ++j)
        ss[i * cols + j] = r.data[sl.offset + (int64_t)i * sl.strides[0] + (int64_t)j * sl.strides[1]];
    DeviceBuffer x(xs), sc(ss), o(n * 2);
    lib_check(exl3_prepare128(x.as<uint16_t>(), (int64_t)n, (int)cols, sc.as<uint16_t>(),
                              (int64_t)n, o.as<uint16_t>(), nullptr));
    return json_list(o.read<uint16_t>(n));
  }
  if (r.op == "metal-prepare128") {  // main.rs:1338-1342, gpu.rs:1537-1558
    // extents checked before any upload, as prepare128_blocks (contracts.rs:2146-2159)
    const uint64_t n = r.x.size(), w = r.cols;
    if (n > UINT32_MAX || w == 0 || w > INT32_MAX || w % 128 || n % w ||
        (r.data.size() != w && r.data.size() != n))
      bail("expected complete 128-aligned rows and column or element scales");
    if (n == 0) return "[]";
    DeviceBuffer x(r.x), sc(r.data), o(r.x.size() * 2);
    lib_check(exl3_prepare128(x.as<uint16_t>(), (int64_t)n, (int)w, sc.as<uint16_t>(),
                              (int64_t)r.data.size(), o.as<uint16_t>(), nullptr));
    return json_list(o.read<uint16_t>(r.x.size()));
  }
  if (r.op == "mlx-linear") {  // main.rs:310-334
    check_k(r.k);
    const uint64_t rows = r.suh.size();
    if (!(rows > 0 && r.x.size() % rows == 0)) bail("invalid linear input rows");
    const uint64_t m = r.x.size() / rows, cols = r.cols;
    if (rows > INT32_MAX || cols > INT32_MAX || m > INT32_MAX) bail("out of range integral type conversion attempted");
    if (r.data.size() != rows / 16 * (cols / 16) * 16 * r.k || rows % 16 || cols % 16)
      bail("invalid trellis shape");
    if (r.svh.size() != cols) bail("EXL3 scales have wrong dimensions");
    DeviceBuffer tr(r.data), su(r.suh), sv(r.svh), x(r.x), y(m * cols * 2);
    exl3_linear* h = nullptr;
    lib_check(exl3_linear_create(tr.as<uint16_t>(), (int)rows, (int)cols, (int)r.k, cb,
                                 su.as<uint16_t>(), sv.as<uint16_t>(), nullptr, &h));
    struct Guard {
      exl3_linear* h;
      ~Guard() { exl3_linear_destroy(h); }
    } guard{h};
    if (m == 0) bail("EXL3 linear input cannot be empty");
    const size_t wb = exl3_linear_workspace_bytes(h, (int64_t)m);
    DeviceBuffer ws(wb);
    zero_workspace(ws);
    lib_check(exl3_linear_forward(h, x.p, EXL3_F16, (int64_t)m, y.p, EXL3_F16, ws.p, wb, nullptr));
    return json_list(y.read<uint16_t>(m * cols));
  }
  if (r.op == "mlx-group") {  // main.rs:336-426
    check_k(r.k);
    if (r.widths.empty()) bail("missing group widths");
    if (r.suh.size() % r.widths.size()) bail("invalid grouped input scales");
    const uint64_t rows = r.suh.size() / r.widths.size();
    if (!(rows > 0 && rows % 128 == 0 && r.x.size() % rows == 0)) bail("invalid grouped input size");
    const uint64_t m = r.x.size() / rows;
    if (!(r.widths.size() >= 2 && r.k != 7)) bail("unsupported group");
    if (r.widths.size() > 8) bail("EXL3 groups of more than 8 projections are not supported");
    if (rows > INT32_MAX || m > INT32_MAX) bail("out of range integral type conversion attempted");
    uint64_t data_off = 0, scale_off = 0;
    std::vector<exl3_linear*> parts;
    std::vector<DeviceBuffer*> bufs;
    struct Cleanup {
      std::vector<exl3_linear*>& parts;
      std::vector<DeviceBuffer*>& bufs;
      ~Cleanup() {
        for (auto* h : parts) exl3_linear_destroy(h);
        for (auto* b : bufs) delete b;
      }
    } cleanup{parts, bufs};
    for (size_t i = 0; i < r.widths.size(); ++i) {
      const uint64_t width = r.widths[i];
      if (!(width > 0 && width % 128 == 0)) bail("invalid group width");
      const uint64_t words = rows / 16 * (width / 16) * 16 * r.k;
      if (data_off + words > r.data.size()) bail("truncated grouped trellis");
      if (scale_off + width > r.svh.size()) bail("truncated grouped scales");
      auto* tr = new DeviceBuffer(std::vector<uint16_t>(r.data.begin() + data_off,
                                                        r.data.begin() + data_off + words));
      bufs.push_back(tr);
      auto* su = new DeviceBuffer(std::vector<uint16_t>(r.suh.begin() + i * rows,
                                                        r.suh.begin() + (i + 1) * rows));
      bufs.push_back(su);
      auto* sv = new DeviceBuffer(std::vector<uint16_t>(r.svh.begin() + scale_off,
                                                        r.svh.begin() + scale_off + width));
      bufs.push_back(sv);
      exl3_linear* h = nullptr;
      lib_check(exl3_linear_create(tr->as<uint16_t>(), (int)rows, (int)width, (int)r.k, cb,
                                   su->as<uint16_t>(), sv->as<uint16_t>(), nullptr, &h));
      parts.push_back(h);
      data_off += words;
      scale_off += width;
    }
    if (data_off != r.data.size() || scale_off != r.svh.size()) bail("extra grouped data");
    DeviceBuffer x(r.x);
    std::vector<DeviceBuffer*> ys;
    std::vector<void*> yp;
    for (uint64_t w : r.widths) {
      ys.push_back(new DeviceBuffer(m * w * 2));
      bufs.push_back(ys.back());
      yp.push_back(ys.back()->p);
    }
    if (m == 0) bail("grouped EXL3 input cannot be empty");
    const size_t wb = exl3_group_workspace_bytes(parts.data(), (int)parts.size(), (int64_t)m);
    DeviceBuffer ws(wb);
    zero_workspace(ws);
    lib_check(exl3_group_forward(parts.data(), (int)parts.size(), x.p, EXL3_F16, (int64_t)m,
                                 yp.data(), ws.p, wb, nullptr));
    std::string out = "[";
    for (size_t i = 0; i < ys.size(); ++i) {
      if (i) out += ',';
      out += json_list(ys[i]->read<uint16_t>(m * r.widths[i]));
    }
    return out + "]";
  }
  if (r.op == "mlx-switch") {  // validate_moe_codec main.rs:211-229, run :627-675
    const uint64_t experts = r.key_heads, top_k = r.top_k > 0 ? r.top_k : r.selected.size();
    const int64_t rows = route_rows(r.selected, experts, top_k);
    if (rows < 0) bail("invalid SwitchGLU routes");
    if (r.x.size() % (uint64_t)rows) bail("invalid SwitchGLU rows");
    const uint64_t input = r.x.size() / rows, hidden = r.cols;
    if (!glu_layout_ok(experts, top_k, input, hidden, r.k)) bail("invalid SwitchGLU layout");
    const uint64_t k16 = 16 * r.k;
    expect_len(r.data.size(), input / 16 * (experts * hidden / 8) * k16);
    expect_len(r.down_data.size(), hidden / 16 * (experts * input / 16) * k16);
    expect_len(r.suh.size(), experts * 2 * input);
    expect_len(r.svh.size(), experts * 2 * hidden);
    expect_len(r.down_suh.size(), experts * hidden);
    expect_len(r.down_svh.size(), experts * input);
    expect_len(r.beta.size(), (uint64_t)rows * top_k);
    DeviceBuffer gu(r.data), gs(r.suh), gv(r.svh), dn(r.down_data), ds(r.down_suh),
        dv(r.down_svh);
    MoeGuard g;
    lib_check(exl3_moe_create(gu.as<uint16_t>(), gs.as<uint16_t>(), gv.as<uint16_t>(),
                              dn.as<uint16_t>(), ds.as<uint16_t>(), dv.as<uint16_t>(), (int)input,
                              (int)hidden, (int)experts, (int)top_k, (int)r.k, cb, &g.h));
    return json_list(moe_run(g.h, r.x, r.selected, r.beta, rows));
  }
  if (r.op == "mlx-expert") {  // main.rs:540-597
    check_k(r.k);
    if (r.projections_per_route == 0 || r.projections_per_route > INT32_MAX)
      bail(r.projections_per_route ? "out of range integral type conversion attempted"
                                   : "invalid projection count");
    const uint64_t rows = (uint64_t)r.selected.size() * r.projections_per_route;
    if (rows / r.projections_per_route != r.selected.size()) bail("expert row count overflow");
    if (rows > INT32_MAX) bail("out of range integral type conversion attempted");
    if (rows == 0) bail("missing expert routes");
    const uint64_t input_dims = r.x.size() / rows, output_dims = r.cols;
    if (r.x.size() > INT32_MAX || output_dims > INT32_MAX || r.projection_stride_tiles > INT32_MAX)
      bail("out of range integral type conversion attempted");
    const uint64_t input_tiles = input_dims / 16, per_tile = 16 * r.k;
    if (input_tiles * per_tile == 0) bail("invalid expert trellis dimensions");
    const uint64_t source_tiles = r.data.size() / (input_tiles * per_tile);
    // Array::from_u16 / from_f16_bits of each tensor (array.rs:884-888)
    expect_len(r.data.size(), input_tiles * source_tiles * per_tile);
    expect_len(r.x.size(), rows * input_dims);
    expect_len(r.suh.size(), rows * input_dims);
    if (!r.return_raw) expect_len(r.svh.size(), rows * output_dims);
    DeviceBuffer tr(r.data), x(r.x), su(r.suh), sel(r.selected),
        sv(r.return_raw ? std::vector<uint16_t>() : r.svh),
        y(rows * output_dims * (r.return_raw ? 4 : 2));
    const size_t wb = exl3_expert_mapped_workspace_bytes((int)input_dims, (int)output_dims,
                                                         (int64_t)rows);
    DeviceBuffer ws(wb);
    lib_check(exl3_expert_mapped(tr.as<uint16_t>(), (int)input_dims, (int)source_tiles, (int)r.k,
                                 cb, x.p, EXL3_F16, (int64_t)rows, su.as<uint16_t>(),
                                 sel.as<uint32_t>(), (int)r.selected.size(),
                                 (int)r.projections_per_route, (int)output_dims,
                                 (int)r.projection_stride_tiles,
                                 r.return_raw ? nullptr : sv.as<uint16_t>(), r.return_raw ? 1 : 0,
                                 y.p, ws.p, wb, nullptr));
    if (r.return_raw) return "{\"f32\":" + json_f32_list(y.read<float>(rows * output_dims)) + "}";
    return "{\"f16\":" + json_list(y.read<uint16_t>(rows * output_dims)) + "}";
  }
  if (r.op == "mlx-swiglu-prepare") {  // validate_moe_codec main.rs:239-252, run :598-613
    const uint64_t hidden = r.cols, width = hidden * 2;
    if (width == 0 || hidden > INT32_MAX) bail("invalid gate/up width");
    if (r.suh.size() % width) bail("invalid gate/up scales");
    const uint64_t experts = r.suh.size() / width;
    if (route_rows(r.selected, experts, 1) < 0) bail("invalid SwiGLU routes");
    const uint64_t slots = r.selected.size();
    expect_len(r.state.size(), slots * 2 * hidden);
    expect_len(r.svh.size(), experts * hidden);
    if (hidden % 128) bail("invalid fused SwiGLU dimensions");
    DeviceBuffer gu(r.state), sv(r.suh), ds(r.svh), sel(r.selected), out(slots * hidden * 2);
    lib_check(exl3_swiglu_down_input(gu.as<float>(), sv.as<uint16_t>(), ds.as<uint16_t>(),
                                     sel.as<uint32_t>(), (int64_t)slots, (int)hidden,
                                     (int)experts, out.as<uint16_t>(), nullptr));
    return json_list(out.read<uint16_t>(slots * hidden));
  }
  if (r.op == "mlx-expert-reduce") {  // main.rs:615-625
    const uint64_t width = r.cols, slots = r.beta.size();
    if (width == 0 || width > INT32_MAX || width % 128)
      bail("invalid expert reduction dimensions");
    expect_len(r.state.size(), slots * width);
    expect_len(r.svh.size(), slots * width);
    if (slots == 0) return json_list(std::vector<uint16_t>(width, 0));  // an empty sum
    DeviceBuffer raw(r.state), sv(r.svh), sc(r.beta), y(width * 2);
    lib_check(exl3_finish_and_reduce(raw.as<float>(), sv.as<uint16_t>(), sc.p, EXL3_F16, 1,
                                     (int)slots, (int)width, y.p, nullptr));
    return json_list(y.read<uint16_t>(width));
  }
  if (r.op == "mlx-checkpoint-switch") {  // validate_moe_codec main.rs:230-238, run :701-725
    if (r.x.empty()) bail("empty SwitchGLU input");
    if (route_rows(r.selected, r.key_heads, r.selected.size()) < 0)
      bail("invalid checkpoint SwitchGLU routes");
    expect_len(r.beta.size(), r.selected.size());
    CheckpointGuard c;
    lib_check(exl3_checkpoint_open(r.path.c_str(), &c.c));
    const bool lfm = std::strcmp(exl3_checkpoint_model_type(c.c), "lfm2_moe") == 0;
    // Exl3SwitchGlu::forward's shape check (moe.rs:911-918) on the [1, len]
    // row, against the bank's input width (first gate trellis: [in/16, ...]),
    // before the bank is uploaded
    exl3_tensor_info gate0;
    const std::string gate_name = r.prefix + ".0." + (lfm ? "w1" : "gate_proj") + ".trellis";
    if (exl3_checkpoint_tensor(c.c, gate_name.c_str(), &gate0) == EXL3_OK && gate0.ndim == 3 &&
        r.x.size() != (uint64_t)gate0.shape[0] * 16)
      bail("invalid SwitchGLU input/routes");
    MoeGuard g;
    lib_check(exl3_moe_load(c.c, r.prefix.c_str(), (int)r.key_heads, (int)r.selected.size(),
                            lfm ? "w1" : nullptr, lfm ? "w3" : nullptr, lfm ? "w2" : nullptr,
                            &g.h));
    if (r.x.size() != (size_t)exl3_moe_in_features(g.h)) bail("invalid SwitchGLU input/routes");
    return json_list(moe_run(g.h, r.x, r.selected, r.beta, 1));
  }
  if (r.op == "mlx-checkpoint-group") {  // main.rs:677-700
    CheckpointGuard c;
    lib_check(exl3_checkpoint_open(r.path.c_str(), &c.c));
    if (r.prefixes.empty()) bail("empty projection bundle");
    std::vector<exl3_linear*> parts;
    struct Cleanup {
      std::vector<exl3_linear*>& parts;
      ~Cleanup() {
        for (auto* h : parts) exl3_linear_destroy(h);
      }
    } cleanup{parts};
    // K, codebook and input width of each projection, as
    // Exl3Linear::from_checkpoint reads them (trellis [in/16][out/16][16k]),
    // before anything is uploaded; a projection whose trellis is missing or
    // malformed is left to exl3_linear_load's error
    std::vector<std::pair<int64_t, int>> kinds;
    std::vector<int64_t> widths;
    bool described = true;
    for (const std::string& p : r.prefixes) {
      exl3_tensor_info info;
      if (exl3_checkpoint_tensor(c.c, (p + ".trellis").c_str(), &info) != EXL3_OK ||
          info.ndim != 3) {
        described = false;
        break;
      }
      widths.push_back(info.shape[0] * 16);
      const int64_t k16 = info.shape[2];
      const int kcb = exl3_checkpoint_tensor(c.c, (p + ".mul1").c_str(), &info) == EXL3_OK ? 2
                      : exl3_checkpoint_tensor(c.c, (p + ".mcg").c_str(), &info) == EXL3_OK ? 1
                                                                                             : 0;
      kinds.emplace_back(k16 / 16, kcb);
    }
    // Exl3Group::compatible (linear.rs:2303-2311)
    bool grouped = described && r.prefixes.size() >= 2 && kinds[0].first != 7;
    for (size_t i = 0; grouped && i < kinds.size(); ++i)
      grouped = widths[i] == widths[0] && kinds[i] == kinds[0];
    // the input row against every projection's width: Exl3Group::forward
    // (linear.rs:2388-2391) or each Exl3Linear::forward (linear.rs:739-743)
    if (described)
      for (int64_t w : widths)
        if ((uint64_t)w != r.x.size())
          bail(grouped ? std::string("invalid grouped EXL3 input")
                       : "invalid EXL3 linear input for " + std::to_string(w) + " inputs");
    for (const std::string& p : r.prefixes) {
      exl3_linear* h = nullptr;
      lib_check(exl3_linear_load(c.c, p.c_str(), &h));
      parts.push_back(h);
    }
    return group_outputs(parts, grouped, r.x);
  }
  // The direct-Metal projection ops (main.rs:1304-1337): a projection of a
  // checkpoint (FlashProjection::load for a Flash reference checkpoint, load_exl3
  // for any) or a dense expert (FlashExpert: down(swiglu(gate x, up x))) on f16
  // rows or on a strided f16/f32 view, f16 out.  The geometry and input checks
  // are the direct path's (gpu/projection.rs:134-333, :1577-1608); the
  // arithmetic is this library's Exl3Linear, which that path matches bit for bit.
  if (r.op == "metal-checkpoint-linear" || r.op == "metal-exl3-linear" ||
      r.op == "metal-checkpoint-expert") {
    const bool view = r.x_layout.given || r.has_x_f32;
    const char* view_batch = "invalid Flash projection view batch or index overflow";
    std::vector<uint16_t> xs;
    uint32_t vrows = 0, vcols = 0;
    if (view) xs = gather_view(r, &vrows, &vcols, view_batch);
    CheckpointGuard c;
    lib_check(exl3_checkpoint_open(r.path.c_str(), &c.c));
    const bool expert = r.op == "metal-checkpoint-expert";
    const FlashGeometry g = flash_geometry(
        c.c, expert ? r.prefix + ".gate_proj" : r.prefix, r.op == "metal-exl3-linear");
    if (expert) {
      const FlashGeometry u = flash_geometry(c.c, r.prefix + ".up_proj", false);
      const FlashGeometry d = flash_geometry(c.c, r.prefix + ".down_proj", false);
      // contracts::compatible_flash_expert
      if (!(u.input == g.input && u.output == g.output && d.input == g.output &&
            d.output == g.input))
        bail("incompatible Flash expert projection geometry");
    }
    uint64_t rows;
    if (view) {
      if (vcols != g.input) bail("invalid projection view width");
      rows = vrows;
      if (!flash_extents(g, rows)) bail(view_batch);
    } else {
      if (r.x.size() % g.input) bail("input is not a complete row");
      rows = r.x.size() / g.input;
      if (!flash_extents(g, rows)) bail("invalid Flash projection batch or index overflow");
      xs = r.x;
    }
    if (!expert) {
      LinearGuard h;
      lib_check(exl3_linear_load(c.c, r.prefix.c_str(), &h.h));
      return json_list(linear_run(h.h, xs, (int64_t)rows));
    }
    LinearGuard gate, up, down;
    lib_check(exl3_linear_load(c.c, (r.prefix + ".gate_proj").c_str(), &gate.h));
    lib_check(exl3_linear_load(c.c, (r.prefix + ".up_proj").c_str(), &up.h));
    lib_check(exl3_linear_load(c.c, (r.prefix + ".down_proj").c_str(), &down.h));
    const std::vector<uint16_t> gy = linear_run(gate.h, xs, (int64_t)rows);
    const std::vector<uint16_t> uy = linear_run(up.h, xs, (int64_t)rows);
    DeviceBuffer gb(gy), ub(uy), act(gy.size() * 2);
    lib_check(exl3_swiglu(gb.as<uint16_t>(), ub.as<uint16_t>(), act.as<uint16_t>(),
                          (int64_t)gy.size(), nullptr));
    return json_list(linear_run(down.h, act.read<uint16_t>(gy.size()), (int64_t)rows));
  }
  // metal-checkpoint-group (main.rs:1173-1199): ProjectionGroup::load
  // (gpu/projection.rs:2386-2443) of load_exl3 projections sharing one input
  // width, one f16 row (x or a [1, width] view), one f16 output per
  // projection; "grouped" when there are two or more generic projections of
  // one K (not 7) and codebook.
  if (r.op == "metal-checkpoint-group") {
    const bool view = r.x_layout.given || r.has_x_f32;
    std::vector<uint16_t> xs;
    uint32_t vrows = 0, vcols = 0;
    if (view) xs = gather_view(r, &vrows, &vcols, "invalid ordinary projection bundle input");
    CheckpointGuard c;
    lib_check(exl3_checkpoint_open(r.path.c_str(), &c.c));
    std::vector<FlashGeometry> geo;
    for (const std::string& p : r.prefixes) geo.push_back(flash_geometry(c.c, p, true));
    if (geo.empty()) bail("empty projection bundle");
    for (const FlashGeometry& g : geo)
      if (g.input != geo[0].input) bail("projection bundle requires one input width and Metal context");
    bool grouped = geo.size() >= 2 && geo[0].k != 7;
    for (const FlashGeometry& g : geo)
      grouped = grouped && g.generic && g.k == geo[0].k && g.cb == geo[0].cb;
    if (view) {
      if (vrows != 1 || vcols != geo[0].input) bail("invalid ordinary projection bundle input");
    } else if (r.x.size() != geo[0].input) {
      bail("invalid grouped input row length");
    } else {
      xs = r.x;
    }
    std::vector<exl3_linear*> parts;
    struct Cleanup {
      std::vector<exl3_linear*>& parts;
      ~Cleanup() {
        for (auto* h : parts) exl3_linear_destroy(h);
      }
    } cleanup{parts};
    for (const std::string& p : r.prefixes) {
      parts.push_back(nullptr);
      lib_check(exl3_linear_load(c.c, p.c_str(), &parts.back()));
    }
    return group_outputs(parts, grouped, xs);
  }
  bail("unknown or unavailable codec operation " + r.op);
}

}  // namespace

int main(int argc, char** argv) {
  // `exl3_codec` or `exl3_codec codec` (the reference's subcommand form)
  if (argc > 2 || (argc == 2 && std::strcmp(argv[1], "codec") != 0)) {
    std::fprintf(stderr, "usage: %s [codec] < requests.jsonl\n", argv[0]);
    return 2;
  }
  std::ios::sync_with_stdio(false);
  std::string line;
  while (std::getline(std::cin, line)) {
    std::string out;
    try {
      out = "{\"data\":" + run(parse_request(line)) + "}";
    } catch (const Failure& f) {
      out = "{\"error\":" + json_string(f.msg) + "}";
    } catch (const std::bad_alloc&) {
      out = "{\"error\":\"out of host memory\"}";
    }
    std::cout << out << '\n' << std::flush;
  }
  return 0;
}
