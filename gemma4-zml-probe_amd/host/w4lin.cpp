// w4lin.cpp -- see w4lin.hpp.
#include "w4lin.hpp"

#include <algorithm>
#include <cstring>

#include "../../include/w4a16.h"

namespace w4 {

namespace {

void check(int rc, const char* what) {
  if (rc != W4A16_OK) throw Error(rc, std::string(what) + ": " + w4a16_last_error());
}

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(W4A16_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}

const char* const kPacked = ".weight_packed";
const char* const kScale = ".weight_scale";
const char* const kShape = ".weight_shape";

bool ends_with(const std::string& s, const char* suffix) {
  const size_t n = std::strlen(suffix);
  return s.size() >= n && s.compare(s.size() - n, n, suffix) == 0;
}

// Checks of one linear; returns "" when consistent, else the first failure.  On
// success fills n, k, group.
std::string check_linear(const SafeTensorsFile& f, const std::string& name, int64_t& n, int64_t& k, int32_t& group,
                         bool& has_shape) {
  const std::string pkn = name + kPacked, scn = name + kScale, shn = name + kShape;
  if (!f.has(pkn)) return name + ": no " + pkn;
  const TensorInfo& pk = f.info(pkn);
  if (pk.dtype != "I32") return pkn + ": dtype " + pk.dtype + " != I32";
  if (pk.shape.size() != 2) return pkn + ": not 2-D";
  n = pk.shape[0];
  k = 8 * pk.shape[1];
  if (!f.has(scn)) return name + ": weight_packed without weight_scale";
  const TensorInfo& sc = f.info(scn);
  if (sc.dtype != "BF16") return scn + ": dtype " + sc.dtype + " != BF16";
  if (sc.shape.size() != 2 || sc.shape[0] != n) return scn + ": shape does not match weight_packed rows";
  const int64_t g = sc.shape[1];
  if (g <= 0 || k % g != 0 || (k / g) % 32 != 0)
    return scn + ": " + std::to_string(g) + " groups do not divide K=" + std::to_string(k) + " into multiples of 32";
  group = (int32_t)(k / g);
  has_shape = f.has(shn);
  if (has_shape) {
    const TensorInfo& sh = f.info(shn);
    if (sh.dtype != "I64" || sh.shape.size() != 1 || sh.shape[0] != 2) return shn + ": not I64 [2]";
    int64_t v[2];
    std::memcpy(v, f.data(shn), sizeof v);
    if (v[0] != n || v[1] != k)
      return shn + ": [" + std::to_string(v[0]) + ", " + std::to_string(v[1]) + "] != packed [" + std::to_string(n) +
             ", " + std::to_string(k) + "]";
  }
  if (f.has(name + ".weight_zero_point")) return name + ": weight_zero_point present (only symmetric w4a16 is supported)";
  if (f.has(name + ".weight_g_idx")) return name + ": weight_g_idx present (act-order is not supported)";
  return "";
}

}  // namespace

void unpackW4(const int32_t* pk, int8_t* q, int64_t n, int64_t k, hipStream_t stream) {
  check(w4a16_unpack(pk, q, n, k, stream), "unpackW4");
}

void dequantW4(const int32_t* pk, const uint16_t* sc, uint16_t* w, int64_t n, int64_t k, int32_t group,
               hipStream_t stream) {
  check(w4a16_dequant(pk, sc, w, n, k, group, stream), "dequantW4");
}

DeviceStore::~DeviceStore() {
  for (auto& kv : dev_) (void)hipFree(kv.second);
}

const void* DeviceStore::device(const std::string& name) {
  auto it = dev_.find(name);
  if (it != dev_.end()) return it->second;
  const TensorInfo& t = file_.info(name);
  void* p = nullptr;
  hip_check(hipMalloc(&p, std::max<size_t>(t.nbytes(), 16)), "DeviceStore: hipMalloc");
  dev_[name] = p;
  hip_check(hipMemcpy(p, file_.data(name), t.nbytes(), hipMemcpyHostToDevice), "DeviceStore: hipMemcpy");
  return p;
}

W4Lin W4Lin::init(DeviceStore& store, const std::string& name) {
  W4Lin lin;
  bool has_shape = false;
  const std::string err = check_linear(store.file(), name, lin.n, lin.k, lin.group, has_shape);
  if (!err.empty()) throw Error(W4A16_EINVAL_SHAPE, "W4Lin.init: " + err);
  lin.pk = static_cast<const int32_t*>(store.device(name + kPacked));
  lin.sc = static_cast<const uint16_t*>(store.device(name + kScale));
  return lin;
}

void W4Lin::toW(uint16_t* w, hipStream_t stream) const { dequantW4(pk, sc, w, n, k, group, stream); }

void W4Lin::linear(const uint16_t* x, uint16_t* y, int64_t m, hipStream_t stream) const {
  check(w4a16_linear(x, W4A16_DTYPE_BF16, pk, sc, y, W4A16_DTYPE_BF16, m, n, k, group, 0, nullptr, 0, stream),
        "W4Lin.linear");
}

void W4Lin::linear(const uint16_t* x, float* y, int64_t m, hipStream_t stream) const {
  check(w4a16_linear(x, W4A16_DTYPE_BF16, pk, sc, y, W4A16_DTYPE_F32, m, n, k, group, 0, nullptr, 0, stream),
        "W4Lin.linear");
}

size_t W4Lin::workspace(int64_t m) const { return w4a16_workspace_size(m, n, k, W4A16_DTYPE_BF16); }

void W4Lin::linear(const uint16_t* x, uint16_t* y, int64_t m, void* workspace, size_t ws_bytes,
                   hipStream_t stream) const {
  check(w4a16_linear(x, W4A16_DTYPE_BF16, pk, sc, y, W4A16_DTYPE_BF16, m, n, k, group, 0, workspace, ws_bytes, stream),
        "W4Lin.linear");
}

void W4Lin::linear(const uint16_t* x, float* y, int64_t m, void* workspace, size_t ws_bytes,
                   hipStream_t stream) const {
  check(w4a16_linear(x, W4A16_DTYPE_BF16, pk, sc, y, W4A16_DTYPE_F32, m, n, k, group, 0, workspace, ws_bytes, stream),
        "W4Lin.linear");
}

size_t W4Lin::workspace_f32(int64_t m) const { return w4a16_workspace_size(m, n, k, W4A16_DTYPE_F32); }

void W4Lin::linear_f32(const float* x, float* y, int64_t m, void* workspace, size_t ws_bytes,
                       hipStream_t stream) const {
  check(w4a16_linear(x, W4A16_DTYPE_F32, pk, sc, y, W4A16_DTYPE_F32, m, n, k, group, 0, workspace, ws_bytes, stream),
        "W4Lin.linear_f32");
}

namespace {
void gate_up_call(const W4Lin& gate, const W4Lin& up, const void* x, int32_t x_dtype, void* h, int32_t h_dtype,
                  int64_t m, void* workspace, size_t ws_bytes, hipStream_t stream, bool bf16_dots) {
  if (up.n != gate.n || up.k != gate.k || up.group != gate.group)
    throw Error(W4A16_EINVAL_SHAPE, "gate_up_gelu: up [" + std::to_string(up.n) + ", " + std::to_string(up.k) +
                                        "] / group " + std::to_string(up.group) + " does not match gate [" +
                                        std::to_string(gate.n) + ", " + std::to_string(gate.k) + "] / group " +
                                        std::to_string(gate.group));
  check(w4a16_gate_up_gelu(x, x_dtype, gate.pk, gate.sc, up.pk, up.sc, h, h_dtype, m, gate.n, gate.k,
                           gate.group, bf16_dots ? W4A16_GATE_UP_BF16_DOTS : 0, workspace, ws_bytes, stream),
        "gate_up_gelu");
}
}  // namespace

size_t gate_up_workspace(const W4Lin& gate, int64_t m) {
  return w4a16_gate_up_workspace_size(m, gate.n, gate.k, W4A16_DTYPE_BF16);
}

void gate_up_gelu(const W4Lin& gate, const W4Lin& up, const uint16_t* x, uint16_t* h, int64_t m, void* workspace,
                  size_t ws_bytes, hipStream_t stream, bool bf16_dots) {
  gate_up_call(gate, up, x, W4A16_DTYPE_BF16, h, W4A16_DTYPE_BF16, m, workspace, ws_bytes, stream, bf16_dots);
}

void gate_up_gelu(const W4Lin& gate, const W4Lin& up, const uint16_t* x, float* h, int64_t m, void* workspace,
                  size_t ws_bytes, hipStream_t stream, bool bf16_dots) {
  gate_up_call(gate, up, x, W4A16_DTYPE_BF16, h, W4A16_DTYPE_F32, m, workspace, ws_bytes, stream, bf16_dots);
}

size_t gate_up_workspace_f32(const W4Lin& gate, int64_t m) {
  return w4a16_gate_up_workspace_size(m, gate.n, gate.k, W4A16_DTYPE_F32);
}

void gate_up_gelu_f32(const W4Lin& gate, const W4Lin& up, const float* x, float* h, int64_t m, void* workspace,
                      size_t ws_bytes, hipStream_t stream) {
  gate_up_call(gate, up, x, W4A16_DTYPE_F32, h, W4A16_DTYPE_F32, m, workspace, ws_bytes, stream, false);
}

void linear_group(const std::vector<W4Lin>& lins, const uint16_t* x, const std::vector<uint16_t*>& ys, int64_t m,
                  hipStream_t stream) {
  linear_group(lins, x, ys, m, nullptr, 0, stream);
}

size_t linear_group_workspace(const std::vector<W4Lin>& lins, int64_t m) {
  size_t ws = 0;
  for (const W4Lin& lin : lins) ws = std::max(ws, lin.workspace(m));
  return ws;
}

namespace {
void group_call(const std::vector<W4Lin>& lins, const void* x, int32_t x_dtype, void* const* ys, size_t nys,
                int32_t y_dtype, int64_t m, void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (lins.empty() || lins.size() > 4 || nys != lins.size())
    throw Error(W4A16_EINVAL_ARG, "linear_group: 1 to 4 linears, one output each");
  const int32_t* pk[4];
  const uint16_t* sc[4];
  void* y[4];
  int64_t n[4];
  for (size_t j = 0; j < lins.size(); ++j) {
    if (lins[j].k != lins[0].k || lins[j].group != lins[0].group)
      throw Error(W4A16_EINVAL_SHAPE, "linear_group: every linear needs the same k and group");
    pk[j] = lins[j].pk;
    sc[j] = lins[j].sc;
    y[j] = ys[j];
    n[j] = lins[j].n;
  }
  check(w4a16_linear_group(x, x_dtype, (int32_t)lins.size(), pk, sc, y, n, y_dtype, m, lins[0].k, lins[0].group, 0,
                           workspace, ws_bytes, stream),
        "linear_group");
}
}  // namespace

void linear_group(const std::vector<W4Lin>& lins, const uint16_t* x, const std::vector<uint16_t*>& ys, int64_t m,
                  void* workspace, size_t ws_bytes, hipStream_t stream) {
  std::vector<void*> y(ys.begin(), ys.end());
  group_call(lins, x, W4A16_DTYPE_BF16, y.data(), y.size(), W4A16_DTYPE_BF16, m, workspace, ws_bytes, stream);
}

size_t linear_group_workspace_f32(const std::vector<W4Lin>& lins, int64_t m) {
  return lins.empty() ? 0 : w4a16_workspace_size(m, 0, lins[0].k, W4A16_DTYPE_F32);
}

void linear_group_f32(const std::vector<W4Lin>& lins, const float* x, const std::vector<float*>& ys, int64_t m,
                      void* workspace, size_t ws_bytes, hipStream_t stream) {
  std::vector<void*> y(ys.begin(), ys.end());
  group_call(lins, x, W4A16_DTYPE_F32, y.data(), y.size(), W4A16_DTYPE_F32, m, workspace, ws_bytes, stream);
}

size_t lm_head_workspace(int64_t m, int64_t v, int64_t k, int topk) {
  return w4a16_lm_head_workspace_size(m, v, k, W4A16_DTYPE_BF16, topk);
}

void lm_head(const uint16_t* embed, int64_t v, int64_t k, const uint16_t* x, int64_t m, float softcap, int topk,
             float* logits, float* top_values, int32_t* top_indices, void* workspace, size_t ws_bytes,
             hipStream_t stream) {
  check(w4a16_lm_head(x, W4A16_DTYPE_BF16, embed, logits, m, v, k, softcap, topk, top_values, top_indices, workspace,
                      ws_bytes, stream),
        "lm_head");
}

Census census(const SafeTensorsFile& f) {
  Census c;
  for (const auto& kv : f.tensors()) {
    const std::string& key = kv.first;
    if (ends_with(key, kPacked)) {
      CensusEntry e;
      e.name = key.substr(0, key.size() - std::strlen(kPacked));
      const std::string err = check_linear(f, e.name, e.n, e.k, e.group, e.has_shape);
      if (err.empty()) c.linears.push_back(e);
      else c.errors.push_back(err);
    } else if (ends_with(key, kScale) || ends_with(key, kShape)) {
      const size_t cut = key.rfind('.');
      if (!f.has(key.substr(0, cut) + kPacked)) c.errors.push_back(key + ": no matching weight_packed");
    }
  }
  return c;
}

std::vector<std::string> g12_layer_linears(const std::string& prefix, int j) {
  const std::string l = prefix + "." + std::to_string(j) + ".";
  std::vector<std::string> v = {l + "self_attn.q_proj", l + "self_attn.k_proj"};
  if (!g12_is_full(j)) v.push_back(l + "self_attn.v_proj");
  v.push_back(l + "self_attn.o_proj");
  v.push_back(l + "mlp.gate_proj");
  v.push_back(l + "mlp.up_proj");
  v.push_back(l + "mlp.down_proj");
  return v;
}

}  // namespace w4
