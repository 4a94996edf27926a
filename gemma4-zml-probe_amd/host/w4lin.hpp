// w4lin.hpp -- C++ host mirror of the reference's W4 brick (zml_runner/w4.zig) over
// the C ABI of libw4a16.so (include/w4a16.h).
//
// The reference's host language is Zig; this is the same interface for a compiled
// host in this image (no Zig toolchain):
//   W4Lin{pk, sc}, W4Lin.init(store, name), W4Lin.toW   zml_runner/w4.zig:16-31
//   unpackW4 / dequantW4                               zml_runner/w4.zig:33-54
//   W4Lin.linear = x.dot(lin.toW()) at the engine sites zml_runner/engine.zig:552-661
//   DeviceStore = the TensorStore + load of W4Model     zml_runner/w4.zig:150-168
//   census = the packed-checkpoint plan and asserts     scripts/63_u_dequant_export.py:92-114
//   g12 layer wiring (which layers carry v_proj)        zml_runner/g12.zig:94-166
// Errors are exceptions (the reference's error unions); every call is
// stream-ordered on the caller's hipStream_t and allocates nothing on the device
// except DeviceStore, which owns the uploaded checkpoint tensors.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "safetensors.hpp"

namespace w4 {

// A failed libw4a16 call (negative w4a16_status) or a bad checkpoint.
class Error : public std::runtime_error {
 public:
  Error(int status, const std::string& msg) : std::runtime_error(msg), status_(status) {}
  int status() const { return status_; }

 private:
  int status_;
};

// unpackW4 (w4.zig:33-45): int32 pk [n, k/8] -> int8 q [n, k], device pointers.
void unpackW4(const int32_t* pk, int8_t* q, int64_t n, int64_t k, hipStream_t stream);
// dequantW4 (w4.zig:47-54): pk + bf16 sc [n, k/group] -> bf16 w [n, k] (uint16_t bits).
void dequantW4(const int32_t* pk, const uint16_t* sc, uint16_t* w, int64_t n, int64_t k, int32_t group,
               hipStream_t stream);

// Device copies of checkpoint tensors, uploaded on first use and freed with the store.
class DeviceStore {
 public:
  explicit DeviceStore(const std::string& path) : file_(path) {}
  ~DeviceStore();
  DeviceStore(const DeviceStore&) = delete;
  DeviceStore& operator=(const DeviceStore&) = delete;

  const SafeTensorsFile& file() const { return file_; }
  // Device pointer of tensor `name` (uploaded once, synchronously, 16-byte aligned).
  const void* device(const std::string& name);

 private:
  SafeTensorsFile file_;
  std::map<std::string, void*> dev_;
};

// Packed linear: the two store tensors of one compressed-tensors Linear [n out, k in].
struct W4Lin {
  const int32_t* pk = nullptr;   // device int32 [n, k/8]
  const uint16_t* sc = nullptr;  // device bf16 [n, k/group]
  int64_t n = 0, k = 0;
  int32_t group = 32;

  // W4Lin.init (w4.zig:20-25): "<name>.weight_packed" / "<name>.weight_scale", with the
  // census checks of one linear (dtypes, shapes, weight_shape when present).
  static W4Lin init(DeviceStore& store, const std::string& name);

  // toW without the engine retag (w4.zig:28-30): bf16 [n, k] into the caller's buffer.
  void toW(uint16_t* w, hipStream_t stream) const;
  // y[m, n] = x[m, k] . toW()^T, fp32 accumulate; bf16 x, bf16 or f32 y.
  void linear(const uint16_t* x, uint16_t* y, int64_t m, hipStream_t stream) const;
  void linear(const uint16_t* x, float* y, int64_t m, hipStream_t stream) const;
  // The same with optional workspace: given workspace(m) bytes, batched shapes whose
  // one-pass grid cannot fill the GPU (the smaller rows, m up to a few hundred) split K
  // across workgroups; 0 bytes or nullptr takes the one-pass route.
  size_t workspace(int64_t m) const;
  void linear(const uint16_t* x, uint16_t* y, int64_t m, void* workspace, size_t ws_bytes, hipStream_t stream) const;
  void linear(const uint16_t* x, float* y, int64_t m, void* workspace, size_t ws_bytes, hipStream_t stream) const;
  // f32 activations (dotPrec with fam = null, engine.zig:530-533): caller workspace of
  // workspace_f32(m) bytes.
  size_t workspace_f32(int64_t m) const;
  void linear_f32(const float* x, float* y, int64_t m, void* workspace, size_t ws_bytes, hipStream_t stream) const;
};

// The MLP front half (engine.zig:653, dotPrec(xff, gate).gelu().mul(dotPrec(xff, up))):
// h[m, F] = gelu_tanh(x . gate.toW()^T) * (x . up.toW()^T) in one call; gate and up
// must both be [F, K] with the same group.  bf16_dots rounds both dot outputs to
// bf16 first (dotPrec with fam = bf16).  Shapes that no fused kernel takes need
// gate_up_workspace(gate, m) bytes of caller workspace (0 on the Gemma shapes).
size_t gate_up_workspace(const W4Lin& gate, int64_t m);
void gate_up_gelu(const W4Lin& gate, const W4Lin& up, const uint16_t* x, uint16_t* h, int64_t m, void* workspace,
                  size_t ws_bytes, hipStream_t stream, bool bf16_dots = false);
void gate_up_gelu(const W4Lin& gate, const W4Lin& up, const uint16_t* x, float* h, int64_t m, void* workspace,
                  size_t ws_bytes, hipStream_t stream, bool bf16_dots = false);

// The same with f32 activations (dotPrec with fam = null: xff stays in the compute
// dtype, engine.zig:530-533): x f32 [m, K], h f32; gate_up_workspace_f32(gate, m) bytes
// of workspace are required (the three bf16 planes of x).
size_t gate_up_workspace_f32(const W4Lin& gate, int64_t m);
void gate_up_gelu_f32(const W4Lin& gate, const W4Lin& up, const float* x, float* h, int64_t m, void* workspace,
                      size_t ws_bytes, hipStream_t stream);

// Linears that read the same x (q, k, v at engine.zig:552,571,583): ys[j][m, lins[j].n] =
// x . lins[j].toW()^T, one launch at decode; 1..4 linears with the same k and group.
void linear_group(const std::vector<W4Lin>& lins, const uint16_t* x, const std::vector<uint16_t*>& ys, int64_t m,
                  hipStream_t stream);
// The same with optional workspace: given linear_group_workspace(lins, m) bytes (the
// largest member's W4Lin::workspace), members that run as their own launch take the
// split-K route; 0 bytes or nullptr keeps them one-pass.
size_t linear_group_workspace(const std::vector<W4Lin>& lins, int64_t m);
void linear_group(const std::vector<W4Lin>& lins, const uint16_t* x, const std::vector<uint16_t*>& ys, int64_t m,
                  void* workspace, size_t ws_bytes, hipStream_t stream);
// f32 activations, f32 outputs (the fam = null flow): linear_group_workspace_f32(lins, m)
// bytes of workspace are required.
size_t linear_group_workspace_f32(const std::vector<W4Lin>& lins, int64_t m);
void linear_group_f32(const std::vector<W4Lin>& lins, const float* x, const std::vector<float*>& ys, int64_t m,
                      void* workspace, size_t ws_bytes, hipStream_t stream);

// The decode head (engine.zig:765-766) and its topK (gemma4_g12auto.zig:1532): logits[m, v] =
// softcap * tanh(x . embed^T / softcap) (f32), top-k values (descending, ties by index) and
// indices.  embed is the tied bf16 [v, k] embedding on the device; workspace of
// lm_head_workspace(m, v, k, topk) bytes.
size_t lm_head_workspace(int64_t m, int64_t v, int64_t k, int topk);
void lm_head(const uint16_t* embed, int64_t v, int64_t k, const uint16_t* x, int64_t m, float softcap, int topk,
             float* logits, float* top_values, int32_t* top_indices, void* workspace, size_t ws_bytes,
             hipStream_t stream);

// ---------------------------------------------------------------- checkpoint census
struct CensusEntry {
  std::string name;  // module name, without ".weight_packed"
  int64_t n = 0, k = 0;
  int32_t group = 0;
  bool has_shape = false;  // "<name>.weight_shape" present (and checked)
};
struct Census {
  std::vector<CensusEntry> linears;  // sorted by name
  std::vector<std::string> errors;   // one line per failed check; empty = clean
};
// Every "<name>.weight_packed" must be I32 [n, k/8] with a "<name>.weight_scale" BF16
// [n, k/group] (group a multiple of 32 dividing k) and, when present, "<name>.weight_shape"
// I64 [2] == [n, k]; no weight_zero_point / weight_g_idx (symmetric, no act-order); no
// orphan scale or shape tensors.
Census census(const SafeTensorsFile& f);

// ---------------------------------------------------------------- 12B layer wiring
constexpr int G12_LAYERS = 48;
// Full-attention layers: (j + 1) % 6 == 0 (8 of 48); they have no v_proj (K = V).
inline bool g12_is_full(int j) { return (j + 1) % 6 == 0; }
// Linear modules of layer j that the decode step consumes, in engine order
// (q, k, [v], o, gate, up, down), under `prefix` (e.g. "model.language_model.layers").
std::vector<std::string> g12_layer_linears(const std::string& prefix, int j);
// 48 * 6 + 40 sliding v_proj = 328 packed linears in the 12B checkpoint.
constexpr int G12_PACKED = G12_LAYERS * 6 + (G12_LAYERS - G12_LAYERS / 6);

}  // namespace w4
