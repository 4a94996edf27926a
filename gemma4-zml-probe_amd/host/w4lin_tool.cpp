// w4lin_tool -- command-line front end of the C++ host mirror (w4lin.hpp).
//
//   w4lin_tool census <file.safetensors> [--expect N]
//       one JSON line per packed linear, then a summary line; exit 1 on any failed
//       check or when the count differs from N (328 for the 12B checkpoint).
//   w4lin_tool layer12 <file.safetensors> <prefix> <j>
//       the linears layer j of the 12B model consumes (g12.zig wiring), each checked.
//   w4lin_tool linear <file.safetensors> <name> <M> <x.bin> <y.bin> [bf16|f32]
//       y[M, n] = x[M, k] . toW()^T on the GPU; x.bin holds M*k bf16 values, y.bin
//       receives M*n bf16 (default) or f32 values.
//   w4lin_tool dequant <file.safetensors> <name> <w.bin>
//       w[n, k] = toW() (bf16) on the GPU.
//   w4lin_tool mlp <file.safetensors> <gate> <up> <M> <x.bin> <h.bin> [bf16|f32]
//       h[M, F] = gelu_tanh(x . gate^T) * (x . up^T) on the GPU (engine.zig:653).
//   w4lin_tool qkv <file.safetensors> <prefix> <j> <M> <x.bin> <out_prefix>
//       q, k (and v on sliding layers) of layer j as one grouped call (engine.zig:552-583);
//       writes <out_prefix>.q.bin, .k.bin[, .v.bin] (bf16).
//   w4lin_tool head <file.safetensors> <embed_name> <M> <x.bin> <softcap> <topk> <out_prefix>
//       logits (f32) and top-k of the tied-embedding head (engine.zig:765-766);
//       writes <out_prefix>.logits.bin, .values.bin (f32), .indices.bin (i32).
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <string>
#include <vector>

#include "w4lin.hpp"

namespace {

int usage() {
  std::fprintf(stderr,
               "usage: w4lin_tool census <file> [--expect N]\n"
               "       w4lin_tool layer12 <file> <prefix> <j>\n"
               "       w4lin_tool linear <file> <name> <M> <x.bin> <y.bin> [bf16|f32]\n"
               "       w4lin_tool dequant <file> <name> <w.bin>\n"
               "       w4lin_tool mlp <file> <gate> <up> <M> <x.bin> <h.bin> [bf16|f32]\n"
               "       w4lin_tool qkv <file> <prefix> <j> <M> <x.bin> <out_prefix>\n"
               "       w4lin_tool head <file> <embed_name> <M> <x.bin> <softcap> <topk> <out_prefix>\n");
  return 2;
}

std::vector<char> read_file(const std::string& path, size_t expect) {
  std::ifstream f(path, std::ios::binary);
  if (!f) throw std::runtime_error("cannot read " + path);
  std::vector<char> b((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
  if (b.size() != expect)
    throw std::runtime_error(path + ": " + std::to_string(b.size()) + " bytes, expected " + std::to_string(expect));
  return b;
}

void write_file(const std::string& path, const void* p, size_t n) {
  std::ofstream f(path, std::ios::binary);
  f.write(static_cast<const char*>(p), (std::streamsize)n);
  if (!f) throw std::runtime_error("cannot write " + path);
}

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

std::string json_escape(const std::string& s) {
  std::string o;
  for (char c : s) {
    if (c == '"' || c == '\\') o.push_back('\\');
    o.push_back(c);
  }
  return o;
}

int cmd_census(int argc, char** argv) {
  if (argc < 3) return usage();
  long expect = -1;
  for (int i = 3; i + 1 < argc; ++i)
    if (!std::strcmp(argv[i], "--expect")) expect = std::atol(argv[i + 1]);
  w4::SafeTensorsFile f(argv[2]);
  const w4::Census c = w4::census(f);
  for (const auto& e : c.linears)
    std::printf("{\"name\": \"%s\", \"n\": %lld, \"k\": %lld, \"group\": %d, \"weight_shape\": %s}\n",
                json_escape(e.name).c_str(), (long long)e.n, (long long)e.k, e.group, e.has_shape ? "true" : "false");
  std::printf("{\"linears\": %zu, \"errors\": [", c.linears.size());
  for (size_t i = 0; i < c.errors.size(); ++i) std::printf("%s\"%s\"", i ? ", " : "", json_escape(c.errors[i]).c_str());
  std::printf("]}\n");
  if (!c.errors.empty()) return 1;
  if (expect >= 0 && (long)c.linears.size() != expect) {
    std::fprintf(stderr, "census: %zu linears, expected %ld\n", c.linears.size(), expect);
    return 1;
  }
  return 0;
}

int cmd_layer12(int argc, char** argv) {
  if (argc < 5) return usage();
  w4::SafeTensorsFile f(argv[2]);
  const w4::Census c = w4::census(f);
  const int j = std::atoi(argv[4]);
  int bad = 0;
  for (const std::string& name : w4::g12_layer_linears(argv[3], j)) {
    bool found = false;
    for (const auto& e : c.linears)
      if (e.name == name) {
        std::printf("{\"name\": \"%s\", \"n\": %lld, \"k\": %lld}\n", json_escape(name).c_str(), (long long)e.n,
                    (long long)e.k);
        found = true;
      }
    if (!found) {
      std::printf("{\"name\": \"%s\", \"missing\": true}\n", json_escape(name).c_str());
      ++bad;
    }
  }
  return bad ? 1 : 0;
}

int cmd_linear(int argc, char** argv) {
  if (argc < 7) return usage();
  const bool f32 = argc > 7 && !std::strcmp(argv[7], "f32");
  const int64_t M = std::atoll(argv[4]);
  w4::DeviceStore store(argv[2]);
  const w4::W4Lin lin = w4::W4Lin::init(store, argv[3]);
  const auto x = read_file(argv[5], (size_t)(M * lin.k * 2));
  const size_t ybytes = (size_t)(M * lin.n * (f32 ? 4 : 2));
  const size_t ws = lin.workspace(M);  // optional: the split-K route on batched shapes
  void *dx = nullptr, *dy = nullptr, *dws = nullptr;
  hip_ok(hipMalloc(&dx, std::max<size_t>(x.size(), 16)), "hipMalloc x");
  hip_ok(hipMalloc(&dy, std::max<size_t>(ybytes, 16)), "hipMalloc y");
  if (ws) hip_ok(hipMalloc(&dws, ws), "hipMalloc workspace");
  hip_ok(hipMemcpy(dx, x.data(), x.size(), hipMemcpyHostToDevice), "copy x");
  if (f32) lin.linear(static_cast<const uint16_t*>(dx), static_cast<float*>(dy), M, dws, ws, nullptr);
  else lin.linear(static_cast<const uint16_t*>(dx), static_cast<uint16_t*>(dy), M, dws, ws, nullptr);
  std::vector<char> y(ybytes);
  hip_ok(hipMemcpy(y.data(), dy, ybytes, hipMemcpyDeviceToHost), "copy y");
  write_file(argv[6], y.data(), ybytes);
  (void)hipFree(dx);
  (void)hipFree(dy);
  if (dws) (void)hipFree(dws);
  std::printf("{\"name\": \"%s\", \"M\": %lld, \"n\": %lld, \"k\": %lld, \"group\": %d, \"y\": \"%s\", "
              "\"workspace\": %zu}\n",
              json_escape(argv[3]).c_str(), (long long)M, (long long)lin.n, (long long)lin.k, lin.group,
              f32 ? "f32" : "bf16", ws);
  return 0;
}

int cmd_mlp(int argc, char** argv) {
  if (argc < 8) return usage();
  const bool f32 = argc > 8 && !std::strcmp(argv[8], "f32");
  const int64_t M = std::atoll(argv[5]);
  w4::DeviceStore store(argv[2]);
  const w4::W4Lin gate = w4::W4Lin::init(store, argv[3]);
  const w4::W4Lin up = w4::W4Lin::init(store, argv[4]);
  const auto x = read_file(argv[6], (size_t)(M * gate.k * 2));
  const size_t hbytes = (size_t)(M * gate.n * (f32 ? 4 : 2));
  const size_t ws = w4::gate_up_workspace(gate, M);
  void *dx = nullptr, *dh = nullptr, *dws = nullptr;
  hip_ok(hipMalloc(&dx, std::max<size_t>(x.size(), 16)), "hipMalloc x");
  hip_ok(hipMalloc(&dh, std::max<size_t>(hbytes, 16)), "hipMalloc h");
  if (ws) hip_ok(hipMalloc(&dws, ws), "hipMalloc workspace");
  hip_ok(hipMemcpy(dx, x.data(), x.size(), hipMemcpyHostToDevice), "copy x");
  if (f32) w4::gate_up_gelu(gate, up, static_cast<const uint16_t*>(dx), static_cast<float*>(dh), M, dws, ws, nullptr);
  else w4::gate_up_gelu(gate, up, static_cast<const uint16_t*>(dx), static_cast<uint16_t*>(dh), M, dws, ws, nullptr);
  std::vector<char> h(hbytes);
  hip_ok(hipMemcpy(h.data(), dh, hbytes, hipMemcpyDeviceToHost), "copy h");
  write_file(argv[7], h.data(), hbytes);
  (void)hipFree(dx);
  (void)hipFree(dh);
  if (dws) (void)hipFree(dws);
  std::printf("{\"gate\": \"%s\", \"up\": \"%s\", \"M\": %lld, \"F\": %lld, \"k\": %lld, \"workspace\": %zu, \"h\": \"%s\"}\n",
              json_escape(argv[3]).c_str(), json_escape(argv[4]).c_str(), (long long)M, (long long)gate.n,
              (long long)gate.k, ws, f32 ? "f32" : "bf16");
  return 0;
}

int cmd_qkv(int argc, char** argv) {
  if (argc < 8) return usage();
  const int j = std::atoi(argv[4]);
  const int64_t M = std::atoll(argv[5]);
  w4::DeviceStore store(argv[2]);
  const std::string l = std::string(argv[3]) + "." + std::to_string(j) + ".self_attn.";
  std::vector<std::string> names = {"q_proj", "k_proj"};
  if (!w4::g12_is_full(j)) names.push_back("v_proj");  // full layers: V = K (g12.zig)
  std::vector<w4::W4Lin> lins;
  for (const auto& n : names) lins.push_back(w4::W4Lin::init(store, l + n));
  const auto x = read_file(argv[6], (size_t)(M * lins[0].k * 2));
  void* dx = nullptr;
  hip_ok(hipMalloc(&dx, std::max<size_t>(x.size(), 16)), "hipMalloc x");
  hip_ok(hipMemcpy(dx, x.data(), x.size(), hipMemcpyHostToDevice), "copy x");
  std::vector<uint16_t*> ys;
  for (const auto& lin : lins) {
    void* p = nullptr;
    hip_ok(hipMalloc(&p, std::max<size_t>((size_t)(M * lin.n * 2), 16)), "hipMalloc y");
    ys.push_back(static_cast<uint16_t*>(p));
  }
  const size_t ws = w4::linear_group_workspace(lins, M);  // optional: split-K members
  void* dws = nullptr;
  if (ws) hip_ok(hipMalloc(&dws, ws), "hipMalloc workspace");
  w4::linear_group(lins, static_cast<const uint16_t*>(dx), ys, M, dws, ws, nullptr);
  if (dws) (void)hipFree(dws);
  for (size_t i = 0; i < lins.size(); ++i) {
    std::vector<char> h((size_t)(M * lins[i].n * 2));
    hip_ok(hipMemcpy(h.data(), ys[i], h.size(), hipMemcpyDeviceToHost), "copy y");
    write_file(std::string(argv[7]) + "." + names[i].substr(0, 1) + ".bin", h.data(), h.size());
    (void)hipFree(ys[i]);
  }
  (void)hipFree(dx);
  std::printf("{\"layer\": %d, \"linears\": %zu, \"M\": %lld, \"workspace\": %zu}\n", j, lins.size(),
              (long long)M, ws);
  return 0;
}

int cmd_head(int argc, char** argv) {
  if (argc < 9) return usage();
  const int64_t M = std::atoll(argv[4]);
  const float cap = (float)std::atof(argv[6]);
  const int topk = std::atoi(argv[7]);
  w4::DeviceStore store(argv[2]);
  const w4::TensorInfo& ti = store.file().info(argv[3]);
  if (ti.dtype != "BF16" || ti.shape.size() != 2) throw std::runtime_error(std::string(argv[3]) + ": not bf16 [V, K]");
  const int64_t V = ti.shape[0], K = ti.shape[1];
  const uint16_t* e = static_cast<const uint16_t*>(store.device(argv[3]));
  const auto x = read_file(argv[5], (size_t)(M * K * 2));
  const size_t ws = w4::lm_head_workspace(M, V, K, topk);
  void *dx = nullptr, *dl = nullptr, *dv = nullptr, *di = nullptr, *dws = nullptr;
  hip_ok(hipMalloc(&dx, std::max<size_t>(x.size(), 16)), "hipMalloc x");
  hip_ok(hipMalloc(&dl, std::max<size_t>((size_t)(M * V * 4), 16)), "hipMalloc logits");
  hip_ok(hipMalloc(&dv, std::max<size_t>((size_t)(M * topk * 4), 16)), "hipMalloc values");
  hip_ok(hipMalloc(&di, std::max<size_t>((size_t)(M * topk * 4), 16)), "hipMalloc indices");
  if (ws) hip_ok(hipMalloc(&dws, ws), "hipMalloc workspace");
  hip_ok(hipMemcpy(dx, x.data(), x.size(), hipMemcpyHostToDevice), "copy x");
  w4::lm_head(e, V, K, static_cast<const uint16_t*>(dx), M, cap, topk, static_cast<float*>(dl),
              static_cast<float*>(dv), static_cast<int32_t*>(di), dws, ws, nullptr);
  const std::string out = argv[8];
  std::vector<char> b((size_t)(M * V * 4));
  hip_ok(hipMemcpy(b.data(), dl, b.size(), hipMemcpyDeviceToHost), "copy logits");
  write_file(out + ".logits.bin", b.data(), b.size());
  b.resize((size_t)(M * topk * 4));
  hip_ok(hipMemcpy(b.data(), dv, b.size(), hipMemcpyDeviceToHost), "copy values");
  write_file(out + ".values.bin", b.data(), b.size());
  hip_ok(hipMemcpy(b.data(), di, b.size(), hipMemcpyDeviceToHost), "copy indices");
  write_file(out + ".indices.bin", b.data(), b.size());
  for (void* p : {dx, dl, dv, di, dws})
    if (p) (void)hipFree(p);
  std::printf("{\"V\": %lld, \"K\": %lld, \"M\": %lld, \"topk\": %d}\n", (long long)V, (long long)K, (long long)M, topk);
  return 0;
}

int cmd_dequant(int argc, char** argv) {
  if (argc < 5) return usage();
  w4::DeviceStore store(argv[2]);
  const w4::W4Lin lin = w4::W4Lin::init(store, argv[3]);
  const size_t bytes = (size_t)(lin.n * lin.k * 2);
  void* dw = nullptr;
  hip_ok(hipMalloc(&dw, std::max<size_t>(bytes, 16)), "hipMalloc w");
  lin.toW(static_cast<uint16_t*>(dw), nullptr);
  std::vector<char> w(bytes);
  hip_ok(hipMemcpy(w.data(), dw, bytes, hipMemcpyDeviceToHost), "copy w");
  write_file(argv[4], w.data(), bytes);
  (void)hipFree(dw);
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) return usage();
  try {
    const std::string cmd = argv[1];
    if (cmd == "census") return cmd_census(argc, argv);
    if (cmd == "layer12") return cmd_layer12(argc, argv);
    if (cmd == "linear") return cmd_linear(argc, argv);
    if (cmd == "dequant") return cmd_dequant(argc, argv);
    if (cmd == "mlp") return cmd_mlp(argc, argv);
    if (cmd == "qkv") return cmd_qkv(argc, argv);
    if (cmd == "head") return cmd_head(argc, argv);
    return usage();
  } catch (const w4::Error& e) {
    std::fprintf(stderr, "w4lin_tool: %s (status %d)\n", e.what(), e.status());
    return 3;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "w4lin_tool: %s\n", e.what());
    return 3;
  }
}
