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
//   w4lin_tool chain <file.safetensors> <prefix> <j> <M> <g12|e2b> <bf16|f32> <in_prefix> <out_prefix>
//       the linears of decoder layer j in engine order (engine.zig:552-663): q, k, v as one
//       grouped call on x (per the model's wiring: 12B full layers have no v, g12.zig;
//       E2B KV-shared layers j >= 15 only q, engine.zig:560-567), o on the attention
//       context a, gate_up_gelu on xff, down fed by its output h, and for E2B the
//       per-layer-embedding pair: pg = h2 . per_layer_input_gate^T, g = gelu(pg) * ple
//       (host f32, the engine's elementwise glue), then g . per_layer_projection^T.
//       Flow bf16 is dotPrec with fam = bf16 (bf16 inputs and outputs, h and g rounded to
//       bf16 before their consumer); flow f32 is fam = null (f32 throughout).
//       Reads <in>.x/.a/.xff[/.h2].bin (bf16 or f32 per flow) and <in>.ple.bin (f32);
//       writes <out>.q/.k/.v/.o/.h/.mlp[/.pg/.g/.ple].bin in the flow's dtype.
//   w4lin_tool head <file.safetensors> <embed_name> <M> <x.bin> <softcap> <topk> <out_prefix>
//       logits (f32) and top-k of the tied-embedding head (engine.zig:765-766);
//       writes <out_prefix>.logits.bin, .values.bin (f32), .indices.bin (i32).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iostream>
#include <memory>
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
               "       w4lin_tool head <file> <embed_name> <M> <x.bin> <softcap> <topk> <out_prefix>\n"
               "       w4lin_tool chain <file> <prefix> <j> <M> <g12|e2b> <bf16|f32> <in_prefix> <out_prefix>\n");
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

// Device buffer freed on scope exit.
struct DevBuf {
  void* p = nullptr;
  size_t n = 0;
  explicit DevBuf(size_t bytes) : n(bytes) { hip_ok(hipMalloc(&p, std::max<size_t>(bytes, 16)), "hipMalloc"); }
  ~DevBuf() { (void)hipFree(p); }
  DevBuf(const DevBuf&) = delete;
  DevBuf& operator=(const DevBuf&) = delete;
  template <class T>
  T* as() const { return static_cast<T*>(p); }
  void upload(const std::vector<char>& h) { hip_ok(hipMemcpy(p, h.data(), h.size(), hipMemcpyHostToDevice), "upload"); }
  std::vector<char> download() const {
    std::vector<char> h(n);
    hip_ok(hipMemcpy(h.data(), p, n, hipMemcpyDeviceToHost), "download");
    return h;
  }
};

float bf16_bits_to_float(uint16_t h) {
  const uint32_t u = (uint32_t)h << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

uint16_t float_to_bf16_rne(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// gelu with the tanh approximation (ZML's Tensor.gelu), in double, rounded to f32.
float gelu_tanh_host(float g) {
  const double x = g, z = 0.7978845608028654 * (x + 0.044715 * x * x * x);
  return (float)(x / (1.0 + std::exp(-2.0 * z)));
}

int cmd_chain(int argc, char** argv) {
  if (argc < 10) return usage();
  const std::string prefix = argv[3], model = argv[6], flow = argv[7], in = argv[8], out = argv[9];
  const int j = std::atoi(argv[4]);
  const int64_t M = std::atoll(argv[5]);
  if ((model != "g12" && model != "e2b") || (flow != "bf16" && flow != "f32") || M < 1) return usage();
  const bool e2b = model == "e2b", f32 = flow == "f32";
  const size_t es = f32 ? 4 : 2;
  w4::DeviceStore store(argv[2]);
  const std::string l = prefix + "." + std::to_string(j) + ".";
  // q/k/v wiring: 12B full layers take V from k_proj (no v_proj, g12.zig); E2B layers from
  // first_kv_shared = 15 on read the writer's cache and project only q (engine.zig:560-567).
  std::vector<std::string> qkv = {"q"};
  if (!(e2b && j >= 15)) {
    qkv.push_back("k");
    if (e2b || !w4::g12_is_full(j)) qkv.push_back("v");
  }
  std::vector<w4::W4Lin> lins;
  for (const auto& n : qkv) lins.push_back(w4::W4Lin::init(store, l + "self_attn." + n + "_proj"));
  const w4::W4Lin o = w4::W4Lin::init(store, l + "self_attn.o_proj");
  const w4::W4Lin gate = w4::W4Lin::init(store, l + "mlp.gate_proj");
  const w4::W4Lin up = w4::W4Lin::init(store, l + "mlp.up_proj");
  const w4::W4Lin down = w4::W4Lin::init(store, l + "mlp.down_proj");
  const int64_t D = lins[0].k;

  DevBuf x(M * D * es), a(M * o.k * es), xff(M * gate.k * es);
  x.upload(read_file(in + ".x.bin", x.n));
  a.upload(read_file(in + ".a.bin", a.n));
  xff.upload(read_file(in + ".xff.bin", xff.n));

  // q, k, v: one grouped call
  std::vector<std::unique_ptr<DevBuf>> ys;
  for (const auto& lin : lins) ys.emplace_back(new DevBuf(M * lin.n * es));
  if (f32) {
    DevBuf ws(w4::linear_group_workspace_f32(lins, M));
    std::vector<float*> yp;
    for (auto& y : ys) yp.push_back(y->as<float>());
    w4::linear_group_f32(lins, x.as<float>(), yp, M, ws.p, ws.n, nullptr);
  } else {
    DevBuf ws(w4::linear_group_workspace(lins, M));
    std::vector<uint16_t*> yp;
    for (auto& y : ys) yp.push_back(y->as<uint16_t>());
    w4::linear_group(lins, x.as<uint16_t>(), yp, M, ws.p, ws.n, nullptr);
  }
  // o on the attention context
  DevBuf yo(M * o.n * es);
  if (f32) {
    DevBuf ws(o.workspace_f32(M));
    o.linear_f32(a.as<float>(), yo.as<float>(), M, ws.p, ws.n, nullptr);
  } else {
    DevBuf ws(o.workspace(M));
    o.linear(a.as<uint16_t>(), yo.as<uint16_t>(), M, ws.p, ws.n, nullptr);
  }
  // MLP: h = gelu(xff . gate^T) * (xff . up^T), then down fed by h
  DevBuf h(M * gate.n * es), ymlp(M * down.n * es);
  if (down.k != gate.n) throw std::runtime_error("down_proj K != gate_proj N");
  if (f32) {
    DevBuf ws(w4::gate_up_workspace_f32(gate, M));
    w4::gate_up_gelu_f32(gate, up, xff.as<float>(), h.as<float>(), M, ws.p, ws.n, nullptr);
    DevBuf ws2(down.workspace_f32(M));
    down.linear_f32(h.as<float>(), ymlp.as<float>(), M, ws2.p, ws2.n, nullptr);
  } else {
    DevBuf ws(w4::gate_up_workspace(gate, M));
    w4::gate_up_gelu(gate, up, xff.as<uint16_t>(), h.as<uint16_t>(), M, ws.p, ws.n, nullptr, true);
    DevBuf ws2(down.workspace(M));
    down.linear(h.as<uint16_t>(), ymlp.as<uint16_t>(), M, ws2.p, ws2.n, nullptr);
  }
  for (size_t i = 0; i < lins.size(); ++i) {
    const auto b = ys[i]->download();
    write_file(out + "." + qkv[i] + ".bin", b.data(), b.size());
  }
  for (auto* kv : {&yo, &h, &ymlp}) {
    const auto b = kv->download();
    const char* tag = kv == &yo ? ".o.bin" : kv == &h ? ".h.bin" : ".mlp.bin";
    write_file(out + tag, b.data(), b.size());
  }
  if (e2b) {
    const w4::W4Lin pgate = w4::W4Lin::init(store, l + "per_layer_input_gate");
    const w4::W4Lin pproj = w4::W4Lin::init(store, l + "per_layer_projection");
    if (pproj.k != pgate.n) throw std::runtime_error("per_layer_projection K != per_layer_input_gate N");
    const int64_t P = pgate.n;
    DevBuf h2(M * pgate.k * es), pg(M * P * es), g(M * P * es), yple(M * pproj.n * es);
    h2.upload(read_file(in + ".h2.bin", h2.n));
    const auto ple = read_file(in + ".ple.bin", (size_t)(M * P * 4));
    if (f32) {
      DevBuf ws(pgate.workspace_f32(M));
      pgate.linear_f32(h2.as<float>(), pg.as<float>(), M, ws.p, ws.n, nullptr);
    } else {
      DevBuf ws(pgate.workspace(M));
      pgate.linear(h2.as<uint16_t>(), pg.as<uint16_t>(), M, ws.p, ws.n, nullptr);
    }
    const auto pgh = pg.download();
    std::vector<char> gh(g.n);
    for (int64_t i = 0; i < M * P; ++i) {
      float v, pi;
      std::memcpy(&pi, ple.data() + 4 * i, 4);
      if (f32) std::memcpy(&v, pgh.data() + 4 * i, 4);
      else {
        uint16_t b;
        std::memcpy(&b, pgh.data() + 2 * i, 2);
        v = bf16_bits_to_float(b);
      }
      const float r = gelu_tanh_host(v) * pi;
      if (f32) std::memcpy(gh.data() + 4 * i, &r, 4);
      else {
        const uint16_t b = float_to_bf16_rne(r);
        std::memcpy(gh.data() + 2 * i, &b, 2);
      }
    }
    g.upload(gh);
    if (f32) {
      DevBuf ws(pproj.workspace_f32(M));
      pproj.linear_f32(g.as<float>(), yple.as<float>(), M, ws.p, ws.n, nullptr);
    } else {
      DevBuf ws(pproj.workspace(M));
      pproj.linear(g.as<uint16_t>(), yple.as<uint16_t>(), M, ws.p, ws.n, nullptr);
    }
    write_file(out + ".pg.bin", pgh.data(), pgh.size());
    write_file(out + ".g.bin", gh.data(), gh.size());
    const auto b = yple.download();
    write_file(out + ".ple.bin", b.data(), b.size());
  }
  std::printf("{\"layer\": %d, \"model\": \"%s\", \"flow\": \"%s\", \"M\": %lld, \"qkv\": %zu, \"F\": %lld}\n", j,
              model.c_str(), flow.c_str(), (long long)M, lins.size(), (long long)gate.n);
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
    if (cmd == "chain") return cmd_chain(argc, argv);
    return usage();
  } catch (const w4::Error& e) {
    std::fprintf(stderr, "w4lin_tool: %s (status %d)\n", e.what(), e.status());
    return 3;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "w4lin_tool: %s\n", e.what());
    return 3;
  }
}
