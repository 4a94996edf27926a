"""The linears of one decoder layer as a chain, through the C++ host mirror
(w4lin_tool chain -> w4lin.hpp -> libw4a16.so), against the oracle's chain.

Reference chain (TheCause/gemma4-zml-probe, zml_runner/engine.zig:540-663):
  q, k, v = dotPrec(h0, q/k/v_proj)           :552,571,583  (one grouped call here)
  attn_out = dotPrec(ctx, o_proj)             :649
  h = gelu(dotPrec(xff, gate)) * dotPrec(xff, up); mlp = dotPrec(h, down)   :653
  E2B: g = gelu(dotPrec(h2, per_layer_input_gate)) * ple_i;
       ple = dotPrec(g, per_layer_projection)                               :658-661
with the wiring of the two models: 12B full layers ((j + 1) % 6 == 0) have no v_proj
(zml_runner/g12.zig:139-166); E2B layers j >= first_kv_shared = 15 read the writer's
K/V cache and project only q (engine.zig:52,560-567), and use the double-wide MLP
(F = 12288, gemma4-e2b-it-meta/config.json use_double_wide_mlp; the unpack fixture's
deq_dn20 [1536, 12288], scripts/57_w4_unpack_fixture.py:74).  The attention context,
xff, h2 and ple_i come from parts of the layer outside the W4 path (attention, norms,
residuals), so the test supplies them; the chain links on the path are h -> down and
g -> per_layer_projection.

Flows: "bf16" is dotPrec with fam = bf16 (inputs rounded to bf16, each dot output
rounded to bf16, h and g rounded to bf16 before their consumer), "f32" is fam = null
(f32 activations and outputs).

Tolerances (eps = 2^-24, gamma_K = K eps / (1 - K eps), mag = sum_k |x_k||w_k|):
  linear, bf16 out:  |y - y_oracle32| <= ulp_bf16(y_oracle32) + 2 gamma_K mag
  linear, f32 out:   |y - y64| <= 2 gamma_K mag
  h: the gate/up bound of tests/test_gpu_gate_up.py
  down / per_layer_projection are checked twice: against the oracle applied to the
  host's own h (resp. g) with the linear bound, and end to end against the oracle
  applied to the oracle's h (resp. g) with that bound plus sum_k |w_k| |dh_k|, where
  dh is the measured difference of the two inputs.
Weights and activations are synthetic (the checkpoints are not in this container) at
the real layer shapes.
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import PKG

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from safetensors.torch import save_file  # noqa: E402

from oracle import w4a16_oracle as o  # noqa: E402

TOOL = os.path.join(PKG, "w4lin_tool")
PREFIX = "model.language_model.layers"
EPS = 2.0 ** -24

# geometry (engine.zig:50-80 for E2B, g12.zig for 12B)
MODELS = {
    "g12": dict(D=3840, nh=16, hd=(256, 512), kvh=(8, 1), full_period=6, F=(15360, 15360)),
    "e2b": dict(D=1536, nh=8, hd=(256, 512), kvh=(1, 1), full_period=5, F=(6144, 12288), P=256),
}


def say(msg: str) -> None:
    print(f"[gpu-chain] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not os.path.exists(TOOL):
        subprocess.run(["make", "-s", "-C", os.path.join(PKG, "host")], check=True)


def layer_modules(model: str, j: int) -> dict:
    """module name -> (n, k) of layer j, in engine order."""
    g = MODELS[model]
    full = (j + 1) % g["full_period"] == 0
    hd, kvh = g["hd"][full], g["kvh"][full]
    D, nh = g["D"], g["nh"]
    reader = model == "e2b" and j >= 15
    F = g["F"][reader]
    mods = {"self_attn.q_proj": (nh * hd, D)}
    if not reader:
        mods["self_attn.k_proj"] = (kvh * hd, D)
        if model == "e2b" or not full:
            mods["self_attn.v_proj"] = (kvh * hd, D)
    mods["self_attn.o_proj"] = (D, nh * hd)
    mods["mlp.gate_proj"] = (F, D)
    mods["mlp.up_proj"] = (F, D)
    mods["mlp.down_proj"] = (D, F)
    if model == "e2b":
        mods["per_layer_input_gate"] = (g["P"], D)
        mods["per_layer_projection"] = (D, g["P"])
    return mods


def write_layer(path: str, model: str, j: int, seed: int) -> dict:
    """Synthetic packed checkpoint of layer j; returns name -> (pk, sc) as numpy."""
    tensors, weights = {}, {}
    for i, (m, (n, k)) in enumerate(layer_modules(model, j).items()):
        _, pk, sc = o.synth_weights(n, k, seed + i)
        base = f"{PREFIX}.{j}.{m}"
        tensors[base + ".weight_packed"] = torch.from_numpy(pk)
        tensors[base + ".weight_scale"] = torch.from_numpy(sc.view(np.int16)).view(torch.bfloat16)
        tensors[base + ".weight_shape"] = torch.tensor([n, k], dtype=torch.int64)
        weights[m] = (pk, sc)
    save_file(tensors, path)
    return weights


def ulp_bf16(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def gam(K):
    return K * EPS / (1 - K * EPS)


def act(M, K, seed, f32):
    """Activations: bf16 N(0,1) or f32 N(0,1) (f32 values off the bf16 grid)."""
    if f32:
        return np.random.Generator(np.random.PCG64(seed)).standard_normal((M, K), dtype=np.float32)
    return o.synth_x(M, K, seed)


def as64(x):
    return x.astype(np.float64) if x.dtype == np.float32 else o.bf16_to_f32(x).astype(np.float64)


def load(path, M, n, f32):
    if f32:
        return np.fromfile(path, dtype=np.float32).reshape(M, n).astype(np.float64)
    return o.bf16_to_f32(np.fromfile(path, dtype=np.uint16).reshape(M, n)).astype(np.float64)


def check_linear(y, x, w, f32, what):
    """y (float64 view of the tool's output) against the oracle linear on input x."""
    K = w.shape[1]
    if f32:
        y64, mag = o.matmul_f32x(x, w, f64=True)
        b = 2 * gam(K) * mag
        ref = y64
    else:
        ref = o.matmul_f32(x, w).astype(np.float64)
        _, mag = o.matmul_f64(x, w)
        b = ulp_bf16(ref) + 2 * gam(K) * mag
    excess = np.abs(y - ref) - b
    assert np.all(excess <= 0), (what, float(np.max(excess)), np.unravel_index(np.argmax(excess), excess.shape))
    return ref, b


def check_end_to_end(y, w, x_host, x_oracle, f32, what):
    """y = consumer(x_host) from the tool; compare with the oracle's consumer(x_oracle):
    the linear bound on x_oracle plus sum_k |w_k| |x_host - x_oracle|_k."""
    wf = np.abs(o.bf16_to_f32(w).astype(np.float64))
    prop = np.abs(as64(x_host) - as64(x_oracle)) @ wf.T
    K = w.shape[1]
    if f32:
        ref, mag = o.matmul_f32x(x_oracle, w, f64=True)
        b = 2 * gam(K) * (mag + prop) + prop
    else:
        ref = o.matmul_f32(x_oracle, w).astype(np.float64)
        _, mag = o.matmul_f64(x_oracle, w)
        b = ulp_bf16(ref) + 2 * gam(K) * (mag + prop) + prop + ulp_bf16(np.abs(ref) + prop)
    excess = np.abs(y - ref) - b
    assert np.all(excess <= 0), (what, float(np.max(excess)))


def run_chain(tmp_path, model, j, M, flow, seed=5000):
    f32 = flow == "f32"
    ck = str(tmp_path / f"{model}_{j}.safetensors")
    say(f"chain {model} layer {j} M={M} flow={flow}: writing checkpoint")
    W = write_layer(ck, model, j, seed)
    mods = layer_modules(model, j)
    D = MODELS[model]["D"]
    ins = {"x": act(M, D, seed + 101, f32), "a": act(M, mods["self_attn.o_proj"][1], seed + 102, f32),
           "xff": act(M, D, seed + 103, f32)}
    if model == "e2b":
        ins["h2"] = act(M, D, seed + 104, f32)
        P = MODELS["e2b"]["P"]
        ins["ple"] = np.random.Generator(np.random.PCG64(seed + 105)).standard_normal((M, P), dtype=np.float32)
    for k, v in ins.items():
        v.tofile(tmp_path / f"in.{k}.bin")
    say(f"chain {model} layer {j} M={M} flow={flow}: running the C++ host")
    p = subprocess.run([TOOL, "chain", ck, PREFIX, str(j), str(M), model, flow, str(tmp_path / "in"),
                        str(tmp_path / "out")], capture_output=True, text=True, timeout=300)
    assert p.returncode == 0, p.stderr
    info = json.loads(p.stdout)
    w = {m: o.dequant(pk, sc) for m, (pk, sc) in W.items()}
    out = lambda tag, n: load(tmp_path / f"out.{tag}.bin", M, n, f32)  # noqa: E731

    # q, k, v: one grouped call on x
    qkv = [m for m in mods if m.startswith("self_attn.") and m != "self_attn.o_proj"]
    assert info["qkv"] == len(qkv)
    for m in qkv:
        check_linear(out(m[10], mods[m][0]), ins["x"], w[m], f32, m)
    for m in ("k", "v"):
        if f"self_attn.{m}_proj" not in mods:
            assert not (tmp_path / f"out.{m}.bin").exists()
    check_linear(out("o", D), ins["a"], w["self_attn.o_proj"], f32, "o_proj")

    # MLP: h within the gate/up bound, then down fed by h
    from test_gpu_gate_up import bound
    F = mods["mlp.gate_proj"][0]
    assert info["F"] == F
    pg, sg = W["mlp.gate_proj"]
    pu, su = W["mlp.up_proj"]
    h64, g, u, mg, mu = o.gate_up_gelu(ins["xff"], pg, sg, pu, su, 32, not f32)
    b = bound(g, u, mg, mu, D, not f32)
    h = out("h", F)
    if not f32:
        b = b + ulp_bf16(np.abs(h64) + b)
    assert np.all(np.abs(h - h64) <= b), "gate_up_gelu"
    h_host = (np.fromfile(tmp_path / "out.h.bin", dtype=np.float32).reshape(M, F) if f32
              else np.fromfile(tmp_path / "out.h.bin", dtype=np.uint16).reshape(M, F))
    h_oracle = h64.astype(np.float32) if f32 else o.round_bf16(h64.astype(np.float32))
    y = out("mlp", D)
    check_linear(y, h_host, w["mlp.down_proj"], f32, "down_proj(h)")
    check_end_to_end(y, w["mlp.down_proj"], h_host, h_oracle, f32, "down_proj end to end")

    if model == "e2b":
        P = MODELS["e2b"]["P"]
        pg_ref, _ = check_linear(out("pg", P), ins["h2"], w["per_layer_input_gate"], f32, "per_layer_input_gate")
        g_tool = out("g", P)
        # the host glue: gelu(pg) * ple_i in double, one rounding to f32 (f32 flow) or bf16
        g_exp = o.gelu_tanh(out("pg", P)) * ins["ple"].astype(np.float64)
        tol = (np.abs(g_exp) * 2.0 ** -23 if f32 else ulp_bf16(g_exp)) + 2.0 ** -140
        assert np.all(np.abs(g_tool - g_exp) <= tol), "gelu * ple glue"
        g_host = (np.fromfile(tmp_path / "out.g.bin", dtype=np.float32).reshape(M, P) if f32
                  else np.fromfile(tmp_path / "out.g.bin", dtype=np.uint16).reshape(M, P))
        g64 = o.gelu_tanh(pg_ref) * ins["ple"].astype(np.float64)
        g_oracle = g64.astype(np.float32) if f32 else o.round_bf16(g64.astype(np.float32))
        y = out("ple", D)
        check_linear(y, g_host, w["per_layer_projection"], f32, "per_layer_projection(g)")
        check_end_to_end(y, w["per_layer_projection"], g_host, g_oracle, f32, "per_layer_projection end to end")
    say(f"chain {model} layer {j} M={M} flow={flow}: ok")


@pytest.mark.parametrize("j,M,flow", [(0, 1, "bf16"), (5, 1, "bf16"), (0, 2, "f32")])
def test_chain_12b_layer(tmp_path, j, M, flow):
    """12B sliding layer 0 (q, k, v) and full layer 5 (q, k; V = K), decode."""
    run_chain(tmp_path, "g12", j, M, flow)


@pytest.mark.parametrize("j,M,flow", [(0, 1, "bf16"), (4, 3, "f32"), (15, 1, "bf16"), (15, 8, "bf16")])
def test_chain_e2b_layer(tmp_path, j, M, flow):
    """E2B layers with the per-layer-embedding linears: sliding writer 0, full layer 4
    (head dim 512) on f32 activations, and KV-shared layer 15 (q only, double-wide MLP
    F = 12288) at decode and M = 8."""
    run_chain(tmp_path, "e2b", j, M, flow)
