"""C++ host mirror of the W4 brick (gemma4-zml-probe_amd/host/w4lin.hpp), through its
command-line front end w4lin_tool.

Mirrors (TheCause/gemma4-zml-probe):
  W4Lin.init / toW, unpackW4 / dequantW4      zml_runner/w4.zig:16-54
  packed-checkpoint census and asserts         scripts/63_u_dequant_export.py:85-114
  12B wiring: v_proj only on sliding layers    zml_runner/g12.zig:94-166, docs/U_12B_CONTRACT.md:54-71
The checkpoints here are small synthetic safetensors files with the reference's key names
(the real checkpoints are not in this container).
"""
from __future__ import annotations

import json
import os
import subprocess

import numpy as np
import pytest

from conftest import PKG

torch = pytest.importorskip("torch")
from safetensors.torch import save_file  # noqa: E402

from oracle import w4a16_oracle as o  # noqa: E402

TOOL = os.path.join(PKG, "w4lin_tool")
PREFIX = "model.language_model.layers"


@pytest.fixture(scope="module")
def tool():
    if not os.path.exists(TOOL):
        subprocess.run(["make", "-s", "-C", os.path.join(PKG, "host")], check=True)
    return TOOL


def run(tool, *args):
    p = subprocess.run([tool, *map(str, args)], capture_output=True, text=True)
    return p.returncode, p.stdout, p.stderr


def packed_linear(n, k, seed, group=32, shape=True):
    """weight_packed I32 [n, k/8], weight_scale BF16 [n, k/group], weight_shape I64 [2]."""
    _, pk, sc = o.synth_weights(n, k, seed, group)
    t = {"weight_packed": torch.from_numpy(pk.copy()),
         "weight_scale": torch.from_numpy(sc.view(np.int16).copy()).view(torch.bfloat16)}
    if shape:
        t["weight_shape"] = torch.tensor([n, k], dtype=torch.int64)
    return t


def g12_like(path, layers=6, n=32, k=64):
    """Layers 0..layers-1 of the 12B key layout at a small size; layer 5 is full (no v_proj)."""
    tensors = {}
    s = 0
    for j in range(layers):
        mods = ["self_attn.q_proj", "self_attn.k_proj", "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj",
                "mlp.down_proj"]
        if (j + 1) % 6 != 0:
            mods.append("self_attn.v_proj")
        for m in mods:
            s += 1
            for suffix, t in packed_linear(n, k, 100 + s).items():
                tensors[f"{PREFIX}.{j}.{m}.{suffix}"] = t
        tensors[f"{PREFIX}.{j}.input_layernorm.weight"] = torch.ones(k, dtype=torch.bfloat16)
    tensors["model.language_model.embed_tokens.weight"] = torch.zeros((16, k), dtype=torch.bfloat16)
    save_file(tensors, path, metadata={"format": "pt", "note": "quo\"ted \\ and é"})
    return tensors


def census(tool, path, *extra):
    rc, out, err = run(tool, "census", path, *extra)
    lines = [json.loads(line) for line in out.strip().splitlines()]
    return rc, lines[:-1], lines[-1], err


def test_census_12b_layout(tool, tmp_path):
    path = str(tmp_path / "g12.safetensors")
    g12_like(path)
    rc, lins, summary, err = census(tool, path, "--expect", 41)
    assert rc == 0, err
    assert summary == {"linears": 41, "errors": []}
    assert all(e["n"] == 32 and e["k"] == 64 and e["group"] == 32 and e["weight_shape"] for e in lins)
    names = [e["name"] for e in lins]
    assert names == sorted(names)
    assert f"{PREFIX}.5.self_attn.v_proj" not in names and f"{PREFIX}.4.self_attn.v_proj" in names
    rc, _, _, _ = census(tool, path, "--expect", 328)
    assert rc == 1  # count mismatch is an error


def test_layer12_wiring(tool, tmp_path):
    path = str(tmp_path / "g12.safetensors")
    g12_like(path)
    rc, out, _ = run(tool, "layer12", path, PREFIX, 0)
    names = [json.loads(line)["name"] for line in out.strip().splitlines()]
    assert rc == 0
    assert [n.split(".", 4)[-1] for n in names] == ["self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                                    "self_attn.o_proj", "mlp.gate_proj", "mlp.up_proj",
                                                    "mlp.down_proj"]
    rc, out, _ = run(tool, "layer12", path, PREFIX, 5)  # full layer: K = V, no v_proj consumed
    assert rc == 0 and len(out.strip().splitlines()) == 6
    rc, out, _ = run(tool, "layer12", path, PREFIX, 6)  # absent layer: every module reported missing
    assert rc == 1 and all(json.loads(line).get("missing") for line in out.strip().splitlines())


@pytest.mark.parametrize("case", ["scale_shape", "scale_dtype", "packed_dtype", "weight_shape", "orphan_scale",
                                  "zero_point", "g_idx", "group_not_32k"])
def test_census_rejects(tool, tmp_path, case):
    t = {f"a.{k}": v for k, v in packed_linear(16, 128, 7).items()}
    if case == "scale_shape":
        t["a.weight_scale"] = t["a.weight_scale"][:, :3].contiguous()
    elif case == "scale_dtype":
        t["a.weight_scale"] = t["a.weight_scale"].float()
    elif case == "packed_dtype":
        t["a.weight_packed"] = t["a.weight_packed"].to(torch.int64)
    elif case == "weight_shape":
        t["a.weight_shape"] = torch.tensor([16, 120], dtype=torch.int64)
    elif case == "orphan_scale":
        t["b.weight_scale"] = t["a.weight_scale"].clone()
    elif case == "zero_point":
        t["a.weight_zero_point"] = torch.zeros((16, 4), dtype=torch.int32)
    elif case == "g_idx":
        t["a.weight_g_idx"] = torch.zeros(128, dtype=torch.int32)
    elif case == "group_not_32k":
        t["a.weight_scale"] = torch.zeros((16, 8), dtype=torch.bfloat16)  # 128 / 8 = 16-column groups
    path = str(tmp_path / f"{case}.safetensors")
    save_file(t, path)
    rc, _, summary, _ = census(tool, path)
    assert rc == 1 and len(summary["errors"]) == 1, summary


def test_census_groups_and_missing_shape(tool, tmp_path):
    t = {f"a.{k}": v for k, v in packed_linear(8, 256, 1, group=128, shape=False).items()}
    t.update({f"b.{k}": v for k, v in packed_linear(8, 256, 2, group=64).items()})
    path = str(tmp_path / "g.safetensors")
    save_file(t, path)
    rc, lins, summary, _ = census(tool, path)
    assert rc == 0 and summary["errors"] == []
    assert [(e["name"], e["group"], e["weight_shape"]) for e in lins] == [("a", 128, False), ("b", 64, True)]


@pytest.mark.parametrize("blob", [b"", b"\x05\x00\x00\x00\x00\x00\x00\x00{}", b"\xff" * 8 + b"{}",
                                  b"\x02\x00\x00\x00\x00\x00\x00\x00{]"])
def test_malformed_files_fail_cleanly(tool, tmp_path, blob):
    path = tmp_path / "bad.safetensors"
    path.write_bytes(blob)
    rc, _, err = run(tool, "census", str(path))
    assert rc == 3 and "safetensors" in err


def test_empty_header_and_offsets_checked(tool, tmp_path):
    path = tmp_path / "empty.safetensors"
    path.write_bytes(b"\x02\x00\x00\x00\x00\x00\x00\x00{}")
    rc, _, summary, _ = census(tool, str(path))
    assert rc == 0 and summary == {"linears": 0, "errors": []}
    hdr = b'{"a.weight_packed":{"dtype":"I32","shape":[2,1],"data_offsets":[0,16]}}'
    path.write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 8)  # 8 data bytes, offsets say 16
    rc, _, err = run(tool, "census", str(path))
    assert rc == 3 and "data_offsets" in err


@pytest.mark.parametrize("shape", ["[4611686018427387904,4]", "[2147483648,2147483648,4]",
                                   "[9223372036854775807,2]"])
def test_overflowing_shape_rejected(tool, tmp_path, shape):
    """A shape whose element count times the element size wraps 64 bits (e.g. [2^62, 4] of I8
    would wrap to 0 bytes and pass the data_offsets check) is rejected before any use."""
    path = tmp_path / "ovf.safetensors"
    hdr = ('{"a.weight_packed":{"dtype":"I8","shape":%s,"data_offsets":[0,0]}}' % shape).encode()
    path.write_bytes(len(hdr).to_bytes(8, "little") + hdr)
    rc, _, err = run(tool, "census", str(path))
    assert rc == 3 and "overflows" in err, err


@pytest.mark.gpu
@pytest.mark.parametrize("M,out", [(1, "bf16"), (5, "f32"), (70, "bf16"), (24, "f32")])
def test_cpp_w4lin_linear_and_dequant_on_gpu(tool, tmp_path, M, out):
    """W4Lin::init -> linear / toW through the C++ mirror vs the oracle (tolerances of
    test_gpu_parity.py: bit-exact dequant; fp32-accumulate bound for the linear)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    n, k = 96, 512
    t = {f"blk.{kk}": v for kk, v in packed_linear(n, k, 3).items()}
    path = str(tmp_path / "one.safetensors")
    save_file(t, path)
    pk = t["blk.weight_packed"].numpy()
    sc = t["blk.weight_scale"].view(torch.int16).numpy().view(np.uint16)
    w = o.dequant(pk, sc)
    rc, _, err = run(tool, "dequant", path, "blk", tmp_path / "w.bin")
    assert rc == 0, err
    assert np.array_equal(np.fromfile(tmp_path / "w.bin", dtype=np.uint16).reshape(n, k), w)
    x = o.synth_x(M, k, 5)
    x.tofile(tmp_path / "x.bin")
    rc, outp, err = run(tool, "linear", path, "blk", M, tmp_path / "x.bin", tmp_path / "y.bin", out)
    assert rc == 0, err
    # M = 24 and 70 at N = 96: the split-K route (skinny form, LDS prefill form)
    assert (json.loads(outp)["workspace"] > 0) == (M in (24, 70))
    ref32 = o.matmul_f32(x, w)
    y64, mag = o.matmul_f64(x, w)
    gam = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    if out == "f32":
        y = np.fromfile(tmp_path / "y.bin", dtype=np.float32).reshape(M, n)
        assert np.all(np.abs(y - y64) <= 2 * gam * mag + 1e-30)
    else:
        y = o.bf16_to_f32(np.fromfile(tmp_path / "y.bin", dtype=np.uint16).reshape(M, n)).astype(np.float64)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref32), 2.0 ** -126))) - 7)
        assert np.all(np.abs(y - ref32) <= ulp + 2 * gam * mag)


@pytest.mark.gpu
def test_cpp_mlp_rejects_mismatched_up(tool, tmp_path):
    """gate [32, 64] with up [16, 64]: gate_up_gelu throws before any kernel runs (W4Lin.init
    uploads the weights first, hence the GPU mark)."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    t = {f"g.{k}": v for k, v in packed_linear(32, 64, 1).items()}
    t.update({f"u.{k}": v for k, v in packed_linear(16, 64, 2).items()})
    path = str(tmp_path / "mm.safetensors")
    save_file(t, path)
    (tmp_path / "x.bin").write_bytes(b"\0" * (2 * 64))
    rc, _, err = run(tool, "mlp", path, "g", "u", 1, tmp_path / "x.bin", tmp_path / "h.bin")
    assert rc == 3 and "does not match gate" in err


@pytest.mark.gpu
@pytest.mark.parametrize("M,out", [(1, "f32"), (3, "bf16"), (70, "f32"), (8, "bf16")])
def test_cpp_gate_up_gelu_on_gpu(tool, tmp_path, M, out):
    """gate_up_gelu through the C++ mirror (the fused routes, the split-K route at M = 70
    and, at K = 320, M = 8, the unfused one with tool-allocated workspace) against the
    oracle, with the bound of
    tests/test_gpu_gate_up.py."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from test_gpu_gate_up import bound, ulp_bf16
    F, K = 72, (320 if M == 8 else 512)
    t = {f"mlp.gate_proj.{kk}": v for kk, v in packed_linear(F, K, 11).items()}
    t.update({f"mlp.up_proj.{kk}": v for kk, v in packed_linear(F, K, 12).items()})
    path = str(tmp_path / "mlp.safetensors")
    save_file(t, path)
    x = o.synth_x(M, K, 13)
    x.tofile(tmp_path / "x.bin")
    rc, outp, err = run(tool, "mlp", path, "mlp.gate_proj", "mlp.up_proj", M, tmp_path / "x.bin",
                        tmp_path / "h.bin", out)
    assert rc == 0, err
    ws = json.loads(outp)["workspace"]
    # K = 320 at M = 8 takes the unfused route (required workspace); M = 70 the optional
    # split-K route of the LDS prefill kernel (144 virtual rows: one workgroup one-pass)
    assert (ws > 0) if M in (8, 70) else (ws == 0)
    pg = t["mlp.gate_proj.weight_packed"].numpy()
    sg = t["mlp.gate_proj.weight_scale"].view(torch.int16).numpy().view(np.uint16)
    pu = t["mlp.up_proj.weight_packed"].numpy()
    su = t["mlp.up_proj.weight_scale"].view(torch.int16).numpy().view(np.uint16)
    h64, g, u, mg, mu = o.gate_up_gelu(x, pg, sg, pu, su)
    b = bound(g, u, mg, mu, K, False)
    if out == "f32":
        h = np.fromfile(tmp_path / "h.bin", dtype=np.float32).reshape(M, F).astype(np.float64)
    else:
        h = o.bf16_to_f32(np.fromfile(tmp_path / "h.bin", dtype=np.uint16).reshape(M, F)).astype(np.float64)
        b = b + ulp_bf16(np.abs(h64) + b)
    assert np.all(np.abs(h - h64) <= b)


@pytest.mark.gpu
@pytest.mark.parametrize("layer,M,k", [(0, 1, 64), (5, 3, 64), (0, 24, 512)])
def test_cpp_qkv_group_on_gpu(tool, tmp_path, layer, M, k):
    """linear_group through the C++ mirror on the 12B key layout: q, k and (sliding layer 0)
    v, or q and k only (full layer 5, K = V), each against the oracle's single linear with
    the bf16-output bound of test_cpp_w4lin_linear_and_dequant_on_gpu.  At M = 24, K = 512
    the members run one launch each on the split-K route with the tool's workspace."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    n = 32
    path = str(tmp_path / "g12.safetensors")
    t = g12_like(path, layers=6, n=n, k=k)
    x = o.synth_x(M, k, 21)
    x.tofile(tmp_path / "x.bin")
    rc, outp, err = run(tool, "qkv", path, PREFIX, layer, M, tmp_path / "x.bin", tmp_path / "y")
    assert rc == 0, err
    mods = ["q", "k"] if layer == 5 else ["q", "k", "v"]
    assert json.loads(outp)["linears"] == len(mods)
    assert (json.loads(outp)["workspace"] > 0) == (M == 24)
    assert not (tmp_path / "y.v.bin").exists() if layer == 5 else True
    gam = k * 2.0 ** -24 / (1 - k * 2.0 ** -24)
    for mname in mods:
        base = f"{PREFIX}.{layer}.self_attn.{mname}_proj"
        w = o.dequant(t[base + ".weight_packed"].numpy(),
                      t[base + ".weight_scale"].view(torch.int16).numpy().view(np.uint16))
        ref32 = o.matmul_f32(x, w)
        _, mag = o.matmul_f64(x, w)
        y = o.bf16_to_f32(np.fromfile(tmp_path / f"y.{mname}.bin", dtype=np.uint16).reshape(M, n)).astype(np.float64)
        ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(ref32), 2.0 ** -126))) - 7)
        assert np.all(np.abs(y - ref32) <= ulp + 2 * gam * mag), mname


@pytest.mark.gpu
def test_cpp_lm_head_on_gpu(tool, tmp_path):
    """lm_head through the C++ mirror on the tied embedding of a checkpoint file: logits
    within the bound of tests/test_gpu_lm_head.py, top-k equal to the oracle's top-k of
    the same logits."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    V, K, M, k = 3000, 256, 2, 7
    rng = np.random.Generator(np.random.PCG64(31))
    e = o.f32_to_bf16(rng.standard_normal((V, K), dtype=np.float32) * np.float32(0.05))
    name = "model.language_model.embed_tokens.weight"
    path = str(tmp_path / "head.safetensors")
    save_file({name: torch.from_numpy(e.view(np.int16).copy()).view(torch.bfloat16)}, path)
    x = o.synth_x(M, K, 32)
    x.tofile(tmp_path / "x.bin")
    rc, outp, err = run(tool, "head", path, name, M, tmp_path / "x.bin", 30.0, k, tmp_path / "h")
    assert rc == 0, err
    assert json.loads(outp) == {"V": V, "K": K, "M": M, "topk": k}
    lg = np.fromfile(tmp_path / "h.logits.bin", dtype=np.float32).reshape(M, V)
    vals = np.fromfile(tmp_path / "h.values.bin", dtype=np.float32).reshape(M, k)
    idx = np.fromfile(tmp_path / "h.indices.bin", dtype=np.int32).reshape(M, k)
    ref, raw, mag = o.lm_head(x, e, 30.0)
    eps = 2.0 ** -24
    gam = K * eps / (1 - K * eps)
    tol = 2 * gam * mag + 4 * eps * (np.abs(raw) + np.abs(ref)) + 2.0 ** -140
    assert np.all(np.abs(lg.astype(np.float64) - ref) <= tol)
    ov, oi = o.topk(lg, k)
    assert np.array_equal(oi, idx) and np.array_equal(ov.view(np.uint32), vals.view(np.uint32))


def test_cpp_head_rejects_non_bf16_embedding(tool, tmp_path):
    """A head tensor that is not bf16 [V, K] fails before any device call."""
    path = str(tmp_path / "bad.safetensors")
    save_file({"e": torch.zeros((4, 8), dtype=torch.float32)}, path)
    (tmp_path / "x.bin").write_bytes(b"\0" * 16)
    rc, _, err = run(tool, "head", path, "e", 1, tmp_path / "x.bin", 30.0, 1, tmp_path / "h")
    assert rc != 0 and "not bf16" in err
