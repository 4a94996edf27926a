"""Pins the CPU oracle (oracle/w4a16_oracle.c) before it is trusted as the checker.

Each check uses something other than the oracle's own formula: the committed
golden fixtures (built with torch by tests/golden/make_golden.py from the
reference's fixture recipes), hand-derived known answers, an independent
little-endian byte-view packing, torch's bf16 multiply over every q and every
bf16 scale pattern, float64 contractions with a rounding-error bound, and
closed forms.  Planted-mistake checks show each gate can fail.
"""
from __future__ import annotations

import hashlib

import numpy as np
import pytest
import torch

from conftest import load_fixture
from oracle import w4a16_oracle as o


def _bf16_np(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


# ------------------------------------------------------------------ W1 gate
# zml_runner/gemma4_w4gate.zig:50-175 on the fixture of scripts/57_w4_unpack_fixture.py:33-44

def test_w1_fixture_pack_unpack_dequant():
    f = load_fixture("w4_unpack.safetensors")
    assert np.array_equal(o.pack(f["q_expected"]), f["packed"])
    assert np.array_equal(o.unpack(f["packed"]), f["q_expected"])
    assert np.array_equal(o.dequant(f["packed"], f["scales"]), f["deq_expected"])  # u16 bit-exact


def test_w1_corrupt_nibble_diverges_exactly_once():
    f = load_fixture("w4_unpack.safetensors")
    q_bad = o.unpack(f["packed_corrupt"])
    diff = np.argwhere(q_bad != f["q_expected"])
    assert diff.tolist() == [[0, 1]], diff  # nibble 1 of word 0, row 0 (57:43-44)


def test_known_answer_words():
    # row 0 = [-8..7, 7..-8] -> nibbles [0..15, 15..0]: hand-derived words
    row0 = np.array(list(range(-8, 8)) + list(range(7, -9, -1)), dtype=np.int8)[None]
    words = [int(w) & 0xFFFFFFFF for w in o.pack(row0)[0]]
    assert words == [0x76543210, 0xFEDCBA98, 0x89ABCDEF, 0x01234567]
    assert o.pack(row0)[0, 1] < 0  # bit 31 set: negative int32 (the sign trap of 57:36-37)


def test_pack_matches_little_endian_byte_view():
    rng = np.random.default_rng(7)
    q = rng.integers(-8, 8, size=(37, 96), dtype=np.int8)
    n = (q.astype(np.int16) + 8).astype(np.uint8)
    bytes_ = (n[:, 0::2] | (n[:, 1::2] << 4)).astype(np.uint8)  # two nibbles per byte, low first
    words = np.ascontiguousarray(bytes_).view("<i4")            # four bytes per word, little endian
    assert np.array_equal(o.pack(q), words)


def test_unpack_every_nibble_at_every_position():
    pk = np.zeros((16 * 8, 1), dtype=np.uint32)
    for v in range(16):
        for j in range(8):
            # all other nibbles 8 (q = 0), nibble j = v
            word = 0
            for jj in range(8):
                word |= (v if jj == j else 8) << (4 * jj)
            pk[v * 8 + j, 0] = word
    q = o.unpack(pk.view(np.int32))
    for v in range(16):
        for j in range(8):
            expect = np.zeros(8, dtype=np.int8)
            expect[j] = v - 8
            assert np.array_equal(q[v * 8 + j], expect)


def test_logical_shift_matters():
    """Planted mistake: an arithmetic shift (sign-propagating) breaks nibbles of
    negative words -- the reason w4.zig:38-39 uses shiftRightLogical."""
    f = load_fixture("w4_unpack.safetensors")
    pk = f["packed"]
    arith = np.stack([((pk >> (4 * j)) & 0xF) for j in range(8)], -1)  # numpy >> on int32 is arithmetic
    # masking with 0xF hides the sign fill, so emulate the reference's hazard: no mask on the top nibble
    top_arith = (pk >> 28) - 8
    top_logical = ((pk.view(np.uint32) >> 28).astype(np.int32)) - 8
    assert not np.array_equal(top_arith, top_logical)
    assert np.array_equal(arith.reshape(pk.shape[0], -1) - 8, o.unpack(pk))


# ------------------------------------------------------------------ dequant

def _all_scales_case():
    s = torch.arange(65536, dtype=torch.int32).to(torch.int16).view(torch.bfloat16).reshape(-1, 1)
    q = torch.arange(-8, 8, dtype=torch.int8).repeat(2).reshape(1, 32).expand(65536, 32).contiguous()
    return q, s


def test_dequant_exhaustive_vs_torch_bf16_multiply():
    """Every q in [-8, 7] times every bf16 scale pattern (1 048 576 cases) against
    torch's bf16 x bf16 -> bf16 (the operation of scripts/57_w4_unpack_fixture.py:41,85).
    NaN results are compared by position (libraries disagree on NaN bits)."""
    q, s = _all_scales_case()
    ref = _bf16_np(q.to(torch.bfloat16) * s)
    got = o.dequant(o.pack(q.numpy()), _bf16_np(s))
    nan_ref, nan_got = o.is_nan_bf16(ref), o.is_nan_bf16(got)
    assert np.array_equal(nan_ref, nan_got)
    assert np.array_equal(got[~nan_ref], ref[~nan_ref])
    # the case is not vacuous: about 37 % of finite products need rounding
    exact = q.numpy().astype(np.float64) * o.bf16_to_f32(_bf16_np(s)).astype(np.float64)
    fin = np.isfinite(exact)
    frac = np.mean(o.bf16_to_f32(got)[fin] != exact[fin])
    assert 0.30 < frac < 0.45, frac


def test_dequant_truncation_would_fail():
    """Planted mistake: truncating q*s to bf16 instead of rounding to nearest even."""
    q, s = _all_scales_case()
    ref = _bf16_np(q.to(torch.bfloat16) * s)
    prod = (q.to(torch.float32) * s.to(torch.float32)).numpy()
    trunc = (prod.view(np.uint32) >> 16).astype(np.uint16)
    ok = ~o.is_nan_bf16(ref)
    assert np.count_nonzero(trunc[ok] != ref[ok]) > 100_000


def test_dequant_special_values():
    for sbits in (0x0000, 0x8000):                 # +0 / -0 scale
        for qv in range(-8, 8):
            r = o.dequant_one(qv, sbits)
            assert r & 0x7FFF == 0                  # a signed zero
    # powers of two and q = -8 are exact: bits shift only in the exponent
    for qv in (-8, -4, -2, -1, 1, 2, 4):
        s = 0x3F80  # 1.0
        assert o.bf16_to_f32(np.uint16(o.dequant_one(qv, s))) == float(qv)
    # the reference fixture's second scale, 0.033203125 = 0x3D08, times 7 rounds
    assert o.dequant_one(7, 0x3D08) == _bf16_np(torch.tensor([7.0]).to(torch.bfloat16) *
                                                 torch.tensor([0.033203125], dtype=torch.bfloat16))[0]


def test_dequant_golden_small_cases():
    f = load_fixture("w4_linear_small.safetensors")
    i = 0
    while f"c{i}.packed" in f:
        K = f[f"c{i}.packed"].shape[1] * 8
        group = K // f[f"c{i}.scales"].shape[1]
        assert np.array_equal(o.dequant(f[f"c{i}.packed"], f[f"c{i}.scales"], group), f[f"c{i}.deq_expected"])
        i += 1
    assert i >= 8


# ------------------------------------------------------------------ linear

def _gamma_bound(K: int, mag: np.ndarray) -> np.ndarray:
    u = 2.0 ** -24
    return (K * u / (1 - K * u)) * mag


def test_linear_golden_small_cases_vs_torch():
    f = load_fixture("w4_linear_small.safetensors")
    i = 0
    while f"c{i}.packed" in f:
        pk, sc, x = f[f"c{i}.packed"], f[f"c{i}.scales"], f[f"c{i}.x"]
        K = pk.shape[1] * 8
        y = o.linear(x, pk, sc, K // sc.shape[1])
        y64, mag = o.matmul_f64(x, o.dequant(pk, sc, K // sc.shape[1]))
        ref = f[f"c{i}.out_expected"]
        b = _gamma_bound(K, mag)
        assert np.all(np.abs(y - y64) <= b + 1e-30)
        assert np.all(np.abs(ref - y64) <= b + 1e-30)   # torch's fp32 matmul lies in the same bound
        i += 1


def test_linear_f64_error_bound_random():
    rng = np.random.default_rng(3)
    q, pk, sc = o.synth_weights(64, 1536, 5)
    x = o.synth_x(4, 1536, 99)
    w = o.dequant(pk, sc)
    y = o.matmul_f32(x, w)
    y64, mag = o.matmul_f64(x, w)
    assert np.all(np.abs(y - y64) <= _gamma_bound(1536, mag))
    # and the f64 contraction agrees with numpy's own float64 matmul
    y64np = o.bf16_to_f32(x).astype(np.float64) @ o.bf16_to_f32(w).astype(np.float64).T
    assert np.allclose(y64, y64np, rtol=1e-12, atol=1e-12)
    del rng, q


def test_linear_one_hot_selects_a_column():
    q, pk, sc = o.synth_weights(48, 256, 21)
    w = o.dequant(pk, sc)
    x = np.zeros((256, 256), dtype=np.uint16)
    x[np.arange(256), np.arange(256)] = 0x3F80  # 1.0
    y = o.linear(x, pk, sc)
    assert np.array_equal(y, o.bf16_to_f32(w).T)


def test_linear_zero_scale_and_constant_q():
    N, K = 8, 128
    x = o.synth_x(3, K, 5)
    sc0 = np.zeros((N, K // 32), dtype=np.uint16)
    rng = np.random.default_rng(1)
    pk = o.pack(rng.integers(-8, 8, size=(N, K), dtype=np.int8))
    assert np.array_equal(o.linear(x, pk, sc0), np.zeros((3, N), np.float32))
    # constant q = 3 everywhere: y[m, n] = sum_g bf16(3 * s_g) * sum_{k in g} x_k
    q3 = np.full((N, K), 3, dtype=np.int8)
    _, _, sc = o.synth_weights(N, K, 8)
    y = o.linear(x, o.pack(q3), sc)
    wg = np.array([[float(torch.tensor(3.0, dtype=torch.bfloat16) * torch.tensor(v, dtype=torch.float32).to(torch.bfloat16))
                    for v in o.bf16_to_f32(row)] for row in sc])          # [N, G] via torch bf16 multiply
    xs = o.bf16_to_f32(x).astype(np.float64).reshape(3, K // 32, 32).sum(-1)   # [M, G]
    closed = xs @ wg.T
    _, mag = o.matmul_f64(x, o.dequant(o.pack(q3), sc))
    assert np.all(np.abs(y - closed) <= _gamma_bound(K, mag) * 2 + 1e-30)


# ------------------------------------------------------------------ W3 gate (synthetic weights)
# zml_runner/gemma4_w4gate.zig:259-363; x from scripts/58_w4_gemm_oracle.py:23-24

def test_w3_synth_fixture(manifest):
    f = load_fixture("w4_gemm_synth.safetensors")
    meta = manifest["w4_gemm_synth"]["weights"]
    q, pk, sc = o.synth_weights(meta["N"], meta["K"], meta["seed"])
    assert hashlib.sha256(pk.tobytes()).hexdigest() == meta["packed_sha256"]
    assert hashlib.sha256(sc.tobytes()).hexdigest() == meta["scale_sha256"]
    x = f["x"].reshape(1, -1)
    # the activation recipe of 58:23-24 reproduced with torch
    torch.manual_seed(1337)
    assert np.array_equal(x, _bf16_np(torch.randn(1, 1, 1536).to(torch.bfloat16)).reshape(1, -1))
    y = o.linear(x, pk, sc)[0]
    exp = f["out_expected"].reshape(-1)
    assert np.max(np.abs(y - exp)) <= 1e-4
    assert np.mean(np.abs(y - exp)) <= 1e-6
    fp = np.array(manifest["w4_gemm_synth"]["fixed_points_out_0_0_0_8"], dtype=np.float32)
    assert np.max(np.abs(y[:8] - fp)) <= 1e-4


def test_w3_gate_rejects_factored_scale():
    """Planted mistake: applying the scale after the group sum (skipping the
    bf16 rounding of each q*s) must fail the reference's W3 tolerance."""
    f = load_fixture("w4_gemm_synth.safetensors")
    q, pk, sc = o.synth_weights(2048, 1536, 1001)
    x = o.bf16_to_f32(f["x"].reshape(1, -1)).astype(np.float64)
    s = o.bf16_to_f32(sc).astype(np.float64)
    fact = (x.reshape(1, 48, 32)[:, None] * q.reshape(2048, 48, 32)).sum(-1)   # [1, N, G]
    y_fact = (fact * s[None]).sum(-1)[0]
    exp = f["out_expected"].reshape(-1)
    assert np.max(np.abs(y_fact - exp)) > 1e-4 or np.mean(np.abs(y_fact - exp)) > 1e-6


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(100_000) * 10.0 ** rng.integers(-30, 30, 100_000)).astype(np.float32)
    v[:6] = [0.0, -0.0, np.inf, -np.inf, 3.4e38, 1e-40]
    got = o.round_bf16(v)
    ref = _bf16_np(torch.from_numpy(v).to(torch.bfloat16))
    assert np.array_equal(got, ref)
