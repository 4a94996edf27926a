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
import math

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


def _f32_x_not_bf16(M: int, K: int, seed: int) -> np.ndarray:
    """f32 activations whose low 16 bits are nonzero almost everywhere (not bf16-representable),
    spread over several binades, as the engine's f32 residual stream carries them."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, K)) * 2.0 ** rng.integers(-6, 6, (M, K))).astype(np.float32)
    assert np.mean((x.view(np.uint32) & 0xFFFF) != 0) > 0.99
    return x


def test_matmul_magnitudes_match_numpy():
    """The sum |x||w| that sizes every gamma_K bound of the GPU tests, checked from both sides
    against numpy's own float64 contraction of the absolute values: an inflated magnitude
    would make every bound vacuous, a deflated one would reject correct kernels."""
    _, pk, sc = o.synth_weights(96, 1024, 31)
    w = o.dequant(pk, sc)
    w64 = o.bf16_to_f32(w).astype(np.float64)
    xb = o.synth_x(5, 1024, 32)
    y, mag = o.matmul_f64(xb, w)
    x64 = o.bf16_to_f32(xb).astype(np.float64)
    assert np.allclose(mag, np.abs(x64) @ np.abs(w64).T, rtol=1e-13, atol=0)
    assert np.allclose(y, x64 @ w64.T, rtol=1e-12, atol=1e-12)
    xf = _f32_x_not_bf16(5, 1024, 33)
    yf, magf = o.matmul_f32x(xf, w, f64=True)
    xf64 = xf.astype(np.float64)
    assert np.allclose(magf, np.abs(xf64) @ np.abs(w64).T, rtol=1e-13, atol=0)
    # planted mistake: a magnitude built from |sum x w| instead of sum |x w| is smaller and must differ
    assert np.max(np.abs(magf - np.abs(xf64 @ w64.T))) > 1.0


def test_matmul_f32x_pinned_by_numpy_and_torch():
    """The f32-activation contraction (dotPrec fam = null with an f32 lhs, engine.zig:530-533):
    the float64 form equals numpy's float64 x64 @ w64.T (rtol 1e-12), and the fp32 form lies
    within gamma_K * sum |x||w| of it, as does torch's own fp32 matmul of the same operands."""
    _, pk, sc = o.synth_weights(80, 1536, 41)
    w = o.dequant(pk, sc)
    w64 = o.bf16_to_f32(w).astype(np.float64)
    x = _f32_x_not_bf16(6, 1536, 42)
    x64 = x.astype(np.float64)
    y64, mag = o.matmul_f32x(x, w, f64=True)
    ref64 = x64 @ w64.T
    assert np.allclose(y64, ref64, rtol=1e-12, atol=1e-12)
    y32 = o.matmul_f32x(x, w)
    b = _gamma_bound(1536, mag)
    assert np.all(np.abs(y32.astype(np.float64) - ref64) <= b)
    yt = (torch.from_numpy(x) @ torch.from_numpy(o.bf16_to_f32(w)).T).numpy().astype(np.float64)
    assert np.all(np.abs(yt - ref64) <= b)
    # o.linear routes f32 x through the same contraction
    assert np.array_equal(o.linear(x, pk, sc), y32)
    # planted mistake: rounding x to bf16 before the f32 contraction must leave the bound
    xr = o.bf16_to_f32(o.round_bf16(x))
    y_bad = o.matmul_f32x(xr, w).astype(np.float64)
    assert np.max(np.abs(y_bad - ref64) - b) > 0


def test_matmul_f32x_non_finite_activations():
    """IEEE f32 semantics of the f32-activation dot: +-inf in x gives +-inf times w (NaN where
    w is +-0, or where infinities of both signs meet); NaN in x gives NaN."""
    _, pk, sc = o.synth_weights(32, 256, 51)
    w = o.dequant(pk, sc)
    wf = o.bf16_to_f32(w).astype(np.float64)
    x = _f32_x_not_bf16(3, 256, 52)
    x[0, 7] = np.inf
    x[1, 100] = -np.inf
    x[2, 5] = np.nan
    with np.errstate(invalid="ignore", over="ignore"):
        ref = x.astype(np.float64) @ wf.T
    y32 = o.matmul_f32x(x, w)
    y64, _ = o.matmul_f32x(x, w, f64=True)
    for y in (y32.astype(np.float64), y64):
        assert np.array_equal(np.isnan(y), np.isnan(ref))
        fin = ~np.isnan(ref)
        assert np.array_equal(np.isinf(y[fin]), np.isinf(ref[fin]))
        assert np.array_equal(np.sign(y[np.isinf(ref)]), np.sign(ref[np.isinf(ref)]))
    assert np.all(np.isnan(y32[2]))
    assert np.isnan(y32[0][wf[:, 7] == 0]).all() and np.isinf(y32[0][wf[:, 7] != 0]).all()


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


# ------------------------------------------------------------------ MLP front half
# engine.zig:653: dot(xff, gate).gelu().mul(dot(xff, up)); Tensor.gelu = gelu_pytorch_tanh
# (docs/ROADMAP_to_full_forward.md:30).  ZML is not vendored in the reference, so the
# activation is pinned against torch's independent implementation of the same function
# (the HF ACT2FN["gelu_pytorch_tanh"] the reference's MLP gate used as its oracle,
# PLANNING.md:345) and against closed forms.

def test_gelu_tanh_matches_torch_gelu_tanh():
    """Against torch's float64 gelu(approximate="tanh"), which evaluates the literal tanh
    form: equal to its rounding (absolute eps64 |g| from the cancelling 1 + tanh)."""
    rng = np.random.default_rng(5)
    g = np.concatenate([rng.standard_normal(20_000) * 3, rng.uniform(-40, 40, 20_000),
                        [0.0, -0.0, 1e-30, -1e-30, 1e4, -1e4]])
    ref = torch.nn.functional.gelu(torch.from_numpy(g), approximate="tanh").numpy()
    got = o.gelu_tanh(g)
    assert np.all(np.abs(got - ref) <= 4e-16 * np.maximum(1e-300, np.abs(g)) + 1e-300)


def _gelu_tanh_decimal(g: float) -> float:
    """The defining formula 0.5 g (1 + tanh z) with tanh z = (e^2z - 1) / (e^2z + 1), in
    400-digit decimal arithmetic (no float cancellation down to g = -20)."""
    from decimal import Decimal, getcontext
    getcontext().prec = 400
    G = Decimal(g)
    c = (Decimal(2) / Decimal("3.14159265358979323846264338327950288419716939937510582097494")).sqrt()
    z = c * (G + Decimal("0.044715") * G ** 3)
    e2 = (2 * z).exp()
    return float(Decimal("0.5") * G * (1 + (e2 - 1) / (e2 + 1)))


def test_gelu_tanh_negative_tail_vs_high_precision():
    """Where the float tanh form has no correct digit left (g < -5.5) the oracle still
    matches the definition to float64 precision (far below fp32's)."""
    for g in [-1.0, -3.0, -5.5, -6.7, -8.37, -9.7, -12.0, -20.0, 0.3, 2.0, 7.0]:
        ref = _gelu_tanh_decimal(g)
        got = float(o.gelu_tanh(g))
        # exp amplifies the argument's rounding: relative error <= (8 + 16 |z|) eps64
        z = math.sqrt(2 / math.pi) * abs(g + 0.044715 * g ** 3)
        assert abs(got - ref) <= (8 + 16 * z) * 2.0 ** -52 * abs(ref) + 1e-320, (g, got, ref)
    # the float tanh form fails this at g = -8.37 (it returns 0): the check can see it
    t = 0.5 * -8.37 * (1 + math.tanh(math.sqrt(2 / math.pi) * (-8.37 + 0.044715 * -8.37 ** 3)))
    assert abs(t - _gelu_tanh_decimal(-8.37)) > 0.5 * abs(_gelu_tanh_decimal(-8.37))


def test_gelu_tanh_closed_forms():
    # odd part: gelu(x) - gelu(-x) = 0.5x(1+t) + 0.5x(1-t) = x for every x
    x = np.linspace(-12, 12, 2401)
    assert np.max(np.abs(o.gelu_tanh(x) - o.gelu_tanh(-x) - x)) <= 1e-14 * 12
    assert o.gelu_tanh(0.0) == 0.0
    # value at 1 from the definition with the constants written out independently
    z = math.sqrt(2 / math.pi) * (1 + 0.044715)
    assert abs(float(o.gelu_tanh(1.0)) - 0.5 * (1 + math.tanh(z))) <= 1e-16
    # the tanh form, not the erf form (0.841344746...): they differ by ~1.5e-4 at 1
    erf_form = 0.5 * (1 + math.erf(1 / math.sqrt(2)))
    assert abs(float(o.gelu_tanh(1.0)) - erf_form) > 1e-4
    # limits: identity for large g, 0 for very negative g
    assert abs(float(o.gelu_tanh(30.0)) - 30.0) <= 1e-12
    assert abs(float(o.gelu_tanh(-30.0))) <= 1e-30


def _torch_mlp_front(x_u16, pk_g, sc_g, pk_u, sc_u):
    """gelu(gate) * up with torch only: bf16 multiply dequant, float64 matmul, torch gelu."""
    def wt(pk, sc):
        q = torch.from_numpy(o.unpack(pk).astype(np.float32)).to(torch.bfloat16)
        s = torch.from_numpy(sc.view(np.int16)).view(torch.bfloat16)
        return (q * s.repeat_interleave(32, dim=1)).double()
    x = torch.from_numpy(x_u16.view(np.int16)).view(torch.bfloat16).double()
    g = x @ wt(pk_g, sc_g).T
    u = x @ wt(pk_u, sc_u).T
    return torch.nn.functional.gelu(g, approximate="tanh") * u, g, u


def test_gate_up_gelu_matches_torch_composition():
    _, pk_g, sc_g = o.synth_weights(40, 256, 71)
    _, pk_u, sc_u = o.synth_weights(40, 256, 72)
    x = o.synth_x(3, 256, 73)
    h, g, u, mg, mu = o.gate_up_gelu(x, pk_g, sc_g, pk_u, sc_u)
    ref, rg, ru = _torch_mlp_front(x, pk_g, sc_g, pk_u, sc_u)
    assert np.allclose(g, rg.numpy(), rtol=0, atol=1e-12) and np.allclose(u, ru.numpy(), rtol=0, atol=1e-12)
    assert np.all(mg >= np.abs(g)) and np.all(mu >= np.abs(u))
    assert np.max(np.abs(h - ref.numpy())) <= 1e-12 * max(1.0, float(np.max(np.abs(h))))
    # planted mistakes the check must see: gelu(gate * up), gelu(up) * gate
    assert np.max(np.abs(o.gelu_tanh(g * u) - ref.numpy())) > 1e-3
    assert np.max(np.abs(o.gelu_tanh(u) * g - ref.numpy())) > 1e-3


def test_gate_up_gelu_bf16_dots_rounds_both_dots():
    _, pk_g, sc_g = o.synth_weights(24, 128, 81)
    _, pk_u, sc_u = o.synth_weights(24, 128, 82)
    x = o.synth_x(2, 128, 83)
    h, g, u, _, _ = o.gate_up_gelu(x, pk_g, sc_g, pk_u, sc_u, bf16_dots=True)
    gb = torch.from_numpy(g).float().to(torch.bfloat16).double()
    ub = torch.from_numpy(u).float().to(torch.bfloat16).double()
    ref = torch.nn.functional.gelu(gb, approximate="tanh") * ub
    assert np.max(np.abs(h - ref.numpy())) <= 1e-12 * max(1.0, float(np.max(np.abs(h))))
    h_plain = o.gate_up_gelu(x, pk_g, sc_g, pk_u, sc_u)[0]
    assert np.max(np.abs(h - h_plain)) > 0


# ------------------------------------------------------------------ lm_head: softcap and topK
# engine.zig:193-195,765-766; gemma4_g12auto.zig:1532

def test_softcap_matches_torch_and_closed_forms():
    x = np.linspace(-200, 200, 40001)
    ref = (30.0 * torch.tanh(torch.from_numpy(x) / 30.0)).numpy()
    assert np.max(np.abs(o.softcap(x, 30.0) - ref)) <= 1e-13
    assert np.all(np.abs(o.softcap(x, 30.0)) < 30.0)
    assert np.allclose(o.softcap(-x, 30.0), -o.softcap(x, 30.0), rtol=0, atol=0)
    small = np.array([1e-6, -3e-4])
    assert np.allclose(o.softcap(small, 30.0), small, rtol=1e-9)
    assert np.array_equal(o.softcap(x, 0.0), x)


def test_topk_matches_torch_on_distinct_values():
    rng = np.random.default_rng(17)
    lg = rng.standard_normal((3, 5000)).astype(np.float32)
    v, i = o.topk(lg, 7)
    tv, ti = torch.topk(torch.from_numpy(lg), 7, dim=1, sorted=True)
    assert np.array_equal(i, ti.numpy()) and np.array_equal(v, tv.numpy())


def test_topk_tie_and_nan_order():
    neg_nan = np.array([0xFFC00000], dtype=np.uint32).view(np.float32)[0]
    lg = np.array([[1.0, 3.0, 3.0, np.nan, -np.inf, 3.0, np.inf, -0.0, 0.0, neg_nan]], dtype=np.float32)
    v, i = o.topk(lg, 10)
    # every NaN first (ties by index), +inf, equal values ascending, +0 above -0
    assert i[0].tolist() == [3, 9, 6, 1, 2, 5, 0, 8, 7, 4]
    assert np.isnan(v[0, 0]) and np.isnan(v[0, 1]) and v[0, 2] == np.inf
