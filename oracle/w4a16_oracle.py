"""NumPy front end of the C oracle (oracle/w4a16_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by bench.py's ``cpu_baseline`` leg, always as the checker.  The product
path (``w4a16`` package / libw4a16.so) never imports it.

bf16 values travel as ``uint16`` bit patterns, as the reference's W1/W2 gates
compare them (zml_runner/gemma4_w4gate.zig:98-111).

Reference functions restated (file:line in TheCause/gemma4-zml-probe):
  pack     compressed-tensors pack_to_int32 call, scripts/57_w4_unpack_fixture.py:39
  unpack   unpackW4, zml_runner/w4.zig:33-45
  dequant  dequantW4, zml_runner/w4.zig:47-54; dequant_manual,
           scripts/63_u_dequant_export.py:83-89
  linear   G3.forward, zml_runner/gemma4_w4gate.zig:288-292;
           scripts/58_w4_gemm_oracle.py:29 (x.f32 @ w.f32.T)
  gelu_tanh     ZML Tensor.gelu = gelu_pytorch_tanh, docs/ROADMAP_to_full_forward.md:30
                (ZML itself is a dependency that is not vendored in the reference)
  gate_up_gelu  the MLP front half, zml_runner/engine.zig:653:
                dot(xff, gate).gelu().mul(dot(xff, up)), gating gelu(gate) * up
                (PLANNING.md:345), dots through dotPrec (engine.zig:530-533)
  softcap       softcapPrec, zml_runner/engine.zig:193-195: raw.scale(1/cap).tanh().scale(cap)
  topk          logits.topK(.voc, K), zml_runner/gemma4_g12auto.zig:1532: descending; ties in
                ascending index order and every NaN above +inf (totalOrder of +NaN), which ZML leaves to
                its sort (parity of tie order unpinned: the reference's own topK test uses
                distinct values, gemma4_bbatch.zig:766-824)
  lm_head       engine.zig:765-766: dotPrec(head, last_hidden, embed_tokens) then softcap
Pins of gelu_tanh / gate_up_gelu (tests/test_oracle.py): gelu_tanh against torch's independent
gelu(approximate="tanh") in float64, against the defining tanh formula in 400-digit
decimal arithmetic on the negative tail (where float tanh forms cancel), the odd-part
identity gelu(x) - gelu(-x) = x, the limits and the closed-form values at 0 and 1;
gate_up_gelu against a torch-only composition (bf16 dequant, float64 matmul, torch
gelu) with planted mistakes (gelu(gate * up), gelu(up) * gate) that the check sees.
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle_w4a16.so")
_lib = None

GROUP = 32


def build() -> str:
    """Compile the C oracle in place (make -C oracle)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        I64 = ctypes.c_int64
        L.oracle_pack.argtypes = [P, P, I64, I64]
        L.oracle_pack.restype = ctypes.c_int
        L.oracle_unpack.argtypes = [P, P, I64, I64]
        L.oracle_unpack.restype = ctypes.c_int
        L.oracle_dequant.argtypes = [P, P, P, I64, I64, I64]
        L.oracle_dequant.restype = ctypes.c_int
        L.oracle_dequant_one.argtypes = [ctypes.c_int32, ctypes.c_uint16]
        L.oracle_dequant_one.restype = ctypes.c_uint16
        L.oracle_matmul_bf16_f32.argtypes = [P, P, P, I64, I64, I64]
        L.oracle_matmul_bf16_f32.restype = None
        L.oracle_matmul_bf16_f64.argtypes = [P, P, P, P, I64, I64, I64]
        L.oracle_matmul_bf16_f64.restype = None
        L.oracle_matmul_f32x_f32.argtypes = [P, P, P, I64, I64, I64]
        L.oracle_matmul_f32x_f32.restype = None
        L.oracle_matmul_f32x_f64.argtypes = [P, P, P, P, I64, I64, I64]
        L.oracle_matmul_f32x_f64.restype = None
        L.oracle_round_bf16.argtypes = [P, P, I64]
        L.oracle_round_bf16.restype = None
        L.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def pack(q: np.ndarray) -> np.ndarray:
    """int8 q [N, K] in [-8, 7] -> int32 [N, K/8] (nibble j of word w = column 8w+j, q+8)."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    N, K = q.shape
    pk = np.empty((N, K // 8), dtype=np.int32)
    if lib().oracle_pack(_p(q), _p(pk), N, K) != 0:
        raise ValueError("pack: K % 8 != 0 or value outside [-8, 7]")
    return pk


def unpack(pk: np.ndarray, K: int | None = None) -> np.ndarray:
    """int32 [N, K/8] -> int8 q [N, K] in [-8, 7]."""
    pk = np.ascontiguousarray(pk, dtype=np.int32)
    N, W = pk.shape
    K = 8 * W if K is None else K
    q = np.empty((N, K), dtype=np.int8)
    if lib().oracle_unpack(_p(pk), _p(q), N, K) != 0:
        raise ValueError("unpack: bad K")
    return q


def dequant(pk: np.ndarray, sc: np.ndarray, group: int = GROUP) -> np.ndarray:
    """int32 pk [N, K/8] + uint16 (bf16) sc [N, K/group] -> uint16 (bf16) w [N, K]."""
    pk = np.ascontiguousarray(pk, dtype=np.int32)
    sc = np.ascontiguousarray(sc, dtype=np.uint16)
    N, W = pk.shape
    K = 8 * W
    assert sc.shape == (N, K // group), (sc.shape, N, K, group)
    w = np.empty((N, K), dtype=np.uint16)
    if lib().oracle_dequant(_p(pk), _p(sc), _p(w), N, K, group) != 0:
        raise ValueError("dequant: bad shape / group")
    return w


def dequant_one(q: int, s_bits: int) -> int:
    return int(lib().oracle_dequant_one(int(q), int(s_bits)))


def matmul_f32(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """x bf16 [M, K] (uint16), w bf16 [N, K] (uint16) -> f32 [M, N], fp32 accumulate."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    M, K = x.shape
    N, K2 = w.shape
    assert K == K2
    y = np.empty((M, N), dtype=np.float32)
    lib().oracle_matmul_bf16_f32(_p(x), _p(w), _p(y), M, N, K)
    return y


def matmul_f64(x: np.ndarray, w: np.ndarray):
    """float64-accumulate contraction and per-output sum |x||w| (error-bound magnitude)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    M, K = x.shape
    N, _ = w.shape
    y = np.empty((M, N), dtype=np.float64)
    mag = np.empty((M, N), dtype=np.float64)
    lib().oracle_matmul_bf16_f64(_p(x), _p(w), _p(y), _p(mag), M, N, K)
    return y, mag


def matmul_f32x(x: np.ndarray, w: np.ndarray, f64: bool = False):
    """f32 activations x [M, K] . bf16 w [N, K]^T; fp32 accumulate, or float64 (+ sum |x||w|)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.uint16)
    M, K = x.shape
    N, _ = w.shape
    if not f64:
        y = np.empty((M, N), dtype=np.float32)
        lib().oracle_matmul_f32x_f32(_p(x), _p(w), _p(y), M, N, K)
        return y
    y = np.empty((M, N), dtype=np.float64)
    mag = np.empty((M, N), dtype=np.float64)
    lib().oracle_matmul_f32x_f64(_p(x), _p(w), _p(y), _p(mag), M, N, K)
    return y, mag


def linear(x: np.ndarray, pk: np.ndarray, sc: np.ndarray, group: int = GROUP) -> np.ndarray:
    """The reference flow: dequant (bf16, bit-exact) then x.f32 @ w.f32^T -> f32 [M, N].
    x is bf16 (uint16) or float32."""
    w = dequant(pk, sc, group)
    if np.asarray(x).dtype == np.float32:
        return matmul_f32x(x, w)
    return matmul_f32(x, w)


SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)


def gelu_tanh(g) -> np.ndarray:
    """0.5 g (1 + tanh(z)), z = sqrt(2/pi) (g + 0.044715 g^3), in float64, evaluated as
    g / (1 + exp(-2 z)) (the same function: 0.5 (1 + tanh z) = 1 / (1 + e^(-2z))).  The
    literal tanh form cancels once 1 + tanh(z) < ~1e-16 (g below about -5.5) and loses
    every digit of the negative tail; this form keeps full relative precision there."""
    g = np.asarray(g, dtype=np.float64)
    z = SQRT_2_OVER_PI * (g + 0.044715 * g ** 3)
    with np.errstate(over="ignore"):
        return g / (1.0 + np.exp(-2.0 * z))


def gate_up_gelu(x: np.ndarray, pk_g: np.ndarray, sc_g: np.ndarray, pk_u: np.ndarray, sc_u: np.ndarray,
                 group: int = GROUP, bf16_dots: bool = False):
    """h[M, F] = gelu(x . Wg^T) * (x . Wu^T) with float64 dots (the exact values the fp32
    kernels approximate) and the error-bound magnitudes sum |x||w| of each dot.
    bf16_dots: g and u rounded to bf16 first (dotPrec with fam = bf16, engine.zig:531).
    Returns (h64, g64, u64, mag_g, mag_u)."""
    wg, wu = dequant(pk_g, sc_g, group), dequant(pk_u, sc_u, group)
    if np.asarray(x).dtype == np.float32:
        g, mg = matmul_f32x(x, wg, f64=True)
        u, mu = matmul_f32x(x, wu, f64=True)
    else:
        g, mg = matmul_f64(x, wg)
        u, mu = matmul_f64(x, wu)
    if bf16_dots:
        gr = bf16_to_f32(round_bf16(g.astype(np.float32))).astype(np.float64)
        ur = bf16_to_f32(round_bf16(u.astype(np.float32))).astype(np.float64)
        return gelu_tanh(gr) * ur, g, u, mg, mu
    return gelu_tanh(g) * u, g, u, mg, mu


def softcap(raw, cap: float) -> np.ndarray:
    """cap * tanh(raw / cap) in float64 (cap = 0: raw unchanged)."""
    raw = np.asarray(raw, dtype=np.float64)
    return cap * np.tanh(raw / cap) if cap > 0 else raw


def total_order_key(v: np.ndarray) -> np.ndarray:
    """f32 values -> uint32 keys in IEEE totalOrder (-inf < ... < -0 < +0 < ... < +inf < NaN),
    every NaN taken as the canonical quiet NaN 0x7FC00000."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    u = np.where(np.isnan(v), np.uint32(0x7FC00000), v.view(np.uint32)).astype(np.uint32)
    return np.where(u & 0x80000000, ~u, u | 0x80000000).astype(np.uint32)


def topk(logits: np.ndarray, k: int):
    """Per row: the k largest f32 values in totalOrder, descending, ties by ascending index.
    Returns (values f32 [M, k], indices int32 [M, k])."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    M, V = lg.shape
    keys = total_order_key(lg)
    idx = np.empty((M, k), dtype=np.int32)
    for m in range(M):
        order = np.lexsort((np.arange(V), -keys[m].astype(np.int64)))
        idx[m] = order[:k]
    return np.take_along_axis(lg, idx.astype(np.int64), axis=1), idx


def lm_head(x: np.ndarray, embed: np.ndarray, cap: float):
    """float64 logits softcap(x . embed^T) and the error-bound magnitudes sum |x||e|;
    x bf16 (uint16) or float32 [M, K], embed bf16 (uint16) [V, K]."""
    if np.asarray(x).dtype == np.float32:
        raw, mag = matmul_f32x(x, embed, f64=True)
    else:
        raw, mag = matmul_f64(x, embed)
    return softcap(raw, cap), raw, mag


def is_nan_bf16(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16) & 0x7FFF) > 0x7F80


def round_bf16(y: np.ndarray) -> np.ndarray:
    """f32 -> bf16 (uint16) with round-to-nearest-even; NaN -> 0x7FC0."""
    y = np.ascontiguousarray(y, dtype=np.float32)
    out = np.empty(y.shape, dtype=np.uint16)
    lib().oracle_round_bf16(_p(y), _p(out), y.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 (exact widening)."""
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(f: np.ndarray) -> np.ndarray:
    return round_bf16(np.asarray(f, dtype=np.float32))


# --------------------------------------------------------------------------
# Synthetic inputs of the benchmark configurations.
# q ~ U{-8..7}; scale = bf16(|N(0,1)| * 0.02) [N, K/32]; x = bf16(N(0,1)) [M, K].
# Seeds: weights 1000 + config index, activations 2000 + M.

def synth_weights(N: int, K: int, seed: int, group: int = GROUP):
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    s = (np.abs(rng.standard_normal((N, K // group), dtype=np.float32)) * np.float32(0.02))
    return q, pack(q), f32_to_bf16(s)


def synth_x(M: int, K: int, seed: int | None = None) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(2000 + M if seed is None else seed))
    return f32_to_bf16(rng.standard_normal((M, K), dtype=np.float32))
