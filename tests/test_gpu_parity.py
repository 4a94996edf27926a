"""GPU parity: libw4a16.so (HIP, gfx950) against the CPU oracle on identical inputs.

Mirrors the reference's gates (TheCause/gemma4-zml-probe):
  W1  zml_runner/gemma4_w4gate.zig:50-175   unpack/dequant bit-exact + corrupt-nibble counter-test
  W2  zml_runner/gemma4_w4gate.zig:179-255  dequant of the 5 E2B shape families, u16 bit-exact
  U1b zml_runner/gemma4_g12gate.zig:134-170 the same on three 12B shapes
  W3  zml_runner/gemma4_w4gate.zig:259-363  linear, max_abs <= 1e-4, mean_abs <= 1e-6, 8 fixed points
The real checkpoint tensors are not available, so the W2/U1b shapes carry the
synthetic benchmark weights (q ~ U{-8..7}, scale = bf16(|N(0,1)| * 0.02)).

Stated tolerances for the linear (fp32 accumulate, only the summation order differs):
  y f32:  |y - y_f64| <= 2 * gamma_K * sum_k |x_k w_k| elementwise,
          max_abs(y - y_oracle32) <= 1e-4 * sqrt(K / 1536) * max(1, rms(y) / 4),
          rel_L2(y, y_oracle32) <= 1e-5
  y bf16: |y - RNE(y_oracle32)| <= 1 bf16 ulp for >= 99.9 % of elements, and for every
          element |y - y_oracle32| <= ulp_bf16(y_oracle32) + 2 * gamma_K * sum_k |x_k w_k|
          (one final rounding plus the fp32 bound; near-cancelling outputs are bounded
          absolutely, not in ulps of their tiny value), rel_L2 <= 4e-3
  argmax of a random bf16 head [4096, N] (seed 3000) unchanged on rows whose
  top1 - top2 margin exceeds 1e-3 * |top1|.
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

from conftest import load_fixture

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

import w4a16  # noqa: E402
from oracle import w4a16_oracle as o  # noqa: E402


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    w4a16.lib()


def say(msg: str) -> None:
    print(f"[gpu-parity] {msg}", flush=True)
    sys.stdout.flush()


def dev_u16(a: np.ndarray, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(dtype).cuda()


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host_u16(t) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def gpu_linear(x_np, pk, sc, out="f32", group=32, x_f32=False):
    x = dev(x_np) if x_f32 else dev_u16(x_np)
    y = w4a16.linear(x, dev(pk), dev_u16(sc), group=group,
                     out_dtype=torch.float32 if out == "f32" else torch.bfloat16)
    torch.cuda.synchronize()
    return y.cpu().numpy() if out == "f32" else host_u16(y)


def check_f32(y, x, w, K, y_ref32=None, x_f32=False):
    """The stated f32 tolerance (module docstring)."""
    if x_f32:
        y64, mag = o.matmul_f32x(x, w, f64=True)
        ref32 = o.matmul_f32x(x, w) if y_ref32 is None else y_ref32
    else:
        y64, mag = o.matmul_f64(x, w)
        ref32 = o.matmul_f32(x, w) if y_ref32 is None else y_ref32
    u = 2.0 ** -24
    gam = K * u / (1 - K * u)
    err64 = np.abs(y.astype(np.float64) - y64)
    assert np.all(err64 <= 2 * gam * mag + 1e-30), float(np.max(err64 - 2 * gam * mag))
    rms = float(np.sqrt(np.mean(ref32.astype(np.float64) ** 2))) if ref32.size else 0.0
    tol_abs = 1e-4 * math.sqrt(K / 1536) * max(1.0, rms / 4)
    assert float(np.max(np.abs(y - ref32))) <= tol_abs
    den = float(np.linalg.norm(ref32.astype(np.float64)))
    if den > 0:
        assert float(np.linalg.norm((y - ref32).astype(np.float64))) / den <= 1e-5
    return y64


def check_bf16(yb, ref32, mag, K):
    rb = o.round_bf16(ref32)
    a = o.bf16_to_f32(yb).astype(np.float64)
    b = o.bf16_to_f32(rb).astype(np.float64)
    r = ref32.astype(np.float64)

    def ulp(v):
        e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
        return 2.0 ** (e - 7)

    assert np.mean(np.abs(a - b) <= ulp(b)) >= 0.999
    u = 2.0 ** -24
    gam = K * u / (1 - K * u)
    excess = np.abs(a - r) - (ulp(r) + 2 * gam * mag)
    assert np.all(excess <= 0), float(np.max(excess))
    den = np.linalg.norm(r)
    if den > 0:
        assert np.linalg.norm(a - r) / den <= 4e-3


def check_head_argmax(y, y_ref, N, seed=3000, V=4096):
    rng = np.random.Generator(np.random.PCG64(seed))
    head = o.bf16_to_f32(o.f32_to_bf16(rng.standard_normal((V, N), dtype=np.float32))).astype(np.float64)
    la = y.astype(np.float64) @ head.T
    lb = y_ref.astype(np.float64) @ head.T
    top = np.sort(lb, axis=1)
    margin = top[:, -1] - top[:, -2]
    decisive = margin > 1e-3 * np.abs(top[:, -1])
    assert np.array_equal(np.argmax(la, 1)[decisive], np.argmax(lb, 1)[decisive])


# ------------------------------------------------------------------ W1

def test_w1_unpack_dequant_fixture():
    say("W1 fixture")
    f = load_fixture("w4_unpack.safetensors")
    q = w4a16.unpackW4(dev(f["packed"])).cpu().numpy()
    assert np.array_equal(q, f["q_expected"])
    d = host_u16(w4a16.dequantW4(dev(f["packed"]), dev_u16(f["scales"])))
    assert np.array_equal(d, f["deq_expected"])
    qc = w4a16.unpackW4(dev(f["packed_corrupt"])).cpu().numpy()
    assert np.argwhere(qc != f["q_expected"]).tolist() == [[0, 1]]


def test_dequant_exhaustive_all_scale_patterns():
    say("dequant: 16 q x 65536 scale patterns")
    q = np.tile(np.arange(-8, 8, dtype=np.int8), 2)[None].repeat(65536, 0)
    sc = np.arange(65536, dtype=np.uint32).astype(np.uint16)[:, None].copy()
    pk = o.pack(q)
    got = host_u16(w4a16.dequantW4(dev(pk), dev_u16(sc)))
    assert np.array_equal(got, o.dequant(pk, sc))  # canonical NaN on both sides: all bits equal
    qg = w4a16.unpackW4(dev(pk)).cpu().numpy()
    assert np.array_equal(qg, q)


W2_SHAPES = {  # scripts/57_w4_unpack_fixture.py:75-81 (E2B) and 63:231-236 (12B, U1b)
    "deq_q0": (2048, 1536), "deq_q4": (4096, 1536), "deq_dn20": (1536, 12288),
    "deq_plp0": (1536, 256), "deq_plmp": (8960, 1536),
    "u1b_q0": (4096, 3840), "u1b_q5": (8192, 3840), "u1b_dn0": (3840, 15360),
}


@pytest.mark.parametrize("name", list(W2_SHAPES))
def test_w2_u1b_dequant_shape_families(name):
    N, K = W2_SHAPES[name]
    say(f"W2/U1b dequant {name} N={N} K={K}")
    _, pk, sc = o.synth_weights(N, K, 4000 + N % 97)
    got = host_u16(w4a16.dequantW4(dev(pk), dev_u16(sc)))
    assert np.array_equal(got, o.dequant(pk, sc))
    assert np.array_equal(w4a16.unpackW4(dev(pk)).cpu().numpy(), o.unpack(pk))


@pytest.mark.parametrize("N,K,group", [
    (3, 24 * 4, 32), (5, 96, 96), (7, 256, 128), (333, 96, 32),     # word counts not a multiple of 256
    (1024, 4096, 64), (2048, 3072, 96), (2048, 2048, 32),          # one word per thread
    (4096, 8192, 64), (4096, 8448, 96), (4099, 8192, 32)])         # four words per thread (>= 1 Mi words)
def test_dequant_unpack_launch_forms_and_groups(N, K, group):
    """Both launch forms of the flat dequant/unpack (one or four words per thread),
    the scale index as a shift (group / 8 a power of two) and as a division, and word
    counts that leave partial workgroups: bit-exact against the oracle."""
    say(f"dequant/unpack N={N} K={K} group={group}")
    _, pk, sc = o.synth_weights(N, K, 4100 + N % 89, group=group)
    ref = o.dequant(pk, sc, group)
    got = host_u16(w4a16.dequantW4(dev(pk), dev_u16(sc), group=group))
    assert np.array_equal(got, ref)
    assert np.array_equal(w4a16.unpackW4(dev(pk)).cpu().numpy(), o.unpack(pk))
    # caller-supplied outputs (filled with a pattern first): written in place
    wbuf = torch.full((N, K), -1.0, dtype=torch.bfloat16, device="cuda")
    assert w4a16.dequantW4(dev(pk), dev_u16(sc), group=group, out=wbuf) is wbuf
    assert np.array_equal(host_u16(wbuf), ref)
    qbuf = torch.full((N, K), 99, dtype=torch.int8, device="cuda")
    assert w4a16.unpackW4(dev(pk), out=qbuf) is qbuf
    assert np.array_equal(qbuf.cpu().numpy(), o.unpack(pk))
    with pytest.raises(w4a16.W4A16Error):
        w4a16.unpackW4(dev(pk), out=qbuf[:, :8])


# ------------------------------------------------------------------ linear: exactness probes

def test_linear_one_hot_reproduces_dequant_exactly():
    """One-hot rows of x select single weights: y must equal the bf16 weight
    exactly.  Over every bf16 scale pattern in the fused kernels' exact range
    this pins the in-register dequant of the M > 4 kernels (32 rows of x: the
    skinny kernel's f16 form) to dequantW4's rounding.  Stated range:
    2^-126 <= |s| < 2^117.  Subnormal scales may be flushed (weights of magnitude
    <= 8 * 2^-126 come out as 0); from 2^117 the intermediate (1024 + n) * s
    overflows fp32.  Checkpoint scales are max_abs / 7.5 of bf16 weights, around
    2^-20..2^-3."""
    say("linear one-hot over all finite scale patterns")
    q = np.tile(np.arange(-8, 8, dtype=np.int8), 2)[None].repeat(65536, 0)
    sc = np.arange(65536, dtype=np.uint32).astype(np.uint16)[:, None].copy()
    expo = (sc[:, 0] >> 7) & 0xFF                     # biased exponent
    in_range = (expo >= 1) & (expo < 127 + 117)
    subnormal = (expo == 0) & ((sc[:, 0] & 0x7F) != 0)
    assert subnormal.sum() == 254
    sc[~(in_range | subnormal), 0] = 0                # drop huge / non-finite scales
    pk = o.pack(q)
    x = np.zeros((32, 32), dtype=np.uint16)
    x[np.arange(32), np.arange(32)] = 0x3F80
    y = gpu_linear(x, pk, sc, "f32")               # [32, 65536]
    w = o.bf16_to_f32(o.dequant(pk, sc)).T         # [32, 65536]
    ok = ~subnormal
    bad = np.argwhere(y[:, ok] != w[:, ok])
    assert bad.size == 0, (bad[:5].tolist(), [hex(int(v)) for v in sc[ok][bad[:5, 1], 0]])
    assert np.all(np.abs(y[:, subnormal] - w[:, subnormal]) <= 8 * 2.0 ** -126)


def test_decode_gemv_one_hot_reproduces_dequant_exactly():
    """The decode GEMV (M <= 4, K % 256 == 0) expands weights with v_fma_mix_f32 from f16
    nibble pairs, not with the v_dot2 form above.  One-hot rows of x over the first 16
    columns (all 16 q values, all 8 nibble positions of a word) of 65536 rows, one bf16
    scale pattern per row: y must equal the bf16 weight exactly for every scale with
    2^-122 <= |s| < 2^117 (s / 16 normal, 1039 |s| finite) and for s = +-0.  Scales of
    2^-126..2^-122 (s / 16 subnormal) are outside the stated range; the check there only
    bounds the error by what flushing s / 16 could cost, 80 * 2^-122."""
    say("decode GEMV one-hot over all finite scale patterns")
    N, K = 65536, 256
    q = np.tile(np.arange(-8, 8, dtype=np.int8), K // 16)[None].repeat(N, 0)
    s_bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expo = (s_bits >> 7) & 0xFF
    exact = ((expo >= 127 - 122) & (expo < 127 + 117)) | ((s_bits & 0x7FFF) == 0)
    low = (expo >= 1) & (expo < 127 - 122)
    s_bits = np.where(exact | low, s_bits, 0).astype(np.uint16)   # drop huge, non-finite, subnormal scales
    sc = np.repeat(s_bits[:, None], K // 32, axis=1).copy()
    pk = o.pack(q)
    w = o.bf16_to_f32(o.dequant(pk, sc))                             # [N, K]
    pkd, scd = dev(pk), dev_u16(sc)
    for k0 in range(0, 16, 4):
        x = np.zeros((4, K), dtype=np.uint16)
        x[np.arange(4), k0 + np.arange(4)] = 0x3F80
        y = w4a16.linear(dev_u16(x), pkd, scd, out_dtype=torch.float32)
        torch.cuda.synchronize()
        y = y.cpu().numpy()                                         # [4, N]
        ref = w[:, k0:k0 + 4].T
        bad = np.argwhere(y[:, exact] != ref[:, exact])
        assert bad.size == 0, (k0, bad[:5].tolist(), [hex(int(v)) for v in s_bits[exact][bad[:5, 1]]])
        say(f"  columns {k0}..{k0 + 3}: {int(np.sum(y[:, low] != ref[:, low]))} inexact below 2^-122")
        assert np.all(np.abs(y[:, low] - ref[:, low]) <= 80 * 2.0 ** -122)


def test_w3_synth_gate():
    say("W3 synthetic gate (q_proj L0 shape)")
    f = load_fixture("w4_gemm_synth.safetensors")
    _, pk, sc = o.synth_weights(2048, 1536, 1001)
    x = f["x"].reshape(1, -1)
    y = gpu_linear(x, pk, sc, "f32")[0]
    exp = f["out_expected"].reshape(-1)
    assert np.max(np.abs(y - exp)) <= 1e-4
    assert np.mean(np.abs(y - exp)) <= 1e-6
    from conftest import load_manifest
    fp = np.array(load_manifest()["w4_gemm_synth"]["fixed_points_out_0_0_0_8"], dtype=np.float32)
    assert np.max(np.abs(y[:8] - fp)) <= 1e-4


def test_linear_golden_small_cases():
    f = load_fixture("w4_linear_small.safetensors")
    i = 0
    while f"c{i}.packed" in f:
        pk, sc, x = f[f"c{i}.packed"], f[f"c{i}.scales"], f[f"c{i}.x"]
        K = pk.shape[1] * 8
        g = K // sc.shape[1]
        say(f"small case {i}: M={x.shape[0]} N={pk.shape[0]} K={K} group={g}")
        y = gpu_linear(x, pk, sc, "f32", group=g)
        check_f32(y, x, f[f"c{i}.deq_expected"], K, y_ref32=None)
        assert np.max(np.abs(y - f[f"c{i}.out_expected"])) <= 1e-4 * max(1.0, np.abs(f[f"c{i}.out_expected"]).max() / 4)
        yb = gpu_linear(x, pk, sc, "bf16", group=g)
        _, mag = o.matmul_f64(x, f[f"c{i}.deq_expected"])
        check_bf16(yb, o.linear(x, pk, sc, g), mag, K)
        i += 1


# ------------------------------------------------------------------ linear: BASELINE configs at M=1

C123 = {  # (K, N)
    "C1": (1536, 6144),
    "E2B_q": (1536, 2048), "E2B_kv": (1536, 256), "E2B_o": (2048, 1536),
    "E2B_gateup": (1536, 12288), "E2B_down": (6144, 1536),
    "12B_gateup": (3840, 30720), "12B_down": (15360, 3840), "12B_q": (3840, 4096),
    "12B_kv": (3840, 2048), "12B_o": (4096, 3840),
    # 12B full-attention layers (g12.zig:139-166: no v_proj; q 3840->8192, k 3840->512, o 8192->3840)
    "12B_full_q": (3840, 8192), "12B_full_k": (3840, 512), "12B_full_o": (8192, 3840),
    # E2B per-layer-embedding linears (engine.zig:659 gate 1536->256, :661 projection 256->1536,
    # :723 per_layer_model_projection 1536->35*256)
    "E2B_ple_gate": (1536, 256), "E2B_ple_proj": (256, 1536), "E2B_plmp": (1536, 8960),
    # E2B double-wide MLP of the KV-shared layers 15-34 (config.json use_double_wide_mlp,
    # scripts/57_w4_unpack_fixture.py:74 deq_dn20 [1536, 12288]): gate + up 1536->12288 each
    # (24576 fused rows) and down 12288->1536
    "E2B_dw_gateup": (1536, 24576), "E2B_dw_down": (12288, 1536),
}


@pytest.mark.parametrize("name", list(C123))
def test_linear_configs_m1(name):
    K, N = C123[name]
    say(f"linear M=1 {name} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 1000 + (K * 7 + N) % 1000)
    x = o.synth_x(1, K)
    w = o.dequant(pk, sc)
    ref32 = o.matmul_f32(x, w)
    y = gpu_linear(x, pk, sc, "f32")
    y64 = check_f32(y, x, w, K, ref32)
    _, mag = o.matmul_f64(x, w)
    yb = gpu_linear(x, pk, sc, "bf16")
    check_bf16(yb, ref32, mag, K)
    check_head_argmax(y, ref32, N)
    del y64


# ------------------------------------------------------------------ skinny and prefill

@pytest.mark.parametrize("M", [2, 3, 8, 16, 17, 32, 33, 63, 64])
def test_linear_skinny_small_shapes(M):
    K, N = 1536, 2048
    say(f"skinny M={M} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 77)
    x = o.synth_x(M, K)
    w = o.dequant(pk, sc)
    ref32 = o.matmul_f32(x, w)
    y = gpu_linear(x, pk, sc, "f32")
    check_f32(y, x, w, K, ref32)
    _, mag = o.matmul_f64(x, w)
    check_bf16(gpu_linear(x, pk, sc, "bf16"), ref32, mag, K)


@pytest.mark.parametrize("M", [8, 16, 32, 64])
def test_linear_c4_12b_gateup(M):
    """12B gate/up weights at M in {8,16,32,64}; the oracle
    runs on every 61st output row (a size-independent sample)."""
    K, N = 3840, 30720
    say(f"C4 M={M} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 1002)
    x = o.synth_x(M, K)
    y = gpu_linear(x, pk, sc, "f32")
    rows = np.arange(0, N, 61)
    w = o.dequant(pk[rows], sc[rows])
    ref32 = o.matmul_f32(x, w)
    check_f32(y[:, rows], x, w, K, ref32)
    check_head_argmax(y[:, rows], ref32, len(rows))


C4_LAYER = {"q": (3840, 4096), "kv": (3840, 2048), "o": (4096, 3840), "down": (15360, 3840)}


@pytest.mark.parametrize("M", [8, 16, 32, 64])
@pytest.mark.parametrize("name", list(C4_LAYER))
def test_linear_c4_12b_layer(name, M):
    """BASELINE config 3 on the other 12B linears (q, k/v, o, down) at M in {8,16,32,64}:
    every route these rows take (16-row GEMV, skinny, split-K) against the oracle on
    every 13th output row, f32 and bf16 outputs."""
    K, N = C4_LAYER[name]
    say(f"C4 {name} M={M} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 1010 + len(name))
    x = o.synth_x(M, K)
    rows = np.arange(0, N, 13)
    w = o.dequant(pk[rows], sc[rows])
    ref32 = o.matmul_f32(x, w)
    y = gpu_linear(x, pk, sc, "f32")
    check_f32(y[:, rows], x, w, K, ref32)
    _, mag = o.matmul_f64(x, w)
    check_bf16(gpu_linear(x, pk, sc, "bf16")[:, rows], ref32, mag, K)


@pytest.mark.parametrize("M,K,N", [
    (5, 3840, 4096), (8, 4096, 3840), (13, 1536, 2048), (16, 3840, 2048), (16, 2048, 1536), (12, 256, 40),
    (4, 3840, 4096),    # M = 4 beyond the 4-row plan (x over 8 vectors per thread)
    (3, 15360, 1000),   # M = 3 with x over the 4-row form's 64 KiB of LDS
])
def test_linear_gemv16_route(M, K, N):
    """M <= 16 on the smaller rows (M <= 4 where the 4-row plan does not hold): the
    straight-line GEMV with its 16-row epilogue (x whole in LDS, up to 160 KB), one
    pass (empty workspace), against the oracle, f32 and bf16 outputs."""
    say(f"gemv16 M={M} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 1300 + N)
    x = o.synth_x(M, K, 1400 + M)
    w = o.dequant(pk, sc)
    ref32 = o.matmul_f32(x, w)
    none = torch.empty(0, dtype=torch.uint8, device="cuda")
    xt, pkt, sct = dev_u16(x), dev(pk), dev_u16(sc)
    y = w4a16.linear(xt, pkt, sct, out_dtype=torch.float32, workspace=none)
    yb = w4a16.linear(xt, pkt, sct, out_dtype=torch.bfloat16, workspace=none)
    torch.cuda.synchronize()
    check_f32(y.cpu().numpy(), x, w, K, ref32)
    _, mag = o.matmul_f64(x, w)
    check_bf16(host_u16(yb), ref32, mag, K)


@pytest.mark.parametrize("M,K,N,step", [
    (64, 15360, 3840, 13),  # 12B down at M = 64: skinny form, 60 W blocks x 4 K parts
    (8, 15360, 3840, 13),   # M = 8 at K >= 8192: skinny form, 4 parts
    (40, 3840, 2048, 1),    # 12B k/v rows, 64-row x block with 24 repeated rows, 5 parts
    (33, 4096, 1000, 1),    # ragged N (last W tile partial), one real row in the x block's second half, 16 parts
    (20, 1536, 300, 1),     # small: 6 parts of one 256-column chunk
    (16, 6144, 1536, 5),    # E2B down at M = 16 (beyond the 16-row GEMV), 8 parts
    (4, 15360, 520, 1),     # M = 4 with x beyond the decode GEMV's LDS: 20 parts, ragged N
    (3, 12288, 256, 1),     # M = 3: 48 parts of one chunk
    (24, 1152, 700, 1),     # prefill form: K % 256 != 0, 9 parts of 128 columns
    (65, 15360, 3840, 13),  # 64 < M <= 128: skinny form, two 64-row x blocks (one real row in the second), 2 parts
    (128, 6144, 1536, 5),   # E2B down at M = 128: skinny form, 24 W blocks x 2 x blocks x 4 parts
    (100, 4160, 1000, 1),   # K % 256 != 0 above M = 64: LDS prefill form, 13 parts
    (200, 4096, 1000, 1),   # skinny form over four x blocks (8 real rows in the last), ragged N, 4 parts
    (300, 4096, 1000, 1),   # M > 256: LDS form, ragged N, 16 parts
    (300, 1152, 700, 3),    # LDS form, two x blocks, K % 256 != 0, 9 parts of 2 steps
])
def test_linear_splitk_route(M, K, N, step):
    """The split-K route (bf16 x, a one-pass grid too small to fill the GPU; the
    skinny kernel over K parts, also over two 64-row x blocks up to M = 128, the
    32x32 kernel when K % 256 != 0, and above M = 64 the LDS prefill kernel): the
    default call (the wrapper allocates the optional workspace) and the one-pass
    route (no workspace) both meet the stated f32 tolerance against the oracle on
    every `step`-th row n; bf16 outputs meet the bf16 bound."""
    say(f"split-K M={M} K={K} N={N}")
    assert w4a16.workspace_size(M, N, K, w4a16.DTYPE_BF16) > 0
    _, pk, sc = o.synth_weights(N, K, 1100 + N)
    x = o.synth_x(M, K, 1200 + M)
    rows = np.arange(0, N, step)
    w = o.dequant(pk[rows], sc[rows])
    ref32 = o.matmul_f32(x, w)
    xt, pkt, sct = dev_u16(x), dev(pk), dev_u16(sc)
    for ws in (None, torch.empty(0, dtype=torch.uint8, device="cuda")):
        y = w4a16.linear(xt, pkt, sct, out_dtype=torch.float32, workspace=ws)
        torch.cuda.synchronize()
        check_f32(y.cpu().numpy()[:, rows], x, w, K, ref32)
    yb = w4a16.linear(xt, pkt, sct, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    _, mag = o.matmul_f64(x, w)
    check_bf16(host_u16(yb)[:, rows], ref32, mag, K)


@pytest.mark.parametrize("M,K,N,group", [(300, 640, 8000, 32), (257, 448, 700, 64), (2048, 128, 520, 128)])
def test_prefill_lds_form(M, K, N, group):
    """The prefill kernel that expands W into LDS (8 waves; 256 x 128 tiles on these
    grids of under 240 workgroups, one pass, no workspace): ragged M (x rows past M
    repeat row M - 1) and N (the last W block partial), K steps that end in the
    ring's tail (10 = 2 * 4 + 2, 7, 2), group sizes 32 / 64 / 128; every row m and n
    against the oracle, f32 and bf16 outputs."""
    say(f"prefill LDS form M={M} K={K} N={N} group={group}")
    _, pk, sc = o.synth_weights(N, K, 1500 + N, group=group)
    x = o.synth_x(M, K, 1600 + M)
    w = o.dequant(pk, sc, group)
    ref32 = o.matmul_f32(x, w)
    check_f32(gpu_linear(x, pk, sc, "f32", group=group), x, w, K, ref32)
    _, mag = o.matmul_f64(x, w)
    check_bf16(gpu_linear(x, pk, sc, "bf16", group=group), ref32, mag, K)


@pytest.mark.parametrize("K,N", [(3840, 30720), (15360, 3840)])
def test_linear_c5_prefill(K, N):
    """M = 2048; oracle on a sample of rows m and n."""
    M = 2048
    say(f"C5 prefill M={M} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 1004)
    x = o.synth_x(M, K)
    y = gpu_linear(x, pk, sc, "f32")
    ms = np.arange(0, M, 53)
    ns = np.arange(0, N, 97)
    w = o.dequant(pk[ns], sc[ns])
    ref32 = o.matmul_f32(x[ms], w)
    check_f32(y[np.ix_(ms, ns)], x[ms], w, K, ref32)
    _, mag = o.matmul_f64(x[ms], w)
    yb = gpu_linear(x, pk, sc, "bf16")
    check_bf16(yb[np.ix_(ms, ns)], ref32, mag, K)


# ------------------------------------------------------------------ edge cases

@pytest.mark.parametrize("M,N,K,group", [(1, 17, 32, 32), (5, 33, 96, 32), (2, 1, 160, 32),
                                         (3, 48, 256, 64), (1, 64, 512, 128), (4, 24, 384, 128),
                                         (1, 1, 32, 32),
                                         # M > 4, K % 256 == 0 (skinny path): chunk counts 1, 2,
                                         # 3, 5, 7 (prefetch tails), partial row blocks of W and x
                                         (5, 33, 256, 32), (65, 70, 512, 128), (17, 100, 768, 64),
                                         (40, 129, 1280, 32), (100, 64, 1792, 256), (7, 16, 256, 256),
                                         # M > 64, K % 64 == 0 (prefill path): partial 256-row x
                                         # blocks and 128-row W blocks, 1 / 3 / 5 / 32 steps of 64
                                         (300, 200, 192, 64), (129, 33, 64, 32), (257, 130, 320, 32),
                                         (70, 300, 2048, 128)])
def test_linear_ragged(M, N, K, group):
    say(f"ragged M={M} N={N} K={K} group={group}")
    _, pk, sc = o.synth_weights(N, K, 55, group)
    x = o.synth_x(M, K, 9)
    w = o.dequant(pk, sc, group)
    y = gpu_linear(x, pk, sc, "f32", group=group)
    check_f32(y, x, w, K)
    assert np.array_equal(host_u16(w4a16.dequantW4(dev(pk), dev_u16(sc), group)), w)


def _random_linear_cases(n=64, seed=20261202):
    """Seeded shapes over every route: M in the decode (1-4), 16-row (5-16), skinny
    (17-64), mid (65-300) and prefill (512-1100) ranges, N ragged up to 6000, K a
    multiple of the group up to 4096, groups 32 / 64 / 128, bf16 or f32 x, bf16 or f32 y,
    with the optional split-K workspace or without it (one pass)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ranges = [(1, 4), (5, 16), (17, 64), (65, 300), (512, 1100)]
    cases = []
    for i in range(n):
        lo, hi = ranges[i % len(ranges)]
        M = int(rng.integers(lo, hi + 1))
        group = int(rng.choice([32, 32, 64, 128]))
        K = group * int(rng.integers(1, 4096 // group + 1))
        N = int(rng.integers(1, 6001))
        while M * N * K > 2_500_000_000:
            N = max(1, N // 2)
        x_f32 = bool(rng.random() < 0.25)
        out = "f32" if (x_f32 or rng.random() < 0.5) else "bf16"
        one_pass = (not x_f32) and bool(rng.random() < 0.5)
        cases.append((i, M, N, K, group, x_f32, out, one_pass))
    return cases


@pytest.mark.parametrize("i,M,N,K,group,x_f32,out,one_pass", _random_linear_cases())
def test_linear_random_shapes(i, M, N, K, group, x_f32, out, one_pass):
    """Seeded random shapes through w4a16_linear against the oracle at the stated
    tolerances (every output element)."""
    say(f"random case {i}: M={M} N={N} K={K} group={group} x_f32={x_f32} out={out} one_pass={one_pass}")
    _, pk, sc = o.synth_weights(N, K, 7000 + i, group)
    xb = o.synth_x(M, K, 8000 + i)
    x_np = (o.bf16_to_f32(xb) * np.float32(1.0 + 2.0 ** -10)).astype(np.float32) if x_f32 else xb
    x = dev(x_np) if x_f32 else dev_u16(x_np)
    ws = torch.empty(0, dtype=torch.uint8, device="cuda") if one_pass else None
    odt = torch.float32 if out == "f32" else torch.bfloat16
    y = w4a16.linear(x, dev(pk), dev_u16(sc), group=group, out_dtype=odt, workspace=ws)
    torch.cuda.synchronize()
    w = o.dequant(pk, sc, group)
    if out == "f32":
        check_f32(y.cpu().numpy(), x_np, w, K, x_f32=x_f32)
    else:
        ref32 = o.matmul_f32(xb, w)
        _, mag = o.matmul_f64(xb, w)
        check_bf16(host_u16(y), ref32, mag, K)


def test_empty_and_k_zero():
    say("empty shapes / K = 0")
    x = torch.zeros((0, 64), dtype=torch.bfloat16, device="cuda")
    pk = torch.zeros((16, 8), dtype=torch.int32, device="cuda")
    sc = torch.zeros((16, 2), dtype=torch.bfloat16, device="cuda")
    y = w4a16.linear(x, pk, sc)
    assert y.shape == (0, 16)
    # K = 0: y = 0 (the dot over an empty contraction)
    y = torch.full((3, 5), 7.0, dtype=torch.float32, device="cuda")
    st = w4a16.lib().w4a16_linear(y.data_ptr(), 0, y.data_ptr(), y.data_ptr(), y.data_ptr(), 1,
                                  3, 5, 0, 32, 0, None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(y).item() == 0
    yb = torch.full((3, 5), 7.0, dtype=torch.bfloat16, device="cuda")
    st = w4a16.lib().w4a16_linear(yb.data_ptr(), 0, yb.data_ptr(), yb.data_ptr(), yb.data_ptr(), 0,
                                  3, 5, 0, 32, 0, None, 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(yb).item() == 0


def test_nan_scale_propagates_to_its_row_only():
    say("NaN scale")
    _, pk, sc = o.synth_weights(32, 256, 3)
    sc[5, 2] = 0x7FC0
    x = o.synth_x(2, 256, 4)
    y = gpu_linear(x, pk, sc, "f32")
    assert np.all(np.isnan(y[:, 5]))
    assert not np.any(np.isnan(np.delete(y, 5, axis=1)))


def test_linear_f32_activations():
    """x in f32 (the engine's compute dtype): carried exactly as three bf16 terms."""
    say("f32 activations")
    for M, K, N in [(1, 1536, 2048), (7, 3840, 512), (64, 256, 96)]:
        _, pk, sc = o.synth_weights(N, K, 31)
        rng = np.random.default_rng(M)
        x = rng.standard_normal((M, K), dtype=np.float32)
        w = o.dequant(pk, sc)
        y = gpu_linear(x, pk, sc, "f32", x_f32=True)
        check_f32(y, x, w, K, x_f32=True)


@pytest.mark.parametrize("M,K,N", [(1, 15360, 3840), (1, 12288, 1536), (1, 3840, 30720)])
def test_linear_f32_activations_decode_shapes(M, K, N):
    """f32 x at decode on the 12B down, E2B double-wide down and 12B gate/up shapes: the
    decode GEMV with three bf16 planes of x in LDS (92 KB of planes for K = 15360, beyond
    the 64 KB that bf16 x keeps to) and, for gate/up, the tile loop; every row against
    the oracle."""
    say(f"f32 activations decode M={M} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 37)
    x = np.random.default_rng(K).standard_normal((M, K), dtype=np.float32)
    w = o.dequant(pk, sc)
    y = gpu_linear(x, pk, sc, "f32", x_f32=True)
    check_f32(y, x, w, K, x_f32=True)


def test_linear_f32_activations_non_finite():
    """+-inf and NaN in f32 x follow the f32 dot (engine.zig:531-532): +-inf * w (NaN where
    w = +-0 or where infinities of both signs meet), NaN * w = NaN; the other rows are
    untouched and meet the f32 bound."""
    say("f32 activations with +-inf / NaN")
    for M, K, N in [(1, 1536, 2048), (3, 3840, 512), (7, 3840, 512), (64, 256, 96)]:
        _, pk, sc = o.synth_weights(N, K, 37)
        rng = np.random.default_rng(100 + M)
        x = rng.standard_normal((M, K), dtype=np.float32)
        x[0, 5] = np.inf
        x[0, K - 1] = np.inf
        if M > 1:
            x[1, 17] = -np.inf
            x[M - 1, K // 2] = np.nan if M > 2 else x[M - 1, K // 2]
        w = o.dequant(pk, sc)
        y = gpu_linear(x, pk, sc, "f32", x_f32=True)
        ref = o.matmul_f32x(x, w)
        assert np.array_equal(np.isnan(y), np.isnan(ref)), (M, K, N)
        inf = np.isinf(ref)
        assert np.array_equal(np.isinf(y), inf) and np.array_equal(np.sign(y[inf]), np.sign(ref[inf]))
        bad = ~np.isfinite(x).all(axis=1)
        if (~bad).any():
            check_f32(y[~bad], x[~bad], w, K, x_f32=True)


def test_deterministic_and_stream_ordered():
    say("determinism + non-default stream")
    K, N = 3840, 4096
    _, pk, sc = o.synth_weights(N, K, 12)
    x = dev_u16(o.synth_x(4, K))
    pkd, scd = dev(pk), dev_u16(sc)
    a = w4a16.linear(x, pkd, scd, out_dtype=torch.float32)
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        b = w4a16.linear(x, pkd, scd, out_dtype=torch.float32)
    s.synchronize()
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int32), b.view(torch.int32))


def test_w4lin_interface():
    say("W4Lin init/toW/linear")
    _, pk, sc = o.synth_weights(256, 512, 8)
    store = {"m.q_proj.weight_packed": dev(pk), "m.q_proj.weight_scale": dev_u16(sc),
             "m.q_proj.weight_shape": torch.tensor([256, 512])}
    lin = w4a16.W4Lin.init(store, "m.q_proj")
    assert (lin.out_features, lin.in_features) == (256, 512)
    assert np.array_equal(host_u16(lin.toW()), o.dequant(pk, sc))
    x = o.synth_x(3, 512)
    y = lin.linear(dev_u16(x), out_dtype=torch.float32).cpu().numpy()
    check_f32(y, x, o.dequant(pk, sc), 512)


def test_graph_capture_replays_match_eager():
    """The linear captured in a HIP graph (how a decode step would run it) gives
    the eager result on every replay, with other eager work in between."""
    say("graph capture / replay")
    K, N = 3840, 4096
    _, pk, sc = o.synth_weights(N, K, 21)
    pkd, scd = dev(pk), dev_u16(sc)
    x = dev_u16(o.synth_x(1, K))
    y = torch.empty((1, N), dtype=torch.float32, device="cuda")
    ref = w4a16.linear(x, pkd, scd, out_dtype=torch.float32).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w4a16.linear(x, pkd, scd, out=y)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w4a16.linear(x, pkd, scd, out=y)
    for rep in range(4):
        y.fill_(float("nan"))
        junk = w4a16.linear(x, pkd, scd, out_dtype=torch.bfloat16)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), ref.view(torch.int32)), rep
        del junk


@pytest.mark.parametrize("M,K,N", [(8, 15360, 1000), (24, 1152, 700), (300, 2048, 700), (100, 2048, 700)])
def test_splitk_graph_replays_match_eager(M, K, N):
    """The split-K route (main kernel + finalize over the caller's workspace; the
    skinny form with 15 parts, the 32x32 form with 9, the LDS prefill form with 16,
    the skinny form over two 64-row x blocks with 8) captured in a HIP graph:
    every replay equals the eager result bit for bit, since the parts are added
    in a fixed order, with other eager work between the replays."""
    say(f"split-K graph capture / replay M={M} K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 51)
    pkd, scd = dev(pk), dev_u16(sc)
    x = dev_u16(o.synth_x(M, K, 52))
    nws = w4a16.workspace_size(M, N, K, w4a16.DTYPE_BF16)
    assert nws > 0
    ws = torch.empty(nws, dtype=torch.uint8, device="cuda")
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    ref = w4a16.linear(x, pkd, scd, out_dtype=torch.bfloat16, workspace=ws).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w4a16.linear(x, pkd, scd, out=y, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        w4a16.linear(x, pkd, scd, out=y, workspace=ws)
    for rep in range(4):
        y.fill_(float("nan"))
        ws.fill_(0xFF)  # the partial planes hold other data between replays
        junk = w4a16.linear(x, pkd, scd, out_dtype=torch.float32)  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16)), rep
        del junk
    w = o.dequant(pk, sc)
    _, mag = o.matmul_f64(o.synth_x(M, K, 52), w)
    check_bf16(host_u16(y), o.matmul_f32(o.synth_x(M, K, 52), w), mag, K)


@pytest.mark.parametrize("N", [16, 48, 400, 30720])
def test_gemv_tile_counts(N):
    """The straight-line GEMV over one to 1920 16-row tiles, with ragged N (rows past
    N are recomputed from row N - 1 and not written)."""
    K = 3840
    tpw = 1
    _, pk, sc = o.synth_weights(N, K, 43)
    x = o.synth_x(1, K, 44)
    w = o.dequant(pk, sc)
    ref32 = o.matmul_f32(x, w)
    say(f"tiles per workgroup {tpw}: N={N}")
    y = gpu_linear(x, pk, sc, "f32")
    check_f32(y, x, w, K, ref32)
    yb = gpu_linear(x, pk, sc, "bf16")
    _, mag = o.matmul_f64(x, w)
    check_bf16(yb, ref32, mag, K)


@pytest.mark.parametrize("N,K,group", [
    # two K segments (8-row tiles, K % 512 == 0): one step per segment, ragged N, 5 and
    # 15 steps per segment over as many waves, 30 over 16 waves (runs 2,..,2,1,1),
    # groups 64 / 128
    (1, 512, 32), (7, 512, 32), (9, 1024, 32), (1001, 2560, 32), (300, 7680, 32),
    (3840, 15360, 32), (200, 1536, 64), (136, 3072, 128),
    # one K segment, uneven runs: 17 steps over 16 waves (one run of 2), 15 steps over
    # 8 waves (runs 2,..,2,1) with a ragged last tile
    (2000, 4352, 32), (16390, 3840, 32)])
def test_decode_gemv_k_segments_and_uneven_runs(N, K, group):
    """M = 1 decode GEMV plans: K in two segments where K % 512 == 0 (the B operand's
    16 columns are 8 rows x 2 halves of K, A row s carries x of half s), and runs of
    steps that differ by one between the waves of a workgroup (a short run loads its
    last step twice and computes it once).  Against the oracle, f32 and bf16 out."""
    say(f"decode segments / uneven runs N={N} K={K} group={group}")
    _, pk, sc = o.synth_weights(N, K, 62, group)
    x = o.synth_x(1, K, 63)
    w = o.dequant(pk, sc, group)
    ref32 = o.matmul_f32(x, w)
    y = gpu_linear(x, pk, sc, "f32", group=group)
    check_f32(y, x, w, K, ref32)
    yb = gpu_linear(x, pk, sc, "bf16", group=group)
    _, mag = o.matmul_f64(x, w)
    check_bf16(yb, ref32, mag, K)


def test_decode_gemv_segments_one_hot():
    """M = 1, K = 512: two K segments of one step each.  A one-hot x at column k selects
    weight k of every row, so y must reproduce the bf16 weight exactly, for columns in
    either segment and at both ends of each (pins which half of K each A row and each
    B column carries)."""
    N, K = 4096, 512
    _, pk, sc = o.synth_weights(N, K, 61)
    w = o.bf16_to_f32(o.dequant(pk, sc))
    pkd, scd = dev(pk), dev_u16(sc)
    for k in (0, 7, 200, 255, 256, 263, 400, 511):
        x = np.zeros((1, K), dtype=np.uint16)
        x[0, k] = 0x3F80
        y = w4a16.linear(dev_u16(x), pkd, scd, out_dtype=torch.float32)
        torch.cuda.synchronize()
        y = y.cpu().numpy()[0]
        bad = np.flatnonzero(y != w[:, k])
        assert bad.size == 0, (k, bad[:5].tolist())


@pytest.mark.parametrize("M,N,K", [(17, 200, 640), (32, 130, 640), (48, 2048, 1344), (64, 300, 960)])
def test_prefill_kernel_small_m(M, N, K):
    """The 32x32 kernel with 32 or 64 rows of x per workgroup over K parts (the split-K
    route when K % 256 != 0 at 16 < M <= 64; the wrapper passes the workspace),
    including x rows past M and ragged N."""
    assert w4a16.workspace_size(M, N, K, w4a16.DTYPE_BF16) > 0
    _, pk, sc = o.synth_weights(N, K, 45)
    x = o.synth_x(M, K, 46)
    w = o.dequant(pk, sc)
    ref32 = o.matmul_f32(x, w)
    say(f"prefill kernel, small M: M={M} N={N} K={K}")
    y = gpu_linear(x, pk, sc, "f32")
    check_f32(y, x, w, K, ref32)
    yb = gpu_linear(x, pk, sc, "bf16")
    _, mag = o.matmul_f64(x, w)
    check_bf16(yb, ref32, mag, K)


def test_linear_m4_beyond_both_gemv_plans():
    """12B gate/up rows at M = 4: the decode GEMV's 4-row form, whose 1 920 tiles are more
    than one round of workgroups holds, so its tile loop (x rows past M repeating row
    M - 1); every 11th row n against the oracle, f32 and bf16 outputs."""
    M, K, N = 4, 3840, 30720
    say(f"M=4 beyond both GEMV plans K={K} N={N}")
    _, pk, sc = o.synth_weights(N, K, 1700)
    x = o.synth_x(M, K, 1701)
    rows = np.arange(0, N, 11)
    w = o.dequant(pk[rows], sc[rows])
    ref32 = o.matmul_f32(x, w)
    check_f32(gpu_linear(x, pk, sc, "f32")[:, rows], x, w, K, ref32)
    _, mag = o.matmul_f64(x, w)
    check_bf16(gpu_linear(x, pk, sc, "bf16")[:, rows], ref32, mag, K)


@pytest.mark.parametrize("M,N,K", [(3, 20001, 3840), (4, 30000, 1536), (3, 30720, 3840)])
def test_linear_decode_tile_loop(M, N, K):
    """M = 3, 4 with more 16-row tiles than one round of workgroups holds: the decode
    GEMV's tile loop (each workgroup walks tiles b, b + grid, ..., the next tile's loads
    issued before the current tile's epilogue, partial sums in alternating LDS halves).
    Every row against the oracle (f32 out), and the bf16 output equal to the f32 one
    rounded once."""
    say(f"decode tile loop M={M} N={N} K={K}")
    _, pk, sc = o.synth_weights(N, K, 1800 + M)
    x = o.synth_x(M, K, 1801 + M)
    w = o.dequant(pk, sc)
    ref32 = o.matmul_f32(x, w)
    y32 = gpu_linear(x, pk, sc, "f32")
    check_f32(y32, x, w, K, ref32)
    yb = gpu_linear(x, pk, sc, "bf16")
    assert np.array_equal(yb, o.f32_to_bf16(y32))


@pytest.mark.parametrize("M,Ns,K,x_f32,out", [
    (1, (4096, 2048, 2048), 3840, False, "bf16"),   # 12B q, k, v at decode: one launch
    (1, (8192, 512), 3840, False, "f32"),           # 12B full-attention q, k at decode: one launch
    (1, (2048, 256, 256), 1536, False, "f32"),      # E2B q, k, v at decode (K % 512 == 0: the single linears split K in two)
    (3, (17, 0, 33, 5), 512, False, "f32"),        # ragged N, an empty member
    (2, (64, 48), 1536, True, "f32"),               # f32 x
    (4, (4096, 2048, 2048), 3840, True, "f32"),     # f32 x at M = 4, planes beyond 64 KB: each member as 3M rows
    (20, (40, 24, 16), 256, False, "bf16"),         # above M = 16: one launch per weight
    (8, (4096, 2048, 2048), 3840, False, "f32"),     # batched decode M = 8: one launch (16-row GEMV)
    (13, (17, 0, 33, 5), 512, False, "f32"),        # M = 13, ragged N, an empty member
    (32, (4096, 2048, 2048), 3840, False, "bf16"),  # M = 32: each member split-K (skinny form)
    (128, (4096, 2048, 0), 3840, False, "f32"),     # M = 128: each member split-K (LDS prefill form)
])
def test_linear_group_equals_single_linears(M, Ns, K, x_f32, out):
    """w4a16_linear_group (q, k, v read the same x, engine.zig:552,571,583): every output
    equals w4a16_linear of that weight bit for bit (same per-row arithmetic), and the
    first member is checked against the oracle."""
    say(f"linear_group M={M} Ns={Ns} K={K} x_f32={x_f32} out={out}")
    ws = [o.synth_weights(n, K, 60 + j)[1:] for j, n in enumerate(Ns)]
    x_np = o.synth_x(M, K, 61)
    if x_f32:
        x_np = (o.bf16_to_f32(x_np) * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)
    x = dev(x_np) if x_f32 else dev_u16(x_np)
    lins = [w4a16.W4Lin(dev(pk), dev_u16(sc)) for pk, sc in ws]
    odt = torch.float32 if out == "f32" else torch.bfloat16
    ys = w4a16.linear_group(x, lins, out_dtype=odt)
    singles = [w4a16.linear(x, lin.pk, lin.sc, out_dtype=odt) for lin in lins]
    torch.cuda.synchronize()
    for y, y1 in zip(ys, singles):
        assert torch.equal(y.view(torch.int32 if out == "f32" else torch.int16),
                           y1.view(torch.int32 if out == "f32" else torch.int16))
    if Ns[0] and out == "f32":
        w = o.dequant(*ws[0])
        check_f32(ys[0].cpu().numpy(), x_np, w, K, x_f32=x_f32)


def _random_group_cases(n=24, seed=20261204):
    """Seeded weight groups: 1-4 members of ragged N (an empty one now and then), M 1-20,
    K a multiple of 32 up to 4096 (K % 512 == 0 half the time: the K-segment plans), bf16
    or f32 x, bf16 or f32 y."""
    rng = np.random.Generator(np.random.PCG64(seed))
    cases = []
    for i in range(n):
        M = int(rng.choice([1, 1, 1, 2, 3, 4, 5, 8, 13, 16, 20]))
        K = 512 * int(rng.integers(1, 9)) if rng.random() < 0.5 else 32 * int(rng.integers(1, 129))
        Ns = tuple(int(v) if rng.random() > 0.1 else 0 for v in rng.integers(1, 9000, size=int(rng.integers(1, 5))))
        x_f32 = bool(rng.random() < 0.2)
        out = "f32" if rng.random() < 0.5 else "bf16"
        cases.append((i, M, Ns, K, x_f32, out))
    return cases


@pytest.mark.parametrize("i,M,Ns,K,x_f32,out", _random_group_cases())
def test_linear_group_random_equals_single_linears(i, M, Ns, K, x_f32, out):
    """Seeded random groups: every output of w4a16_linear_group equals w4a16_linear of
    that weight bit for bit (fused or not)."""
    say(f"random linear_group {i}: M={M} Ns={Ns} K={K} x_f32={x_f32} out={out}")
    ws = [o.synth_weights(n, K, 300 + 7 * i + j)[1:] for j, n in enumerate(Ns)]
    x_np = o.synth_x(M, K, 400 + i)
    if x_f32:
        x_np = (o.bf16_to_f32(x_np) * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)
    x = dev(x_np) if x_f32 else dev_u16(x_np)
    lins = [w4a16.W4Lin(dev(pk), dev_u16(sc)) for pk, sc in ws]
    odt = torch.float32 if out == "f32" else torch.bfloat16
    ys = w4a16.linear_group(x, lins, out_dtype=odt)
    singles = [w4a16.linear(x, lin.pk, lin.sc, out_dtype=odt) for lin in lins]
    torch.cuda.synchronize()
    for y, y1 in zip(ys, singles):
        assert torch.equal(y.view(torch.int32 if out == "f32" else torch.int16),
                           y1.view(torch.int32 if out == "f32" else torch.int16))
