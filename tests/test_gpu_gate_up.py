"""GPU parity of the fused MLP front half, w4a16_gate_up_gelu (engine.zig:653:
dot(xff, gate).gelu().mul(dot(xff, up))), against the oracle (oracle.gate_up_gelu,
float64 dots and float64 gelu_pytorch_tanh).

Stated tolerance, elementwise, with eps = 2^-24 and gamma_K = K eps / (1 - K eps):
  eg = 2 gamma_K sum|x||wg|, eu = 2 gamma_K sum|x||wu|      (the linear's fp32 bound on g, u)
  with bf16 dots, eg += ulp_bf16(|g| + eg) (and eu alike): rounding both sides to bf16
  adds at most one bf16 ulp
  ev = (16 + 16 |z|) eps, z = sqrt(2/pi)(g + 0.044715 g^3)  (fp32 evaluation of the
  activation, exp2 and reciprocal included, and of the product)
  |h - h64| <= 1.2 eg (|u| + eu) + |gelu(g)| eu + (|gelu(g)| + 1.2 eg)(|u| + eu) ev
               + 2^-118 (1 + |u| + eu)
  (1.2 bounds |gelu'|; the last term is fp32 underflow of gelu(g) for g < about -10);
  h bf16: plus ulp_bf16(|h64| + that bound).
  rel_L2(h, h64) <= 1e-5 for h f32 with f32 dots, else 4e-3 (bf16 h or bf16 dots).
Shapes that no fused kernel takes run the unfused route (two linears + activation) and
meet the same bound.  At the 12B prefill shape the fused result is compared with the
composition of two plain w4a16_linear calls and a float64 activation (a size-independent
property: same g and u, only the activation's fp32 evaluation error apart).
"""
from __future__ import annotations

import math
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

import w4a16  # noqa: E402
from oracle import w4a16_oracle as o  # noqa: E402

EPS = 2.0 ** -24
# gelu(g) below ~2^-120 (g < about -10) is at fp32's underflow threshold and may come
# out as 0 (so does the tanh form in fp32, where 1 + tanh(z) rounds to 0 from g < -4.5)
UNDERFLOW = 2.0 ** -118


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    w4a16.lib()


def say(msg: str) -> None:
    print(f"[gpu-gate-up] {msg}", flush=True)
    sys.stdout.flush()


def dev_bf16(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def host_u16(t) -> np.ndarray:
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def ulp_bf16(v):
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -126)))
    return 2.0 ** (e - 7)


def weights(F, K, seed, group):
    _, pk_g, sc_g = o.synth_weights(F, K, seed, group)
    _, pk_u, sc_u = o.synth_weights(F, K, seed + 1, group)
    return pk_g, sc_g, pk_u, sc_u


def w4lin(pk, sc, group):
    return w4a16.W4Lin(torch.from_numpy(pk).cuda(), dev_bf16(sc), group)


def run_gpu(x, pk_g, sc_g, pk_u, sc_u, group, x_f32, h_f32, bf16_dots):
    xt = torch.from_numpy(x).cuda() if x_f32 else dev_bf16(x)
    h = w4a16.gate_up_gelu(xt, w4lin(pk_g, sc_g, group), w4lin(pk_u, sc_u, group),
                           out_dtype=torch.float32 if h_f32 else torch.bfloat16, bf16_dots=bf16_dots)
    torch.cuda.synchronize()
    return h.cpu().numpy().astype(np.float64) if h_f32 else o.bf16_to_f32(host_u16(h)).astype(np.float64)


def bound(g, u, mg, mu, K, bf16_dots):
    gam = K * EPS / (1 - K * EPS)
    eg, eu = 2 * gam * mg, 2 * gam * mu
    if bf16_dots:
        eg = eg + ulp_bf16(np.abs(g) + eg)
        eu = eu + ulp_bf16(np.abs(u) + eu)
        g = o.bf16_to_f32(o.round_bf16(g.astype(np.float32))).astype(np.float64)
        u = o.bf16_to_f32(o.round_bf16(u.astype(np.float32))).astype(np.float64)
    z = math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)
    ev = (16 + 16 * np.abs(z)) * EPS
    gel = np.abs(o.gelu_tanh(g))
    return (1.2 * eg * (np.abs(u) + eu) + gel * eu + (gel + 1.2 * eg) * (np.abs(u) + eu) * ev
            + UNDERFLOW * (1 + np.abs(u) + eu))


def check(h, x, pk_g, sc_g, pk_u, sc_u, K, group, h_f32, bf16_dots):
    h64, g, u, mg, mu = o.gate_up_gelu(x, pk_g, sc_g, pk_u, sc_u, group, bf16_dots)
    b = bound(g, u, mg, mu, K, bf16_dots)
    if not h_f32:
        b = b + ulp_bf16(np.abs(h64) + b)
    excess = np.abs(h - h64) - b
    assert np.all(excess <= 0), (float(np.max(excess)), np.unravel_index(np.argmax(excess), excess.shape))
    den = float(np.linalg.norm(h64))
    if den > 0:
        # bf16 dots round g and u to bf16 before the activation, so an fp32 difference in g
        # or u that crosses a bf16 rounding boundary moves h by a bf16 ulp: the bf16 flow's
        # relative bound applies, as for h in bf16
        assert float(np.linalg.norm(h - h64)) / den <= (1e-5 if h_f32 and not bf16_dots else 4e-3)


# (M, F, K, group, x f32, h f32, bf16 dots): the route each shape takes is in the comment
CASES = [
    (1, 1000, 3840, 32, False, True, False),    # straight-line GEMV
    (2, 70, 1536, 32, False, False, False),     # GEMV, h bf16
    (3, 33, 512, 64, False, True, True),        # GEMV, group 64, bf16 dots
    (1, 72, 1024, 32, True, True, False),       # GEMV on f32 x (three bf16 planes)
    (1, 15360, 3840, 32, False, True, False),   # 12B gate/up decode
    (4, 70, 3840, 32, False, True, False),      # M = 4 at K = 3840: beyond the 4-row plan -> 16-row GEMV
    (4, 15360, 3840, 32, False, False, False),  # 12B gate/up at M = 4: beyond both GEMV plans -> skinny
    (5, 33, 256, 32, False, False, False),      # 16-row GEMV pair mode
    (8, 6144, 1536, 32, False, True, False),    # 16-row GEMV pair mode: E2B gate/up at M = 8
    (1, 12288, 1536, 32, False, True, False),   # E2B double-wide gate/up (layers 15-34) at decode
    (1, 12288, 1536, 32, False, False, True),   # the same, bf16 dots, h bf16 (fam = bf16 flow)
    (4, 12288, 1536, 32, False, False, True),   # E2B double-wide at M = 4
    (16, 72, 1024, 64, False, False, True),     # 16-row GEMV pair mode, group 64, bf16 dots, h bf16
    (17, 9, 512, 32, False, True, False),       # split-K (skinny form, 2 parts), one real row in the second x block
    (40, 129, 1280, 32, False, True, True),     # split-K (skinny form, 5 parts), bf16 dots
    (64, 200, 768, 128, False, True, False),    # split-K (skinny form, 400 virtual rows), group 128
    (16, 1000, 6144, 32, False, False, False),  # split-K at M = 16 beyond the 16-row GEMV (8 parts), h bf16
    (32, 6144, 1536, 32, False, True, False),   # E2B gate/up at M = 32: one-pass skinny (no split part count)
    (65, 50, 64, 32, False, True, False),       # prefill
    (100, 6144, 1536, 32, False, True, False),  # E2B gate/up at M = 100: one-pass skinny over two 64-row x blocks
    (96, 40, 512, 64, False, False, True),      # skinny over two x blocks, group 64, bf16 dots, h bf16
    (160, 300, 1024, 32, False, True, False),   # skinny over three x blocks
    (250, 40, 512, 128, False, False, True),    # skinny over four x blocks, group 128, bf16 dots, h bf16
    (300, 130, 192, 64, False, False, False),   # prefill, h bf16
    (257, 17, 320, 32, False, True, True),      # prefill, bf16 dots
    (4096, 4096, 64, 32, False, True, False),   # prefill with two W blocks per wave
    (8, 40, 320, 32, False, True, False),       # unfused: K % 256 != 0 at M <= 64
    (2, 24, 96, 32, False, False, True),        # unfused, bf16 dots, h bf16
    (6, 20, 512, 32, True, True, False),        # unfused: f32 x above M = 4
    (8, 15360, 3840, 32, True, True, False),    # 12B at M = 8, f32 x: g and u each from the planes run as 3M rows
]


@pytest.mark.parametrize("M,F,K,group,x_f32,h_f32,bf16_dots", CASES)
def test_gate_up_gelu_vs_oracle(M, F, K, group, x_f32, h_f32, bf16_dots):
    say(f"gate_up_gelu M={M} F={F} K={K} group={group} x_f32={x_f32} h_f32={h_f32} bf16_dots={bf16_dots}")
    pk_g, sc_g, pk_u, sc_u = weights(F, K, 4000 + F, group)
    x = o.synth_x(M, K, 4100 + M)
    if x_f32:
        x = (o.bf16_to_f32(x) * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)  # not bf16-representable
    h = run_gpu(x, pk_g, sc_g, pk_u, sc_u, group, x_f32, h_f32, bf16_dots)
    check(h, x, pk_g, sc_g, pk_u, sc_u, K, group, h_f32, bf16_dots)


def _random_gate_up_cases(n=40, seed=20261203):
    """Seeded shapes over every gate/up route: M in the decode, 16-row, skinny, mid and
    prefill ranges, ragged F up to 3000, K a multiple of the group up to 4096, groups
    32 / 64 / 128, bf16 or f32 x, h bf16 or f32, with or without bf16 dots."""
    rng = np.random.Generator(np.random.PCG64(seed))
    ranges = [(1, 4), (5, 16), (17, 64), (65, 300), (512, 1100)]
    cases = []
    for i in range(n):
        lo, hi = ranges[i % len(ranges)]
        M = int(rng.integers(lo, hi + 1))
        group = int(rng.choice([32, 32, 64, 128]))
        K = group * int(rng.integers(1, 4096 // group + 1))
        F = int(rng.integers(1, 3001))
        while M * 2 * F * K > 2_500_000_000:
            F = max(1, F // 2)
        x_f32 = bool(rng.random() < 0.2)
        h_f32 = bool(rng.random() < 0.5)
        bf16_dots = bool(rng.random() < 0.3)
        cases.append((i, M, F, K, group, x_f32, h_f32, bf16_dots))
    return cases


@pytest.mark.parametrize("i,M,F,K,group,x_f32,h_f32,bf16_dots", _random_gate_up_cases())
def test_gate_up_gelu_random_shapes(i, M, F, K, group, x_f32, h_f32, bf16_dots):
    """Seeded random shapes through w4a16_gate_up_gelu against the oracle at the stated
    bound (every output element)."""
    say(f"gate_up_gelu random case {i}: M={M} F={F} K={K} group={group} x_f32={x_f32} h_f32={h_f32} "
        f"bf16_dots={bf16_dots}")
    pk_g, sc_g, pk_u, sc_u = weights(F, K, 9000 + 2 * i, group)
    x = o.synth_x(M, K, 9500 + i)
    if x_f32:
        x = (o.bf16_to_f32(x) * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)
    h = run_gpu(x, pk_g, sc_g, pk_u, sc_u, group, x_f32, h_f32, bf16_dots)
    check(h, x, pk_g, sc_g, pk_u, sc_u, K, group, h_f32, bf16_dots)


@pytest.mark.parametrize("M", [20, 64])
def test_gate_up_gelu_12b_skinny_eight_waves(M):
    """12B gate/up (F = 15360, K = 3840) at M = 20 and 64: the skinny kernel with eight
    waves (128 W rows) per workgroup, pair mode; the oracle on every 7th row f."""
    F, K = 15360, 3840
    say(f"gate_up_gelu 12B skinny M={M}")
    pk_g, sc_g, pk_u, sc_u = weights(F, K, 4700, 32)
    x = o.synth_x(M, K, 4701 + M)
    h = run_gpu(x, pk_g, sc_g, pk_u, sc_u, 32, False, True, False)
    f = np.arange(0, F, 7)
    check(h[:, f], x, pk_g[f], sc_g[f], pk_u[f], sc_u[f], K, 32, True, False)


@pytest.mark.parametrize("h_f32", [True, False])
def test_gate_up_gelu_one_pass_without_workspace(h_f32):
    """Gate/up at M = 48, F = 1000, K = 1536 (split-K, skinny form, 6 parts by default):
    with an empty workspace the call takes the one-pass skinny route instead; both
    meet the bound."""
    M, F, K = 48, 1000, 1536
    say(f"gate_up_gelu one-pass M={M} F={F} K={K} h_f32={h_f32}")
    assert w4a16.gate_up_workspace_size(M, F, K, w4a16.DTYPE_BF16) > 0
    pk_g, sc_g, pk_u, sc_u = weights(F, K, 4600, 32)
    x = o.synth_x(M, K, 4601)
    h = w4a16.gate_up_gelu(dev_bf16(x), w4lin(pk_g, sc_g, 32), w4lin(pk_u, sc_u, 32),
                           out_dtype=torch.float32 if h_f32 else torch.bfloat16,
                           workspace=torch.empty(0, dtype=torch.uint8, device="cuda"))
    torch.cuda.synchronize()
    h = h.cpu().numpy().astype(np.float64) if h_f32 else o.bf16_to_f32(host_u16(h)).astype(np.float64)
    check(h, x, pk_g, sc_g, pk_u, sc_u, K, 32, h_f32, False)


def test_gate_up_gelu_equals_two_linears_at_12b_prefill():
    """M = 2048, F = 15360, K = 3840 (the prefill config): fused h against gelu64(g) * u of
    two plain w4a16_linear calls (g, u in f32)."""
    M, F, K = 2048, 15360, 3840
    say(f"gate_up_gelu vs two linears M={M} F={F} K={K}")
    gen = torch.Generator(device="cuda").manual_seed(7)
    pk_g = torch.randint(-2 ** 31, 2 ** 31 - 1, (F, K // 8), dtype=torch.int32, device="cuda", generator=gen)
    pk_u = torch.randint(-2 ** 31, 2 ** 31 - 1, (F, K // 8), dtype=torch.int32, device="cuda", generator=gen)
    sc_g = (torch.rand((F, K // 32), device="cuda", generator=gen) * 0.04).to(torch.bfloat16)
    sc_u = (torch.rand((F, K // 32), device="cuda", generator=gen) * 0.04).to(torch.bfloat16)
    x = torch.randn((M, K), device="cuda", generator=gen).to(torch.bfloat16)
    gate, up = w4a16.W4Lin(pk_g, sc_g), w4a16.W4Lin(pk_u, sc_u)
    h = w4a16.gate_up_gelu(x, gate, up, out_dtype=torch.float32)
    g = gate.linear(x, out_dtype=torch.float32).double()
    u = up.linear(x, out_dtype=torch.float32).double()
    torch.cuda.synchronize()
    z = math.sqrt(2 / math.pi) * (g + 0.044715 * g ** 3)
    ref = g * torch.sigmoid(2 * z) * u  # 0.5 g (1 + tanh z) without the float cancellation of 1 + tanh z
    tol = (16 + 16 * z.abs()) * EPS * ref.abs() + UNDERFLOW * (1 + u.abs())
    ex = (h.double() - ref).abs() - tol
    excess = ex.max().item()
    if excess > 0:
        bad = (ex > 0).nonzero()
        i, j = (int(v) for v in bad[ex[bad[:, 0], bad[:, 1]].argmax()])
        say(f"{bad.shape[0]} elements over; worst [{i},{j}] g={g[i, j].item()!r} u={u[i, j].item()!r} "
            f"h={h[i, j].item()!r} ref={ref[i, j].item()!r} tol={tol[i, j].item()!r}")
        for r in bad[:8].tolist():
            say(f"  [{r[0]},{r[1]}] g={g[r[0], r[1]].item()!r} u={u[r[0], r[1]].item()!r} "
                f"h={h[r[0], r[1]].item()!r} ref={ref[r[0], r[1]].item()!r}")
    assert excess <= 0, excess


def test_gate_up_gelu_k_zero_and_empty():
    gate = w4a16.W4Lin(torch.zeros((24, 0), dtype=torch.int32, device="cuda"),
                       torch.zeros((24, 0), dtype=torch.bfloat16, device="cuda"))
    up = w4a16.W4Lin(torch.zeros((24, 0), dtype=torch.int32, device="cuda"),
                     torch.zeros((24, 0), dtype=torch.bfloat16, device="cuda"))
    x = torch.zeros((3, 0), dtype=torch.bfloat16, device="cuda")
    h = torch.full((3, 24), 7.0, dtype=torch.float32, device="cuda")
    w4a16.gate_up_gelu(x, gate, up, out=h)
    torch.cuda.synchronize()
    assert torch.count_nonzero(h).item() == 0
    e = w4a16.gate_up_gelu(torch.zeros((0, 0), dtype=torch.bfloat16, device="cuda"), gate, up)
    assert e.shape == (0, 24)


def test_gate_up_gelu_graph_replays_match_eager():
    """Decode shape captured in a HIP graph and replayed with eager work in between."""
    F, K = 2048, 1536
    pk_g, sc_g, pk_u, sc_u = weights(F, K, 4200, 32)
    gate, up = w4lin(pk_g, sc_g, 32), w4lin(pk_u, sc_u, 32)
    x = dev_bf16(o.synth_x(1, K, 4201))
    eager = w4a16.gate_up_gelu(x, gate, up, out_dtype=torch.float32)
    out = torch.empty_like(eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        w4a16.gate_up_gelu(x, gate, up, out=out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        w4a16.gate_up_gelu(x, gate, up, out=out)
    for i in range(4):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = (x.float() * 2).sum().item()  # eager work between replays
