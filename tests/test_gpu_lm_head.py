"""GPU parity of the decode head, w4a16_lm_head (engine.zig:765-766 logits + softcap,
gemma4_g12auto.zig:1532 topK), against the oracle.

Stated tolerance, elementwise, with eps = 2^-24 and gamma_K = K eps / (1 - K eps):
  |logits - softcap(raw64)| <= 2 gamma_K sum_k |x_k e_k| + 4 eps (|raw64| + |logit|) + 2^-140
(softcap is 1-Lipschitz; the rest bounds the fp32 scaling, tanh and final scaling).
Top-k: the GPU's (values, indices) equal the oracle's top-k of the GPU's own logits
bit for bit (same total order: descending, ties by ascending index, NaN above +inf),
and its indices equal the top-k of the float64 logits on every row whose k-th and
(k+1)-th float64 logits differ by more than the logits tolerance.
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


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    w4a16.lib()


def say(msg: str) -> None:
    print(f"[gpu-lm-head] {msg}", flush=True)
    sys.stdout.flush()


def dev_bf16(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).cuda()


def synth_embed(V, K, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    return o.f32_to_bf16((rng.standard_normal((V, K), dtype=np.float32) * np.float32(0.05)))


def run(x, e_dev, cap, k):
    xt = torch.from_numpy(x).cuda() if x.dtype == np.float32 else dev_bf16(x)
    logits, vals, idx = w4a16.lm_head(xt, e_dev, softcap=cap, topk=k)
    torch.cuda.synchronize()
    return (logits.cpu().numpy(), vals.cpu().numpy() if k else None, idx.cpu().numpy() if k else None)


def check(x, e, lg, vals, idx, K, cap, k):
    ref, raw, mag = o.lm_head(x, e, cap)
    gam = K * EPS / (1 - K * EPS)
    tol = 2 * gam * mag + 4 * EPS * (np.abs(raw) + np.abs(ref)) + 2.0 ** -140
    err = np.abs(lg.astype(np.float64) - ref)
    assert np.all(err <= tol), float(np.max(err - tol))
    if not k:
        return
    ov, oi = o.topk(lg, k)
    assert np.array_equal(oi, idx), (oi[:, :8], idx[:, :8])
    assert np.array_equal(ov.view(np.uint32), vals.view(np.uint32))
    # against the float64 ranking on decisive rows
    srt = np.sort(ref, axis=1)[:, ::-1]
    margin = srt[:, k - 1] - srt[:, k] if ref.shape[1] > k else np.full(ref.shape[0], np.inf)
    decisive = margin > 2 * np.max(tol, axis=1)
    ref_idx = np.argsort(-ref, axis=1, kind="stable")[:, :k]
    assert np.array_equal(np.sort(idx[decisive], axis=1), np.sort(ref_idx[decisive], axis=1))


# (M, V, K, x f32, softcap, topk)
CASES = [
    (1, 1000, 256, False, 30.0, 5),
    (3, 4097, 512, True, 30.0, 8),      # two top-k slices, f32 x
    (4, 333, 64, False, 0.0, 1),        # no softcap, argmax
    (2, 9000, 1536, True, 30.0, 64),    # three slices, the largest k
    (3, 2000, 3840, True, 30.0, 5),     # f32 x at K = 3840: rows in chunks of 2
    (6, 1500, 3840, False, 30.0, 5),    # bf16 x, rows in chunks of 4
    (1, 777, 1536, False, 30.0, 0),     # logits only
    (1, 262144, 256, False, 30.0, 64),  # 64 candidates from 4096-logit slices
    (16, 3000, 3840, False, 30.0, 5),   # one launch of 16 rows (16-row epilogue, 138 KB of LDS)
    (11, 777, 1536, False, 0.0, 3),     # 11 rows in one launch, no softcap
    (20, 600, 3840, False, 30.0, 4),    # 16 + 4 rows: the 16-row and the 4-row forms
    (7, 900, 3840, True, 30.0, 5),      # f32 x: chunks of 5 + 2 rows
]


@pytest.mark.parametrize("M,V,K,x_f32,cap,k", CASES)
def test_lm_head_vs_oracle(M, V, K, x_f32, cap, k):
    say(f"lm_head M={M} V={V} K={K} x_f32={x_f32} cap={cap} k={k}")
    e = synth_embed(V, K, 5000 + V)
    x = o.synth_x(M, K, 5100 + M)
    if x_f32:
        x = (o.bf16_to_f32(x) * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)
    lg, vals, idx = run(x, dev_bf16(e), cap, k)
    check(x, e, lg, vals, idx, K, cap, k)


def _random_head_cases(n=24, seed=20261205):
    """Seeded heads: M 1-24, V ragged up to 40000, K a multiple of 32 up to 4096, bf16 or
    f32 x, softcap 30 or none, top-k 0-64."""
    rng = np.random.Generator(np.random.PCG64(seed))
    cases = []
    for i in range(n):
        M = int(rng.integers(1, 25))
        V = int(rng.integers(1, 40001))
        K = 32 * int(rng.integers(1, 129))
        while M * V * K > 1_500_000_000:
            V = max(1, V // 2)
        x_f32 = bool(rng.random() < 0.3)
        cap = 30.0 if rng.random() < 0.7 else 0.0
        k = int(rng.choice([0, 1, 2, 5, 8, 17, 64]))
        cases.append((i, M, V, K, x_f32, cap, min(k, V)))
    return cases


@pytest.mark.parametrize("i,M,V,K,x_f32,cap,k", _random_head_cases())
def test_lm_head_random_shapes(i, M, V, K, x_f32, cap, k):
    """Seeded random heads against the oracle at the stated tolerance; top-k bit-equal
    to the oracle's top-k of the GPU logits and to the float64 ranking on decisive rows."""
    say(f"random lm_head {i}: M={M} V={V} K={K} x_f32={x_f32} cap={cap} k={k}")
    e = synth_embed(V, K, 6000 + i)
    x = o.synth_x(M, K, 6100 + i)
    if x_f32:
        x = (o.bf16_to_f32(x) * np.float32(1.0 + 2.0 ** -10)).astype(np.float32)
    lg, vals, idx = run(x, dev_bf16(e), cap, k)
    check(x, e, lg, vals, idx, K, cap, k)


def test_lm_head_12b_vocab():
    """The 12B head: V = 262144, K = 3840 (a 2 GB bf16 embedding), M = 1, top-5."""
    V, K = 262144, 3840
    say(f"lm_head 12B V={V} K={K}")
    gen = torch.Generator(device="cuda").manual_seed(11)
    e_dev = (torch.randn((V, K), device="cuda", generator=gen) * 0.05).to(torch.bfloat16)
    x = o.synth_x(1, K, 5200)
    lg, vals, idx = run(x, e_dev, 30.0, 5)
    e = e_dev.view(torch.int16).cpu().numpy().view(np.uint16)
    del e_dev
    torch.cuda.empty_cache()
    check(x, e, lg, vals, idx, K, 30.0, 5)


def test_lm_head_ties_and_nan():
    """Duplicate embedding rows give bit-equal logits: the smaller index ranks first.
    A NaN row ranks above every finite logit."""
    V, K = 600, 64
    e = synth_embed(V // 2, K, 5300)
    e = np.repeat(e, 2, axis=0)                  # rows 2j and 2j+1 equal
    e[100:102] = 0x7FC0                          # a NaN pair of rows
    x = o.synth_x(1, K, 5301)
    lg, vals, idx = run(x, dev_bf16(e), 30.0, 12)
    assert lg[0, 100:102].view(np.uint32).tolist() == [0x7FC00000] * 2 and idx[0, :2].tolist() == [100, 101]
    pairs = idx[0, 2:].reshape(5, 2)
    assert np.all(pairs[:, 1] == pairs[:, 0] + 1) and np.all(pairs[:, 0] % 2 == 0)
    ov, oi = o.topk(lg, 12)
    assert np.array_equal(oi, idx)


def test_lm_head_k_zero_and_empty():
    e = dev_bf16(synth_embed(40, 32, 5400))
    x = torch.zeros((2, 0), dtype=torch.bfloat16, device="cuda")
    lg, v, i = w4a16.lm_head(torch.zeros((2, 32), dtype=torch.bfloat16, device="cuda"), e, topk=3)
    torch.cuda.synchronize()
    assert torch.count_nonzero(lg).item() == 0 and sorted(i[0].tolist()) == [0, 1, 2]
    lg0, v0, i0 = w4a16.lm_head(torch.zeros((0, 32), dtype=torch.bfloat16, device="cuda"), e, topk=3)
    assert lg0.shape == (0, 40) and v0.shape == (0, 3)
    del x
