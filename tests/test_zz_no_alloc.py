"""The allocation-free entry point w4a16_linear_noalloc, called through the C ABI:
its output equals w4a16_linear's (given a workspace as large as its static scratch)
bit for bit, on two calls in a row whose second input is smaller, for bf16 x on the
split-K route (partials in the scratch), bf16 x one-pass, and f32 x (x planes in the
scratch).  Sizes beyond the scratch are rejected before any HIP call."""
from __future__ import annotations

import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

import w4a16  # noqa: E402
from oracle import w4a16_oracle as o  # noqa: E402

SCRATCH = 8 << 20


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    w4a16.lib()


def say(msg: str) -> None:
    print(f"[no-alloc] {msg}", flush=True)
    sys.stdout.flush()


def _inputs(M, N, K, x_f32, seed):
    _, pk, sc = o.synth_weights(N, K, seed)
    if x_f32:
        x = torch.from_numpy(np.random.default_rng(seed).standard_normal((M, K), dtype=np.float32)).cuda()
    else:
        x = torch.from_numpy(o.synth_x(M, K, seed).view(np.int16)).view(torch.bfloat16).cuda()
    return x, torch.from_numpy(pk).cuda(), torch.from_numpy(sc.view(np.int16)).view(torch.bfloat16).cuda()


def _call_both(x, pk, sc, M, N, K, out_f32):
    L = w4a16.lib()
    xd = w4a16.DTYPE_F32 if x.dtype == torch.float32 else w4a16.DTYPE_BF16
    yd = w4a16.DTYPE_F32 if out_f32 else w4a16.DTYPE_BF16
    dt = torch.float32 if out_f32 else torch.bfloat16
    st = torch.cuda.current_stream().cuda_stream
    ref = torch.empty((M, N), dtype=dt, device="cuda")
    got = torch.full((M, N), float("nan"), dtype=dt, device="cuda")
    ws = torch.empty(SCRATCH, dtype=torch.uint8, device="cuda")
    w4a16.check(L.w4a16_linear(x.data_ptr(), xd, pk.data_ptr(), sc.data_ptr(), ref.data_ptr(), yd, M, N, K, 32, 0,
                               ws.data_ptr(), SCRATCH, st))
    w4a16.check(L.w4a16_linear_noalloc(x.data_ptr(), xd, pk.data_ptr(), sc.data_ptr(), got.data_ptr(), yd, M, N, K,
                                       32, 0, st))
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("case", [
    # (label, first call (M, N, K), second call, smaller), x f32, out f32
    ("bf16 x, split-K route", (32, 3840, 15360), (8, 2048, 3840), False, True),
    ("bf16 x, decode GEMV", (1, 30720, 3840), (1, 4096, 3840), False, False),
    ("f32 x, planes in scratch", (16, 4096, 3840), (3, 2048, 1536), True, True),
    ("bf16 x, decode GEMV tile loop", (4, 30720, 3840), (3, 20001, 3840), False, False),
])
def test_noalloc_matches_linear(case):
    label, first, second, x_f32, out_f32 = case
    for i, (M, N, K) in enumerate((first, second)):
        say(f"{label}: call {i + 1} M={M} N={N} K={K}")
        if not x_f32:
            sk = w4a16.workspace_size(M, N, K, w4a16.DTYPE_BF16)
            assert sk <= SCRATCH
        x, pk, sc = _inputs(M, N, K, x_f32, 900 + 7 * i)
        ref, got = _call_both(x, pk, sc, M, N, K, out_f32)
        a = ref.view(torch.int32 if out_f32 else torch.int16).cpu().numpy()
        b = got.view(torch.int32 if out_f32 else torch.int16).cpu().numpy()
        assert np.array_equal(a, b), (label, i, int(np.sum(a != b)))


def test_noalloc_rejects_f32_beyond_scratch():
    """6 * M * K bytes of f32-activation planes beyond 8 MiB: W4A16_EWORKSPACE, nothing launched."""
    L = w4a16.lib()
    M, K, N = 128, 15360, 64
    assert 6 * M * K > SCRATCH
    rc = L.w4a16_linear_noalloc(0x10000, w4a16.DTYPE_F32, 0x10000, 0x10000, 0x10000, w4a16.DTYPE_F32, M, N, K, 32, 0,
                                None)
    assert rc == w4a16.EWORKSPACE
    assert "scratch" in L.w4a16_last_error().decode()


def test_noalloc_random_sequence():
    """Sixteen seeded calls in a row with random shapes (M 1-64, ragged N, K up to 8192,
    bf16 or f32 x within the scratch, bf16 or f32 y): each output equals w4a16_linear's
    with an 8 MiB workspace bit for bit, whatever the previous call left in the scratch."""
    rng = np.random.Generator(np.random.PCG64(20261206))
    for i in range(16):
        M = int(rng.integers(1, 65))
        K = 32 * int(rng.integers(1, 257))
        N = int(rng.integers(1, 6001))
        x_f32 = bool(rng.random() < 0.3) and 6 * M * K <= SCRATCH
        out_f32 = bool(rng.random() < 0.5)
        say(f"random call {i}: M={M} N={N} K={K} x_f32={x_f32} out_f32={out_f32}")
        x, pk, sc = _inputs(M, N, K, x_f32, 1000 + i)
        ref, got = _call_both(x, pk, sc, M, N, K, out_f32)
        a = ref.view(torch.int32 if out_f32 else torch.int16).cpu().numpy()
        b = got.view(torch.int32 if out_f32 else torch.int16).cpu().numpy()
        assert np.array_equal(a, b), (i, int(np.sum(a != b)))
