"""Non-vacuity of the GPU parity gates: each gate must be able to fail.

The reference's doctrine is that a gate counts only once it has been shown to reject
a wrong result (docs/superpowers/plans/2026-07-24-w4-j1-brique-e2b.md:121-127); its
counter-tests corrupt the checkpoint -- one packed byte XOR 0xF0
(scripts/57_w4_unpack_fixture.py:44) and a scale multiplied up
(scripts/59_w4_corrupt_ckpt.py:24,31) -- and the corruption targets gate_proj, whose
output passes through gelu, rather than up_proj alone (docs/DOCUMENTATION.md:673-678).

Here the HIP kernels run on corrupted weights while the oracle keeps the clean ones,
and the checks of tests/test_gpu_parity.py (check_f32, check_bf16) and
tests/test_gpu_gate_up.py (the gate/up bound) must raise.  Each case first shows that
the same check passes on the clean weights, so a failure is the corruption's doing.
The corrupted nibble sits where x is largest and flips q by at least 9, so its effect
(|x_k| |dq| s) clears the checks' elementwise bounds; the x100 scale moves a whole
group of 32 weights.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

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
    print(f"[gpu-nonvacuity] {msg}", flush=True)
    sys.stdout.flush()


def corrupt_nibble(pk: np.ndarray, sc: np.ndarray, x: np.ndarray, row: int) -> np.ndarray:
    """XOR 0xF0 on one byte of row `row` (the reference's corruption), at the column
    where the change |x_k| |dq| s is largest among those whose nibble moves by >= 9."""
    q = o.unpack(pk[row:row + 1])[0].astype(np.int64)
    xa = np.abs(o.bf16_to_f32(x[0]).astype(np.float64))
    s = np.repeat(np.abs(o.bf16_to_f32(sc[row]).astype(np.float64)), 32)
    # XOR 0xF0 on a byte flips its high nibble n -> 15 - n, i.e. q -> -1 - q
    cols = np.arange(q.size)
    dq = np.abs(2 * q + 1)
    cand = np.where((cols % 2 == 1) & (dq >= 9))[0]
    k = int(cand[np.argmax((xa * dq * s)[cand])])
    out = pk.copy()
    out[row:row + 1].view(np.uint8)[0, k // 2] ^= 0xF0
    return out


def scale_group(sc: np.ndarray, row: int, g: int, factor: float = 100.0) -> np.ndarray:
    out = sc.copy()
    s = o.bf16_to_f32(out[row, g:g + 1])
    out[row, g] = o.f32_to_bf16(s * np.float32(factor))[0]
    return out


def both_outputs(x, pk, sc):
    from test_gpu_parity import gpu_linear
    return gpu_linear(x, pk, sc, "f32"), gpu_linear(x, pk, sc, "bf16")


@pytest.mark.parametrize("M,K,N", [(1, 3840, 1024), (16, 3840, 1024), (64, 1536, 512)])
@pytest.mark.parametrize("kind", ["nibble", "scale"])
def test_linear_gates_reject_corrupted_weights(M, K, N, kind):
    from test_gpu_parity import check_bf16, check_f32
    say(f"linear M={M} K={K} N={N} corruption={kind}")
    _, pk, sc = o.synth_weights(N, K, 4242)
    x = o.synth_x(M, K, 4243)
    w = o.dequant(pk, sc)
    ref32 = o.matmul_f32(x, w)
    _, mag = o.matmul_f64(x, w)
    y, yb = both_outputs(x, pk, sc)
    check_f32(y, x, w, K, ref32)
    check_bf16(yb, ref32, mag, K)
    row = N // 3
    if kind == "nibble":
        pk_bad, sc_bad = corrupt_nibble(pk, sc, x, row), sc
    else:
        pk_bad, sc_bad = pk, scale_group(sc, row, (K // 32) // 2)
    yc, ycb = both_outputs(x, pk_bad, sc_bad)
    # the corruption shows in its own row only
    assert np.array_equal(np.delete(yc, row, axis=1), np.delete(y, row, axis=1))
    with pytest.raises(AssertionError):
        check_f32(yc, x, w, K, ref32)
    with pytest.raises(AssertionError):
        check_bf16(ycb, ref32, mag, K)


@pytest.mark.parametrize("M,F,K", [(1, 2048, 3840), (4, 1024, 1536), (64, 512, 1536)])
@pytest.mark.parametrize("kind", ["nibble", "scale"])
def test_gate_up_bound_rejects_corrupted_gate(M, F, K, kind):
    from test_gpu_gate_up import check, run_gpu, weights
    say(f"gate/up M={M} F={F} K={K} corruption={kind} (gate_proj)")
    pk_g, sc_g, pk_u, sc_u = weights(F, K, 4300, 32)
    x = o.synth_x(M, K, 4301)
    h = run_gpu(x, pk_g, sc_g, pk_u, sc_u, 32, False, True, False)
    check(h, x, pk_g, sc_g, pk_u, sc_u, K, 32, True, False)
    # a row with g > 1 (gelu' near 1) and the largest |u| at m = 0, so that
    # gelu(g) * u carries the change of g
    g = o.matmul_f32(x, o.dequant(pk_g, sc_g)).astype(np.float64)
    u = o.matmul_f32(x, o.dequant(pk_u, sc_u)).astype(np.float64)
    row = int(np.argmax(np.abs(u[0]) * (g[0] > 1)))
    if kind == "nibble":
        pg_bad, sg_bad = corrupt_nibble(pk_g, sc_g, x, row), sc_g
    else:
        pg_bad, sg_bad = pk_g, scale_group(sc_g, row, (K // 32) // 2)
    hc = run_gpu(x, pg_bad, sg_bad, pk_u, sc_u, 32, False, True, False)
    with pytest.raises(AssertionError):
        check(hc, x, pk_g, sc_g, pk_u, sc_u, K, 32, True, False)
