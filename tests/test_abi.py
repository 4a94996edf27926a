"""C-ABI checks that need no GPU: the library loads, exports every function
include/w4a16.h declares, and rejects bad arguments on the host before any
HIP call (the reference fails such calls at graph-compile time,
zml_runner/w4.zig:116-117)."""
from __future__ import annotations

import ctypes
import os
import re

import pytest

from conftest import ROOT

import w4a16

HEADER = os.path.join(ROOT, "include", "w4a16.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(w4a16_[a-z_0-9]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    return w4a16.lib()


def test_exports_every_declared_symbol(L):
    decl = _declared_functions()
    assert decl, "no declarations parsed"
    assert sorted(w4a16.EXPORTS) == decl
    for name in decl:
        assert hasattr(L, name), name


def test_version_matches_header(L):
    m = re.search(r"#define W4A16_ABI_VERSION (\d+)", open(HEADER).read())
    assert L.w4a16_version() == int(m.group(1))


def test_status_codes_match_header():
    text = open(HEADER).read()
    for name, val in (("W4A16_OK", 0), ("W4A16_EINVAL_SHAPE", -1), ("W4A16_EINVAL_PTR", -2),
                      ("W4A16_EINVAL_ARG", -3), ("W4A16_EWORKSPACE", -4), ("W4A16_EHIP", -5)):
        assert re.search(rf"{name} = {val}\b", text), name
        assert w4a16.STATUS_NAMES[val] == name


A = 0x10000          # a 16-byte aligned fake device address (never dereferenced)
MIS = 0x10004        # misaligned


def _lin(L, x=A, xd=0, pk=A, sc=A, y=A, yd=0, M=1, N=16, K=64, group=32, flags=0, ws=None, wsb=0):
    return L.w4a16_linear(x, xd, pk, sc, y, yd, M, N, K, group, flags, ws, wsb, None)


def test_linear_validation(L):
    assert _lin(L, M=-1) == w4a16.EINVAL_SHAPE
    assert _lin(L, K=60) == w4a16.EINVAL_SHAPE            # K % 8
    assert _lin(L, K=80) == w4a16.EINVAL_SHAPE            # K % group
    assert _lin(L, group=16) == w4a16.EINVAL_ARG
    assert _lin(L, group=48) == w4a16.EINVAL_ARG
    assert _lin(L, xd=7) == w4a16.EINVAL_ARG
    assert _lin(L, yd=2) == w4a16.EINVAL_ARG
    assert _lin(L, flags=1) == w4a16.EINVAL_ARG
    assert _lin(L, M=2**31) == w4a16.EINVAL_SHAPE
    assert _lin(L, x=None) == w4a16.EINVAL_PTR
    assert _lin(L, pk=None) == w4a16.EINVAL_PTR
    assert _lin(L, sc=MIS) == w4a16.EINVAL_PTR
    assert _lin(L, y=MIS) == w4a16.EINVAL_PTR
    assert "not 16-byte aligned" in L.w4a16_last_error().decode()
    assert _lin(L, xd=1) == w4a16.EWORKSPACE                # f32 x needs workspace
    assert _lin(L, xd=1, ws=A, wsb=16) == w4a16.EWORKSPACE  # too small
    assert _lin(L, ws=MIS, wsb=1024) == w4a16.EINVAL_PTR
    # empty problems are no-ops and touch nothing (no GPU call is made)
    assert _lin(L, M=0, x=None, pk=None, sc=None, y=None) == 0
    assert _lin(L, N=0, x=None, pk=None, sc=None, y=None) == 0
    assert L.w4a16_last_error().decode() == ""


def test_unpack_dequant_validation(L):
    assert L.w4a16_unpack(A, A, -1, 64, None) == w4a16.EINVAL_SHAPE
    assert L.w4a16_unpack(A, A, 4, 12, None) == w4a16.EINVAL_SHAPE
    assert L.w4a16_unpack(None, A, 4, 64, None) == w4a16.EINVAL_PTR
    assert L.w4a16_unpack(A, MIS, 4, 64, None) == w4a16.EINVAL_PTR
    assert L.w4a16_unpack(None, None, 0, 64, None) == 0
    assert L.w4a16_dequant(A, A, A, 4, 64, 24, None) == w4a16.EINVAL_ARG
    assert L.w4a16_dequant(A, A, A, 4, 96, 64, None) == w4a16.EINVAL_SHAPE
    assert L.w4a16_dequant(A, None, A, 4, 64, 32, None) == w4a16.EINVAL_PTR
    assert L.w4a16_dequant(None, None, None, 0, 64, 32, None) == 0


def gemv_ok(M, K):
    """Decode GEMV: 1 <= M <= 4 with x and the reduction tile in 64 KiB of LDS."""
    return 1 <= M <= 4 and M * K * 2 + 16 * 4 * 16 * 4 <= 65536


def gemv16_ok(M, N, K):
    """16-row GEMV (4 < M <= 16): steps of 256 columns, the fewest steps per wave
    p <= 6 with steps / p <= 16 waves, at most 8 x vectors per thread, x whole in
    160 KB of LDS with the reduction tile, and every tile's re-read of x under
    40 MiB."""
    if not (4 < M <= 16 and K % 256 == 0 and N > 0):
        return False
    steps = K // 256
    nst = next((p for p in range(1, 7) if steps % p == 0 and steps // p <= 16), 0)
    if not nst:
        return False
    waves = steps // nst
    per = -(-(M * K // 8) // (64 * waves))
    xpt = 1
    while xpt < per:
        xpt *= 2
    if xpt > 8 or M * K * 2 + waves * 16 * 16 * 4 > 160 * 1024:
        return False
    return -(-N // 16) * M * K * 2 <= 40 << 20


def splitk_bytes(M, N, K):
    """Optional split-K workspace of a bf16 linear (kq f32 partial planes).  At
    64 < M <= 128, or up to 256 with K <= 8192, with K % 256 == 0: the skinny form
    over 64-row x blocks, kq = the largest divisor q <= 64 of K / 256 with
    ceil(M / 64) * ceil(N / 64) * q <= 256 (none: no split).  Otherwise above M = 64: when the LDS prefill kernel's grid (256 x 128 tiles) is under 240
    workgroups (and N <= 8192 up to M = 128), kq = the largest divisor q <= 16 of
    K / 64 with grid * q <= 256; else
    the largest.  Else taken when N < 16384, K % 64 == 0 and: 16 < M <= 64; or 4 < M <= 16 outside the
    16-row GEMV with K >= 8192 or N < 8192; or M <= 4 outside the decode GEMV
    with K % 256 == 0.  Skinny form (K % 256 == 0): kq = the largest divisor
    q <= 64 of K / 256 with ceil(N / 64) * (x blocks of 16, 32 or 64 rows) * q
    <= 256 (none: no split).  K % 256 != 0 (M > 4): the 32x32 form, the smallest divisor q <= 16 of
    K / 64 with tiles * q >= 240 (tiles of 256 W rows at M > 32, 128 below),
    else the largest."""
    if 64 < M <= 256 and N > 0 and K % 256 == 0 and (M <= 128 or K <= 8192):
        nk = K // 256
        per_part = -(-N // 64) * -(-M // 64)
        fits = [c for c in range(2, min(nk, 64) + 1) if nk % c == 0 and per_part * c <= 256]
        return -(-(fits[-1] * M * N * 4) // 256) * 256 if fits else 0
    if M > 64 and N > 0 and K % 64 == 0:
        # 256 x 128 tiles of the LDS prefill kernel over K parts when its grid is under 240
        grid = -(-N // 128) * -(-M // 256)
        if grid >= 240 or (M <= 128 and N > 8192):
            return 0
        fits = [c for c in range(2, 17) if (K // 64) % c == 0 and grid * c <= 256]
        q = fits[-1] if fits else 0
        return -(-(q * M * N * 4) // 256) * 256 if q else 0
    if not (1 <= M <= 64 and 0 < N < 16384 and K % 64 == 0):
        return 0
    if M <= 4 and (gemv_ok(M, K) or K % 256 != 0):
        return 0
    if 4 < M <= 16 and (gemv16_ok(M, N, K) or (K < 8192 and N >= 8192)):
        return 0
    q = 0
    if K % 256 == 0:
        nk = K // 256
        mt = 1 if M <= 16 else 2 if M <= 32 else 4
        per_part = -(-N // 64) * -(-M // (16 * mt))
        fits = [c for c in range(2, min(nk, 64) + 1) if nk % c == 0 and per_part * c <= 256]
        if not fits:
            return 0  # the one-pass grid already has > 128 workgroups
        q = fits[-1]
    if not q:
        if M <= 4:
            return 0
        tiles = -(-N // (256 if M > 32 else 128))
        steps = K // 64
        divs = [c for c in range(2, 17) if steps % c == 0]
        if not divs:
            return 0
        fill = [c for c in divs if tiles * c >= 240]
        q = fill[0] if fill else divs[-1]
    return -(-(q * M * N * 4) // 256) * 256


def test_workspace_size(L):
    assert L.w4a16_workspace_size(1, 4096, 3840, w4a16.DTYPE_BF16) == 0
    n = L.w4a16_workspace_size(3, 4096, 3840, w4a16.DTYPE_F32)
    assert n >= 6 * 3 * 3840 and n % 256 == 0
    assert L.w4a16_workspace_size(0, 4096, 3840, w4a16.DTYPE_F32) == 0


@pytest.mark.parametrize("M,N,K,expect", [
    (64, 3840, 15360, 4 * 64 * 3840 * 4),   # 12B down: 60 W blocks of 64 rows x 4 parts
    (8, 3840, 15360, 4 * 8 * 3840 * 4),     # M = 8 at K >= 8192: 60 x 4
    (64, 4096, 3840, 3 * 64 * 4096 * 4),    # 12B q: 64 blocks, 3 | 15 chunks
    (64, 2048, 3840, 5 * 64 * 2048 * 4),    # k/v: 32 blocks x 5
    (32, 12288, 1536, 0),                   # E2B gate/up rows at M = 32: 192 blocks one-pass, no skinny part count
    (16, 1536, 6144, 8 * 16 * 1536 * 4),    # E2B down at M = 16: beyond the 16-row GEMV, 24 x 8
    (4, 3840, 15360, 4 * 4 * 3840 * 4),     # M = 4: x beyond the decode GEMV's LDS
    (24, 700, 1152, 604928),                # K % 256 != 0: 32x32 form, 9 parts (9 * 24 * 700 * 4 rounded up to 256)
    (2, 3840, 15360, 0),                    # decode GEMV (x fits its LDS)
    (16, 4096, 3840, 0),                    # 16-row GEMV
    (8, 6144, 1536, 0),                     # 16-row GEMV (E2B gate/up rows)
    (16, 8192, 3840, 0),                    # beyond the 16-row GEMV, N >= 8192 at K < 8192: one-pass skinny
    (64, 30720, 3840, 0),                   # the skinny grid fills the GPU
    (65, 3840, 15360, 2 * 65 * 3840 * 4),   # 64 < M <= 128: skinny form, 60 W blocks x 2 x blocks x 2 parts
    (96, 1536, 6144, 4 * 96 * 1536 * 4),    # E2B down at M = 96: 24 W blocks x 2 x blocks x 4 parts
    (100, 1000, 4160, 5200128),             # K % 256 != 0 above M = 64: LDS prefill form, 8 W blocks x 13 parts (rounded up to 256)
    (256, 3840, 15360, 8 * 256 * 3840 * 4), # M > 128: LDS prefill form, 30 W blocks x 8 parts
    (200, 1000, 4096, 4 * 200 * 1000 * 4),  # skinny form, 16 W blocks x 4 x blocks x 4 parts
    (300, 1000, 4096, 16 * 300 * 1000 * 4), # M > 256: LDS prefill form, 8 W blocks x 2 x blocks x 16 parts
    (256, 1536, 6144, 2 * 256 * 1536 * 4),  # E2B down at M = 256: skinny form, 24 x 4 x 2 parts
    (160, 4096, 3840, 0),                   # no part count fits 192 skinny workgroups: one-pass skinny
    (128, 4096, 3840, 0),                   # q at M = 128: no part count of K / 256 = 15 fits, one-pass skinny
    (2048, 3840, 15360, 0),                 # 240 workgroups one-pass: no split
    (128, 30720, 3840, 0),                  # 240 W blocks
    (128, 12288, 1536, 0),                  # 384 skinny workgroups one-pass
    (128, 8192, 3840, 0),                   # full-layer q at M = 128: one-pass skinny (256 workgroups)
    (64, 3840, 15360 + 32, 0),              # K % 64 != 0
])
def test_workspace_size_splitk(L, M, N, K, expect):
    """bf16 x: the optional split-K workspace (a call with less takes the
    one-pass route); f32 x: the planes, plus above M = 4 the optional room for the
    three planes' results (12 * M * N bytes, rounded up to 256), and no split-K part."""
    assert splitk_bytes(M, N, K) == expect
    assert L.w4a16_workspace_size(M, N, K, w4a16.DTYPE_BF16) == expect
    planes = -(-(6 * M * K) // 256) * 256
    wide = M > 4 or (M >= 2 and 6 * M * K + 4096 > 65536) or K % 256 != 0
    rows = -(-(12 * M * N) // 256) * 256 + splitk_bytes(3 * M, N, K) if wide else 0
    assert L.w4a16_workspace_size(M, N, K, w4a16.DTYPE_F32) == planes + rows


_TUNING_ENV = ("W4A16_GEMV16_XBYTES", "W4A16_GEMV_NST", "W4A16_GEMV_TPW", "W4A16_GEMV16", "W4A16_GEMV_W",
               "W4A16_GEMV_STREAM", "W4A16_SKINNY_MT", "W4A16_SKINNY_NW", "W4A16_PF_WS", "W4A16_PF_KS",
               "W4A16_PF_LDS", "W4A16_SKINNY_MID", "W4A16_SPLITK_SKINNY", "W4A16_SPLITK", "W4A16_PF_KQ",
               "W4A16_PF_SMALL", "W4A16_HEAD_LOOP", "W4A16_HEAD_WG")


def test_dispatch_reads_no_environment():
    """Route and workspace size are functions of (M, N, K, group, dtypes) only: the library
    imports no getenv, and every workspace size is the same in a process where all the
    former tuning variables are set."""
    import subprocess
    import sys
    syms = subprocess.run(["nm", "-D", "--undefined-only", w4a16.LIB_PATH], capture_output=True, text=True,
                          check=True).stdout
    assert not re.search(r"\bgetenv\b|secure_getenv", syms)
    code = ("import sys, json; sys.path.insert(0, %r); import w4a16; L = w4a16.lib(); out = []\n"
            "for M in (1, 3, 4, 8, 16, 17, 32, 64, 65, 96, 128, 160, 256, 300, 1024, 2048):\n"
            "  for N, K in ((3840, 15360), (4096, 3840), (2048, 3840), (30720, 3840), (1536, 6144),\n"
            "               (12288, 1536), (700, 1152), (1000, 4160), (8192, 3840)):\n"
            "    for xd in (0, 1):\n"
            "      out.append(L.w4a16_workspace_size(M, N, K, xd))\n"
            "      out.append(L.w4a16_gate_up_workspace_size(M, N // 2, K, xd))\n"
            "print(json.dumps(out))\n") % os.path.dirname(os.path.dirname(w4a16.__file__))
    clean = {k: v for k, v in os.environ.items() if not k.startswith("W4A16_")}
    runs = []
    for env in (clean, dict(clean, **{k: "1" for k in _TUNING_ENV}),
                dict(clean, **{k: "0" for k in _TUNING_ENV})):
        runs.append(subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                                   check=True).stdout)
    assert runs[0] == runs[1] == runs[2]


def test_python_wrapper_refuses_cpu_tensors():
    import torch
    pk = torch.zeros((16, 8), dtype=torch.int32)
    sc = torch.zeros((16, 2), dtype=torch.bfloat16)
    x = torch.zeros((1, 64), dtype=torch.bfloat16)
    with pytest.raises(w4a16.W4A16Error) as e:
        w4a16.linear(x, pk, sc)
    assert e.value.status == w4a16.EINVAL_PTR
    with pytest.raises(w4a16.W4A16Error):
        w4a16.dequantW4(pk, sc)
    with pytest.raises(w4a16.W4A16Error):
        w4a16.unpackW4(pk)


def test_last_error_is_thread_local(L):
    import threading
    assert _lin(L, M=-1) == w4a16.EINVAL_SHAPE
    seen = {}

    def other():
        seen["msg"] = L.w4a16_last_error().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == ""
    assert "negative dimension" in L.w4a16_last_error().decode()


def _gu(L, x=A, xd=0, pg=A, sg=A, pu=A, su=A, h=A, hd=0, M=1, F=16, K=256, group=32, flags=0, ws=None, wsb=0):
    return L.w4a16_gate_up_gelu(x, xd, pg, sg, pu, su, h, hd, M, F, K, group, flags, ws, wsb, None)


def test_gate_up_gelu_validation(L):
    assert _gu(L, M=-1) == w4a16.EINVAL_SHAPE
    assert _gu(L, K=60) == w4a16.EINVAL_SHAPE
    assert _gu(L, K=96, group=64) == w4a16.EINVAL_SHAPE
    assert _gu(L, F=2**30) == w4a16.EINVAL_SHAPE            # 16 * ceil(F / 8) virtual rows overflow int
    assert _gu(L, group=48) == w4a16.EINVAL_ARG
    assert _gu(L, xd=3) == w4a16.EINVAL_ARG
    assert _gu(L, hd=5) == w4a16.EINVAL_ARG
    assert _gu(L, flags=2) == w4a16.EINVAL_ARG
    for kw in ("x", "pg", "sg", "pu", "su", "h"):
        assert _gu(L, **{kw: None}) == w4a16.EINVAL_PTR, kw
        assert _gu(L, **{kw: MIS}) == w4a16.EINVAL_PTR, kw
    # the unfused route (K % 256 != 0 at M <= 64) needs f32 g and u in the workspace
    assert _gu(L, M=8, K=320) == w4a16.EWORKSPACE
    assert "workspace" in L.w4a16_last_error().decode()
    assert _gu(L, xd=1) == w4a16.EWORKSPACE                  # f32 x: the split
    assert _gu(L, ws=MIS, wsb=1024) == w4a16.EINVAL_PTR
    assert _gu(L, M=0, x=None, pg=None, sg=None, pu=None, su=None, h=None) == 0
    assert _gu(L, F=0, x=None, pg=None, sg=None, pu=None, su=None, h=None) == 0
    assert L.w4a16_last_error().decode() == ""


@pytest.mark.parametrize("M,F,K,xd,fused", [
    (1, 15360, 3840, 0, True),     # 12B decode: straight-line GEMV
    (4, 15360, 3840, 0, True),     # M = 4 at K = 3840: x too large for the GEMV plan -> skinny
    (2, 6144, 1536, 0, True),      # E2B
    (64, 15360, 3840, 0, True),    # skinny
    (2048, 15360, 3840, 0, True),  # prefill
    (300, 130, 192, 0, True),      # prefill, K % 256 != 0
    (8, 40, 320, 0, False),        # K % 256 != 0 at M <= 64
    (2, 24, 96, 0, False),
    (1, 72, 1024, 1, True),        # f32 x in the decode GEMV
    (8, 40, 512, 1, False),        # f32 x above M = 4
    (32, 6144, 1536, 0, True),     # E2B at M = 32: split-K partials over 12288 virtual rows
])
def test_gate_up_workspace_size(L, M, F, K, xd, fused):
    n = L.w4a16_gate_up_workspace_size(M, F, K, xd)
    planes = -(-(6 * M * K) // 256) * 256 if xd == 1 else 0
    extra = splitk_bytes(M, 16 * -(-F // 8), K) if xd == 0 else 0  # over the virtual rows
    assert n % 256 == 0
    if fused:
        assert n == planes + extra
    else:
        assert n >= planes + 8 * M * F
    assert L.w4a16_gate_up_workspace_size(0, F, K, xd) == 0


def _lm(L, x=A, xd=0, e=A, lg=A, M=1, V=1000, K=256, cap=30.0, k=5, tv=A, ti=A, ws=A, wsb=1 << 20):
    return L.w4a16_lm_head(x, xd, e, lg, M, V, K, cap, k, tv, ti, ws, wsb, None)


def test_lm_head_validation(L):
    assert _lm(L, M=-1) == w4a16.EINVAL_SHAPE
    assert _lm(L, K=48) == w4a16.EINVAL_SHAPE              # K % 32
    assert _lm(L, K=8224) == w4a16.EINVAL_SHAPE            # K > 8192: no launch plan (bf16 x: before any HIP call)
    assert _lm(L, xd=2) == w4a16.EINVAL_ARG
    assert _lm(L, cap=-1.0) == w4a16.EINVAL_ARG
    assert _lm(L, cap=float("nan")) == w4a16.EINVAL_ARG
    assert _lm(L, cap=float("inf")) == w4a16.EINVAL_ARG
    assert _lm(L, k=65) == w4a16.EINVAL_ARG
    assert _lm(L, k=-1) == w4a16.EINVAL_ARG
    assert _lm(L, V=3, k=4) == w4a16.EINVAL_ARG           # topk > V
    assert _lm(L, V=4096 * 65, k=64) == w4a16.EINVAL_ARG  # 65 slices * 64 candidates > 4096
    assert _lm(L, lg=None) == w4a16.EINVAL_PTR
    assert _lm(L, tv=MIS) == w4a16.EINVAL_PTR
    assert _lm(L, ti=None) == w4a16.EINVAL_PTR
    assert _lm(L, ws=None, wsb=0) == w4a16.EWORKSPACE      # top-k candidates need workspace
    assert _lm(L, ws=A, wsb=64) == w4a16.EWORKSPACE
    # K == 0 with top-k: the logits are zeros and the top-k still needs its candidates
    # (the check returns before any HIP call)
    assert _lm(L, V=100, K=0, ws=None, wsb=0) == w4a16.EWORKSPACE
    assert _lm(L, M=0, x=None, e=None, lg=None, tv=None, ti=None, ws=None, wsb=0) == 0
    assert L.w4a16_last_error().decode() == ""


def test_lm_head_workspace_size(L):
    assert L.w4a16_lm_head_workspace_size(1, 262144, 3840, w4a16.DTYPE_BF16, 0) == 0
    n = L.w4a16_lm_head_workspace_size(1, 262144, 3840, w4a16.DTYPE_BF16, 5)
    assert n == 10240  # 256 slices of 1024 x 5 candidates x 8 B
    assert L.w4a16_lm_head_workspace_size(1, 262144, 3840, w4a16.DTYPE_BF16, 64) == 64 * 64 * 8  # 4096-slices
    split = L.w4a16_workspace_size(2, 262144, 3840, w4a16.DTYPE_F32)
    assert L.w4a16_lm_head_workspace_size(2, 262144, 3840, w4a16.DTYPE_F32, 5) == split + 20480
    # the candidates do not depend on K (K == 0 included); the x planes do
    assert L.w4a16_lm_head_workspace_size(1, 100, 0, w4a16.DTYPE_BF16, 5) == 256
    assert L.w4a16_lm_head_workspace_size(1, 100, 0, w4a16.DTYPE_F32, 5) == 256
    assert L.w4a16_lm_head_workspace_size(1, 100, 0, w4a16.DTYPE_BF16, 0) == 0


def test_linear_group_validation(L):
    arr = lambda *v: (ctypes.c_void_p * len(v))(*v)
    Ns = (ctypes.c_int64 * 2)(16, 32)

    def grp(n=2, pk=None, sc=None, y=None, N=Ns, M=1, K=64, xd=0, yd=0, flags=0, x=A):
        pk = arr(A, A) if pk is None else pk
        sc = arr(A, A) if sc is None else sc
        y = arr(A, A) if y is None else y
        return L.w4a16_linear_group(x, xd, n, pk, sc, y, N, yd, M, K, 32, flags, None, 0, None)

    assert grp(n=0) == w4a16.EINVAL_ARG
    assert grp(n=5) == w4a16.EINVAL_ARG
    assert L.w4a16_linear_group(A, 0, 2, None, arr(A, A), arr(A, A), Ns, 0, 1, 64, 32, 0, None, 0, None) \
        == w4a16.EINVAL_PTR
    assert grp(N=(ctypes.c_int64 * 2)(16, -1)) == w4a16.EINVAL_SHAPE
    assert grp(K=80) == w4a16.EINVAL_SHAPE
    assert grp(yd=3) == w4a16.EINVAL_ARG
    assert grp(flags=1) == w4a16.EINVAL_ARG
    assert grp(y=arr(A, MIS)) == w4a16.EINVAL_PTR
    assert grp(pk=arr(A, None)) == w4a16.EINVAL_PTR
    assert grp(xd=1) == w4a16.EWORKSPACE
    assert grp(M=0, x=None) == 0
    assert L.w4a16_last_error().decode() == ""
