"""ctypes binding of libw4a16.so (the C ABI in include/w4a16.h).

Host-side mirror of the reference's W4 brick interface
(TheCause/gemma4-zml-probe, zml_runner/w4.zig):

  unpackW4(pk)            w4.zig:33-45   -> int8 q [N, K]
  dequantW4(pk, sc)       w4.zig:47-54   -> bf16 w [N, K]
  W4Lin(pk, sc)           w4.zig:16-31   packed pair; .init(store, name) reads
                                         "<name>.weight_packed" / ".weight_scale";
                                         .toW() dequantizes; .linear(x) is the fused call
  linear(x, pk, sc)       G3.forward, zml_runner/gemma4_w4gate.zig:288-292:
                          y = x . dequantW4(pk, sc)^T with fp32 accumulation
  gate_up_gelu(x, gate, up)  the MLP front half, zml_runner/engine.zig:653:
                          h = gelu_tanh(x . Wg^T) * (x . Wu^T) in one call
  lm_head(x, embed)       the decode head, engine.zig:765-766 + gemma4_g12auto.zig:1532:
                          logits = cap * tanh((x . embed^T) / cap) and their topK

Tensors are torch tensors on the GPU; torch is only the device-memory and
stream plumbing.  Every call goes through libw4a16.so on the current torch
stream.  There is no CPU fallback: without the built library or a GPU the
calls raise.  In the reference a shape/tag mismatch fails the trace at compile
time (w4.zig:116-117); here the library's status code is raised as
W4A16Error before any kernel runs.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(_PKG_DIR, "libw4a16.so")
CSRC = os.path.join(_PKG_DIR, "csrc")

OK, EINVAL_SHAPE, EINVAL_PTR, EINVAL_ARG, EWORKSPACE, EHIP = 0, -1, -2, -3, -4, -5
STATUS_NAMES = {OK: "W4A16_OK", EINVAL_SHAPE: "W4A16_EINVAL_SHAPE", EINVAL_PTR: "W4A16_EINVAL_PTR",
                EINVAL_ARG: "W4A16_EINVAL_ARG", EWORKSPACE: "W4A16_EWORKSPACE", EHIP: "W4A16_EHIP"}
DTYPE_BF16, DTYPE_F32 = 0, 1
GROUP = 32

# Every symbol include/w4a16.h declares.
EXPORTS = ("w4a16_version", "w4a16_last_error", "w4a16_unpack", "w4a16_dequant",
           "w4a16_workspace_size", "w4a16_linear", "w4a16_gate_up_workspace_size",
           "w4a16_gate_up_gelu", "w4a16_lm_head_workspace_size", "w4a16_lm_head", "w4a16_linear_group",
           "w4a16_linear_noalloc")
GATE_UP_BF16_DOTS = 1


class W4A16Error(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


def build(jobs: int = 4) -> str:
    """Compile libw4a16.so for gfx950 in place (make -C csrc)."""
    subprocess.run(["make", "-s", f"-j{jobs}", "-C", CSRC], check=True)
    return LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    """Load libw4a16.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"libw4a16.so not built ({LIB_PATH}); run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        P, I64, I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
        L.w4a16_version.argtypes = []
        L.w4a16_version.restype = ctypes.c_int
        L.w4a16_last_error.argtypes = []
        L.w4a16_last_error.restype = ctypes.c_char_p
        L.w4a16_unpack.argtypes = [P, P, I64, I64, P]
        L.w4a16_unpack.restype = ctypes.c_int
        L.w4a16_dequant.argtypes = [P, P, P, I64, I64, I32, P]
        L.w4a16_dequant.restype = ctypes.c_int
        L.w4a16_workspace_size.argtypes = [I64, I64, I64, I32]
        L.w4a16_workspace_size.restype = ctypes.c_size_t
        L.w4a16_linear.argtypes = [P, I32, P, P, P, I32, I64, I64, I64, I32, I32, P, ctypes.c_size_t, P]
        L.w4a16_linear.restype = ctypes.c_int
        L.w4a16_gate_up_workspace_size.argtypes = [I64, I64, I64, I32]
        L.w4a16_gate_up_workspace_size.restype = ctypes.c_size_t
        L.w4a16_gate_up_gelu.argtypes = [P, I32, P, P, P, P, P, I32, I64, I64, I64, I32, I32, P,
                                         ctypes.c_size_t, P]
        L.w4a16_gate_up_gelu.restype = ctypes.c_int
        L.w4a16_lm_head_workspace_size.argtypes = [I64, I64, I64, I32, I32]
        L.w4a16_lm_head_workspace_size.restype = ctypes.c_size_t
        L.w4a16_lm_head.argtypes = [P, I32, P, P, I64, I64, I64, ctypes.c_float, I32, P, P, P, ctypes.c_size_t, P]
        L.w4a16_lm_head.restype = ctypes.c_int
        L.w4a16_linear_group.argtypes = [P, I32, I32, P, P, P, P, I32, I64, I64, I32, I32, P, ctypes.c_size_t, P]
        L.w4a16_linear_group.restype = ctypes.c_int
        L.w4a16_linear_noalloc.argtypes = [P, I32, P, P, P, I32, I64, I64, I64, I32, I32, P]
        L.w4a16_linear_noalloc.restype = ctypes.c_int
        _lib = L
    return _lib


def check(status: int) -> None:
    if status != OK:
        raise W4A16Error(status, lib().w4a16_last_error().decode())


def version() -> int:
    return int(lib().w4a16_version())


def workspace_size(M: int, N: int, K: int, x_dtype: int = DTYPE_BF16) -> int:
    return int(lib().w4a16_workspace_size(M, N, K, x_dtype))


def gate_up_workspace_size(M: int, F: int, K: int, x_dtype: int = DTYPE_BF16) -> int:
    return int(lib().w4a16_gate_up_workspace_size(M, F, K, x_dtype))


def lm_head_workspace_size(M: int, V: int, K: int, x_dtype: int = DTYPE_BF16, topk: int = 0) -> int:
    return int(lib().w4a16_lm_head_workspace_size(M, V, K, x_dtype, topk))


# ------------------------------------------------------------ torch-facing API

def _torch():
    import torch
    return torch


def _stream_ptr(t) -> int:
    torch = _torch()
    return torch.cuda.current_stream(t.device).cuda_stream


def _dev_check(*ts) -> None:
    for t in ts:
        if not t.is_cuda:
            raise W4A16Error(EINVAL_PTR, "tensor is not on a GPU (libw4a16 has no CPU path)")
        if not t.is_contiguous():
            raise W4A16Error(EINVAL_SHAPE, "tensor must be contiguous (dense row-major)")


def _out_check(out, shape, dtype, device, name):
    """A caller-supplied output: the exact shape and dtype, dense, on pk's GPU."""
    if tuple(out.shape) != tuple(shape) or out.dtype != dtype:
        raise W4A16Error(EINVAL_SHAPE, f"{name} must be {dtype} {tuple(shape)}, got {out.dtype} {tuple(out.shape)}")
    _dev_check(out)
    if out.device != device:
        raise W4A16Error(EINVAL_PTR, f"{name} is on {out.device}, pk on {device}")


def unpackW4(pk, out=None):
    """int32 [N, K/8] -> int8 q [N, K] (w4.zig:33-45).  out: optional int8 [N, K]."""
    torch = _torch()
    _dev_check(pk)
    if pk.dtype != torch.int32 or pk.dim() != 2:
        raise W4A16Error(EINVAL_ARG, "pk must be a 2-D int32 tensor")
    N, W = pk.shape
    if out is None:
        q = torch.empty((N, 8 * W), dtype=torch.int8, device=pk.device)
    else:
        _out_check(out, (N, 8 * W), torch.int8, pk.device, "out")
        q = out
    check(lib().w4a16_unpack(pk.data_ptr(), q.data_ptr(), N, 8 * W, _stream_ptr(pk)))
    return q


def dequantW4(pk, sc, group: int = GROUP, out=None):
    """int32 pk [N, K/8] + bf16 sc [N, K/group] -> bf16 w [N, K] (w4.zig:47-54).
    out: optional bf16 [N, K]."""
    torch = _torch()
    _dev_check(pk, sc)
    if pk.dtype != torch.int32 or sc.dtype != torch.bfloat16 or pk.dim() != 2 or sc.dim() != 2:
        raise W4A16Error(EINVAL_ARG, "pk must be int32 [N, K/8] and sc bf16 [N, K/group]")
    N, W = pk.shape
    K = 8 * W
    if sc.shape[0] != N or sc.shape[1] * group != K:
        raise W4A16Error(EINVAL_SHAPE, f"sc shape {tuple(sc.shape)} does not match pk {tuple(pk.shape)} / group {group}")
    if out is None:
        w = torch.empty((N, K), dtype=torch.bfloat16, device=pk.device)
    else:
        _out_check(out, (N, K), torch.bfloat16, pk.device, "out")
        w = out
    check(lib().w4a16_dequant(pk.data_ptr(), sc.data_ptr(), w.data_ptr(), N, K, group, _stream_ptr(pk)))
    return w


def linear(x, pk, sc, out_dtype=None, group: int = GROUP, out=None, workspace=None):
    """y[..., N] = x[..., K] . dequantW4(pk, sc)^T, fp32 accumulate.

    x: bf16 or f32 [..., K] (leading dims flattened to M rows).  out_dtype
    bf16 (default for bf16 x) or f32 (default for f32 x).  f32 activations
    need workspace; bf16 activations on rows whose one-pass grid cannot fill
    the GPU (12B down at M >= 3, q/k/v/o at M > 16, up to a few hundred rows)
    can use it for the split-K route (allocated here when not given; pass an
    empty tensor to take the one-pass route instead).
    """
    torch = _torch()
    _dev_check(x, pk, sc)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise W4A16Error(EINVAL_ARG, "x must be bf16 or f32")
    N, W = pk.shape
    K = 8 * W
    if x.shape[-1] != K:
        raise W4A16Error(EINVAL_SHAPE, f"x last dim {x.shape[-1]} != K {K}")
    if sc.shape[0] != N or sc.shape[1] * group != K:
        raise W4A16Error(EINVAL_SHAPE, f"sc shape {tuple(sc.shape)} does not match pk {tuple(pk.shape)} / group {group}")
    lead = tuple(x.shape[:-1])
    M = 1
    for d in lead:
        M *= d
    x_dtype = DTYPE_BF16 if x.dtype == torch.bfloat16 else DTYPE_F32
    if out is not None:
        if out_dtype is not None and out_dtype != out.dtype:
            raise W4A16Error(EINVAL_ARG, f"out_dtype {out_dtype} != out.dtype {out.dtype}")
        out_dtype = out.dtype
        _dev_check(out)
        if out.numel() != M * N or out.shape[-1] != N:
            raise W4A16Error(EINVAL_SHAPE, f"out shape {tuple(out.shape)} != {lead + (N,)}")
    elif out_dtype is None:
        out_dtype = x.dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise W4A16Error(EINVAL_ARG, "output must be bf16 or f32")
    y_dtype = DTYPE_BF16 if out_dtype == torch.bfloat16 else DTYPE_F32
    if out is None:
        out = torch.empty(lead + (N,), dtype=out_dtype, device=x.device)
    ws_need = workspace_size(M, N, K, x_dtype)
    ws_ptr, ws_bytes = None, 0
    if ws_need:
        if workspace is None:
            workspace = torch.empty(ws_need, dtype=torch.uint8, device=x.device)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    check(lib().w4a16_linear(x.data_ptr(), x_dtype, pk.data_ptr(), sc.data_ptr(), out.data_ptr(),
                             y_dtype, M, N, K, group, 0, ws_ptr, ws_bytes, _stream_ptr(x)))
    return out


def linear_group(x, lins, out_dtype=None, outs=None, workspace=None):
    """[x . lin.toW()^T for lin in lins]: 1 to 4 linears that read the same x (q, k, v at
    engine.zig:552,571,583), one launch at decode.  Each output equals linear(x, lin);
    above the fused sizes the members take the split-K route with the workspace
    (allocated here when not given; an empty tensor keeps them one-pass)."""
    torch = _torch()
    if not 1 <= len(lins) <= 4:
        raise W4A16Error(EINVAL_ARG, "linear_group takes 1 to 4 linears")
    _dev_check(x, *[t for lin in lins for t in (lin.pk, lin.sc)])
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise W4A16Error(EINVAL_ARG, "x must be bf16 or f32")
    K = lins[0].in_features
    group = lins[0].group
    for lin in lins:
        if lin.in_features != K or lin.group != group:
            raise W4A16Error(EINVAL_SHAPE, "every linear of a group has the same K and group")
        if lin.sc.shape[0] != lin.out_features or lin.sc.shape[1] * group != K:
            raise W4A16Error(EINVAL_SHAPE, f"sc shape {tuple(lin.sc.shape)} does not match pk / group {group}")
    if x.shape[-1] != K:
        raise W4A16Error(EINVAL_SHAPE, f"x last dim {x.shape[-1]} != K {K}")
    lead = tuple(x.shape[:-1])
    M = 1
    for d in lead:
        M *= d
    if out_dtype is None:
        out_dtype = x.dtype if outs is None else outs[0].dtype
    if outs is None:
        outs = [torch.empty(lead + (lin.out_features,), dtype=out_dtype, device=x.device) for lin in lins]
    for o_, lin in zip(outs, lins):
        _dev_check(o_)
        if o_.dtype != out_dtype or o_.numel() != M * lin.out_features:
            raise W4A16Error(EINVAL_SHAPE, "outs must match the linears' [M, N] and one dtype")
    x_dtype = DTYPE_BF16 if x.dtype == torch.bfloat16 else DTYPE_F32
    # f32 x: the x planes (required); bf16 x: the largest member's optional split-K space
    ws_need = max(workspace_size(M, lin.out_features, K, x_dtype) for lin in lins)
    ws_ptr, ws_bytes = None, 0
    if workspace is None and ws_need:
        workspace = torch.empty(ws_need, dtype=torch.uint8, device=x.device)
    if workspace is not None and workspace.numel():
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    n = len(lins)
    arr = lambda vals: (ctypes.c_void_p * n)(*vals)
    Ns = (ctypes.c_int64 * n)(*[lin.out_features for lin in lins])
    check(lib().w4a16_linear_group(x.data_ptr(), x_dtype, n, arr([lin.pk.data_ptr() for lin in lins]),
                                   arr([lin.sc.data_ptr() for lin in lins]), arr([o_.data_ptr() for o_ in outs]), Ns,
                                   DTYPE_BF16 if out_dtype == torch.bfloat16 else DTYPE_F32, M, K, group, 0,
                                   ws_ptr, ws_bytes, _stream_ptr(x)))
    return outs


def gate_up_gelu(x, gate: "W4Lin", up: "W4Lin", out_dtype=None, bf16_dots: bool = False, out=None,
                 workspace=None):
    """h[..., F] = gelu_tanh(x . gate.toW()^T) * (x . up.toW()^T) in one call: the front half
    of the MLP, engine.zig:653 (``dotPrec(xff, gate_proj).gelu().mul(dotPrec(xff, up_proj))``).

    gelu_tanh is ZML's Tensor.gelu (gelu_pytorch_tanh).  x bf16 or f32 [..., K]; out_dtype
    bf16 (default for bf16 x) or f32 (default for f32 x).  bf16_dots rounds both dot
    outputs to bf16 before the activation (dotPrec with fam = bf16).  Shapes no fused
    kernel takes need workspace (allocated here when not given)."""
    torch = _torch()
    _dev_check(x, gate.pk, gate.sc, up.pk, up.sc)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise W4A16Error(EINVAL_ARG, "x must be bf16 or f32")
    if gate.group != up.group:
        raise W4A16Error(EINVAL_ARG, f"gate group {gate.group} != up group {up.group}")
    for w in (gate, up):
        if w.pk.dtype != torch.int32 or w.sc.dtype != torch.bfloat16 or w.pk.dim() != 2 or w.sc.dim() != 2:
            raise W4A16Error(EINVAL_ARG, "pk must be int32 [F, K/8] and sc bf16 [F, K/group]")
    F, K = gate.out_features, gate.in_features
    if (up.out_features, up.in_features) != (F, K):
        raise W4A16Error(EINVAL_SHAPE, f"up [{up.out_features}, {up.in_features}] != gate [{F}, {K}]")
    for w in (gate, up):
        if w.sc.shape[0] != F or w.sc.shape[1] * w.group != K:
            raise W4A16Error(EINVAL_SHAPE, f"sc shape {tuple(w.sc.shape)} does not match [{F}, {K}] / {w.group}")
    if x.shape[-1] != K:
        raise W4A16Error(EINVAL_SHAPE, f"x last dim {x.shape[-1]} != K {K}")
    lead = tuple(x.shape[:-1])
    M = 1
    for d in lead:
        M *= d
    x_dtype = DTYPE_BF16 if x.dtype == torch.bfloat16 else DTYPE_F32
    if out is not None:
        if out_dtype is not None and out_dtype != out.dtype:
            raise W4A16Error(EINVAL_ARG, f"out_dtype {out_dtype} != out.dtype {out.dtype}")
        out_dtype = out.dtype
        _dev_check(out)
        if out.numel() != M * F or out.shape[-1] != F:
            raise W4A16Error(EINVAL_SHAPE, f"out shape {tuple(out.shape)} != {lead + (F,)}")
    elif out_dtype is None:
        out_dtype = x.dtype
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise W4A16Error(EINVAL_ARG, "output must be bf16 or f32")
    h_dtype = DTYPE_BF16 if out_dtype == torch.bfloat16 else DTYPE_F32
    if out is None:
        out = torch.empty(lead + (F,), dtype=out_dtype, device=x.device)
    ws_need = gate_up_workspace_size(M, F, K, x_dtype)
    ws_ptr, ws_bytes = None, 0
    if ws_need:
        if workspace is None:
            workspace = torch.empty(ws_need, dtype=torch.uint8, device=x.device)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    check(lib().w4a16_gate_up_gelu(x.data_ptr(), x_dtype, gate.pk.data_ptr(), gate.sc.data_ptr(), up.pk.data_ptr(),
                                   up.sc.data_ptr(), out.data_ptr(), h_dtype, M, F, K, gate.group,
                                   GATE_UP_BF16_DOTS if bf16_dots else 0, ws_ptr, ws_bytes, _stream_ptr(x)))
    return out


def lm_head(x, embed, softcap: float = 30.0, topk: int = 5, logits=None, workspace=None):
    """The decode head (engine.zig:765-766) and its topK (gemma4_g12auto.zig:1532).

    x bf16 or f32 [..., K]; embed bf16 [V, K] (the tied embedding).  Returns
    (logits f32 [..., V], values f32 [..., topk], indices int32 [..., topk]) with
    logits = softcap * tanh((x . embed^T) / softcap) (softcap = 0: no cap); the top-k are
    descending, equal values in ascending index order.  topk = 0 returns only logits."""
    torch = _torch()
    _dev_check(x, embed)
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise W4A16Error(EINVAL_ARG, "x must be bf16 or f32")
    if embed.dtype != torch.bfloat16 or embed.dim() != 2:
        raise W4A16Error(EINVAL_ARG, "embed must be a 2-D bf16 tensor [V, K]")
    V, K = embed.shape
    if x.shape[-1] != K:
        raise W4A16Error(EINVAL_SHAPE, f"x last dim {x.shape[-1]} != K {K}")
    lead = tuple(x.shape[:-1])
    M = 1
    for d in lead:
        M *= d
    x_dtype = DTYPE_BF16 if x.dtype == torch.bfloat16 else DTYPE_F32
    if logits is None:
        logits = torch.empty(lead + (V,), dtype=torch.float32, device=x.device)
    else:
        _dev_check(logits)
        if logits.dtype != torch.float32 or logits.numel() != M * V:
            raise W4A16Error(EINVAL_SHAPE, f"logits must be f32 with {M * V} elements")
    values = torch.empty(lead + (topk,), dtype=torch.float32, device=x.device) if topk else None
    indices = torch.empty(lead + (topk,), dtype=torch.int32, device=x.device) if topk else None
    ws_need = lm_head_workspace_size(M, V, K, x_dtype, topk)
    ws_ptr, ws_bytes = None, 0
    if ws_need:
        if workspace is None:
            workspace = torch.empty(ws_need, dtype=torch.uint8, device=x.device)
        ws_ptr, ws_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    check(lib().w4a16_lm_head(x.data_ptr(), x_dtype, embed.data_ptr(), logits.data_ptr(), M, V, K,
                              float(softcap), topk, values.data_ptr() if topk else None,
                              indices.data_ptr() if topk else None, ws_ptr, ws_bytes, _stream_ptr(x)))
    return logits, values, indices


class W4Lin:
    """Packed linear weight: the two store tensors of one compressed-tensors
    Linear (zml_runner/w4.zig:16-31).  pk int32 [N, K/8], sc bf16 [N, K/group]."""

    def __init__(self, pk, sc, group: int = GROUP):
        self.pk, self.sc, self.group = pk, sc, group

    @classmethod
    def init(cls, store, name: str, group: int = GROUP, device=None) -> "W4Lin":
        """Read "<name>.weight_packed" / "<name>.weight_scale" from a mapping of
        tensors (e.g. a safetensors file), as W4Lin.init does (w4.zig:20-25);
        "<name>.weight_shape" is ignored, as in the reference."""
        pk, sc = store[name + ".weight_packed"], store[name + ".weight_scale"]
        if device is not None:
            pk, sc = pk.to(device), sc.to(device)
        return cls(pk.contiguous(), sc.contiguous(), group)

    @property
    def out_features(self) -> int:
        return int(self.pk.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.pk.shape[1]) * 8

    def toW(self):
        """Dequantized bf16 weight [N, K] (w4.zig:28-30, without the engine retag)."""
        return dequantW4(self.pk, self.sc, self.group)

    def linear(self, x, out_dtype=None, out=None, workspace=None):
        """x . toW()^T fused in one call (replaces x.dot(lin.toW()) at the engine sites)."""
        return linear(x, self.pk, self.sc, out_dtype=out_dtype, group=self.group, out=out,
                      workspace=workspace)
