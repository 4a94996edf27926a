"""The reference's CPU path restated in PyTorch (CPU baseline of bench.py).

TEST / MEASUREMENT INFRASTRUCTURE ONLY: bench.py times it as the reported
``cpu_baseline`` (kind "port"); the product path never calls it.

Restates, per linear and per call (the reference dequantizes every decode
step, docs/W4_RESULTS.md:125-126):
  unpack -> minus 8 -> bf16 -> x scale (bf16)   scripts/57_w4_unpack_fixture.py:84-85,
                                                scripts/63_u_dequant_export.py:83-89
  x.float() @ w.float().T                       scripts/58_w4_gemm_oracle.py:29
"""
from __future__ import annotations

import torch

_SHIFTS = torch.arange(8, dtype=torch.int32) * 4


def dequant(pk: torch.Tensor, sc: torch.Tensor, group: int = 32) -> torch.Tensor:
    """int32 [N, K/8] + bf16 [N, K/group] -> bf16 [N, K]."""
    n, w = pk.shape
    q = ((pk.unsqueeze(-1) >> _SHIFTS) & 0xF).reshape(n, 8 * w) - 8   # & 0xF: logical nibble
    return (q.reshape(n, -1, group).to(torch.bfloat16) * sc.unsqueeze(-1)).reshape(n, 8 * w)


def linear(x: torch.Tensor, pk: torch.Tensor, sc: torch.Tensor, group: int = 32) -> torch.Tensor:
    """y = x.f32 @ dequant(pk, sc).f32^T (f32 [M, N])."""
    return x.to(torch.float32) @ dequant(pk, sc, group).to(torch.float32).t()
