#!/usr/bin/env python3
"""Writes the committed golden fixtures for the W4A16 parity tests.

Run from the repository root:  python tests/golden/make_golden.py

The reference's own fixture tensors are gitignored upstream (only their JSON
manifests are committed), and its fixture scripts import compressed-tensors and
read checkpoints that are not available here.  These fixtures are therefore
rebuilt from the reference's recipes with torch and numpy only, independently
of oracle/ (which the tests then check against them):

  w4_unpack.safetensors  -- the W1 gate fixture, recipe of
      scripts/57_w4_unpack_fixture.py:33-44 (same tensor names): two rows of 32
      chosen q values (all 16 nibbles, the bit-31 sign trap, both extremes),
      packed with the published compressed-tensors pack_to_int32 algorithm
      (q + 8, cast to int32, shifted by 4*j, summed over each group of 8),
      dequantized with torch's bf16 multiply (57:41), and a copy with nibble 1
      of row 0 flipped (57:43-44).
  w4_gemm_synth.safetensors -- the W3 gate shape (q_proj L0, K=1536 -> N=2048),
      x from the reference recipe (scripts/58_w4_gemm_oracle.py:23-24:
      manual_seed(1337), randn(1,1,1536) -> bf16); the real q_proj weights are
      not available, so the weights are the synthetic benchmark distribution
      (seed 1001), regenerated at test time and checked by sha256.
      out_expected = x.f32 @ dequant.f32^T with torch (58:29).
  w4_linear_small.safetensors -- small seeded (M, N, K) cases incl. ragged ones,
      expected outputs from torch (dequant via bf16 multiply, fp32 matmul).
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np
import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))


def ct_pack_to_int32(q: torch.Tensor) -> torch.Tensor:
    """Published compressed-tensors pack_to_int32 (num_bits=4, packed_dim=1)."""
    assert q.dtype == torch.int8 and q.shape[1] % 8 == 0
    v = (q.to(torch.int16) + 8).to(torch.uint8)
    rows, cols = v.shape
    r = v.view(rows, cols // 8, 8).to(torch.int64)
    shifts = torch.arange(8, dtype=torch.int64) * 4
    packed = (r << shifts).sum(dim=2)           # < 2**32, exact in int64
    packed = torch.where(packed >= 2**31, packed - 2**32, packed)
    return packed.to(torch.int32)


def ct_unpack_from_int32(pk: torch.Tensor) -> torch.Tensor:
    """Published compressed-tensors unpack_from_int32 (num_bits=4, packed_dim=1)."""
    rows, groups = pk.shape
    out = torch.zeros((rows, groups * 8), dtype=torch.int32)
    for i in range(8):
        out[:, i::8] = (pk >> (4 * i)) & 0xF
    return (out - 8).to(torch.int8)


def torch_dequant(pk: torch.Tensor, sc: torch.Tensor, group: int = 32) -> torch.Tensor:
    """scripts/63_u_dequant_export.py:83-89 restated with the torch unpack above."""
    q = ct_unpack_from_int32(pk)
    n, k = q.shape
    return (q.reshape(n, k // group, group).to(torch.bfloat16) * sc.unsqueeze(-1)).reshape(n, k)


def synth_weights_np(N: int, K: int, seed: int, group: int = 32):
    """Benchmark weight distribution: q ~ U{-8..7}; scale bf16(|N(0,1)| * 0.02)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.integers(-8, 8, size=(N, K), dtype=np.int8)
    s = np.abs(rng.standard_normal((N, K // group), dtype=np.float32)) * np.float32(0.02)
    return torch.from_numpy(q), torch.from_numpy(s).to(torch.bfloat16)


def synth_x_np(M: int, K: int, seed: int) -> torch.Tensor:
    rng = np.random.Generator(np.random.PCG64(seed))
    return torch.from_numpy(rng.standard_normal((M, K), dtype=np.float32)).to(torch.bfloat16)


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


def make_w1() -> dict:
    row0 = torch.tensor(list(range(-8, 8)) + list(range(7, -9, -1)), dtype=torch.int8)
    torch.manual_seed(1337)
    row1 = torch.randint(-8, 8, (32,), dtype=torch.int8)
    row1[7] = 7
    row1[15] = 7
    q = torch.stack([row0, row1])
    packed = ct_pack_to_int32(q)
    scales = torch.tensor([[0.5], [0.033203125]], dtype=torch.bfloat16)
    deq = q.to(torch.bfloat16) * scales
    corrupt = packed.clone()
    corrupt[0, 0] ^= 0x000000F0
    assert torch.equal(ct_unpack_from_int32(packed), q)
    t = {"packed": packed, "scales": scales, "q_expected": q, "deq_expected": deq,
         "packed_corrupt": corrupt}
    save_file({k: v.contiguous() for k, v in t.items()}, os.path.join(HERE, "w4_unpack.safetensors"))
    return {"w4_unpack": {
        "recipe": "scripts/57_w4_unpack_fixture.py:33-44",
        "packed_hex": [[f"{int(v) & 0xffffffff:08x}" for v in r] for r in packed.tolist()],
        "row1": row1.tolist(),
        "pass": "unpack == q_expected (int); dequant == deq_expected (bf16 u16 bit-exact); "
                "packed_corrupt diverges in exactly one element (row 0, column 1)",
    }}


def make_w3() -> dict:
    torch.manual_seed(1337)
    x = torch.randn(1, 1, 1536, dtype=torch.float32).to(torch.bfloat16)
    q, sc = synth_weights_np(2048, 1536, 1001)
    pk = ct_pack_to_int32(q)
    w = torch_dequant(pk, sc)
    out = x.to(torch.float32) @ w.to(torch.float32).t()
    save_file({"x": x.contiguous(), "out_expected": out.contiguous()},
              os.path.join(HERE, "w4_gemm_synth.safetensors"))
    return {"w4_gemm_synth": {
        "recipe": "x: scripts/58_w4_gemm_oracle.py:23-24; out: 58:29 on synthetic weights",
        "weights": {"N": 2048, "K": 1536, "seed": 1001, "generator": "numpy PCG64",
                    "packed_sha256": sha(pk), "scale_sha256": sha(sc)},
        "pass": "max_abs <= 1e-4, mean_abs <= 1e-6, 8 fixed points (zml_runner/gemma4_w4gate.zig:259-260)",
        "fixed_points_out_0_0_0_8": out[0, 0, :8].tolist(),
        "stats": {"max": float(out.max()), "min": float(out.min()), "mean": float(out.mean())},
    }}


SMALL_CASES = [  # (M, N, K, group, seed)
    (1, 64, 256, 32, 11),
    (1, 48, 96, 32, 12),        # K not a multiple of 128, N not a multiple of 64
    (3, 40, 160, 32, 13),       # ragged everywhere
    (16, 32, 128, 32, 14),
    (17, 24, 64, 32, 15),       # M crosses one 16-row tile
    (64, 96, 512, 32, 16),
    (2, 32, 256, 64, 17),       # coarser group
    (2, 16, 512, 128, 18),
]


def make_small() -> dict:
    t = {}
    meta = []
    for i, (M, N, K, g, seed) in enumerate(SMALL_CASES):
        q, sc = synth_weights_np(N, K, seed, g)
        pk = ct_pack_to_int32(q)
        x = synth_x_np(M, K, seed + 100)
        w = torch_dequant(pk, sc, g)
        y = x.to(torch.float32) @ w.to(torch.float32).t()
        t[f"c{i}.packed"], t[f"c{i}.scales"], t[f"c{i}.x"] = pk, sc, x
        t[f"c{i}.deq_expected"], t[f"c{i}.out_expected"] = w, y
        meta.append({"M": M, "N": N, "K": K, "group": g, "seed": seed})
    save_file({k: v.contiguous() for k, v in t.items()}, os.path.join(HERE, "w4_linear_small.safetensors"))
    return {"w4_linear_small": {"cases": meta}}


def main() -> int:
    manifest = {"generator": "tests/golden/make_golden.py", "torch": torch.__version__}
    manifest.update(make_w1())
    manifest.update(make_w3())
    manifest.update(make_small())
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=2)
    print("golden fixtures written to", HERE)
    return 0


if __name__ == "__main__":
    sys.exit(main())
