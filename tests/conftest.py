"""Shared pytest setup: the `gpu` marker, import paths and fixture loaders."""
from __future__ import annotations

import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "gemma4-zml-probe_amd")
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libw4a16.so")


def load_fixture(name: str) -> dict:
    """safetensors fixture -> dict of numpy arrays; bf16 tensors as uint16 bit patterns."""
    import torch
    from safetensors.torch import load_file
    out = {}
    for k, t in load_file(os.path.join(GOLDEN, name)).items():
        if t.dtype == torch.bfloat16:
            out[k] = t.view(torch.int16).numpy().view(np.uint16)
        else:
            out[k] = t.numpy()
    return out


def load_manifest() -> dict:
    with open(os.path.join(GOLDEN, "manifest.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def manifest():
    return load_manifest()
