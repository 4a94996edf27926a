"""The CPU suite under AddressSanitizer + UndefinedBehaviorSanitizer (tests/sanitize.sh):
the C ABI's host code, the C++ host mirror (safetensors/JSON parser, census) and the C
oracle, built with -fsanitize=address,undefined in a scratch copy of the tree, run every
`-m "not gpu"` test with halt-on-error; a sanitizer report fails this test."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

from conftest import ROOT


@pytest.mark.skipif(os.environ.get("W4A16_SANITIZER_RUN") == "1", reason="already inside the sanitizer run")
@pytest.mark.skipif(shutil.which("make") is None or not os.path.exists("/opt/rocm/llvm/bin/clang")
                    or not os.path.exists(os.path.join(ROOT, "tests", "sanitize.sh")),
                    reason="needs make, ROCm's clang and tests/sanitize.sh")
def test_cpu_suite_under_asan_ubsan(tmp_path):
    p = subprocess.run(["bash", os.path.join(ROOT, "tests", "sanitize.sh"), str(tmp_path / "tree")],
                       capture_output=True, text=True, timeout=1200)
    tail = (p.stdout + p.stderr)[-4000:]
    assert p.returncode == 0, tail
    assert " passed" in p.stdout and "ERROR: AddressSanitizer" not in tail and "runtime error" not in tail, tail
