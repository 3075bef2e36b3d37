"""The C++ host mirror (include/railgun_hip.hpp) on the GPU: runs the test binary that
railgun_amd/build.py compiles from tests/cpp/test_paged_attention_op.cpp.  It exercises
PagedAttentionOp::execute (v1 and v2 branches, fp32 and bf16, fused pool views),
reshape_and_cache (+ IsoQuant metadata), apply_rope, prefill_packed and the CoreError
variants against host computations (see the .cpp for the tolerances)."""
from __future__ import annotations

import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BINARY = os.path.join(ROOT, "tests", "cpp", "test_paged_attention_op")

pytestmark = pytest.mark.gpu


def test_cpp_host_mirror(device):
    assert os.path.exists(BINARY), "C++ test binary missing: run __graft_entry__.build() first"
    r = subprocess.run([BINARY], capture_output=True, text=True, timeout=110)
    print(r.stdout)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "checks passed" in r.stdout
