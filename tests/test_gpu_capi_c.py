"""The C ABI from a plain C program: tests/capi/capi_check (built by __graft_entry__.build()
from tests/capi/capi_check.c) allocates its own device memory with the HIP runtime, calls
rlk_gae (aligned and element-aligned rows), rlk_vtrace and the look-back rlk_prefix_sum
with a workspace it zeroes once and reuses, and checks every result against the float64
CPU oracle (oracle/rlk_oracle.c) at the GPU suite's tolerances.  No Python or torch runs
in that process, so this is the boundary as a C, C++, Go (cgo) or Rust caller sees it."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
EXE = os.path.join(ROOT, "tests", "capi", "capi_check")

pytestmark = pytest.mark.gpu


def test_c_program_matches_the_oracle():
    assert os.path.exists(EXE), "tests/capi/capi_check is not built (run __graft_entry__.build())"
    print(f"running {EXE}", flush=True)
    r = subprocess.run([EXE], capture_output=True, text=True, timeout=100)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "capi_check ok" in r.stdout
