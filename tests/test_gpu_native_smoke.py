"""The native C++ smoke test (tests/native/pkv_smoke.cpp): the reference's eight
smoke_test.cu correctness cases driven through libpkv.so's C ABI by a host-only C++
program, with no Python or torch in the loop.  Built by __graft_entry__.build()."""
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu
BINARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "native", "_build", "pkv_smoke")


def test_native_smoke_binary(gpu):
    if not os.path.exists(BINARY):
        pytest.fail(f"{BINARY} is not built (run __graft_entry__.build())")
    run = subprocess.run([BINARY], capture_output=True, text=True, timeout=120)
    print(run.stdout)
    assert run.returncode == 0, run.stdout + run.stderr
    lines = [ln for ln in run.stdout.splitlines() if ln.startswith("case ")]
    assert len(lines) == 9 and all(ln.endswith("PASS") for ln in lines), run.stdout
