"""Runs the C++ drop-in API test (tests/cpp/test_dia_api.cpp, built by
__graft_entry__.build()) on the GPU: the reference-named C++ functions over
libdiagpu, checked against the oracle inside the program."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "cpp" / "bin" / "test_dia_api"


def test_cpp_drop_in_api(dev):
    assert EXE.exists(), f"{EXE} missing: run __graft_entry__.build() first"
    proc = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ALL TESTS PASSED" in proc.stdout
    assert "[FAIL]" not in proc.stdout
