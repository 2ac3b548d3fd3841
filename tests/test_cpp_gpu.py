"""Runs the C++ GPU test programs (tests/cpp/*.cpp without the _cpu suffix,
built by __graft_entry__.build()): the reference-named C++ drop-in API over
libdiagpu, checked against the oracle inside the program (test_dia_api), and
the matrix-power / Taylor chain checked against dense float64 products
(test_chain)."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "cpp" / "bin"


@pytest.mark.parametrize("program", ["test_dia_api", "test_chain", "test_krylov"])
def test_cpp_program(dev, program):
    exe = BIN / program
    assert exe.exists(), f"{exe} missing: run __graft_entry__.build() first"
    print(f"running {program}", flush=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ALL TESTS PASSED" in proc.stdout
    assert "[FAIL]" not in proc.stdout
