"""The grouped pair schedule of include/diagpu/schedule.hpp (build_schedule
and schedule_from_plan) against the oracle's restatement of
spmspm/bench_spmspm.cu:137-243, on the CPU (tests/cpp/test_schedule_cpu.cpp,
built by __graft_entry__.build()).  The oracle itself is pinned to the
reference planner's own output in tests/test_oracle.py."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "cpp" / "bin" / "test_schedule_cpu"


def test_schedule_header_matches_oracle():
    if not EXE.exists():   # host-only program: cheap to build here if a build step was skipped
        from diagpu_amd import build
        build.build_cpp_tests()
    proc = subprocess.run([str(EXE)], capture_output=True, text=True, timeout=120)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ALL TESTS PASSED" in proc.stdout and "[FAIL]" not in proc.stdout
