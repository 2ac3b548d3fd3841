"""MatrixMarket I/O (include/diagpu/mtx.hpp), CPU only: the band writer
matches the reference's gen_banded_mtx output byte for byte and the reader
inverts it (tests/cpp/test_mtx_cpu.cpp, built by __graft_entry__.build())."""
import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "cpp" / "bin" / "test_mtx_cpu"
REF = ROOT / "oracle" / "_ref" / "gen_banded_mtx"


def test_mtx_round_trip(tmp_path):
    if not EXE.exists():   # host-only program: cheap to build here if a build step was skipped
        from diagpu_amd import build
        build.build_cpp_tests()
    args = [str(EXE), str(ROOT / "tests" / "golden" / "gen_banded_n64.mtx"), str(tmp_path)]
    if REF.exists():
        args.append(str(REF))
    proc = subprocess.run(args, capture_output=True, text=True, timeout=60)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ALL TESTS PASSED" in proc.stdout
