"""MatrixMarket files through the GPU path (tests/cpp/test_mtx_gpu.cpp, built
by __graft_entry__.build()): read_mtx_dia -> build_recon ->
launch_tc_spmv_regdirect, and the file's matrix squared by the SpGEMM,
checked against the CPU oracle inside the program.  Files:
  - tests/golden/gen_banded_n64.mtx, the reference gen_banded_mtx output;
  - a transverse-field Ising chain Hamiltonian (12 spins, n = 4096) written by
    scipy in the symmetric MatrixMarket format: the kind of matrix the
    reference targets (diagonals at 0 and +-2^i);
  - the SpMV bench's 9-diagonal band at 2^16 rows, written by write_mtx_band
    and read back."""
import subprocess
from pathlib import Path

import numpy as np
import pytest
import scipy.io
import scipy.sparse as sp

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "cpp" / "bin" / "test_mtx_gpu"


def tfim(L: int, J: float = 1.0, h: float = 0.7) -> sp.coo_matrix:
    """H = -J sum Z_i Z_{i+1} (periodic) - h sum X_i in the computational basis."""
    n = 1 << L
    b = np.arange(n)
    s = 1 - 2 * ((b[:, None] >> np.arange(L)) & 1)          # spins +-1
    diag = -J * (s * np.roll(s, -1, axis=1)).sum(axis=1)
    rows, cols, vals = [b], [b], [diag.astype(np.float64)]
    for i in range(L):
        rows.append(b)
        cols.append(b ^ (1 << i))
        vals.append(np.full(n, -h))
    return sp.coo_matrix((np.concatenate(vals), (np.concatenate(rows), np.concatenate(cols))),
                         shape=(n, n))


def test_mtx_files_on_gpu(dev, tmp_path):
    assert EXE.exists(), f"{EXE} missing: run __graft_entry__.build() first"
    ham = tmp_path / "tfim12.mtx"
    scipy.io.mmwrite(str(ham), tfim(12), symmetry="symmetric")
    assert "symmetric" in ham.read_text().split("\n")[0]
    args = [str(EXE), str(ROOT / "tests" / "golden" / "gen_banded_n64.mtx"), str(ham),
            "--write-band", str(tmp_path / "band65536.mtx"), "65536"]
    print("running test_mtx_gpu", flush=True)
    proc = subprocess.run(args, capture_output=True, text=True, timeout=110)
    print(proc.stdout)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert "ALL TESTS PASSED" in proc.stdout
    assert proc.stdout.count("[OK]") == 3 * 4     # 3 files x (recon, SpMV, plan, values)
