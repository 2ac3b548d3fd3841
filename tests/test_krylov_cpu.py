"""The host step of the Lanczos propagator, c = exp(-i t T) e_1 for a real
symmetric tridiagonal T (diagpu_amd/csrc/expm_tridiag.hpp, driven through
tests/cpp/test_expm_tridiag_cpu.cpp), against the eigendecomposition of T in
fp64: sub-stepped Taylor for moderate ||t T||, scaling and squaring beyond,
and t up to 1e12 (where a sub-step count would overflow int) answered in
well under a second with a unit-norm result."""
import subprocess
import time
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
EXE = ROOT / "tests" / "cpp" / "bin" / "test_expm_tridiag_cpu"


def run(al, be, t):
    if not EXE.exists():
        from diagpu_amd import build
        build.build_cpp_tests()
    text = (f"{len(al)} {float(t)!r}\n" + " ".join(repr(float(x)) for x in al) + "\n"
            + " ".join(repr(float(x)) for x in be) + "\n")
    t0 = time.perf_counter()
    proc = subprocess.run([str(EXE)], input=text, capture_output=True, text=True, timeout=60)
    dt = time.perf_counter() - t0
    assert proc.returncode == 0, proc.stderr
    if proc.stdout.startswith("NOT FINITE"):
        return None, dt
    v = np.array([[float(x) for x in line.split()] for line in proc.stdout.split("\n") if line])
    return v[:, 0] + 1j * v[:, 1], dt


def eig_ref(al, be, t):
    T = np.diag(al) + np.diag(be, 1) + np.diag(be, -1)
    w, V = np.linalg.eigh(T)
    return V @ (np.exp(-1j * t * w) * V[0, :])


@pytest.mark.parametrize("m,t,tol", [
    (1, 0.7, 1e-14), (2, 3.0, 1e-13), (30, 0.5, 1e-13), (30, 40.0, 1e-12),
    (64, 300.0, 1e-11),       # sub-stepped Taylor: ||t T|| ~ 1e3 < 512 sub-steps
    (64, 2e3, 1e-10),         # scaling and squaring from here on
    (40, 1e6, 1e-7),          # the phases t * lambda carry t * eps * |lambda| of error
])
def test_against_eigendecomposition(m, t, tol):
    rng = np.random.default_rng(m)
    al = rng.uniform(-1, 1, m)
    be = rng.uniform(0.1, 1, m - 1)
    c, _ = run(al, be, t)
    want = eig_ref(al, be, t)
    assert np.abs(c - want).max() <= tol
    assert abs(np.linalg.norm(c) - 1) <= tol


@pytest.mark.parametrize("t", [5e9, 1e12, -3e10])
def test_huge_t_stays_fast_and_unitary(t):
    """||t T|| beyond 2^31 sub-steps: the result is still unit-norm and close
    to the eigendecomposition (up to the t * eps phase error both carry)."""
    m = 12
    rng = np.random.default_rng(3)
    al = rng.uniform(-1, 1, m)
    be = rng.uniform(0.1, 1, m - 1)
    c, dt = run(al, be, t)
    assert dt < 5.0
    # each of the log2 ||t T|| squarings doubles the rounding error: a few
    # t * eps * ||T|| in total, the same order as the phase error
    bound = 1e-8 + 4 * m * abs(t) * 2.2e-16
    assert abs(np.linalg.norm(c) - 1) <= bound
    want = eig_ref(al, be, t)
    assert np.abs(c - want).max() <= bound


def test_not_finite():
    c, _ = run([1.0, float("inf")], [0.5], 1.0)
    assert c is None
