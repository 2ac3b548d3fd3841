"""Pins the CPU oracle (oracle/dia_oracle.c) -- CPU only.

Each restated function is checked against something other than itself:
the reference's own known-answer output (tests/golden, produced by the
reference programs built from its sources), the reference programs run
live where oracle/_ref is built, scipy's independent DIA definition, dense
numpy products, closed forms, and a second traversal of the same algebra.
"""
import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"
REF = Path(__file__).resolve().parents[1] / "oracle" / "_ref"

TC_CASES = [  # spmv/test/test_tc_spmv.cu:168-179
    ("tridiagonal", 48, [-1, 0, 1]),
    ("tridiag ragged", 37, [-1, 0, 1]),
    ("pentadiagonal", 64, [-2, -1, 0, 1, 2]),
    ("9-diag wide band", 80, [-9, -5, -2, -1, 0, 1, 2, 5, 9]),
    ("asymmetric band", 71, [-3, 0, 2, 4, 7]),
    ("main diagonal", 16, [0]),
]


def hm_to_dense(n, offs, starts, vals):
    """hm_to_dense of spmspm/paper_hm.cuh:68-83 (real or complex values)."""
    D = np.zeros((n, n), dtype=np.result_type(np.asarray(vals).dtype, np.float64))
    for d, s in zip(offs, starts):
        sr, sc = (0, d) if d >= 0 else (-d, 0)
        for p in range(n - abs(d)):
            D[sr + p, sc + p] = vals[s + p]
    return D


def hm_random_np(n, offs, rng):
    offs = sorted(set(int(d) for d in offs))
    lens = [n - abs(d) for d in offs]
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    vals = rng.uniform(-1, 1, size=sum(lens)).astype(np.float32)
    return (np.array(offs, np.int32), np.array(lens, np.int32), starts, vals)


# ---------------------------------------------------------------- SpMV ----

def test_known_answer_5x5(oracle):
    kat = json.loads((GOLDEN / "reconstruct_kat.json").read_text())
    H = np.array(kat["H"], dtype=np.float32)
    x = np.array(kat["x"], dtype=np.float32)
    offs, starts, lens, vals = oracle.dense_to_dia(H)
    assert offs.tolist() == kat["dia_offsets"]
    r_off, r_val = oracle.build_recon(5, 5, offs, starts, lens, vals)
    assert r_off.tolist() == kat["recon_offsets"]
    assert r_val.reshape(5, 5).tolist() == kat["recon_rows"]
    y = oracle.spmv_recon_f32(5, 5, r_off, r_val, x)
    assert y.tolist() == kat["y"]
    assert np.array_equal(oracle.recon_to_dense(5, 5, r_off, r_val), H)
    assert kat["checks"] == ["OK", "OK"]


@pytest.mark.skipif(not (REF / "test_reconstruct").exists(), reason="oracle/_ref not built")
def test_known_answer_live_reference():
    """The reference program, built from its sources, still prints the fixture."""
    import sys
    sys.path.insert(0, str(GOLDEN))
    from make_golden import parse_reconstruct
    live = parse_reconstruct(subprocess.run([str(REF / "test_reconstruct")], capture_output=True,
                                            text=True, check=True).stdout)
    kat = json.loads((GOLDEN / "reconstruct_kat.json").read_text())
    for key in ("H", "x", "dia_offsets", "recon_offsets", "recon_rows", "y", "checks"):
        assert live[key] == kat[key], key


def _parse_mtx(path):
    lines = [ln for ln in Path(path).read_text().splitlines() if not ln.startswith("%")]
    rows, cols, nnz = map(int, lines[0].split())
    ents = [ln.split() for ln in lines[1:]]
    assert len(ents) == nnz
    return rows, ents


def test_hash_band_matches_reference_mtx(oracle):
    """hval of bench_cusparse.cu:70-76 vs gen_banded_mtx's printed values."""
    N, ents = _parse_mtx(GOLDEN / "gen_banded_n64.mtx")
    assert N == 64
    for r, c, v in ents:
        r, c = int(r) - 1, int(c) - 1
        assert "%.7g" % oracle.hval(r, c - r) == v
    # the Recon built from the same hash holds those values at [k][c]
    offs = [-9, -5, -2, -1, 0, 1, 2, 5, 9]
    r_off, r_val, x = oracle.hash_band_recon(N, offs)
    assert r_off.tolist() == sorted(offs, reverse=True)
    R = r_val.reshape(len(offs), N)
    k_of = {d: k for k, d in enumerate(r_off.tolist())}
    for r, c, v in ents:
        r, c = int(r) - 1, int(c) - 1
        assert "%.7g" % R[k_of[c - r], c] == v
    assert np.count_nonzero(R) <= len(ents)


@pytest.mark.skipif(not (REF / "gen_banded_mtx").exists(), reason="oracle/_ref not built")
def test_hash_band_live_reference(tmp_path, oracle):
    out = tmp_path / "b.mtx"
    subprocess.run([str(REF / "gen_banded_mtx"), "200", str(out)], check=True,
                   capture_output=True)
    N, ents = _parse_mtx(out)
    for r, c, v in ents:
        r, c = int(r) - 1, int(c) - 1
        assert "%.7g" % oracle.hval(r, c - r) == v


@pytest.mark.parametrize("name,N,offsets", TC_CASES)
def test_tc_cases_against_dense_and_scipy(oracle, name, N, offsets):
    import scipy.sparse as sp
    H, x = oracle.tc_spmv_case(N, offsets)
    offs, starts, lens, vals = oracle.dense_to_dia(H)
    assert sorted(offs.tolist()) == sorted(o for o in offsets if abs(o) < N)
    r_off, r_val = oracle.build_recon(N, N, offs, starts, lens, vals)
    # scipy.sparse.dia_matrix stores data[k][j] = A[j - off_k, j]: the Recon layout.
    S = sp.dia_matrix((r_val.reshape(len(r_off), N), r_off), shape=(N, N)).toarray()
    assert np.array_equal(S, H)
    y_dense = H.astype(np.float64) @ x.astype(np.float64)
    y64, absum = oracle.spmv_recon_ref64(N, N, r_off, r_val, x)
    assert np.allclose(y64, y_dense, rtol=0, atol=1e-12)
    y32 = oracle.spmv_recon_f32(N, N, r_off, r_val, x)
    assert np.all(np.abs(y32 - y64) <= 1e-6 * absum + 1e-30)
    assert np.array_equal(oracle.recon_to_dense(N, N, r_off, r_val), H)
    # fp64 build_recon (orc_build_recon_f64): the same scatter on fp64 data
    # with bits below fp32 resolution, against scipy's layout of the same H
    v64 = vals.astype(np.float64) * (1 + 2.0 ** -40)
    r_off64, r_val64 = oracle.build_recon(N, N, offs, starts, lens, v64)
    assert r_val64.dtype == np.float64 and np.array_equal(r_off64, r_off)
    S64 = sp.dia_matrix((r_val64.reshape(len(r_off), N), r_off), shape=(N, N)).toarray()
    assert np.array_equal(S64, H.astype(np.float64) * (1 + 2.0 ** -40))


def test_spmv_poisson_closed_form(oracle):
    """5-point stencil, x = 1: y = number of grid neighbours missing."""
    import torch
    from diagpu_amd.workloads import recon_poisson5
    side = 8
    R = recon_poisson5(side, seed=0, device="cpu")
    n = side * side
    y, _ = oracle.spmv_recon_ref64(n, n, R.offsets.numpy(), R.values.numpy(), np.ones(n, np.float32))
    i, j = np.divmod(np.arange(n), side)
    missing = (i == 0).astype(int) + (i == side - 1) + (j == 0) + (j == side - 1)
    assert np.array_equal(y, missing.astype(np.float64))
    assert torch.count_nonzero(R.values).item() == 5 * n - 4 * side


def _recon_f64_case(rows, cols, offsets, seed):
    """fp64 Recon values with full 53-bit mantissas (not fp32-representable),
    NaN in every padding slot (column c of diagonal d with row c - d outside
    [0, rows)), the dense matrix scipy's dia_matrix builds from the in-range
    slots, and an fp64 x."""
    import scipy.sparse as sp
    rng = np.random.default_rng(seed)
    K = len(offsets)
    vals = rng.uniform(-1, 1, (K, cols)) + rng.uniform(-1, 1, (K, cols)) * 2.0 ** -30
    c = np.arange(cols)
    for k, d in enumerate(offsets):
        vals[k, (c - d < 0) | (c - d >= rows)] = np.nan
    D = sp.dia_matrix((np.nan_to_num(vals, nan=0.0), offsets), shape=(rows, cols)).toarray()
    x = rng.standard_normal(cols) + rng.standard_normal(cols) * 2.0 ** -29
    return vals.reshape(-1), D, x


F64_CASES = [(n, n, offs) for _, n, offs in TC_CASES] + [
    (31, 45, [-30, -1, 0, 5, 44]), (50, 20, [-49, -6, 0, 1, 19]), (64, 64, [-70, 0, 3, 80])]


@pytest.mark.parametrize("rows,cols,offsets", F64_CASES)
def test_spmv_f64_vs_dense_and_scipy(oracle, rows, cols, offsets):
    """orc_spmv_recon_f64, the fp64 checker of the GPU's fp64 SpMV, against
    the dense fp64 product of scipy's dia_matrix (the column-indexed Recon
    convention of spmv/src/dia_reconstruct.cuh:9-27), summing exactly the
    in-range terms of spmv/test/test_reconstruct.cpp:122-138 (NaN padding
    must never be read); abs_sum against |D| |x|; x shorter than cols drops
    the columns past its end."""
    import scipy.sparse as sp
    vals, D, x = _recon_f64_case(rows, cols, offsets, rows * 131 + cols)
    y, absum = oracle.spmv_recon_ref64(rows, cols, offsets, vals, x)
    assert y.dtype == np.float64 and np.all(np.isfinite(y))
    want = D @ x
    bound = np.abs(D) @ np.abs(x)
    assert np.all(np.abs(y - want) <= 1e-14 * bound + 1e-300)
    assert np.allclose(absum, bound, rtol=1e-13, atol=0)
    S = sp.dia_matrix((np.nan_to_num(vals.reshape(len(offsets), cols)), offsets), shape=(rows, cols))
    assert np.all(np.abs(y - S @ x) <= 1e-14 * bound + 1e-300)
    # a value below fp32 resolution reaches y: fp64 arithmetic throughout
    y32, _ = oracle.spmv_recon_ref64(rows, cols, offsets, vals.astype(np.float32), x.astype(np.float32))
    if np.any(D != 0):
        assert not np.array_equal(y, y32)
    # x of length cols - 3: columns >= cols - 3 contribute nothing
    m = max(cols - 3, 0)
    y_short, _ = oracle.spmv_recon_ref64(rows, cols, offsets, vals, x[:m].copy())
    assert np.all(np.abs(y_short - D[:, :m] @ x[:m]) <= 1e-14 * bound + 1e-300)


def test_spmv_f64_poisson_closed_form(oracle):
    """5-point stencil in fp64: x = 1 gives the count of missing grid
    neighbours exactly; x = i (the row's grid column index) gives 4j - the
    present horizontal neighbours' columns - 2j for the vertical ones."""
    from diagpu_amd.workloads import recon_poisson5
    side = 16
    R = recon_poisson5(side, seed=0, device="cpu")
    n = side * side
    off = R.offsets.numpy()
    v64 = R.values.numpy().astype(np.float64)
    y, _ = oracle.spmv_recon_ref64(n, n, off, v64, np.ones(n))
    i, j = np.divmod(np.arange(n), side)
    missing = (i == 0).astype(int) + (i == side - 1) + (j == 0) + (j == side - 1)
    assert np.array_equal(y, missing.astype(np.float64))
    # x = grid column j: y = 4j - (j-1)[j>0] - (j+1)[j<side-1] - j[i>0] - j[i<side-1]
    y2, _ = oracle.spmv_recon_ref64(n, n, off, v64, j.astype(np.float64))
    want = (4 * j - np.where(j > 0, j - 1, 0) - np.where(j < side - 1, j + 1, 0)
            - np.where(i > 0, j, 0) - np.where(i < side - 1, j, 0))
    assert np.array_equal(y2, want.astype(np.float64))


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("rows,cols,offsets", [(80, 80, [-9, -5, -2, -1, 0, 1, 2, 5, 9]),
                                              (50, 20, [-49, -6, 0, 1, 19]),
                                              (4099, 4099, [-2048, -1, 0, 1, 2048])])
def test_spmv_omp_baseline_vs_dense(oracle, dtype, rows, cols, offsets):
    """The OpenMP CPU baselines (orc_spmv_recon_omp_f32/_f64) compute every
    row of y: compared with the dense product (accumulation in the element
    type, so the bound scales with its epsilon)."""
    vals, D, x = _recon_f64_case(rows, cols, offsets, rows + 7 * cols)
    vals = np.nan_to_num(vals).astype(dtype)
    x = x.astype(dtype)
    D = D.astype(dtype).astype(np.float64)
    y = np.full(rows, np.nan, dtype=dtype)
    threads = oracle.spmv_recon_omp(rows, cols, np.array(offsets, np.int32), vals, x, y)
    assert threads >= 1
    want = D @ x.astype(np.float64)
    bound = np.abs(D) @ np.abs(x.astype(np.float64))
    eps = np.finfo(dtype).eps
    assert np.all(np.abs(y.astype(np.float64) - want) <= 2 * len(offsets) * eps * bound + 1e-300)


def test_spmv_main_diagonal_and_out_of_range(oracle):
    rng = np.random.default_rng(1)
    n = 33
    d = rng.standard_normal(n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    y = oracle.spmv_recon_f32(n, n, [0], d, x)
    assert np.array_equal(y, d * x)
    # offsets with |d| >= cols contribute nothing
    y2 = oracle.spmv_recon_f32(n, n, [n, 0, -n - 5], np.concatenate([d, d, d]), x)
    assert np.array_equal(y2, d * x)


@pytest.mark.parametrize("rows,cols,offsets", [(40, 40, [-3, 0, 2, 7]), (31, 45, [-30, -1, 0, 5, 44]),
                                              (50, 20, [-49, -6, 0, 1, 19, 25])])
def test_complex_spmv_vs_dense_and_scipy(oracle, rows, cols, offsets):
    """Complex Recon SpMV (no reference counterpart): scipy's dia_matrix with
    complex data gives the dense matrix, whose complex128 product the oracle
    must match; a real matrix applied to a complex x must equal the real
    oracle applied to each part."""
    import scipy.sparse as sp
    rng = np.random.default_rng(rows * cols)
    K = len(offsets)
    vals = (rng.uniform(-1, 1, (K, cols)) + 1j * rng.uniform(-1, 1, (K, cols))).astype(np.complex64)
    x = (rng.standard_normal(cols) + 1j * rng.standard_normal(cols)).astype(np.complex64)
    D = sp.dia_matrix((vals, offsets), shape=(rows, cols)).toarray().astype(np.complex128)
    y, absum = oracle.spmv_recon_complex_ref(rows, cols, offsets, vals.reshape(-1), x)
    want = D @ x.astype(np.complex128)
    assert np.allclose(y, want, rtol=0, atol=1e-12)
    ax = np.abs(x.real.astype(np.float64)) + np.abs(x.imag.astype(np.float64))
    dense_abs = np.abs(D.real) @ ax + np.abs(D.imag) @ ax
    assert np.allclose(absum, dense_abs, rtol=1e-12, atol=1e-12)
    # real values, complex x: linearity over the two parts
    rv = vals.real.copy()
    yr, _ = oracle.spmv_recon_complex_ref(rows, cols, offsets, rv.reshape(-1), x)
    p_re, _ = oracle.spmv_recon_ref64(rows, cols, offsets, rv.reshape(-1), x.real.copy())
    p_im, _ = oracle.spmv_recon_ref64(rows, cols, offsets, rv.reshape(-1), x.imag.copy())
    assert np.array_equal(yr.real, p_re) and np.array_equal(yr.imag, p_im)
    # a planted conjugation or swapped part would be caught here
    assert not np.allclose(y, np.conj(D) @ x.astype(np.complex128), atol=1e-6)


# --------------------------------------------------------- SpGEMM plan ----

@pytest.mark.parametrize("seed", range(6))
def test_c_structure_vs_brute_force(oracle, seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(8, 60))
    oa = rng.choice(np.arange(-n + 1, n), size=int(rng.integers(1, 8)), replace=False)
    ob = rng.choice(np.arange(-n + 1, n), size=int(rng.integers(1, 8)), replace=False)
    c_off, c_len, c_st, nnz = oracle.c_structure(n, oa, ob)
    want = sorted({int(a + b) for a in oa for b in ob if abs(a + b) < n})
    assert c_off.tolist() == want
    assert c_len.tolist() == [n - abs(d) for d in want]
    assert c_st.tolist() == np.concatenate([[0], np.cumsum(c_len)[:-1]]).tolist()
    assert nnz == int(c_len.sum())
    # the structural diagonal set of the dense product (random non-zero values)
    A = hm_random_np(n, oa, rng)
    B = hm_random_np(n, ob, rng)
    P = hm_to_dense(n, A[0], A[2], A[3]) @ hm_to_dense(n, B[0], B[2], B[3])
    r, c = np.nonzero(P)
    assert sorted(set((c - r).tolist())) == want
    lk = oracle.c_lookup(n, c_off)
    for k, d in enumerate(want):
        assert lk[d + n - 1] == k
    assert int((lk >= 0).sum()) == len(want)


@pytest.mark.parametrize("seed", range(8))
def test_pair_plan_and_numeric_vs_dense(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    n = int(rng.integers(16, 90))
    oa = rng.choice(np.arange(-n + 1, n), size=int(rng.integers(1, 10)), replace=False)
    ob = rng.choice(np.arange(-n + 1, n), size=int(rng.integers(1, 10)), replace=False)
    A = hm_random_np(n, oa, rng)
    B = list(hm_random_np(n, ob, rng))
    if seed % 2:   # B's order must not matter to the set, only to the pair order
        perm = rng.permutation(len(B[0]))
        B = [B[0][perm], B[1][perm], B[2][perm], B[3]]
    c_off, c_len, c_st, nnz = oracle.c_structure(n, A[0], B[0])
    ptr, pairs = oracle.pairs_only(n, A[0], A[1], A[2], B[0], B[1], B[2], c_off)
    assert ptr[0] == 0 and np.all(np.diff(ptr) >= 1)          # every C diagonal has a pair
    assert ptr[-1] == sum(1 for a in A[0] for b in B[0] if abs(int(a) + int(b)) < n)
    # pairs of one C diagonal follow B's array order
    b_index = {int(s): i for i, s in enumerate(B[2])}
    for k in range(len(c_off)):
        order = [b_index[int(g["bb"])] for g in pairs[ptr[k]:ptr[k + 1]]]
        assert order == sorted(order)
    dense = hm_to_dense(n, A[0], A[2], A[3]) @ hm_to_dense(n, B[0], B[2], B[3])
    want = np.zeros(nnz)
    for d, s, ln in zip(c_off, c_st, c_len):
        sr, sc = (0, d) if d >= 0 else (-d, 0)
        want[s:s + ln] = dense[sr + np.arange(ln), sc + np.arange(ln)]
    got_pairs, ab = oracle.spgemm_pairs_f64(A[3], B[3], c_len, c_st, ptr, pairs, 0, len(c_off))
    assert np.allclose(got_pairs, want, rtol=0, atol=1e-12)
    got_gather, _ = oracle.spgemm_gather_f64(n, A, tuple(B), (c_off, c_len, c_st, nnz))
    assert np.allclose(got_gather, want, rtol=0, atol=1e-12)
    got_atomic = oracle.spgemm_hm_atomic_f64(n, A, tuple(B), c_len, c_st,
                                             oracle.c_lookup(n, c_off), nnz)
    assert np.allclose(got_atomic, want, rtol=0, atol=1e-12)
    assert np.all(ab >= np.abs(got_pairs) - 1e-12)
    # fp32 CPU baseline agrees within the summation bound
    out = np.zeros(nnz, np.float32)
    oracle.spgemm_pairs_omp_f32(A[3], B[3], c_len.astype(np.int32), c_st, ptr, pairs, 0,
                                len(c_off), out)
    assert np.all(np.abs(out - want) <= 1e-5 * ab + 1e-30)


@pytest.mark.parametrize("seed", range(3))
def test_complex_pair_numeric_vs_dense(oracle, seed):
    """Complex plan-driven numeric phase (no reference counterpart): the dense
    complex product gives every C value, and each part equals the real oracle
    on the four real part products (Re = ArBr - AiBi, Im = ArBi + AiBr)."""
    rng = np.random.default_rng(300 + seed)
    n = int(rng.integers(20, 70))
    oa = rng.choice(np.arange(-n + 1, n), size=int(rng.integers(1, 8)), replace=False)
    ob = rng.choice(np.arange(-n + 1, n), size=int(rng.integers(1, 8)), replace=False)
    A = hm_random_np(n, oa, rng)
    B = hm_random_np(n, ob, rng)
    Ai = rng.uniform(-1, 1, A[3].size).astype(np.float32)
    Bi = rng.uniform(-1, 1, B[3].size).astype(np.float32)
    Ac = (A[3] + 1j * Ai).astype(np.complex64)
    Bc = (B[3] + 1j * Bi).astype(np.complex64)
    c_off, c_len, c_st, nnz = oracle.c_structure(n, A[0], B[0])
    ptr, pairs = oracle.pairs_only(n, A[0], A[1], A[2], B[0], B[1], B[2], c_off)
    got, ab = oracle.spgemm_pairs_complex(Ac, Bc, c_len, c_st, ptr, pairs, 0, len(c_off))
    dense = (hm_to_dense(n, A[0], A[2], Ac.astype(np.complex128))
             @ hm_to_dense(n, B[0], B[2], Bc.astype(np.complex128)))
    want = np.zeros(nnz, np.complex128)
    for d, s0, ln in zip(c_off, c_st, c_len):
        sr, sc = (0, d) if d >= 0 else (-d, 0)
        want[s0:s0 + ln] = dense[sr + np.arange(ln), sc + np.arange(ln)]
    assert np.allclose(got, want, rtol=0, atol=1e-12)
    part = lambda a, b: oracle.spgemm_pairs_f64(a, b, c_len, c_st, ptr, pairs, 0, len(c_off))[0]
    assert np.allclose(got.real, part(A[3], B[3]) - part(Ai, Bi), rtol=0, atol=1e-12)
    assert np.allclose(got.imag, part(A[3], Bi) + part(Ai, B[3]), rtol=0, atol=1e-12)
    assert np.all(ab >= np.abs(got.real) - 1e-12) and np.all(ab >= np.abs(got.imag) - 1e-12)


def test_gemm_diag_formula_vs_dense(oracle):
    rng = np.random.default_rng(7)
    n = 40
    for oa, ob in [(list(range(-3, 4)), list(range(-3, 4))), ([-17, -2, 0, 5, 30], [-30, 1, 9])]:
        DA = oracle.pack_diag_matrix(n, oa, 42)
        DB = oracle.pack_diag_matrix(n, ob, 137)
        Ad = np.zeros((n, n)); Bd = np.zeros((n, n))
        for i, d in enumerate(oa):
            for t in range(n):
                if 0 <= t + d < n:
                    Ad[t, t + d] = DA[i, t]
        for j, d in enumerate(ob):
            for t in range(n):
                if 0 <= t + d < n:
                    Bd[t, t + d] = DB[j, t]
        P = Ad @ Bd
        c_off, c_len, c_st, nnz = oracle.c_structure(n, oa, ob)
        got, _ = oracle.gemm_diag_f64(n, DA, oa, DB, ob, oracle.c_lookup(n, c_off), c_st, nnz)
        for d, s, ln in zip(c_off, c_st, c_len):
            sr, sc = (0, d) if d >= 0 else (-d, 0)
            assert np.allclose(got[s:s + ln], P[sr + np.arange(ln), sc + np.arange(ln)],
                               rtol=0, atol=1e-12)


def test_reference_generators(oracle):
    offs, starts, lens, vals = oracle.make_banded(100, 3, 1234)
    assert offs.tolist() == list(range(-3, 4))
    assert lens.tolist() == [100 - abs(d) for d in offs]
    assert starts.tolist() == np.concatenate([[0], np.cumsum(lens)[:-1]]).tolist()
    assert vals.min() >= -1 and vals.max() < 1
    assert np.array_equal(vals, oracle.make_banded(100, 3, 1234)[3])
    assert not np.array_equal(vals, oracle.make_banded(100, 3, 5678)[3])
    DA = oracle.pack_diag_matrix(50, [-4, 0, 7], 42)
    assert np.all(DA[0, :4] == 0) and np.all(DA[2, 43:] == 0)
    nz = DA[DA != 0]
    assert nz.size == 46 + 50 + 43 and nz.min() >= 0.5 and nz.max() < 1.5


# ---------------------------------------------------------------------------
# The reference's input generators: the oracle's restatements against the
# outputs of the reference's own source text (tests/golden/generators.json,
# written by tests/golden/make_generator_golden.py from oracle/_ref/
# ref_generators), and the mt19937 draws against the published algorithm.
# ---------------------------------------------------------------------------

GEN = json.loads((Path(__file__).resolve().parent / "golden" / "generators.json").read_text())


def _sha(a) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def _check_summary(a: np.ndarray, s: dict):
    a = np.ascontiguousarray(a, np.float32)
    assert a.size == s["count"]
    if "bits" in s:
        assert a.view(np.uint32).tolist() == s["bits"]
    else:
        assert a[:64].view(np.uint32).tolist() == s["head_bits"]
    assert _sha(a) == s["sha256"]


def test_xval_hval_match_reference(oracle):
    """orc_xval / orc_hval (dia_oracle.c) against bench_cusparse.cu:70-82
    run as written, value for value (N = 1000) and by digest (N = 2^20); the
    SpMV bench's Recon fill and x (orc_hash_band_recon) use exactly them."""
    for f in GEN["xval"]:
        _check_summary(oracle.xval_array(f["N"]), f)
    for f in GEN["hval"]:
        _check_summary(oracle.hval_band(f["N"], f["offsets"]), f)
    N, offs = 4096, GEN["hval"][0]["offsets"]
    r_off, r_val, x = oracle.hash_band_recon(N, offs)
    assert np.array_equal(x, oracle.xval_array(N))
    band = oracle.hval_band(N, list(r_off))
    o = 0
    for k, d in enumerate(r_off):
        c = np.arange(max(d, 0), min(N, N + d))
        assert np.array_equal(r_val[k * N + c], band[o: o + c.size]), d
        o += c.size


def test_tc_spmv_cases_match_reference(oracle):
    """orc_tc_spmv_case against run_case's LCG fill (test_tc_spmv.cu:86-98)
    for the six structural cases of :168-179: every band entry in fill order,
    the whole dense H by digest, and x."""
    for f in GEN["lcg"]:
        N, offs = f["N"], f["offsets"]
        H, x = oracle.tc_spmv_case(N, offs)
        band = np.array([H[r, r + d] for r in range(N) for d in offs if 0 <= r + d < N],
                        np.float32)
        assert band.view(np.uint32).tolist() == f["band_bits"], N
        assert _sha(H) == f["H_sha256"], N
        assert x.view(np.uint32).tolist() == f["x_bits"], N


def test_make_banded_matches_reference(oracle):
    """orc_make_banded against DiaMatrix + make_banded of
    bench_spmspm.cu:79-106: offsets, int64 starts, lengths and every value,
    including diagonals skipped for n <= |d| and the bench's own operands
    make_banded(100000, 16, 1234 / 5678) (:465-466)."""
    for f in GEN["make_banded"]:
        offs, starts, lens, vals = oracle.make_banded(f["n"], f["w"], f["seed"])
        assert offs.tolist() == f["offsets"]
        assert starts.tolist() == f["starts"]
        assert lens.tolist() == f["lengths"]
        _check_summary(vals, f["values"])


def test_pack_diag_matrix_matches_reference(oracle):
    """orc_pack_diag_matrix against pack_diag_matrix of gemm_diag.cu:361-382,
    including the driver's own operands (n = 4096, -10..10, seeds 42 / 137)."""
    for f in GEN["pack_diag_matrix"]:
        DA = oracle.pack_diag_matrix(f["n"], f["offsets"], f["seed"])
        _check_summary(DA.reshape(-1), f["DA"])


def _mt19937_uniform(seed: int, count: int, a: float, b: float) -> np.ndarray:
    """std::uniform_real_distribution<float>(a, b) over std::mt19937(seed) as
    libstdc++ computes it, from the published algorithms: the MT19937 engine
    with init_genrand seeding (numpy's legacy RandomState seeding), one
    32-bit draw per value for generate_canonical<float, 24>, g / 2^32 in
    float (1.0 replaced by the float just below it), then g * (b - a) + a in
    float."""
    raw = np.random.RandomState(seed).randint(0, 2 ** 32, size=count, dtype=np.uint32)
    c = raw.astype(np.float32) / np.float32(2.0 ** 32)
    c = np.where(c >= 1, np.nextafter(np.float32(1), np.float32(0)), c).astype(np.float32)
    return (c * (np.float32(b) - np.float32(a)) + np.float32(a)).astype(np.float32)


def test_mt19937_draws_follow_published_algorithm(oracle):
    """The fixtures and the oracle's draw loops against MT19937 and
    libstdc++'s uniform mapping computed independently in numpy: the draw
    order of make_banded (diagonal by diagonal, positions ascending) and of
    pack_diag_matrix (row by row, only in-range positions)."""
    for f in GEN["make_banded"]:
        want = _mt19937_uniform(f["seed"], f["values"]["count"], -1.0, 1.0)
        _check_summary(want, f["values"])
    n, w, seed = 100000, 16, 5678
    assert np.array_equal(oracle.make_banded(n, w, seed)[3],
                          _mt19937_uniform(seed, 33 * n - 2 * 136, -1.0, 1.0))
    for f in GEN["pack_diag_matrix"]:
        n, offs = f["n"], f["offsets"]
        lens = [n - abs(d) for d in offs]
        draws = _mt19937_uniform(f["seed"], sum(lens), 0.5, 1.5)
        DA = np.zeros((len(offs), n), np.float32)
        o = 0
        for i, (d, ln) in enumerate(zip(offs, lens)):
            DA[i, max(-d, 0): max(-d, 0) + ln] = draws[o: o + ln]
            o += ln
        _check_summary(DA.reshape(-1), f["DA"])


# ---------------------------------------------------------------------------
# The grouped pair schedule (build_schedule, spmspm/bench_spmspm.cu:137-243):
# orc_build_schedule and orc_c_structure against the reference planner run
# from its own source text (tests/golden/schedule.json, written by
# tests/golden/make_schedule_golden.py from oracle/_ref/ref_schedule).
# ---------------------------------------------------------------------------

SCHED = json.loads((Path(__file__).resolve().parent / "golden" / "schedule.json").read_text())
SCHED_ARRAYS = ("a_count", "b_count", "pair_count", "t_out", "a_globals", "b_globals",
                "c_globals", "block_group", "block_tile")


def _check_int_array(a, f, name):
    a = np.ascontiguousarray(a, np.int32)
    assert a.size == f["count"], name
    if "values" in f:
        assert a.tolist() == f["values"], name
    assert _sha(a) == f["sha256"], name


@pytest.mark.parametrize("idx", range(len(SCHED["cases"])))
def test_schedule_matches_reference(oracle, idx):
    case = SCHED["cases"][idx]
    if "banded" in case:
        n, w, sa, sb = case["banded"]
        a_off = oracle.make_banded(n, w, sa)[0]
        b_off = oracle.make_banded(n, w, sb)[0]
    else:
        n, a_off, b_off = case["n"], case["A"], case["B"]
    c_off = oracle.c_structure(n, a_off, b_off)[0]
    _check_int_array(c_off, case["c_offsets"], "c_offsets")
    T, n_tile = case["scalars"][8], case["scalars"][9]
    S = oracle.build_schedule(n, a_off, b_off, c_off, T, n_tile)
    assert [S[k] for k in ("a_halo", "b_halo", "num_groups", "max_a", "max_b", "max_pairs",
                           "num_ntiles", "num_blocks")] == case["scalars"][:8]
    for k in SCHED_ARRAYS:
        _check_int_array(S[k], case[k], k)
    flat = S["pairs"].view(np.int32).reshape(-1)
    _check_int_array(flat, case["pairs"], "pairs")
