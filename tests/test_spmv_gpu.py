"""SpMV parity on the GPU: diagpu_spmv_recon_f32/_f64 (through the C ABI)
against the CPU oracle.

Tolerance (fp32): |y - y64| <= 1e-5 * sum_k |Recon[k][c] * x[c]| per row,
where y64 is the oracle's fp64 sum; 1e-5 relative to the absolute term sum
is the north-star bound made independent of cancellation (any fp32
summation order of K <= 166 terms satisfies it).  fp64: 1e-13 of the same
sum.  Integer-valued cases must be exact.
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from diagpu_amd import workloads
from diagpu_amd.spmv import spmv_recon

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL32, TOL64 = 1e-5, 1e-13

TC_CASES = [  # spmv/test/test_tc_spmv.cu:168-179
    ("tridiagonal", 48, [-1, 0, 1]),
    ("tridiag ragged", 37, [-1, 0, 1]),
    ("pentadiagonal", 64, [-2, -1, 0, 1, 2]),
    ("9-diag wide band", 80, [-9, -5, -2, -1, 0, 1, 2, 5, 9]),
    ("asymmetric band", 71, [-3, 0, 2, 4, 7]),
    ("main diagonal", 16, [0]),
]


def gpu_spmv(dev, r_off, r_val, rows, cols, x, y_init=None):
    off = torch.as_tensor(np.ascontiguousarray(r_off, np.int32), device=dev)
    val = torch.as_tensor(np.ascontiguousarray(r_val), device=dev)
    xx = torch.as_tensor(np.ascontiguousarray(x), device=dev)
    y = None if y_init is None else torch.as_tensor(y_init, device=dev)
    out = spmv_recon(off, val, rows, cols, xx, y)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def check_bound(y, y64, absum, tol):
    err = np.abs(y.astype(np.float64) - y64)
    bad = err > tol * absum + 1e-300
    assert not bad.any(), (f"{int(bad.sum())} rows out of bound; worst row {int(np.argmax(err - tol * absum))}"
                           f" err={err.max():.3e}")


def test_known_answer_5x5(dev, oracle):
    kat = json.loads((GOLDEN / "reconstruct_kat.json").read_text())
    r_off = np.array(kat["recon_offsets"], np.int32)
    r_val = np.array(kat["recon_rows"], np.float32).reshape(-1)
    y = gpu_spmv(dev, r_off, r_val, 5, 5, np.array(kat["x"], np.float32))
    assert y.tolist() == kat["y"]


@pytest.mark.parametrize("name,N,offsets", TC_CASES)
def test_reference_structural_cases(dev, oracle, name, N, offsets):
    H, x = oracle.tc_spmv_case(N, offsets)
    offs, starts, lens, vals = oracle.dense_to_dia(H)
    r_off, r_val = oracle.build_recon(N, N, offs, starts, lens, vals)
    y = gpu_spmv(dev, r_off, r_val, N, N, x)
    y64, absum = oracle.spmv_recon_ref64(N, N, r_off, r_val, x)
    check_bound(y, y64, absum, TOL32)
    # the reference's own criterion for this case (test_tc_spmv.cu:147-148), far tighter here
    y_dense = H.astype(np.float64) @ x
    assert np.max(np.abs(y - y_dense)) / max(np.max(np.abs(y_dense)), 1e-30) < 1e-6


def test_hash_band_bench_matrix(dev, oracle):
    """The SpMV bench's matrix (bench_cusparse.cu:84-144), N = 2^20, 9 diagonals."""
    N = 1 << 20
    r_off, r_val, x = oracle.hash_band_recon(N, [-9, -5, -2, -1, 0, 1, 2, 5, 9])
    y = gpu_spmv(dev, r_off, r_val, N, N, x)
    y64, absum = oracle.spmv_recon_ref64(N, N, r_off, r_val, x)
    check_bound(y, y64, absum, TOL32)


@pytest.mark.parametrize("cfg,dtype", [(1, torch.float32), (2, torch.float32),
                                       (2, torch.float64), (3, torch.float32)])
def test_baseline_configs_full_size(dev, oracle, cfg, dtype):
    R = workloads.spmv_config(cfg, seed=cfg, device=dev, dtype=dtype)
    y1 = spmv_recon(R.offsets, R.values, R.rows, R.cols, R.x)
    y2 = spmv_recon(R.offsets, R.values, R.rows, R.cols, R.x)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "run-to-run results differ"
    y64, absum = oracle.spmv_recon_ref64(R.rows, R.cols, R.offsets.cpu().numpy(),
                                         R.values.cpu().numpy(), R.x.cpu().numpy())
    check_bound(y1.cpu().numpy(), y64, absum, TOL32 if dtype == torch.float32 else TOL64)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float64])
def test_poisson_closed_form_full_size(dev, dtype):
    """5-point stencil 2048 x 2048, x = 1: y = number of missing grid neighbours."""
    R = workloads.spmv_config(2, seed=0, device=dev, dtype=dtype)
    y = spmv_recon(R.offsets, R.values, R.rows, R.cols, torch.ones_like(R.x))
    side = 2048
    i = torch.arange(R.rows, device=dev) // side
    j = torch.arange(R.rows, device=dev) % side
    missing = (i == 0).to(dtype) + (i == side - 1) + (j == 0) + (j == side - 1)
    assert torch.equal(y, missing)


def _random_rect(oracle, rng, rows, cols, offsets):
    H = np.zeros((rows, cols), np.float32)
    for d in offsets:
        for r in range(rows):
            c = r + d
            if 0 <= c < cols:
                H[r, c] = rng.uniform(-1, 1)
    return H


@pytest.mark.parametrize("rows,cols,offsets", [
    (3000, 2100, [-700, -3, 0, 5, 1500]),          # rows > cols
    (1500, 4099, [-2, 0, 1, 900, 2500, 4000]),     # rows < cols
    (1, 1, [0]),                                   # single row
    (4097, 4097, list(range(-100, 101))),          # K = 201 > 64: several offset groups
])
def test_rectangular_and_wide(dev, oracle, rows, cols, offsets):
    rng = np.random.default_rng(rows + cols)
    H = _random_rect(oracle, rng, rows, cols, offsets)
    x = rng.standard_normal(cols).astype(np.float32)
    offs, starts, lens, vals = oracle.dense_to_dia(H)
    r_off, r_val = oracle.build_recon(rows, cols, offs, starts, lens, vals)
    y = gpu_spmv(dev, r_off, r_val, rows, cols, x)
    y64, absum = oracle.spmv_recon_ref64(rows, cols, r_off, r_val, x)
    check_bound(y, y64, absum, TOL32)
    assert np.allclose(y, H.astype(np.float64) @ x, rtol=0, atol=1e-4)


def test_unsorted_duplicate_and_out_of_range_offsets(dev, oracle):
    """Offsets in any order, repeated, or beyond the matrix: the sum is still
    the Recon identity with out-of-range terms dropped."""
    rng = np.random.default_rng(5)
    n = 5000
    r_off = np.array([3, -4999, 0, 7000, -12, 3, 4999, -9000], np.int32)
    r_val = rng.uniform(-1, 1, size=len(r_off) * n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    y = gpu_spmv(dev, r_off, r_val, n, n, x)
    y64, absum = oracle.spmv_recon_ref64(n, n, r_off, r_val, x)
    check_bound(y, y64, absum, TOL32)


def test_short_x_and_zero_diagonals(dev, oracle):
    rng = np.random.default_rng(9)
    n = 3000
    r_off = np.array([1, 0, -1], np.int32)
    r_val = rng.uniform(-1, 1, size=3 * n).astype(np.float32)
    x = rng.standard_normal(n - 777).astype(np.float32)        # x_size < cols
    y = gpu_spmv(dev, r_off, r_val, n, n, x)
    y64, absum = oracle.spmv_recon_ref64(n, n, r_off, r_val, x)
    check_bound(y, y64, absum, TOL32)
    # K = 0: y is overwritten with zeros
    y0 = gpu_spmv(dev, np.zeros(0, np.int32), np.zeros(0, np.float32), n, n,
                  x, y_init=np.full(n, np.nan, np.float32))
    assert np.array_equal(y0, np.zeros(n, np.float32))


def test_unaligned_pointers_and_side_stream(dev, oracle):
    """Views starting one element into their allocation, launched on a
    non-default stream."""
    rng = np.random.default_rng(11)
    n = 9001
    r_off = np.array([64, 2, 0, -1, -300], np.int32)
    r_val = rng.uniform(-1, 1, size=len(r_off) * n).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    off = torch.as_tensor(r_off, device=dev)
    vbuf = torch.empty(len(r_val) + 1, device=dev)
    vbuf[1:] = torch.as_tensor(r_val, device=dev)
    xbuf = torch.empty(n + 1, device=dev)
    xbuf[1:] = torch.as_tensor(x, device=dev)
    ybuf = torch.full((n + 3,), float("nan"), device=dev)
    s = torch.cuda.Stream()
    torch.cuda.synchronize()
    with torch.cuda.stream(s):
        spmv_recon(off, vbuf[1:], n, n, xbuf[1:], ybuf[3:], stream=s)
    s.synchronize()
    y = ybuf[3:].cpu().numpy()
    assert np.isnan(ybuf[:3].cpu().numpy()).all()
    y64, absum = oracle.spmv_recon_ref64(n, n, r_off, r_val, x)
    check_bound(y, y64, absum, TOL32)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("K", [1, 2, 3, 4, 5, 6, 7, 12, 63, 64, 65, 130])
def test_every_kernel_variant(dev, oracle, K, dtype):
    """Each K path of the library (straight-line kernel for K <= 5, ring for
    6..64, grouped ring above 64) in both precisions, with offsets wide enough
    that several tiles at each end are edge tiles and a ragged last tile
    (rows not a multiple of the tile).  Padding holds NaN, so a read of any
    out-of-range Recon entry would show."""
    rng = np.random.default_rng(1000 * K + (dtype == np.float64))
    rows, cols = 20011, 19997
    offs = rng.choice(np.arange(-2600, 2601), size=K, replace=False).astype(np.int32)
    vals = rng.uniform(-1, 1, size=(K, cols)).astype(dtype)
    for k, d in enumerate(offs):          # NaN where the row c - d is outside [0, rows)
        c = np.arange(cols)
        vals[k][(c - d < 0) | (c - d >= rows)] = np.nan
    x = rng.standard_normal(cols).astype(dtype)
    y = gpu_spmv(dev, offs, vals.reshape(-1), rows, cols, x)
    y64, absum = oracle.spmv_recon_ref64(rows, cols, offs, np.nan_to_num(vals).reshape(-1), x)
    assert not np.isnan(y).any()
    check_bound(y, y64, absum, TOL32 if dtype == np.float32 else TOL64)


@pytest.mark.parametrize("dtype", [np.float32, np.float64])
@pytest.mark.parametrize("cols,xlen", [(1, 1), (2, 2), (3, 3), (3000, 1), (3000, 3)])
def test_narrow_matrix(dev, oracle, dtype, cols, xlen):
    """Fewer columns of x in range than one 16-byte run holds (min(cols,
    x_size) < 16 / element size): the per-element kernel, any K, with rows
    far beyond the columns so most rows see no in-range term.  (f64 with
    two columns is the boundary min(cols, x_size) == 16 / element size of
    the clamped-run kernels instead.)"""
    R = 16 // np.dtype(dtype).itemsize
    rng = np.random.default_rng(cols * 7 + xlen + R)
    rows = 3001
    for offs in ([0], [2, 0, -1], [-2999, -5, -1, 0, 1, 2, 3, 2999], list(range(-40, 30))):
        r_off = np.array(offs, np.int32)
        r_val = rng.uniform(-1, 1, size=len(offs) * cols).astype(dtype)
        x = rng.standard_normal(xlen).astype(dtype)
        y = gpu_spmv(dev, r_off, r_val, rows, cols, x, y_init=np.full(rows, np.nan, dtype))
        y64, absum = oracle.spmv_recon_ref64(rows, cols, r_off, r_val, x)
        assert not np.isnan(y).any()
        check_bound(y, y64, absum, TOL32 if dtype == np.float32 else TOL64)
