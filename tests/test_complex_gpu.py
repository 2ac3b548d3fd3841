"""Complex Hamiltonians on the GPU: complex64 Recon SpMV, real Recon applied
to a complex state, and the Lanczos propagator exp(-i t H) psi_0 built on
them (through the C ABI).

Bounds.  SpMV: each part within 1e-5 of the oracle's fp64 result relative to
the sum of |term parts| (the fp32 bound of any summation order).  The real
matrix applied to a complex x must equal the real kernel applied to each part
bit for bit (same diagonal order, same fused multiply-adds).  Propagator:
against scipy.linalg.expm in complex128 at small n, to 1e-4 of ||psi_0||
(fp32 Lanczos rounding over m <= 40 steps with t ||H|| <= 12; the Krylov
truncation error is below 1e-7 there and is also checked through the
returned estimate); at n = 2^22 through the properties the exact propagator
has (unitarity, time reversal, energy conservation, determinism).
"""
import numpy as np
import pytest
import torch

from diagpu_amd import workloads
from diagpu_amd.krylov import expm_krylov, KrylovWorkspace
from diagpu_amd.spmv import spmv_recon

pytestmark = pytest.mark.gpu


def _nan_padded(rng, rows, cols, offs, dtype):
    K = len(offs)
    if dtype == np.complex64:
        vals = (rng.uniform(-1, 1, (K, cols)) + 1j * rng.uniform(-1, 1, (K, cols))).astype(dtype)
    else:
        vals = rng.uniform(-1, 1, (K, cols)).astype(dtype)
    c = np.arange(cols)
    for k, d in enumerate(offs):          # NaN wherever the row c - d is outside [0, rows)
        vals[k][(c - d < 0) | (c - d >= rows)] = np.nan
    return vals


def _cx(rng, n):
    return (rng.standard_normal(n) + 1j * rng.standard_normal(n)).astype(np.complex64)


@pytest.mark.parametrize("K", [1, 3, 5, 6, 12, 64, 65])
@pytest.mark.parametrize("mat", ["c64", "f32"])
def test_complex_spmv_every_path(dev, oracle, K, mat):
    rng = np.random.default_rng(77 * K + (mat == "f32"))
    rows, cols = 12007, 11993
    offs = rng.choice(np.arange(-2100, 2101), size=K, replace=False).astype(np.int32)
    vals = _nan_padded(rng, rows, cols, offs, np.complex64 if mat == "c64" else np.float32)
    x = _cx(rng, cols)
    y = spmv_recon(torch.as_tensor(offs, device=dev), torch.as_tensor(vals.reshape(-1), device=dev),
                   rows, cols, torch.as_tensor(x, device=dev)).cpu().numpy()
    assert y.dtype == np.complex64 and not np.isnan(y).any()
    want, absum = oracle.spmv_recon_complex_ref(rows, cols, offs, np.nan_to_num(vals).reshape(-1), x)
    for part in (np.real, np.imag):
        err = np.abs(part(y).astype(np.float64) - part(want))
        assert (err <= 1e-5 * absum + 1e-30).all(), float(err.max())


@pytest.mark.parametrize("mat,cols", [("c64", 1), ("f32", 1), ("f32", 3)])
def test_complex_spmv_narrow(dev, oracle, mat, cols):
    """One column: below one run (2 rows per lane for both pairs), so the
    per-element kernel for complex and real-matrix/complex-state operands.
    Three columns: just above one run, so every tile is an edge tile of the
    clamped-run ring with lim barely past R."""
    rng = np.random.default_rng(cols + 10 * (mat == "f32"))
    rows = 2049
    offs = np.array([-1500, -2, -1, 0, 1, 2, 700], np.int32)
    vals = (_cx(rng, len(offs) * cols) if mat == "c64"
            else rng.uniform(-1, 1, len(offs) * cols).astype(np.float32))
    x = _cx(rng, cols)
    y = spmv_recon(torch.as_tensor(offs, device=dev), torch.as_tensor(vals, device=dev),
                   rows, cols, torch.as_tensor(x, device=dev)).cpu().numpy()
    want, absum = oracle.spmv_recon_complex_ref(rows, cols, offs, vals, x)
    for part in (np.real, np.imag):
        err = np.abs(part(y).astype(np.float64) - part(want))
        assert (err <= 1e-5 * absum + 1e-30).all(), float(err.max())


@pytest.mark.parametrize("K", [2, 5, 9, 40, 70])
def test_real_matrix_complex_state_equals_real_kernel_per_part(dev, K):
    """H (real) applied to x = a + ib is H a + i H b with the real kernel's
    exact roundings."""
    rng = np.random.default_rng(500 + K)
    n = 20011
    offs = torch.as_tensor(rng.choice(np.arange(-3000, 3001), size=K, replace=False), dtype=torch.int32, device=dev)
    vals = torch.as_tensor(rng.uniform(-1, 1, K * n).astype(np.float32), device=dev)
    x = torch.as_tensor(_cx(rng, n), device=dev)
    y = spmv_recon(offs, vals, n, n, x)
    yr = spmv_recon(offs, vals, n, n, x.real.contiguous())
    yi = spmv_recon(offs, vals, n, n, x.imag.contiguous())
    assert torch.equal(y.real, yr) and torch.equal(y.imag, yi)


def test_complex_spmv_full_size_poisson(dev, oracle):
    """Benchmark config 2's stencil with complex values (i times the real
    stencil) and a complex state: y = i H x, checked over every row."""
    R = workloads.spmv_config(2, seed=3, device=dev, dtype=torch.float32)
    cv = (1j * R.values.to(torch.complex64)).contiguous()
    x = torch.complex(R.x, torch.roll(R.x, 7)).contiguous()
    y = spmv_recon(R.offsets, cv, R.rows, R.cols, x)
    y2 = spmv_recon(R.offsets, cv, R.rows, R.cols, x)
    assert torch.equal(y, y2)
    want, absum = oracle.spmv_recon_complex_ref(R.rows, R.cols, R.offsets.cpu().numpy(),
                                                cv.cpu().numpy(), x.cpu().numpy())
    got = y.cpu().numpy()
    for part in (np.real, np.imag):
        assert (np.abs(part(got) - part(want)) <= 1e-5 * absum + 1e-30).all()


# ------------------------------------------------------------ propagator --

def _hermitian_band(rng, n, offsets, complex_values=True):
    """Recon arrays of a random Hermitian band: H[r, r+d] = h, H[r+d, r] =
    conj(h); the main diagonal real."""
    pos = sorted({abs(int(d)) for d in offsets})
    H = np.zeros((n, n), np.complex128 if complex_values else np.float64)
    for d in pos:
        for r in range(n - d):
            if d == 0:
                H[r, r] = rng.uniform(-2, 2)
            else:
                h = rng.uniform(-1, 1) + (1j * rng.uniform(-1, 1) if complex_values else 0)
                H[r, r + d] = h
                H[r + d, r] = np.conj(h)
    offs = sorted({d for p in pos for d in (p, -p)}, reverse=True)
    dt = np.complex64 if complex_values else np.float32
    vals = np.zeros((len(offs), n), dt)
    for k, d in enumerate(offs):          # Recon[k][c] = H[c - d, c]
        for c in range(n):
            r = c - d
            if 0 <= r < n:
                vals[k, c] = H[r, c]
    return np.array(offs, np.int32), vals, H.astype(np.complex64).astype(np.complex128)


@pytest.mark.parametrize("complex_values", [True, False])
def test_propagator_matches_expm(dev, complex_values):
    import scipy.linalg as sl
    rng = np.random.default_rng(4 + complex_values)
    n = 500
    offs, vals, H = _hermitian_band(rng, n, [0, 1, 2, 5, 37], complex_values)
    psi0 = _cx(rng, n)
    t, m = 0.8, 40
    res = expm_krylov(torch.as_tensor(offs, device=dev), torch.as_tensor(vals.reshape(-1), device=dev),
                      n, torch.as_tensor(psi0, device=dev), t, m)
    want = sl.expm(-1j * t * H) @ psi0.astype(np.complex128)
    got = res.psi.cpu().numpy().astype(np.complex128)
    nrm = np.linalg.norm(psi0.astype(np.complex128))
    assert np.linalg.norm(got - want) <= 1e-4 * nrm, np.linalg.norm(got - want) / nrm
    assert res.steps == m and not res.breakdown
    assert res.err_estimate <= 1e-6 * nrm
    assert abs(res.psi0_norm - nrm) <= 1e-6 * nrm
    # T_m's leading coefficients against an fp64 Lanczos whose relation
    # V^H H V = T is verified here, so the comparison pins them.
    v = psi0.astype(np.complex128) / nrm
    vp = np.zeros_like(v)
    al, be, V = [], [], [v]
    bprev = 0.0
    for j in range(8):
        w = H @ v
        a = np.vdot(v, w).real
        w = w - a * v - bprev * vp
        b = np.linalg.norm(w)
        al.append(a); be.append(b)
        vp, v, bprev = v, w / b, b
        V.append(v)
    Vm = np.array(V[:8]).T
    T = np.diag(al) + np.diag(be[:7], 1) + np.diag(be[:7], -1)
    assert np.allclose(Vm.conj().T @ H @ Vm, T, atol=1e-9)
    scale = np.abs(np.linalg.eigvalsh(H)).max()
    assert np.allclose(res.alpha[:8], al, rtol=0, atol=1e-4 * scale)
    assert np.allclose(res.beta[:8], be, rtol=0, atol=1e-4 * scale)


def test_propagator_breakdown_is_exact(dev):
    """A diagonal H with three distinct values: the Krylov space of any psi_0
    has dimension 3, Lanczos stops there and the result is exp(-i t d) psi_0."""
    rng = np.random.default_rng(8)
    n = 3000
    d = rng.choice(np.array([-1.0, 0.5, 2.0], np.float32), size=n)
    psi0 = _cx(rng, n)
    t = 1.3
    res = expm_krylov(torch.tensor([0], dtype=torch.int32, device=dev),
                      torch.as_tensor(d, device=dev), n, torch.as_tensor(psi0, device=dev), t, 20)
    assert res.breakdown and res.steps == 3
    want = np.exp(-1j * t * d.astype(np.float64)) * psi0
    got = res.psi.cpu().numpy()
    assert np.abs(got - want).max() <= 2e-6 * np.abs(psi0).max()


@pytest.mark.parametrize("n", [1, 2, 3])
@pytest.mark.parametrize("complex_values", [True, False])
def test_propagator_tiny_n(dev, n, complex_values):
    """n below one 16-byte run (the per-element SpMV with its dot epilogue):
    Lanczos reaches the whole space in <= n steps and is exact there."""
    import scipy.linalg as sl
    rng = np.random.default_rng(20 + n + 5 * complex_values)
    offs, vals, H = _hermitian_band(rng, n, list(range(n)), complex_values)
    psi0 = _cx(rng, n)
    t = 0.9
    res = expm_krylov(torch.as_tensor(offs, device=dev), torch.as_tensor(vals.reshape(-1), device=dev),
                      n, torch.as_tensor(psi0, device=dev), t, 8)
    want = sl.expm(-1j * t * H) @ psi0.astype(np.complex128)
    got = res.psi.cpu().numpy().astype(np.complex128)
    nrm = np.linalg.norm(psi0.astype(np.complex128))
    assert res.steps <= n and np.linalg.norm(got - want) <= 1e-5 * nrm


def test_propagator_pageable_readback(dev):
    """host_scratch = NULL (T_m's entries read back through pageable memory)
    gives the same result, bit for bit, as the pinned buffer the Python
    workspace passes."""
    import ctypes as C
    from diagpu_amd import _lib
    from diagpu_amd.spmv import recon_view
    rng = np.random.default_rng(31)
    n, m, t = 3000, 16, 0.7
    offs, vals, _ = _hermitian_band(rng, n, [0, 1, 9], True)
    d_off = torch.as_tensor(offs, device=dev)
    d_val = torch.as_tensor(vals.reshape(-1), device=dev)
    psi0 = torch.as_tensor(_cx(rng, n), device=dev)
    ws = KrylovWorkspace(n, m, dev)
    pinned = expm_krylov(d_off, d_val, n, psi0, t, m, workspace=ws)
    out = torch.empty_like(psi0)
    info = _lib.KrylovInfo()
    view = recon_view(d_off, d_val, n, n)
    _lib.call("diagpu_expm_krylov_c64", C.byref(view), psi0.data_ptr(), t, m, out.data_ptr(),
              ws.buf.data_ptr(), ws.buf.numel(), None, None, None, C.byref(info),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert info.steps == pinned.steps and info.err_estimate == pinned.err_estimate
    assert torch.equal(out, pinned.psi)


def test_propagator_zero_time_and_zero_state(dev):
    rng = np.random.default_rng(9)
    n = 4097
    offs, vals, _ = _hermitian_band(rng, n, [0, 3])
    o = torch.as_tensor(offs, device=dev)
    v = torch.as_tensor(vals.reshape(-1), device=dev)
    psi0 = torch.as_tensor(_cx(rng, n), device=dev)
    r0 = expm_krylov(o, v, n, psi0, 0.0, 10)
    assert torch.allclose(r0.psi, psi0, rtol=0, atol=1e-6)
    rz = expm_krylov(o, v, n, torch.zeros_like(psi0), 0.7, 10)
    assert rz.steps == 0 and torch.count_nonzero(rz.psi) == 0


def test_propagator_full_size_properties(dev):
    """n = 2^22 (config 2's 5-point stencil, real symmetric H) with a complex
    state: ||psi(t)|| = ||psi_0||, psi(-t) of psi(t) = psi_0, <H> conserved,
    and two runs agree bit for bit."""
    R = workloads.spmv_config(2, seed=5, device=dev, dtype=torch.float32)
    n = R.rows
    g = torch.Generator(device=dev).manual_seed(5)
    psi0 = torch.complex(torch.randn(n, device=dev, generator=g),
                         torch.randn(n, device=dev, generator=g)).contiguous()
    ws = KrylovWorkspace(n, 30, dev)
    t = 0.25
    a = expm_krylov(R.offsets, R.values, n, psi0, t, 30, workspace=ws)
    a2 = expm_krylov(R.offsets, R.values, n, psi0, t, 30, workspace=ws)
    assert torch.equal(a.psi, a2.psi)
    assert a.err_estimate <= 1e-5 * a.psi0_norm
    nrm0 = torch.linalg.vector_norm(psi0.to(torch.complex128)).item()
    assert abs(torch.linalg.vector_norm(a.psi.to(torch.complex128)).item() - nrm0) <= 1e-5 * nrm0
    back = expm_krylov(R.offsets, R.values, n, a.psi, -t, 30, workspace=ws)
    diff = torch.linalg.vector_norm((back.psi - psi0).to(torch.complex128)).item()
    assert diff <= 1e-4 * nrm0, diff / nrm0

    def energy(psi):
        hpsi = spmv_recon(R.offsets, R.values, n, n, psi)
        return torch.vdot(psi.to(torch.complex128), hpsi.to(torch.complex128)).real.item()
    e0, e1 = energy(psi0), energy(a.psi)
    assert abs(e1 - e0) <= 1e-4 * abs(e0)


# ------------------------------------------------------- complex SpGEMM --

def _complexify(M, shift):
    """The same HM structure with complex values v + i * roll(v, shift)."""
    from diagpu_amd.workloads import HM
    v = M.values
    return HM(M.n, M.offsets, M.lengths, M.starts,
              torch.complex(v, torch.roll(v, shift)).contiguous())


def _plan_host(oracle, plan, A, B):
    a_off, a_len, a_st = (t.cpu().numpy() for t in (A.offsets, A.lengths, A.starts))
    b_off, b_len, b_st = (t.cpu().numpy() for t in (B.offsets, B.lengths, B.starts))
    c_off, c_len, c_st, nnz = oracle.c_structure(A.n, a_off, b_off)
    ptr, pairs = oracle.pairs_only(A.n, a_off, a_len, a_st, b_off, b_len, b_st, c_off)
    assert np.array_equal(plan.c_offsets().cpu().numpy(), c_off)
    assert np.array_equal(plan.pair_ptr().cpu().numpy(), ptr)
    return c_len, c_st, ptr, pairs


def _check_complex(got, want, ab):
    for part in (np.real, np.imag):
        err = np.abs(part(got).astype(np.float64) - part(want))
        assert (err <= 1e-5 * ab + 1e-300).all(), float(err.max())


@pytest.mark.parametrize("seed,n,na,nb,span", [
    (0, 37, 5, 4, 36), (1, 1000, 12, 30, 999), (2, 3001, 40, 8, 2999), (3, 1031, 64, 64, 1030)])
def test_complex_spgemm_random(dev, oracle, seed, n, na, nb, span):
    from diagpu_amd.spgemm import SpgemmPlan
    rng = np.random.default_rng(seed)
    oa = rng.choice(np.arange(-span, span + 1), size=na, replace=False)
    ob = rng.choice(np.arange(-span, span + 1), size=nb, replace=False)
    A = _complexify(workloads.hm_random(n, oa, seed=seed, device=dev), 3)
    B = _complexify(workloads.hm_random(n, ob, seed=seed + 50, device=dev), 5)
    plan = SpgemmPlan(A, B)
    c_len, c_st, ptr, pairs = _plan_host(oracle, plan, A, B)
    C1 = plan.multiply(A.values, B.values)
    C2 = plan.multiply(A.values, B.values)
    assert C1.dtype == torch.complex64 and torch.equal(C1, C2)
    want, ab = oracle.spgemm_pairs_complex(A.values.cpu().numpy(), B.values.cpu().numpy(),
                                           c_len, c_st, ptr, pairs, 0, len(c_len))
    _check_complex(C1.cpu().numpy(), want, ab)


def test_complex_spgemm_real_values_equal_real_kernel(dev):
    """Zero imaginary parts: the complex kernel's real part is the real
    kernel's result bit for bit and its imaginary part is zero."""
    from diagpu_amd.spgemm import SpgemmPlan
    from diagpu_amd.workloads import HM
    A, B = workloads.spgemm_config(4, seed=7, device=dev)
    plan = SpgemmPlan(A, B)
    Cr = plan.multiply(A.values, B.values)
    Ac = torch.complex(A.values, torch.zeros_like(A.values)).contiguous()
    Bc = torch.complex(B.values, torch.zeros_like(B.values)).contiguous()
    Cc = plan.multiply(Ac, Bc)
    assert torch.equal(Cc.real, Cr) and torch.count_nonzero(Cc.imag) == 0


def test_complex_spgemm_config4_and_config5(dev, oracle):
    """Config 4's structure with complex values over every C value; config 5
    on a sample of C diagonals (C has 2.4e9 complex values)."""
    from diagpu_amd.spgemm import SpgemmPlan
    for cfg, sample in ((4, None), (5, 24)):
        A, B = workloads.spgemm_config(cfg, seed=cfg, device=dev)
        A, B = _complexify(A, 1), _complexify(B, 2)
        plan = SpgemmPlan(A, B)
        c_len, c_st, ptr, pairs = _plan_host(oracle, plan, A, B)
        Cv = plan.multiply(A.values, B.values)
        torch.cuda.synchronize()
        Av, Bv = A.values.cpu().numpy(), B.values.cpu().numpy()
        if sample is None:
            want, ab = oracle.spgemm_pairs_complex(Av, Bv, c_len, c_st, ptr, pairs, 0, len(c_len))
            _check_complex(Cv.cpu().numpy(), want, ab)
        else:
            rng = np.random.default_rng(cfg)
            ks = sorted({0, len(c_len) - 1, *rng.choice(len(c_len), sample).tolist()})
            for k in ks:
                want, ab = oracle.spgemm_pairs_complex(Av, Bv, c_len, c_st, ptr, pairs, k, k + 1)
                got = Cv[int(c_st[k]):int(c_st[k]) + int(c_len[k])].cpu().numpy()
                _check_complex(got, want, ab)
        del Cv, plan
        torch.cuda.empty_cache()


def _bits(C):
    return torch.view_as_real(C).contiguous().view(torch.int32)


def _offsets(rng, cnt, lo, hi):
    return sorted(rng.choice(np.arange(lo, hi + 1), size=cnt, replace=False).tolist())


@pytest.mark.parametrize("n,case", [
    (4096, "band32"),       # 32 random offsets over +-512 squared: 32 entries per A diagonal
    (37, "edges"),          # smaller than one block, offsets reaching +-(n-1)
    (1000, "wideB"),        # narrow A, B spanning the matrix
    (70001, "ragged"),      # ragged last block, B beyond the A window
    (5000, "maxA"),         # DIAGPU_ASTAT_MAX_A_C64 A diagonals
    (1, "one"),             # a 1 x 1 matrix: one block, 16 lead rows before row 0
    (3, "three"),           # every diagonal of a 3 x 3 matrix
    (1 << 17, "tail"),      # 512 blocks, the last with 5 rows per lane (513 would take 2 rounds)
    (1 << 20, "short"),     # 5 C diagonals: 8 rows per lane, 2048 blocks, the last 9
    (1 << 17, "wideA"),     # 100 A diagonals: 2 rows per lane, 1024 blocks, the last 3
])
def test_complex_astat_same_bits_as_gather(dev, oracle, n, case):
    """The complex A-stationary kernel returns the complex gather's C bit for
    bit (same plan order, same four fused multiply-adds per term, same
    skipped terms), and both agree with the oracle's complex128 products."""
    from diagpu_amd import _lib
    from diagpu_amd.spgemm import SpgemmPlan
    rng = np.random.default_rng(n + 7)
    if case == "band32":
        oa = ob = _offsets(rng, 32, -512, 512)
    elif case == "edges":
        oa, ob = [-36, -3, 0, 2, 36], [-30, -1, 0, 5, 36]
    elif case == "wideB":
        oa, ob = list(range(-40, 41, 3)), [-999, -7, 0, 1, 998]
    elif case == "ragged":
        oa, ob = list(range(-12, 13)), [-65000, -3, 0, 4, 65000]
    elif case == "one":
        oa, ob = [0], [0]
    elif case == "three":
        oa, ob = [-2, -1, 0, 1, 2], [-2, 0, 1]
    elif case == "tail":
        oa, ob = _offsets(rng, 30, -3000, 3000), _offsets(rng, 10, -600, 600)
    elif case == "short":
        oa = ob = [-512, 0, 512]
    elif case == "wideA":
        oa, ob = _offsets(rng, 100, -3000, 3000), _offsets(rng, 8, -300, 300)
    else:
        oa, ob = _offsets(rng, _lib.ASTAT_MAX_A_C64, -2000, 2000), _offsets(rng, 9, -100, 100)
    A = _complexify(workloads.hm_random(n, oa, seed=31, device=dev), 3)
    B = _complexify(workloads.hm_random(n, ob, seed=32, device=dev), 5)
    plan = SpgemmPlan(A, B)
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    Ca = plan.multiply(A.values, B.values, kernel="astat")
    assert Ca.dtype == torch.complex64
    assert torch.equal(_bits(Cg), _bits(Ca))
    if n <= 5000:
        c_len, c_st, ptr, pairs = _plan_host(oracle, plan, A, B)
        want, ab = oracle.spgemm_pairs_complex(A.values.cpu().numpy(), B.values.cpu().numpy(),
                                               c_len, c_st, ptr, pairs, 0, len(c_len))
        _check_complex(Ca.cpu().numpy(), want, ab)


def test_complex_astat_real_values_equal_real_kernel(dev):
    """Zero imaginary parts: the complex A-stationary kernel's real part is
    the real A-stationary kernel's C bit for bit, its imaginary part zero."""
    from diagpu_amd.spgemm import SpgemmPlan
    rng = np.random.default_rng(11)
    offs = _offsets(rng, 24, -300, 300)
    A = workloads.hm_random(20000, offs, seed=1, device=dev)
    B = workloads.hm_random(20000, offs, seed=2, device=dev)
    plan = SpgemmPlan(A, B)
    Cr = plan.multiply(A.values, B.values, kernel="astat")
    Ac = torch.complex(A.values, torch.zeros_like(A.values)).contiguous()
    Bc = torch.complex(B.values, torch.zeros_like(B.values)).contiguous()
    Cc = plan.multiply(Ac, Bc, kernel="astat")
    assert torch.equal(Cc.real.contiguous().view(torch.int32), Cr.view(torch.int32))
    assert torch.count_nonzero(Cc.imag) == 0


def test_complex_astat_choice_and_capacity(dev):
    """auto takes the complex A-stationary kernel where A fits (at most
    DIAGPU_ASTAT_MAX_A_C64 diagonals), n >= 4096, and n >= 2^16 or the plan
    has >= 3 entries per A diagonal; the gather otherwise.  More A diagonals are refused with DIAGPU_ERR_CAPACITY
    before any launch; the band kernel takes fp32 only."""
    from diagpu_amd import _lib
    from diagpu_amd.spgemm import SpgemmPlan
    rng = np.random.default_rng(5)
    offs = _offsets(rng, 40, -512, 512)
    H = _complexify(workloads.hm_random(1 << 16, offs, seed=4, device=dev), 1)
    p = SpgemmPlan(H, H)
    assert p.kernel_for(torch.complex64) == "astat"
    assert torch.equal(_bits(p.multiply(H.values, H.values)),
                       _bits(p.multiply(H.values, H.values, kernel="gather")))
    A4, B4 = workloads.spgemm_config(4, seed=4, device=dev)      # n = 2^20, 63 C diagonals
    p4 = SpgemmPlan(_complexify(A4, 1), _complexify(B4, 2))
    assert p4.kernel_for(torch.complex64) == "astat"
    assert SpgemmPlan(A4, B4).kernel_for(torch.float32) == "astat"    # 63 entries, 47 C diagonals
    lo_a = _offsets(rng, 64, -2000, 2000)                        # 2 entries per A diagonal
    lo = SpgemmPlan(_complexify(workloads.hm_random(8192, lo_a, seed=7, device=dev), 1),
                    _complexify(workloads.hm_random(8192, [-9, 4], seed=8, device=dev), 2))
    assert lo.kernel_for(torch.complex64) == "gather"
    lo16 = SpgemmPlan(_complexify(workloads.hm_random(1 << 16, lo_a, seed=7, device=dev), 1),
                      _complexify(workloads.hm_random(1 << 16, [-9, 4], seed=8, device=dev), 2))
    assert lo16.kernel_for(torch.complex64) == "astat"            # the same at n = 2^16
    five = workloads.hm_random(1 << 18, [-512, -1, 0, 1, 512], seed=9, device=dev)
    p5 = SpgemmPlan(_complexify(five, 1), _complexify(five, 2))    # 13 C diagonals, 25 entries
    assert p5.kernel_for(torch.complex64) == "astat"
    P2 = _complexify(workloads.recon_to_hm(workloads.spmv_config(2, seed=1, device=dev)), 1)
    assert SpgemmPlan(P2, P2).kernel_for(torch.complex64) == "astat"   # the same at n = 2^22
    wide = _complexify(workloads.hm_random(4096, _offsets(rng, _lib.ASTAT_MAX_A_C64 + 1, -300, 300),
                                           seed=6, device=dev), 2)
    pw = SpgemmPlan(wide, wide)
    assert pw.kernel_for(torch.complex64) == "gather"
    with pytest.raises(_lib.DiagpuError) as e:
        pw.multiply(wide.values, wide.values, kernel="astat")
    assert e.value.status == _lib.ERR_CAPACITY
    with pytest.raises(TypeError):
        pw.multiply(wide.values, wide.values, kernel="band")
