"""The explicit propagator U = exp(-i dt H) built by the SpGEMM chain in
complex arithmetic, handed to the SpMV path by build_recon on the device --
the "build U once, apply it cheaply" side of slides/transcript.md:10-18 --
and the pieces it needs (complex axpby, diagpu_hm_to_recon_*).

Checks:
  - HM -> Recon equals the oracle's build_recon (the reference's, pinned to
    its 5x5 known-answer test) value for value, real and complex parts;
  - complex axpby against dense complex128 arithmetic;
  - U against scipy.linalg.expm(-i dt H), elementwise |err| <= 1e-5 * order *
    expm(dt |H|) + the series' truncation bound (fp32 sums of order products);
  - at n = 2^20, U psi (complex SpMV on Recon(U)) against the Lanczos
    propagator of the same H, and ||U psi|| = ||psi||.
"""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from diagpu_amd import chain
from diagpu_amd.krylov import expm_krylov
from diagpu_amd.spmv import spmv_recon
from diagpu_amd.workloads import HM, hm_random, hm_stencil7
from hm_host import dense_of, matvec64

pytestmark = pytest.mark.gpu


def _complex_hm(n, offs, seed, dev):
    a = hm_random(n, offs, seed, dev)
    b = hm_random(n, offs, seed + 1000, dev)
    return HM(n, a.offsets, a.lengths, a.starts, torch.complex(a.values, b.values).contiguous())


def _hermitian_hm(n, pos, seed, dev, complex_values=True):
    """HM of a Hermitian band: diagonal -d holds the conjugates of diagonal d
    (same positions); the main diagonal is real."""
    offs = sorted({s * d for d in pos for s in (1, -1)})
    M = _complex_hm(n, offs, seed, dev) if complex_values else chain.as_complex(hm_random(n, offs, seed, dev))
    v = M.values
    starts = M.starts.cpu().tolist()
    for d in pos:
        i_pos, i_neg = offs.index(d), offs.index(-d)
        ln = n - d
        src = v[starts[i_pos]: starts[i_pos] + ln]
        if d == 0:
            src.imag.zero_()
        else:
            v[starts[i_neg]: starts[i_neg] + ln] = src.conj()
    if not complex_values:
        return HM(n, M.offsets, M.lengths, M.starts, v.real.contiguous())
    return M


def test_hm_to_recon_matches_reference_build_recon(dev, oracle):
    n = 777
    for M in (hm_random(n, [-700, -3, 0, 1, 64], 3, dev), _complex_hm(n, [-5, 0, 2, 776], 4, dev)):
        r_off, r_val = chain.to_recon(M)
        offs, lens = M.offsets.cpu().numpy(), M.lengths.cpu().numpy()
        starts = M.starts.cpu().numpy()
        v = M.values.cpu().numpy()
        parts = (v.real, v.imag) if np.iscomplexobj(v) else (v,)
        got = r_val.cpu().numpy()
        got_parts = (got.real, got.imag) if np.iscomplexobj(got) else (got,)
        for p, gp in zip(parts, got_parts):
            want_off, want_val = oracle.build_recon(n, n, offs, starts, lens, p.astype(np.float32))
            assert np.array_equal(r_off.cpu().numpy(), want_off)
            assert np.array_equal(gp, want_val)
        # and the SpMV of the Recon form is the HM matrix's product
        x = np.random.default_rng(5).standard_normal(n).astype(np.complex64)
        y = spmv_recon(r_off, r_val, n, n, torch.as_tensor(x, device=dev)).cpu().numpy()
        assert np.allclose(y, matvec64(M, x.astype(np.complex128)), rtol=0, atol=1e-4)


@pytest.mark.parametrize("count", [1, 2, 7, 1 << 20, (1 << 20) + 3])
def test_promote_f32_c64(dev, count):
    """diagpu_promote_f32_c64: dst = (src, 0), exactly, for odd and even
    counts and with a one-element offset (unaligned) destination."""
    from diagpu_amd import _lib
    g = torch.Generator(device=dev).manual_seed(count)
    src = torch.randn(count, device=dev, generator=g)
    buf = torch.full((count + 1,), complex("nan+nanj"), dtype=torch.complex64, device=dev)
    _lib.call("diagpu_promote_f32_c64", count, src.data_ptr(), buf[1:].data_ptr(),
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.isnan(buf[0].real)
    assert torch.equal(buf[1:].real, src) and torch.equal(buf[1:].imag, torch.zeros_like(src))


def test_complex_axpby(dev):
    n = 300
    X = _complex_hm(n, [-4, 0, 9], 1, dev)
    Y = _complex_hm(n, [0, 9, 50], 2, dev)
    a, b = 0.5 - 1.25j, -2.0 + 0.5j
    Z = chain.axpby(a, X, b, Y)
    assert Z.values.dtype == torch.complex64 and Z.offsets.cpu().tolist() == [-4, 0, 9, 50]
    Xd, Yd = dense_of(X), dense_of(Y)
    want = a * Xd + b * Yd
    bound = abs(a) * np.abs(Xd) + abs(b) * np.abs(Yd)
    # fp32 complex products and sum: |err| <= sqrt(2) * 4 * 2^-24 * bound
    assert np.all(np.abs(dense_of(Z) - want) <= 4e-7 * bound + 1e-30)
    # a zero complex factor does not read its operand
    Y.values.fill_(complex("nan+nanj"))
    Z0 = chain.axpby(2.0j, X, 0j, Y)
    D0 = dense_of(Z0)
    assert np.isfinite(D0).all() and np.allclose(D0, 2.0j * Xd, rtol=0, atol=1e-6)


@pytest.mark.parametrize("complex_values", [True, False])
def test_propagator_matches_expm(dev, complex_values):
    n, dt, order = 240, 0.05, 10
    H = _hermitian_hm(n, [0, 1, 3, 17], 7, dev, complex_values)
    Hd = dense_of(H).astype(np.complex128)
    assert np.allclose(Hd, Hd.conj().T)
    U = chain.propagator(H, dt, order)
    assert U.values.dtype == torch.complex64
    Ud = dense_of(U)
    want = scipy.linalg.expm(-1j * dt * Hd)
    nrm = np.abs(Hd).sum(axis=1).max() * dt          # ||dt H||_inf
    trunc = nrm ** (order + 1) / math.factorial(order + 1) * math.exp(nrm)
    bound = 1e-5 * order * scipy.linalg.expm(dt * np.abs(Hd)) + trunc
    assert np.all(np.abs(Ud - want) <= bound), float((np.abs(Ud - want) / bound).max())
    assert np.allclose(Ud @ Ud.conj().T, np.eye(n), atol=1e-5)


def test_propagator_applied_by_spmv_matches_lanczos(dev):
    """n = 2^20 (the 7-point stencil of SpGEMM config 4): U psi by the
    complex SpMV on Recon(U) against the Lanczos propagator of the same H."""
    H = hm_stencil7(128, 128, 64, device=dev)
    n = H.n
    dt, order = 0.05, 8
    U = chain.propagator(H, dt, order)
    u_off, u_val = chain.to_recon(U)
    h_off, h_val = chain.to_recon(H)
    g = torch.Generator(device=dev).manual_seed(3)
    psi = torch.complex(torch.randn(n, device=dev, generator=g),
                        torch.randn(n, device=dev, generator=g)).contiguous()
    up = spmv_recon(u_off, u_val, n, n, psi)
    kr = expm_krylov(h_off, h_val, n, psi, dt, 20)
    nrm = torch.linalg.vector_norm(psi.to(torch.complex128)).item()
    diff = torch.linalg.vector_norm((up - kr.psi).to(torch.complex128)).item()
    assert diff <= 2e-5 * nrm, diff / nrm
    assert abs(torch.linalg.vector_norm(up.to(torch.complex128)).item() - nrm) <= 2e-5 * nrm
