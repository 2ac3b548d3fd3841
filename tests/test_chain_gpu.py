"""Matrix-power chain and Taylor series on the GPU (diagpu_amd.chain over
diagpu_spgemm_symbolic / diagpu_spgemm_numeric_f32 / diagpu_dia_axpby_f32).

The reference describes the chain (spmspm/gather_flat.cuh:13-14,110-117) but
ships no driver, so there is no reference output to match; the checks are
the mathematics:
  - powers against dense float64 matrix powers, |err| <= 1e-5 * k * (|H|^k);
  - the Taylor sum against scipy.linalg.expm, |err| <= 1e-5 * order *
    expm(t|H|) + the series' truncation bound;
  - at 2^20 rows, S x against the float64 recurrence sum_k t^k/k! H^k x;
  - the diagonal set of every result equals the offset sumset.
"""
import math

import numpy as np
import pytest
import scipy.linalg
import torch

from diagpu_amd import chain
from diagpu_amd.workloads import HM, hm_random, hm_stencil7
from hm_host import dense_of, matvec64

pytestmark = pytest.mark.gpu


def _sumset(a, b, n):
    return sorted({x + y for x in a for y in b if abs(x + y) < n})


def test_axpby_union(dev):
    n = 333
    X = hm_random(n, [-5, 0, 2], 1, dev)
    Y = hm_random(n, [-5, 1, 2, 100], 2, dev)
    Z = chain.axpby(0.75, X, -1.5, Y)
    assert Z.offsets.cpu().tolist() == [-5, 0, 1, 2, 100]
    Xd, Yd = dense_of(X), dense_of(Y)
    want = 0.75 * Xd - 1.5 * Yd
    bound = 0.75 * np.abs(Xd) + 1.5 * np.abs(Yd)
    assert np.all(np.abs(dense_of(Z) - want) <= 1.2e-7 * bound)


def test_axpby_zero_factor_does_not_read(dev):
    n = 100
    X = hm_random(n, [-1, 0, 1], 3, dev)
    Y = hm_random(n, [0, 4], 4, dev)
    Y.values.fill_(float("nan"))
    Z = chain.axpby(2.0, X, 0.0, Y)
    assert Z.offsets.cpu().tolist() == [-1, 0, 1, 4]
    D = dense_of(Z)
    assert np.isfinite(D).all()
    assert np.array_equal(D, 2.0 * dense_of(X))   # exact: scaling by 2


def test_axpby_rejects_unsorted(dev):
    n = 50
    X = hm_random(n, [0, 1], 5, dev)
    # the same values under descending offsets (no host copy of them)
    X = HM(n, torch.tensor([1, 0], dtype=torch.int32, device=dev), X.lengths, X.starts, X.values)
    with pytest.raises(ValueError):
        chain.axpby(1.0, X, 1.0, None)


@pytest.mark.parametrize("n,offs,k", [
    (257, [-3, -1, 0, 1, 4], 5),
    (300, [-2, 1], 4),                       # no main diagonal: parity classes
    (200, [-150, -2, 0, 7, 120], 3),         # offsets near n: clipped sumset
    (1000, [-16, -4, -1, 0, 1, 4, 16], 6),
])
def test_power_against_dense(dev, n, offs, k):
    H = hm_random(n, offs, 10 + k, dev)
    P = chain.power(H, k)
    Hd = dense_of(H)
    want = np.linalg.matrix_power(Hd, k)
    bound = np.linalg.matrix_power(np.abs(Hd), k)
    expect = offs
    for _ in range(k - 1):
        expect = _sumset(expect, offs, n)
    assert P.offsets.cpu().tolist() == expect
    err = np.abs(dense_of(P) - want)
    assert np.all(err <= 1e-5 * k * bound + 1e-30), float((err / (bound + 1e-30)).max())


@pytest.mark.parametrize("n,offs,t,order", [
    (240, [-3, -1, 0, 1, 4], 0.2, 12),
    (180, [-2, 1], 0.5, 14),
])
def test_taylor_against_expm(dev, n, offs, t, order):
    H = hm_random(n, offs, 7, dev)
    stats = chain.ChainStats()
    S = chain.taylor_expm(H, t, order, stats)
    assert len(stats.numeric) == order - 1 and len(stats.axpby) == 2 * order - 1
    Hd = dense_of(H)
    want = scipy.linalg.expm(t * Hd)
    bound = scipy.linalg.expm(t * np.abs(Hd))
    norm = t * np.abs(Hd).sum(axis=1).max()
    trunc = norm ** (order + 1) / math.factorial(order + 1) * math.exp(norm)
    err = np.abs(dense_of(S) - want)
    assert np.all(err <= 1e-5 * order * bound + trunc)
    # every offset reachable in at most `order` steps is present
    reach, frontier = {0}, [0]
    for _ in range(order):
        frontier = _sumset(frontier, offs, n)
        reach |= set(frontier)
    assert S.offsets.cpu().tolist() == sorted(reach)


def test_host_offsets_follow_the_device(dev):
    """The host copies of the offsets that products and sums carry (so the
    chain needs no device read-back per step) equal the device offsets: the
    sumset for products, sums past n dropped, and the union for axpby."""
    n = 40
    A = hm_random(n, [-39, -7, 0, 3, 30], 14, dev)
    B = hm_random(n, [-20, -1, 0, 9, 39], 15, dev)
    for M in (chain.multiply(A, B), chain.multiply(B, A), chain.power(A, 3),
              chain.axpby(1.0, A, 2.0, B), chain.axpby(3.0, A, 0.0, None),
              chain.taylor_expm(B, 0.1, 3), chain.taylor_expm(A, 0.2j, 2)):
        assert M.host_offsets is not None
        assert M.host_offsets == M.offsets.cpu().tolist()


def test_add_identity_in_place_and_union(dev):
    n = 90
    S = hm_random(n, [-3, 0, 2], 12, dev)
    before = dense_of(S)
    ptr = S.values.data_ptr()
    T = chain.add_identity(S, 0.5)
    assert T is S and T.values.data_ptr() == ptr        # main diagonal present: in place
    want = before.astype(np.float32) + np.float32(0.5) * np.eye(n, dtype=np.float32)  # one fp32 rounding
    assert np.array_equal(dense_of(T), want.astype(np.float64))
    U = hm_random(n, [-3, 2], 13, dev)
    V = chain.add_identity(U, 2.0)                       # no main diagonal: union
    assert V.offsets.cpu().tolist() == [-3, 0, 2]
    assert np.array_equal(dense_of(V), dense_of(U) + 2.0 * np.eye(n))


def test_identity_cache_across_streams(dev):
    """The cached identity is filled on the stream of its first caller; a
    caller on another stream must wait for that fill.  The first stream is
    held busy (a bounded spin) so its fill runs late: the second stream's
    union must still see ones on the main diagonal."""
    n = 700_001
    chain._UNITS.clear()
    s1, s2 = torch.cuda.Stream(device=dev), torch.cuda.Stream(device=dev)
    U1 = hm_random(n, [-3, 2], 21, dev)
    U2 = hm_random(n, [-1, 5], 22, dev)
    torch.cuda.synchronize()
    with torch.cuda.stream(s1):
        torch.cuda._sleep(20_000_000)
    V1 = chain.add_identity(U1, 2.0, stream=s1)
    V2 = chain.add_identity(U2, 3.0, stream=s2)
    torch.cuda.synchronize()
    for V, U, sg, offs in ((V1, U1, 2.0, [-3, 0, 2]), (V2, U2, 3.0, [-1, 0, 5])):
        assert V.offsets.cpu().tolist() == offs
        st = V.starts.cpu().tolist()
        main = V.values[st[1]: st[1] + n]
        assert torch.all(main == sg).item()
        for k, j in ((0, 0), (2, 1)):      # the other diagonals are U's, unchanged
            ln = n - abs(offs[k])
            src = U.values[U.starts[j].item(): U.starts[j].item() + ln]
            assert torch.equal(V.values[st[k]: st[k] + ln], src)
    I, _, readers = next(iter(chain._UNITS.values()))
    assert {s1.cuda_stream, s2.cuda_stream} <= readers
    chain._UNITS.clear()


def test_taylor_order_zero_is_identity(dev):
    H = hm_random(64, [-1, 1], 9, dev)
    S = chain.taylor_expm(H, 1.0, 0)
    assert np.array_equal(dense_of(S), np.eye(64))


def test_taylor_stencil_2pow20(dev):
    """The 7-point stencil of SpGEMM config 4 (n = 2^20), order 4:
    S x against sum_k t^k/k! H^k x in float64 for a random x."""
    H = hm_stencil7(128, 128, 64, dev)
    t, order = 0.05, 4
    S = chain.taylor_expm(H, t, order)
    assert S.ndiag == 129            # |a| + |b| + |c| <= 4 in three dimensions
    rng = np.random.default_rng(0)
    x = rng.uniform(-1.0, 1.0, H.n)
    want, v = x.copy(), x.copy()
    for k in range(1, order + 1):
        v = matvec64(H, v)
        want += t ** k / math.factorial(k) * v
    got = matvec64(S, x)
    # the stencil's absolute row sums are <= 12, so sum_k t^k/k! (|H|^k |x|) <= this
    abs_bound = sum((t * 12) ** k / math.factorial(k) for k in range(order + 1)) * np.abs(x).max()
    assert np.all(np.abs(got - want) <= 1e-5 * order * abs_bound)


def test_complex_chain_order_and_kernel(dev):
    """Complex chain steps put the narrow factor first where the complex
    A-stationary kernel holds it (at most DIAGPU_ASTAT_MAX_A_C64 diagonals),
    and that kernel then takes the 7-point stencil's steps at n = 2^20; the
    narrow-first product equals the wide-first one to fp32 rounding (the
    factors commute; only the order of the terms differs)."""
    from diagpu_amd import _lib
    from diagpu_amd.spgemm import SpgemmPlan
    H = chain.as_complex(hm_stencil7(128, 128, 64, dev))
    Hj = chain.axpby(-0.01j, H, 0.0, None)
    S = chain.axpby(1.0, chain.multiply(Hj, Hj), 1.0, chain.identity(H.n, dev, torch.complex64))
    assert chain._narrow_first(Hj)
    assert SpgemmPlan(Hj, S).kernel_for(torch.complex64) == "astat"
    C1, C2 = chain.multiply(Hj, S), chain.multiply(S, Hj)
    assert C1.offsets.cpu().tolist() == C2.offsets.cpu().tolist()
    err = (C1.values - C2.values).abs().max().item()
    assert err <= 1e-6 * C1.values.abs().max().item()
    wide = chain.as_complex(hm_random(4096, list(range(-_lib.ASTAT_MAX_A_C64, 1)), 3, dev))
    assert not chain._narrow_first(wide)
    assert chain._narrow_first(hm_random(4096, list(range(-200, 1)), 3, dev))   # fp32: always


# ---- the fused Horner step (diagpu_spgemm_numeric_astat_scaled_*) ----------

_S7 = [-16384, -128, -1, 0, 1, 128, 16384]      # the 7-point stencil's offsets at n = 2^20


def _with_main(C_vals, C_offsets, C_starts, n, sigma):
    """C + sigma I where C has a main diagonal (offset 0), in fp32/c64."""
    out = C_vals.clone()
    offs = C_offsets.cpu().tolist()
    if 0 in offs:
        s = int(C_starts[offs.index(0)])
        out[s: s + n] += sigma
    return out


@pytest.mark.parametrize("n,a_offs,b_offs", [
    (8192, [-3, -1, 0, 1, 4], [-40, -2, 0, 5, 9, 33]),             # 4 rows per lane
    (8192, list(range(-20, 21, 2)), list(range(-30, 31, 3))),       # four-entry batches
    (1 << 20, [-16384, -128, -1, 0, 1, 128, 16384], [-2, 0, 3]),    # 16 rows per lane
    (1 << 20, _S7, _sumset(_sumset(_S7, _S7, 1 << 20), _S7, 1 << 20)),  # 8 rows per lane
    (6000, [-2, 1], [-5, 3]),                                       # C without a main diagonal
    (1 << 18, [-700, -3, 0, 2, 900], [-4000, -10, 0, 10, 4000]),    # the longer last block
])
def test_numeric_scaled_f32_bits(dev, n, a_offs, b_offs):
    """C = (alpha A) B + sigma I from one fused pass has the bits of the
    plain A-stationary product on the operand fl(alpha A) (scaled by torch)
    with fl(c + sigma) added to the main diagonal, for every rows-per-lane
    layout the kernel chooses; sigma is dropped where C has no main diagonal."""
    from diagpu_amd.spgemm import SpgemmPlan
    A, B = hm_random(n, a_offs, 21, dev), hm_random(n, b_offs, 22, dev)
    plan = SpgemmPlan(A, B)
    assert plan.kernel_for(torch.float32) == "astat"
    alpha, sigma = 0.37, 1.0
    fused = plan.multiply(A.values, B.values)                     # buffer of the right size
    plan.numeric_scaled(A.values, B.values, fused, alpha, sigma)
    scaled = (A.values * torch.tensor(alpha, dtype=torch.float32, device=dev)).contiguous()
    plain = plan.multiply(scaled, B.values, kernel="astat")
    want = _with_main(plain, plan.c_offsets(), plan.c_starts(), n, sigma)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int32), want.view(torch.int32))
    # a second call on the same C buffer overwrites it (nothing accumulates)
    plan.numeric_scaled(A.values, B.values, fused, alpha, sigma)
    assert torch.equal(fused.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("n,a_offs,b_offs", [
    (1 << 20, [-16384, -128, -1, 0, 1, 128, 16384], [-129, -1, 0, 2, 16385]),
    (8192, [-3, -1, 0, 1, 4], [-40, -2, 0, 5, 9, 33]),
])
def test_numeric_scaled_c64(dev, n, a_offs, b_offs):
    """Complex values: the fused pass against the plain product of the
    operand alpha A scaled by torch, within 1e-6 of |alpha| sum |a| |b|
    (plus |sigma| on the main diagonal); the bound's sums come from the same
    plan on |A|, |B| in fp32."""
    from diagpu_amd.spgemm import SpgemmPlan
    Ar, Br = hm_random(n, a_offs, 23, dev), hm_random(n, b_offs, 24, dev)
    A = chain.as_complex(Ar)
    B = chain.as_complex(Br)
    A.values = torch.complex(Ar.values, torch.roll(Ar.values, 3)).contiguous()
    B.values = torch.complex(Br.values, -torch.roll(Br.values, 5)).contiguous()
    plan = SpgemmPlan(A, B)
    assert plan.kernel_for(torch.complex64) == "astat"
    alpha, sigma = complex(0.0, -0.02), complex(1.0, 0.5)
    fused = plan.multiply(A.values, B.values)
    plan.numeric_scaled(A.values, B.values, fused, alpha, sigma)
    scaled = (A.values * alpha).contiguous()
    want = _with_main(plan.multiply(scaled, B.values, kernel="astat"), plan.c_offsets(),
                      plan.c_starts(), n, sigma)
    ab = plan.multiply(A.values.abs().contiguous(), B.values.abs().contiguous(), kernel="gather")
    bound = 1e-6 * (abs(alpha) * ab + abs(sigma)) + 1e-30
    torch.cuda.synchronize()
    assert bool(((fused - want).abs() <= bound).all())


def test_numeric_scaled_limits_and_forced_plans(dev):
    """numeric_scaled refuses a plan the A-stationary kernel cannot take
    (n < 4096) and takes one the automatic choice leaves to another kernel
    (the tridiagonal square at n = 2^19 goes to the gather), with the same
    bits as the forced plain kernel on the torch-scaled operand."""
    from diagpu_amd.spgemm import SpgemmPlan
    A = hm_random(1000, [-1, 0, 1], 25, dev)
    plan = SpgemmPlan(A, A)
    C = plan.multiply(A.values, A.values)
    with pytest.raises(ValueError):
        plan.numeric_scaled(A.values, A.values, C, 2.0, 1.0)
    n = 1 << 19
    A = hm_random(n, [-1, 0, 1], 26, dev)
    plan = SpgemmPlan(A, A)
    assert plan.kernel_for(torch.float32) == "gather"
    fused = plan.multiply(A.values, A.values)
    plan.numeric_scaled(A.values, A.values, fused, -1.5, 2.0)
    scaled = (A.values * torch.tensor(-1.5, dtype=torch.float32, device=dev)).contiguous()
    want = _with_main(plan.multiply(scaled, A.values, kernel="astat"), plan.c_offsets(),
                      plan.c_starts(), n, 2.0)
    torch.cuda.synchronize()
    assert torch.equal(fused.view(torch.int32), want.view(torch.int32))


@pytest.mark.parametrize("complex_values", [False, True])
def test_fused_chain_matches_unfused(dev, monkeypatch, complex_values):
    """The Taylor chain with its fused Horner steps against the same chain
    with every step unfused (scaling pass, product, identity add): the same
    offsets, the same fp32 bits (no scaled element of the stencil is
    subnormal), complex values within 1e-6 of the result's largest element;
    the phase-synchronised form takes the fused steps too (one axpby: the
    first step's I + (t/order) H) and gives the same values."""
    H = hm_stencil7(128, 128, 64, dev)
    t, order = (complex(0.0, -0.02), 6) if complex_values else (0.05, 6)
    S1 = chain.taylor_expm(H, t, order)
    st = chain.ChainStats()
    S2 = chain.taylor_expm(H, t, order, st)
    monkeypatch.setattr(chain, "_fused", lambda plan, H: False)
    S0 = chain.taylor_expm(H, t, order)
    torch.cuda.synchronize()
    assert len(st.axpby) == 1 and len(st.numeric) == order - 1
    assert S1.offsets.cpu().tolist() == S0.offsets.cpu().tolist() == S2.offsets.cpu().tolist()
    assert torch.equal(S1.values, S2.values)
    if complex_values:
        tol = 1e-6 * S0.values.abs().max().item()
        assert (S1.values - S0.values).abs().max().item() <= tol
    else:
        assert torch.equal(S1.values.view(torch.int32), S0.values.view(torch.int32))


def test_fused_chain_without_main_diagonal(dev, monkeypatch):
    """A Taylor chain whose H has no main diagonal, at an n the fused steps
    take: S_4 = I + (t/4) H gets a structure of its own (the first plan then
    waits for it on the caller's stream), a product without a main diagonal
    takes sigma = 0 and I on the union, the next one sigma = 1 in the kernel;
    the same offsets and bits as with every step unfused, and against the
    float64 recurrence for S x."""
    n, t, order = 8192, 0.3, 4
    H = hm_random(n, [-2, 1], 31, dev)
    S1 = chain.taylor_expm(H, t, order)
    monkeypatch.setattr(chain, "_fused", lambda plan, H: False)
    S0 = chain.taylor_expm(H, t, order)
    torch.cuda.synchronize()
    assert S1.offsets.cpu().tolist() == S0.offsets.cpu().tolist()
    assert torch.equal(S1.values.view(torch.int32), S0.values.view(torch.int32))
    rng = np.random.default_rng(1)
    x = rng.uniform(-1.0, 1.0, n)
    want, v = x.copy(), x.copy()
    for k in range(1, order + 1):
        v = matvec64(H, v)
        want += t ** k / math.factorial(k) * v
    assert np.all(np.abs(matvec64(S1, x) - want) <= 1e-5 * order * math.exp(2 * t))


@pytest.mark.parametrize("complex_values", [False, True])
def test_power_pipelined_matches_synced(dev, complex_values):
    """power() with its plans built beside the products (no stats) against
    the phase-synchronised chain (stats) on the 7-point stencil at n = 2^20:
    the same offsets and the same bits (the same kernels in the same order
    on the same operands), and the host offsets it carries equal the
    device's."""
    H = hm_stencil7(128, 128, 64, dev)
    if complex_values:
        H = chain.as_complex(H)
        H.values = torch.complex(H.values.real, 0.25 * torch.roll(H.values.real, 7)).contiguous()
    P1 = chain.power(H, 5)
    P2 = chain.power(H, 5, chain.ChainStats())
    torch.cuda.synchronize()
    assert P1.offsets.cpu().tolist() == P2.offsets.cpu().tolist() == P1.host_offsets
    assert torch.equal(P1.values.view(torch.int32), P2.values.view(torch.int32))
