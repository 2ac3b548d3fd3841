"""SpGEMM and gemm_diag parity on the GPU, through the C ABI.

Integer outputs (C offsets, lengths, starts, lookup, pair_ptr, every GPair
field, counts) must equal the oracle's restatement of the reference planners
bit for bit.  Values: |C - C64| <= 1e-5 * sum |a * b| per element, C64 the
oracle's fp64 result (1e-5 relative to the absolute term sum; any fp32
summation of <= 166 products satisfies it).
"""
import numpy as np
import pytest
import torch

from diagpu_amd import _lib, workloads
from diagpu_amd.spgemm import SpgemmPlan, gemm_diag

pytestmark = pytest.mark.gpu
TOL = 1e-5


def host(M):
    return (M.offsets.cpu().numpy(), M.lengths.cpu().numpy(), M.starts.cpu().numpy(),
            M.values.cpu().numpy())


def check_plan(oracle, plan, A, B):
    n = A.n
    a, b = host(A), host(B)
    c_off, c_len, c_st, nnz = oracle.c_structure(n, a[0], b[0])
    assert plan.info.c_ndiag == len(c_off)
    assert plan.info.c_nnz == nnz
    assert np.array_equal(plan.c_offsets().cpu().numpy(), c_off)
    assert np.array_equal(plan.c_lengths().cpu().numpy(), c_len)
    assert np.array_equal(plan.c_starts().cpu().numpy(), c_st)
    ptr, pairs = oracle.pairs_only(n, a[0], a[1], a[2], b[0], b[1], b[2], c_off)
    assert np.array_equal(plan.pair_ptr().cpu().numpy(), ptr)
    assert plan.info.n_pairs == ptr[-1]
    got = plan.pairs_numpy()
    for f in ("ab", "bb", "ash", "bsh", "al", "bl"):
        assert np.array_equal(got[f], pairs[f]), f
    counts = np.diff(ptr)
    assert plan.info.max_pairs == (counts.max() if len(counts) else 0)
    for M, ext in ((a, plan.info.a_extent), (b, plan.info.b_extent)):
        assert ext == (int((M[2] + M[1]).max()) if len(M[0]) else 0)
    # useful flops: 2 * sum over pairs of n - max(|da|, |db|, |dc|)
    dc = np.repeat(c_off.astype(np.int64), counts)
    b_of = {int(s): int(o) for s, o in zip(b[2], b[0])}
    db = np.array([b_of[int(s)] for s in pairs["bb"]], np.int64)
    da = dc - db
    assert plan.info.useful_flops == int(2 * (n - np.maximum(np.maximum(abs(da), abs(db)),
                                                               abs(dc))).sum())
    if plan.lookup is not None:
        assert np.array_equal(plan.lookup.cpu().numpy(), oracle.c_lookup(n, c_off))
    return c_off, c_len, c_st, nnz, ptr, pairs


def check_values(got, want, absum):
    err = np.abs(got.astype(np.float64) - want)
    bad = err > TOL * absum + 1e-300
    assert not bad.any(), f"{int(bad.sum())} values out of bound, max err {err.max():.3e}"


def rand_case(rng, n, na, nb, span):
    oa = rng.choice(np.arange(-span, span + 1), size=na, replace=False)
    ob = rng.choice(np.arange(-span, span + 1), size=nb, replace=False)
    return oa, ob


@pytest.mark.parametrize("seed,n,na,nb,span", [
    (0, 16, 3, 3, 15), (1, 37, 5, 4, 36), (2, 257, 9, 7, 256), (3, 1000, 12, 30, 999),
    (4, 3001, 40, 8, 2999), (5, 5000, 3, 60, 100), (6, 1031, 64, 64, 1030),
])
def test_random_products(dev, oracle, seed, n, na, nb, span):
    rng = np.random.default_rng(seed)
    oa, ob = rand_case(rng, n, na, nb, span)
    A = workloads.hm_random(n, oa, seed=seed, device=dev)
    B = workloads.hm_random(n, ob, seed=seed + 100, device=dev)
    if seed % 2:   # B in non-ascending order: plan order must follow B's array order
        perm = torch.as_tensor(rng.permutation(nb), device=dev)
        B = workloads.HM(n, B.offsets[perm].contiguous(), B.lengths[perm].contiguous(),
                         B.starts[perm].contiguous(), B.values)
    plan = SpgemmPlan(A, B, want_lookup=True)
    c_off, c_len, c_st, nnz, ptr, pairs = check_plan(oracle, plan, A, B)
    Cv = plan.multiply(A.values, B.values)
    C2 = plan.multiply(A.values, B.values)
    torch.cuda.synchronize()
    assert torch.equal(Cv, C2), "run-to-run results differ"
    want, ab = oracle.spgemm_pairs_f64(A.values.cpu().numpy(), B.values.cpu().numpy(), c_len,
                                       c_st, ptr, pairs, 0, len(c_off))
    check_values(Cv.cpu().numpy(), want, ab)
    if n <= 300:   # brute-force dense product
        from test_oracle import hm_to_dense
        a, b = host(A), host(B)
        P = hm_to_dense(n, a[0], a[2], a[3]) @ hm_to_dense(n, b[0], b[2], b[3])
        g = Cv.cpu().numpy()
        for d, s, ln in zip(c_off, c_st, c_len):
            sr, sc = (0, d) if d >= 0 else (-d, 0)
            assert np.allclose(g[s:s + ln], P[sr + np.arange(ln), sc + np.arange(ln)],
                               rtol=0, atol=1e-5)


@pytest.mark.parametrize("n,offs_a,offs_b", [
    # offset spans beyond the one-launch path's LDS: the multi-launch symbolic path
    ((1 << 22) + 3, [-(1 << 22) - 2, -5, 0, 7, (1 << 22) + 2], [-3, 0, 1, (1 << 21)]),
    (600_000, [-599_999, 0, 599_999], [-599_999, -1, 2, 599_999]),
])
def test_symbolic_wide_spans(dev, oracle, n, offs_a, offs_b):
    A = workloads.hm_random(n, offs_a, seed=81, device=dev)
    B = workloads.hm_random(n, offs_b, seed=82, device=dev)
    plan = SpgemmPlan(A, B, want_lookup=True)
    c_off, c_len, c_st, nnz, ptr, pairs = check_plan(oracle, plan, A, B)
    Cv = plan.multiply(A.values, B.values)
    want, ab = oracle.spgemm_pairs_f64(A.values.cpu().numpy(), B.values.cpu().numpy(), c_len,
                                       c_st, ptr, pairs, 0, len(c_off))
    check_values(Cv.cpu().numpy(), want, ab)


def test_symbolic_large_product(dev, oracle):
    """1100 x 1000 diagonals (1.1M pairs, more than the one-launch path
    enumerates): the multi-launch path, bit-exact."""
    n = 1200
    rng = np.random.default_rng(17)
    oa = rng.choice(np.arange(-n + 1, n), size=1100, replace=False)
    ob = rng.choice(np.arange(-n + 1, n), size=1000, replace=False)
    A = workloads.hm_random(n, oa, seed=83, device=dev)
    B = workloads.hm_random(n, ob, seed=84, device=dev)
    plan = SpgemmPlan(A, B, want_lookup=True)
    assert plan.info.n_pairs > 1 << 20 or len(oa) * len(ob) > 1 << 20
    check_plan(oracle, plan, A, B)


def test_reference_bench_operands(dev, oracle):
    """make_banded(100000, 16, 1234 / 5678) of spmspm/bench_spmspm.cu:465-466,
    values checked against the cpu_dia_spgemm loop (:376-408) in fp64."""
    n, w = 100000, 16
    A = workloads.hm_from_values(n, oracle.make_banded(n, w, 1234)[0],
                                 torch.as_tensor(oracle.make_banded(n, w, 1234)[3], device=dev),
                                 device=dev)
    B = workloads.hm_from_values(n, oracle.make_banded(n, w, 5678)[0],
                                 torch.as_tensor(oracle.make_banded(n, w, 5678)[3], device=dev),
                                 device=dev)
    plan = SpgemmPlan(A, B)
    c_off, c_len, c_st, nnz, ptr, pairs = check_plan(oracle, plan, A, B)
    assert len(c_off) == 4 * w + 1
    Cv = plan.multiply(A.values, B.values).cpu().numpy()
    want, ab = oracle.spgemm_gather_f64(n, host(A), host(B), (c_off, c_len, c_st, nnz))
    check_values(Cv, want, ab)


def test_config4_full_size(dev, oracle):
    A, B = workloads.spgemm_config(4, seed=4, device=dev)
    plan = SpgemmPlan(A, B)
    c_off, c_len, c_st, nnz, ptr, pairs = check_plan(oracle, plan, A, B)
    assert (len(c_off), int(ptr[-1]), nnz) == (47, 63, 48_985_826)
    Cv = plan.multiply(A.values, B.values).cpu().numpy()
    want, ab = oracle.spgemm_pairs_f64(A.values.cpu().numpy(), B.values.cpu().numpy(), c_len,
                                       c_st, ptr, pairs, 0, len(c_off))
    check_values(Cv, want, ab)


def _c_matvec_gpu(plan, Cv, v, transpose=False):
    """C v (or v^T C) on the device in fp64, diagonal by diagonal."""
    n = plan.n
    vd = torch.as_tensor(v, dtype=torch.float64, device=Cv.device)
    y = torch.zeros(n, dtype=torch.float64, device=Cv.device)
    offs = plan.c_offsets().cpu().tolist()
    lens = plan.c_lengths().cpu().tolist()
    sts = plan.c_starts().cpu().tolist()
    for d, ln, s in zip(offs, lens, sts):
        r0, c0 = (0, d) if d >= 0 else (-d, 0)
        if transpose:
            r0, c0 = c0, r0
        y[r0:r0 + ln] += Cv[s:s + ln].double() * vd[c0:c0 + ln]
    return y.cpu().numpy()


def _hm_matvec(n, M, v, transpose=False):
    """(M v) and (|M| |v|) in fp64 for an HM matrix on the host (M^T with
    transpose)."""
    off, ln, st, val = M
    y = np.zeros(n)
    ya = np.zeros(n)
    for d, l, s in zip(off, ln, st):
        r0, c0 = (0, d) if d >= 0 else (-d, 0)
        if transpose:
            r0, c0 = c0, r0
        seg = val[s:s + l].astype(np.float64)
        y[r0:r0 + l] += seg * v[c0:c0 + l]
        ya[r0:r0 + l] += np.abs(seg) * np.abs(v[c0:c0 + l])
    return y, ya


def _check_products(plan, Cv, A, B, seed):
    """All of C through C v = A (B v) and v^T C = (v^T A) B for a random v:
    a value written to a wrong position or diagonal changes both (a row sum
    alone misses a value moved between two C diagonals of one row).  Bound:
    1e-5 |A| |B| |v| (each C element is within 1e-5 of its term sum)."""
    n = A.n
    v = np.random.default_rng(seed).standard_normal(n)
    got = _c_matvec_gpu(plan, Cv, v)
    bv, bva = _hm_matvec(n, host(B), v)
    want, _ = _hm_matvec(n, host(A), bv)
    _, bound = _hm_matvec(n, host(A), bva)
    assert np.all(np.abs(got - want) <= TOL * bound + 1e-300), "C v"
    got = _c_matvec_gpu(plan, Cv, v, transpose=True)
    av, ava = _hm_matvec(n, host(A), v, transpose=True)
    want, _ = _hm_matvec(n, host(B), av, transpose=True)
    _, bound = _hm_matvec(n, host(B), ava, transpose=True)
    assert np.all(np.abs(got - want) <= TOL * bound + 1e-300), "v^T C"


def test_config5_full_size(dev, oracle):
    """n = 262144, 128 x 128 random offsets: plan exact; the automatic choice
    (the A-stationary kernel, 128 A diagonals in LDS) bit-identical to the
    gather; values exact to the bound on a sample of C diagonals; all of C
    through C v = A (B v) and v^T C = (v^T A) B."""
    A, B = workloads.spgemm_config(5, seed=5, device=dev)
    plan = SpgemmPlan(A, B)
    c_off, c_len, c_st, nnz, ptr, pairs = check_plan(oracle, plan, A, B)
    assert nnz > 2**31                       # int64 starts are required
    assert plan.kernel_for() == "astat"
    Cv = plan.multiply(A.values, B.values)
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    assert torch.equal(Cv.view(torch.int32), Cg.view(torch.int32))
    del Cg
    torch.cuda.synchronize()
    Av, Bv = A.values.cpu().numpy(), B.values.cpu().numpy()
    rng = np.random.default_rng(0)
    counts = np.diff(ptr)
    ks = sorted({0, len(c_off) - 1, int(np.argmax(counts)), *rng.choice(len(c_off), 48).tolist()})
    for k in ks:
        want, ab = oracle.spgemm_pairs_f64(Av, Bv, c_len, c_st, ptr, pairs, k, k + 1)
        got = Cv[int(c_st[k]):int(c_st[k]) + int(c_len[k])].cpu().numpy()
        check_values(got, want, ab)
    _check_products(plan, Cv, A, B, seed=5)


@pytest.mark.parametrize("n,offs_a,offs_b", [
    (4096, list(range(-10, 11)), list(range(-10, 11))),          # gemm_diag.cu:467-486 defaults
    (3000, [-700, -9, -2, 0, 1, 33, 512], [-1000, -5, 0, 3, 4, 900]),   # non-contiguous offsets
    (1025, [-1024, 0, 1024], [-1, 1]),
])
def test_gemm_diag(dev, oracle, n, offs_a, offs_b):
    DA = oracle.pack_diag_matrix(n, offs_a, 42)
    DB = oracle.pack_diag_matrix(n, offs_b, 137)
    oa = torch.tensor(offs_a, dtype=torch.int32, device=dev)
    ob = torch.tensor(offs_b, dtype=torch.int32, device=dev)
    plan, Cv = gemm_diag(n, oa, torch.as_tensor(DA, device=dev).reshape(-1), ob,
                         torch.as_tensor(DB, device=dev).reshape(-1))
    c_off, c_len, c_st, nnz = oracle.c_structure(n, offs_a, offs_b)
    assert np.array_equal(plan.c_offsets().cpu().numpy(), c_off)
    assert np.array_equal(plan.c_starts().cpu().numpy(), c_st)
    lk = oracle.c_lookup(n, c_off)
    assert np.array_equal(plan.lookup.cpu().numpy(), lk)
    want, ab = oracle.gemm_diag_f64(n, DA, offs_a, DB, offs_b, lk, c_st, nnz)
    got = Cv.cpu().numpy()
    check_values(got, want, ab)
    assert np.max(np.abs(got - want)) < 1e-1          # the reference's own bound (:544)


def _hm_dev(dev, n, offs, lens=None):
    offs = list(offs)
    lens = lens or [n - abs(d) for d in offs]
    st = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64)
    return workloads.HM(n, torch.tensor(offs, dtype=torch.int32, device=dev),
                        torch.tensor(lens, dtype=torch.int32, device=dev),
                        torch.tensor(st, device=dev),
                        torch.zeros(max(1, sum(lens)), device=dev))


@pytest.mark.parametrize("offs_a,offs_b,lens_a,status", [
    ([0, 3, 3], [0, 1], None, _lib.ERR_DUPLICATE),
    ([0, 1], [-2, -2], None, _lib.ERR_DUPLICATE),
    ([0, 100], [1], None, _lib.ERR_OFFSET),          # |d| >= n
    ([0, -5], [1], [100, 94], _lib.ERR_OFFSET),      # length != n - |d|
])
def test_invalid_operands(dev, offs_a, offs_b, lens_a, status):
    n = 100
    A = _hm_dev(dev, n, offs_a, lens_a)
    B = _hm_dev(dev, n, offs_b)
    with pytest.raises(_lib.DiagpuError) as ei:
        SpgemmPlan(A, B)
    assert ei.value.status == status


def test_capacity_and_empty(dev):
    n = 64
    A = _hm_dev(dev, n, [-3, 0, 3])
    B = _hm_dev(dev, n, [-1, 1])
    plan = SpgemmPlan(A, B)
    assert plan.info.c_ndiag == 6 and plan.info.n_pairs == 6
    plan.p_cap = 5
    with pytest.raises(_lib.DiagpuError) as ei:
        plan.symbolic()
    assert ei.value.status == _lib.ERR_CAPACITY
    plan.p_cap, plan.c_cap = 6, 5
    with pytest.raises(_lib.DiagpuError) as ei:
        plan.symbolic()
    assert ei.value.status == _lib.ERR_CAPACITY
    E = _hm_dev(dev, n, [])
    p2 = SpgemmPlan(A, E)
    assert (p2.info.c_ndiag, p2.info.n_pairs, p2.info.c_nnz) == (0, 0, 0)
    assert p2.pair_ptr().cpu().tolist() == [0]
    # offsets whose sums all leave the matrix
    F = _hm_dev(dev, n, [60, 63])
    p3 = SpgemmPlan(F, _hm_dev(dev, n, [10, 20]))
    assert p3.info.c_ndiag == 0


def test_symbolic_after_operand_rebinding(dev):
    """symbolic() keeps its call's arguments between calls; a plan whose
    operand is rebound (new structure tensors, same diagonal count) builds
    the new operand's plan, equal to a fresh plan's, and the old tensors'
    memory is not read after they are dropped."""
    n = 4000
    A = workloads.hm_random(n, [-30, -2, 0, 9, 400], 71, dev)
    B = workloads.hm_random(n, [-5, 0, 3, 77], 72, dev)
    plan = SpgemmPlan(A, B)
    first = plan.c_offsets().cpu().tolist()
    A2 = workloads.hm_random(n, [-1000, -7, 0, 12, 2500], 73, dev)
    plan.A = A2
    del A
    torch.cuda.empty_cache()
    junk = torch.full((1 << 20,), -9, dtype=torch.int64, device=dev)   # reuses freed blocks
    plan.symbolic()
    ref = SpgemmPlan(A2, B)
    assert plan.c_offsets().cpu().tolist() == ref.c_offsets().cpu().tolist() != first
    assert torch.equal(plan.pair_ptr(), ref.pair_ptr())
    assert np.array_equal(plan.pairs_numpy(), ref.pairs_numpy())
    del junk


@pytest.mark.parametrize("cfg", [1, 2, 3])
def test_square_of_spmv_configs(dev, oracle, cfg):
    """H H for the SpMV configs' matrices (full size): plan exact; values to
    the bound on every C diagonal (configs 1, 2) or on a sample of them
    (config 3, about 1400 C diagonals of 4.2M values), and all of C through
    C v = H (H v) and v^T C = (v^T H) H."""
    A, B = workloads.spgemm_config(cfg, seed=cfg, device=dev)
    plan = SpgemmPlan(A, B)
    c_off, c_len, c_st, nnz, ptr, pairs = check_plan(oracle, plan, A, B)
    Cv = plan.multiply(A.values, B.values)
    torch.cuda.synchronize()
    Av, Bv = A.values.cpu().numpy(), B.values.cpu().numpy()
    if cfg < 3:
        want, ab = oracle.spgemm_pairs_f64(Av, Bv, c_len, c_st, ptr, pairs, 0, len(c_off))
        check_values(Cv.cpu().numpy(), want, ab)
        return
    rng = np.random.default_rng(3)
    counts = np.diff(ptr)
    ks = sorted({0, len(c_off) - 1, int(np.argmax(counts)), *rng.choice(len(c_off), 24).tolist()})
    for k in ks:
        want, ab = oracle.spgemm_pairs_f64(Av, Bv, c_len, c_st, ptr, pairs, k, k + 1)
        got = Cv[int(c_st[k]):int(c_st[k]) + int(c_len[k])].cpu().numpy()
        check_values(got, want, ab)
    _check_products(plan, Cv, A, B, seed=cfg)


@pytest.mark.parametrize("n,offs_a,offs_b", [
    (4096, list(range(-10, 11)), list(range(-10, 11))),       # gemm_diag.cu:467-486 defaults
    (37, [-36, -3, 0, 2, 36], [-30, -1, 0, 5, 36]),            # smaller than one block, edges
    (1000, list(range(-40, 41, 3)), [-999, -7, 0, 1, 998]),    # narrow A, B spanning the matrix
    (70001, list(range(-12, 13)), [-65000, -3, 0, 4, 65000]),  # ragged last block
    (1, [0], [0]),                                             # a 1 x 1 matrix
    (3, [-2, -1, 0, 1, 2], [-2, 0, 1]),                        # every diagonal of 3 x 3
])
def test_band_kernel_same_bits_as_gather(dev, oracle, n, offs_a, offs_b):
    """The LDS-staged band kernel returns the gather kernel's C bit for bit
    (same plan order, same fused multiply-adds, same skipped terms), and its
    entries point every plan entry at its operand diagonals' LDS rows."""
    A = workloads.hm_random(n, offs_a, 11, dev)
    B = workloads.hm_random(n, offs_b, 12, dev)
    plan = SpgemmPlan(A, B)
    pab, info = plan.band_info()
    assert info.eligible and info.a_off_min == min(offs_a) and info.a_off_max == max(offs_a)
    pairs = plan.pairs_numpy()
    a_st, b_st = A.starts.cpu().numpy(), B.starts.cpu().numpy()
    a_idx = np.searchsorted(a_st, pairs["ab"].astype(np.int64))
    b_idx = np.searchsorted(b_st, pairs["bb"].astype(np.int64))
    da = np.asarray(offs_a)[a_idx]
    wb = (256 + max(offs_a) - min(offs_a) + 3) // 4 * 4
    got = pab[: 4 * plan.info.n_pairs].cpu().numpy().reshape(-1, 4)
    assert np.array_equal(got[:, 0], a_idx * 256)
    assert np.array_equal(got[:, 1], b_idx * wb + da - min(offs_a))
    assert np.array_equal(got[:, 2], da) and not got[:, 3].any()
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    Cb = plan.multiply(A.values, B.values, kernel="band")
    assert torch.equal(Cg.view(torch.int32), Cb.view(torch.int32))
    if n <= 5000:
        ptr, c_len, c_st = plan.pair_ptr().cpu().numpy(), plan.c_lengths().cpu().numpy(), plan.c_starts().cpu().numpy()
        want, ab = oracle.spgemm_pairs_f64(A.values.cpu().numpy(), B.values.cpu().numpy(), c_len,
                                           c_st, ptr, pairs, 0, plan.info.c_ndiag)
        check_values(Cb.cpu().numpy(), want, ab)


def test_band_kernel_choice_and_capacity(dev):
    """auto picks the band kernel for gemm_diag's contiguous bands from 1024
    row blocks on (the A-stationary kernel below that) and the gather for
    config 4 (1.3 entries per C diagonal); a plan whose staged operands
    exceed the LDS budget is refused with DIAGPU_ERR_CAPACITY."""
    n = 1 << 14
    A = workloads.hm_random(1 << 18, range(-10, 11), 1, dev)     # 1024 row blocks
    assert SpgemmPlan(A, A).uses_band()
    A17 = workloads.hm_random(1 << 17, range(-10, 11), 1, dev)   # 512: the A-stationary kernel
    p17 = SpgemmPlan(A17, A17)
    assert not p17.uses_band() and p17.kernel_for() == "astat"
    small = workloads.hm_random(n, range(-10, 11), 1, dev)        # 64 row blocks
    ps = SpgemmPlan(small, small)
    assert not ps.uses_band() and ps.kernel_for() == "astat"
    A4, B4 = workloads.spgemm_config(4, seed=4, device=dev)
    p4 = SpgemmPlan(A4, B4)
    assert not p4.uses_band()
    Cg = p4.multiply(A4.values, B4.values, kernel="gather")
    Cb = p4.multiply(A4.values, B4.values, kernel="band")      # eligible, just not chosen
    assert torch.equal(Cg.view(torch.int32), Cb.view(torch.int32))
    wide = workloads.hm_random(n, [-8000, 0, 8000], 3, dev)      # span 16000: B window too big
    narrow = workloads.hm_random(n, range(-8, 9), 4, dev)
    pw = SpgemmPlan(wide, narrow)
    assert not pw.band_info()[1].eligible and not pw.uses_band()
    with pytest.raises(_lib.DiagpuError) as e:                    # refused before any launch
        pw.multiply(wide.values, narrow.values, kernel="band")
    assert e.value.status == _lib.ERR_CAPACITY


def _random_offsets(rng, cnt, lo, hi, with_zero=True):
    offs = set(rng.choice(np.arange(lo, hi + 1), size=cnt, replace=False).tolist())
    if with_zero:
        offs.add(0)
    return sorted(offs)


@pytest.mark.parametrize("n,case", [
    (4096, "band64"),       # 64 random offsets over +-512: the cfg-3 square, small n
    (37, "edges"),          # smaller than one block, offsets reaching +-(n-1)
    (1000, "wideB"),        # narrow A, B spanning the matrix
    (70001, "ragged"),      # ragged last block, B beyond the A window
    (5000, "maxA"),         # DIAGPU_ASTAT_MAX_A A diagonals
    (1, "one"),             # a 1 x 1 matrix: one block, 32 lead rows before row 0
    (3, "three"),           # every diagonal of a 3 x 3 matrix
    (1 << 17, "tail"),      # 512 blocks, the last with 5 rows per lane (513 would take 2 rounds)
    (1 << 20, "short"),     # 25 short C diagonals: 16 rows per lane, 1024 blocks, the last 17
    (1 << 20, "many"),      # 7 x 40 diagonals, > 64 C diagonals: 8 rows per lane, the last 9
    (1 << 18, "quadpf"),    # 64 x 64 over +-256: metadata prefetch, 4-entry batches, 5-row tail
    (4096, "gd"),           # gemm_diag's band: 10.8 entries per C diagonal, 17 blocks split
                            # over 3 workgroups each, 4-entry batches
])
def test_astat_kernel_same_bits_as_gather(dev, oracle, n, case):
    """The A-stationary kernel returns the gather kernel's C bit for bit
    (same plan order, same fused multiply-adds, same skipped terms), and its
    records point every plan entry at its A diagonal with the positions both
    operands hold."""
    rng = np.random.default_rng(n)
    if case == "band64":
        offs_a = _random_offsets(rng, 63, -512, 512)
        offs_b = _random_offsets(rng, 63, -512, 512)
    elif case == "edges":
        offs_a, offs_b = [-36, -3, 0, 2, 36], [-30, -1, 0, 5, 36]
    elif case == "wideB":
        offs_a, offs_b = list(range(-40, 41, 3)), [-999, -7, 0, 1, 998]
    elif case == "ragged":
        offs_a, offs_b = list(range(-12, 13)), [-65000, -3, 0, 4, 65000]
    elif case == "one":
        offs_a, offs_b = [0], [0]
    elif case == "three":
        offs_a, offs_b = [-2, -1, 0, 1, 2], [-2, 0, 1]
    elif case == "tail":
        offs_a = _random_offsets(rng, 40, -3000, 3000)
        offs_b = _random_offsets(rng, 12, -600, 600)
    elif case == "short":
        offs_a = offs_b = [-1024, -32, -1, 0, 1, 32, 1024]
    elif case == "many":
        offs_a = [-1024, -32, -1, 0, 1, 32, 1024]
        offs_b = _random_offsets(rng, 40, -5000, 5000)
    elif case == "gd":
        offs_a = offs_b = list(range(-10, 11))
    elif case == "quadpf":
        offs_a = _random_offsets(rng, 63, -256, 256)
        offs_b = _random_offsets(rng, 63, -256, 256)
    else:
        offs_a = _random_offsets(rng, _lib.ASTAT_MAX_A, -2000, 2000, with_zero=False)
        offs_b = _random_offsets(rng, 9, -100, 100)
    assert len(offs_a) <= _lib.ASTAT_MAX_A
    A = workloads.hm_random(n, offs_a, 21, dev)
    B = workloads.hm_random(n, offs_b, 22, dev)
    plan = SpgemmPlan(A, B)
    if case == "quadpf":      # >= 3 entries per C diagonal, > 64 per wave's share
        assert plan.info.n_pairs >= 3 * plan.info.c_ndiag and plan.info.c_ndiag >= 64
    full = plan.astat_records().cpu().numpy()
    np_ = plan.info.n_pairs
    # after the records: two clear error flags, then A's smallest and largest offset
    assert full[4 * np_: 4 * np_ + 4].tolist() == [0, 0, min(offs_a), max(offs_a)]
    rec = full[: 4 * np_].reshape(-1, 4)
    pairs = plan.pairs_numpy()
    a_st = A.starts.cpu().numpy()
    a_idx = np.searchsorted(a_st, pairs["ab"].astype(np.int64))
    assert np.array_equal(rec[:, 0], a_idx)
    assert np.array_equal(rec[:, 1], np.maximum(0, np.maximum(-pairs["ash"], -pairs["bsh"])))
    assert np.array_equal(rec[:, 2], np.minimum(pairs["al"] - pairs["ash"], pairs["bl"] - pairs["bsh"]))
    assert np.array_equal(rec[:, 3], pairs["bb"].astype(np.int64) + pairs["bsh"])
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    Ca = plan.multiply(A.values, B.values, kernel="astat")
    assert torch.equal(Cg.view(torch.int32), Ca.view(torch.int32))
    if n <= 5000:
        ptr, c_len, c_st = plan.pair_ptr().cpu().numpy(), plan.c_lengths().cpu().numpy(), plan.c_starts().cpu().numpy()
        want, ab = oracle.spgemm_pairs_f64(A.values.cpu().numpy(), B.values.cpu().numpy(), c_len,
                                           c_st, ptr, pairs, 0, plan.info.c_ndiag)
        check_values(Ca.cpu().numpy(), want, ab)


def test_astat_kernel_choice_and_capacity(dev):
    """auto picks the A-stationary kernel for the square of a 64-diagonal
    band over +-512, for gemm_diag's band below 1024 row blocks, for the
    9-point and 5-point stencils' squares, config 4 and config 2's square,
    the band kernel from 1024 row blocks, the gather below n = 4096 and for
    plans of fewer than 16 entries and at least 1.5 per C diagonal at
    2^19 <= n < 2^20 (the tridiagonal square at n = 2^19, not at 2^20, and
    not a random 3 x 3 product at 2^20); more than DIAGPU_ASTAT_MAX_A A
    diagonals are refused with DIAGPU_ERR_CAPACITY."""
    rng = np.random.default_rng(3)
    n = 1 << 18
    offs = _random_offsets(rng, 63, -512, 512)
    H = workloads.hm_random(n, offs, 5, dev)
    p = SpgemmPlan(H, H)
    assert p.kernel_for() == "astat"
    Cg = p.multiply(H.values, H.values, kernel="gather")
    Ca = p.multiply(H.values, H.values)
    assert torch.equal(Cg.view(torch.int32), Ca.view(torch.int32))
    G = workloads.hm_random(1 << 19, range(-10, 11), 1, dev)
    assert SpgemmPlan(G, G).kernel_for() == "band"
    G4 = workloads.hm_random(4096, range(-10, 11), 1, dev)       # gemm_diag's default size
    assert SpgemmPlan(G4, G4).kernel_for() == "astat"
    g5 = workloads.hm_random(2048, range(-10, 11), 1, dev)       # below n = 4096: the gather
    assert SpgemmPlan(g5, g5).kernel_for() == "gather"
    A4, B4 = workloads.spgemm_config(4, seed=4, device=dev)
    assert SpgemmPlan(A4, B4).kernel_for() == "astat"           # 63 entries over 47 C diagonals
    T = workloads.hm_random(1 << 19, [-1, 0, 1], 7, dev)
    assert SpgemmPlan(T, T).kernel_for() == "gather"            # 9 entries at n = 2^19
    T20 = workloads.hm_random(1 << 20, [-1, 0, 1], 7, dev)
    pt = SpgemmPlan(T20, T20)
    assert pt.kernel_for() == "astat"                            # the same at n = 2^20
    assert torch.equal(pt.multiply(T20.values, T20.values).view(torch.int32),
                       pt.multiply(T20.values, T20.values, kernel="gather").view(torch.int32))
    R3a = workloads.hm_random(1 << 20, [-1500, 7, 1900], 7, dev)
    R3b = workloads.hm_random(1 << 20, [-800, 0, 1200], 8, dev)
    pr = SpgemmPlan(R3a, R3b)                                     # 9 entries, one per C diagonal
    assert pr.info.n_pairs == 9 and pr.info.c_ndiag == 9 and pr.kernel_for() == "astat"
    assert torch.equal(pr.multiply(R3a.values, R3b.values).view(torch.int32),
                       pr.multiply(R3a.values, R3b.values, kernel="gather").view(torch.int32))
    nine = sorted({dy * 256 + dx for dx in (-1, 0, 1) for dy in (-1, 0, 1)})
    S9 = workloads.hm_random(1 << 16, nine, 8, dev)
    p9 = SpgemmPlan(S9, S9)
    assert p9.kernel_for() == "astat"
    assert torch.equal(p9.multiply(S9.values, S9.values).view(torch.int32),
                       p9.multiply(S9.values, S9.values, kernel="gather").view(torch.int32))
    S5 = workloads.hm_random(1 << 16, [-256, -1, 0, 1, 256], 8, dev)
    assert SpgemmPlan(S5, S5).kernel_for() == "astat"           # 25 entries
    P2 = workloads.recon_to_hm(workloads.spmv_config(2, seed=1, device=dev))
    assert SpgemmPlan(P2, P2).kernel_for() == "astat"           # the same, at n = 2^22
    wide = workloads.hm_random(4096, _random_offsets(rng, _lib.ASTAT_MAX_A + 1, -300, 300), 6, dev)
    pw = SpgemmPlan(wide, wide)
    assert pw.kernel_for() != "astat"
    with pytest.raises(_lib.DiagpuError) as e:                    # refused before any launch
        pw.multiply(wide.values, wide.values, kernel="astat")
    assert e.value.status == _lib.ERR_CAPACITY


def test_lds_kernels_with_operands_in_any_order(dev):
    """The band and A-stationary kernels look each plan entry's diagonals up
    by their starts: operands whose diagonals are stored out of offset order
    (starts not ascending) give the gather's bits too, and "auto" still
    works on them."""
    rng = np.random.default_rng(9)
    n = 6000

    def shuffled(offs, seed):
        M = workloads.hm_random(n, offs, seed, dev)
        perm = torch.as_tensor(rng.permutation(len(offs)), device=dev)
        return workloads.HM(n, M.offsets[perm].contiguous(), M.lengths[perm].contiguous(),
                            M.starts[perm].contiguous(), M.values)
    A = shuffled(list(range(-10, 11)), 31)
    B = shuffled(list(range(-8, 9)), 32)
    plan = SpgemmPlan(A, B)
    # A's offset extremes after the records, whatever the storage order
    assert plan.astat_records()[4 * plan.info.n_pairs:].cpu().tolist() == [0, 0, -10, 10]
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    for k in ("band", "astat", "auto"):
        Ck = plan.multiply(A.values, B.values, kernel=k)
        assert torch.equal(Cg.view(torch.int32), Ck.view(torch.int32)), k


def test_plan_entries_without_positions(dev):
    """A caller's plan may hold entries where no position has both operands
    (a symbolic plan never does: |da|, |db|, |dc| < n leaves at least one
    row).  The gather takes each entry's range from its lengths: here
    entries of the first B diagonal (B start 0, where the clamped B load of
    an empty range would fall before the array) get al = 0 on the device,
    and the gather's C differs from the full plan's product on exactly the C
    diagonals of the emptied entries.  The band and A-stationary kernels
    derive each term from the operands' offsets, so their prepare steps
    refuse the edited plan (DIAGPU_ERR_ARG)."""
    n = 3000
    A = workloads.hm_random(n, list(range(-20, 21, 4)), 41, dev)
    B = workloads.hm_random(n, [-2999, -700, 0, 5, 2998], 42, dev)
    plan = SpgemmPlan(A, B)
    pairs = plan.pairs_numpy()
    hit = np.nonzero(pairs["bb"] == 0)[0][:7]
    assert hit.size > 0
    words = plan.pairs[: plan.info.n_pairs * 32].view(torch.int32).view(-1, 8)
    words[torch.as_tensor(hit, device=dev), 6] = 0             # al = 0: empty range
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    for k, fn in (("band", plan.band_info), ("astat", plan.astat_records)):
        plan._band, plan._astat = None, None
        with pytest.raises(_lib.DiagpuError) as e:
            fn()
        assert e.value.status == _lib.ERR_ARG and "symbolic" in str(e.value), k
    full = SpgemmPlan(A, B)
    Cf = full.multiply(A.values, B.values, kernel="gather")
    ptr = full.pair_ptr().cpu().numpy()
    c_st, c_len = full.c_starts().cpu().numpy(), full.c_lengths().cpu().numpy()
    touched = np.zeros(full.info.c_ndiag, bool)
    touched[np.searchsorted(ptr, hit, side="right") - 1] = True
    diff = (Cg != Cf).cpu().numpy()
    for k in range(full.info.c_ndiag):
        assert diff[c_st[k]: c_st[k] + c_len[k]].any() == touched[k], k


@pytest.mark.parametrize("field,delta", [("ash", 1), ("bsh", -1), ("al", -1), ("bl", 1),
                                         ("bb", "next"), ("ptr", None)])
def test_astat_prepare_refuses_edited_plans(dev, field, delta):
    """diagpu_spgemm_astat_prepare checks every entry against the symbolic
    form (A and B starts, da + db = dc, the shifts min0(da) - min0(dc) and
    da + min0(db) - min0(dc), the lengths n - |d|): one edited field of one
    entry, or a pair_ptr that moves an entry to the next C diagonal, gives
    DIAGPU_ERR_ARG; the unedited plan is accepted and multiplies to the
    gather's bits."""
    n = 5000
    A = workloads.hm_random(n, [-9, -4, 0, 3, 11], 51, dev)
    B = workloads.hm_random(n, [-30, -1, 0, 2, 7, 40], 52, dev)
    plan = SpgemmPlan(A, B)
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    Ca = plan.multiply(A.values, B.values, kernel="astat")
    assert torch.equal(Cg.view(torch.int32), Ca.view(torch.int32))
    g = plan.info.n_pairs // 2
    if field == "ptr":
        ptr = plan.pair_ptr().cpu().numpy()
        k = int(np.nonzero(np.diff(ptr)[:-1] >= 2)[0][0])   # a C diagonal with 2+ entries
        g = int(ptr[k]) + 1
        plan.ptr[k + 1] = g          # its entries from g on now count as the next one's
    else:
        words = plan.pairs[: plan.info.n_pairs * 32].view(torch.int32).view(-1, 8)
        col = {"ash": 4, "bsh": 5, "al": 6, "bl": 7}.get(field)
        if col is not None:
            words[g, col] += delta
        else:                        # bb: the start of another B diagonal
            q = plan.pairs[: plan.info.n_pairs * 32].view(torch.int64).view(-1, 4)
            bst = B.starts.cpu().tolist()
            cur = q[g, 1].item()
            q[g, 1] = bst[(bst.index(cur) + 1) % len(bst)]
    plan._astat = None
    with pytest.raises(_lib.DiagpuError) as e:
        plan.astat_records()
    assert e.value.status == _lib.ERR_ARG and "symbolic" in str(e.value)


def test_astat_prepare_b_index_bound(dev):
    """The numeric kernel forms B byte offsets 4 (b + c) in 32 bits, so the
    prepare step accepts a plan while every entry's last B index b + hi stays
    within 2^30 and refuses it with DIAGPU_ERR_CAPACITY one index beyond; the
    automatic choice then falls back to the gather.  B's starts and every
    entry's B start are moved together (the entries keep the symbolic form;
    the prepare step reads no values)."""
    n = 5000
    A = workloads.hm_random(n, [-9, -4, 0, 3, 11], 61, dev)
    B = workloads.hm_random(n, [-30, -1, 0, 2, 7, 40], 62, dev)
    plan = SpgemmPlan(A, B)
    rec = plan.astat_records()[: 4 * plan.info.n_pairs].view(-1, 4).cpu().numpy().astype(np.int64)
    top = int((rec[:, 3] + rec[:, 2]).max())      # largest b + hi
    q = plan.pairs[: plan.info.n_pairs * 32].view(torch.int64).view(-1, 4)
    starts0, bb0 = B.starts.clone(), q[:, 1].clone()
    for shift, ok in ((2**30 - top, True), (2**30 - top + 1, False)):
        B.starts.copy_(starts0 + shift)
        q[:, 1] = bb0 + shift
        plan._astat = None
        if ok:
            got = plan.astat_records()[: 4 * plan.info.n_pairs].view(-1, 4).cpu().numpy()
            assert np.array_equal(got[:, :3], rec[:, :3])
            assert np.array_equal(got[:, 3].astype(np.int64), rec[:, 3] + shift)
        else:
            with pytest.raises(_lib.DiagpuError) as e:
                plan.astat_records()
            assert e.value.status == _lib.ERR_CAPACITY and "2^30" in str(e.value)
            plan._astat = None
            assert not plan.uses_astat()


@pytest.mark.parametrize("case", ["stencil", "band", "random", "wide_a", "wide_b"])
def test_symbolic_astat_records_match_prepare(dev, case):
    """diagpu_spgemm_symbolic_astat builds, inside the symbolic call, the
    records and the 4-int tail that diagpu_spgemm_astat_prepare writes for
    the same plan, on the one-launch symbolic path and on the multi-launch
    path (the wide cases), and the A-stationary product from them has the
    gather's bits."""
    rng = np.random.default_rng(91)
    if case == "stencil":
        n, oa, ob = 1 << 20, list(range(-4, 5)), [-16384, -128, -1, 0, 1, 128, 16384]
    elif case == "band":
        n, oa, ob = 5000, list(range(-10, 11)), list(range(-10, 11))
    elif case == "random":
        n = 70000
        oa = rng.choice(np.arange(-4096, 4097), size=128, replace=False)
        ob = rng.choice(np.arange(-4096, 4097), size=40, replace=False)
    elif case == "wide_a":
        n, oa, ob = 600_000, [-599_999, 0, 599_999], [-599_999, -1, 2, 599_999]
    else:
        n = (1 << 22) + 3
        oa, ob = [-(1 << 22) - 2, -5, 0, 7, (1 << 22) + 2], [-3, 0, 1, (1 << 21)]
    A = workloads.hm_random(n, oa, seed=92, device=dev)
    B = workloads.hm_random(n, ob, seed=93, device=dev)
    plan = SpgemmPlan(A, B)
    assert plan._fused and plan._astat is True    # built by the symbolic call
    fused = plan.astat_records().clone()
    assert fused.numel() == 4 * plan.info.n_pairs + 4
    plan._astat = None                       # the separate prepare step, on the same plan
    sep = plan.astat_records().clone()
    assert torch.equal(fused, sep), case
    plan._astat = fused
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    Ca = plan.multiply(A.values, B.values, kernel="astat")
    assert torch.equal(Cg.view(torch.int32), Ca.view(torch.int32)), case


def test_symbolic_astat_records_b_index_bound(dev):
    """The records step inside the symbolic call applies the prepare step's
    2^30 bound on B indices: with B's starts moved so that the largest b + hi
    is 2^30 the plan's records are those of the unmoved plan with b moved;
    one index further the call still returns the plan (DIAGPU_OK) but reports
    DIAGPU_ERR_CAPACITY for the records, so the automatic choice skips the
    A-stationary kernel and forcing it raises that error."""
    from diagpu_amd.workloads import HM
    n = 5000
    A = workloads.hm_random(n, [-9, -4, 0, 3, 11], 94, dev)
    B = workloads.hm_random(n, [-30, -1, 0, 2, 7, 40], 95, dev)
    plan0 = SpgemmPlan(A, B)
    rec = plan0.astat_records().cpu().numpy().astype(np.int64)
    body = rec[: 4 * plan0.info.n_pairs].reshape(-1, 4)
    top = int((body[:, 3] + body[:, 2]).max())
    for shift, ok in ((2**30 - top, True), (2**30 - top + 1, False)):
        Bs = HM(n, B.offsets, B.lengths, B.starts + shift, B.values, None)
        plan = SpgemmPlan(A, Bs)
        assert plan.info.n_pairs == plan0.info.n_pairs
        if ok:
            got = plan.astat_records().cpu().numpy().astype(np.int64)
            gb = got[: 4 * plan.info.n_pairs].reshape(-1, 4)
            assert np.array_equal(gb[:, :3], body[:, :3])
            assert np.array_equal(gb[:, 3], body[:, 3] + shift)
            assert np.array_equal(got[-4:], rec[-4:])
        else:
            assert plan._astat is False and not plan.uses_astat()
            with pytest.raises(_lib.DiagpuError) as e:
                plan.astat_records()
            assert e.value.status == _lib.ERR_CAPACITY and "2^30" in str(e.value)


def _drop_diagonals(plan, empty):
    """Remove every plan entry of the C diagonals `empty` (their pair_ptr
    ranges become empty); returns the kept entries' mask."""
    nc, npair = plan.info.c_ndiag, plan.info.n_pairs
    ptr = plan.pair_ptr().cpu().numpy()
    pairs = plan.pairs_numpy().copy()
    keep = np.ones(npair, bool)
    counts = np.diff(ptr)
    for k in empty:
        keep[ptr[k]: ptr[k + 1]] = False
        counts[k] = 0
    new_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int64)
    kept = pairs[keep]
    plan.ptr[: nc + 1].copy_(torch.as_tensor(new_ptr))
    plan.pairs[: kept.size * 32].copy_(torch.as_tensor(kept.view(np.uint8)))
    plan.info.n_pairs = int(kept.size)
    plan.info.max_pairs = int(counts.max())
    plan._band = None
    plan._astat = None
    return keep


@pytest.mark.parametrize("n", [5000, 1 << 17])
def test_empty_c_diagonals_written_as_zero(dev, n):
    """A caller's plan may give a C diagonal no entry at all (pair_ptr[k] ==
    pair_ptr[k + 1]), or a whole batch of diagonals none: every kernel still
    writes every C value, zeros there, and the other diagonals keep the full
    plan's bits.  C starts out as NaN so an unwritten value shows."""
    A = workloads.hm_random(n, list(range(-10, 11)), 51, dev)
    B = workloads.hm_random(n, list(range(-8, 9)), 52, dev)
    full = SpgemmPlan(A, B)
    Cf = full.multiply(A.values, B.values, kernel="gather")
    plan = SpgemmPlan(A, B)
    nc = plan.info.c_ndiag
    assert nc == 37
    empty = [0, *range(5, 23), nc - 2, nc - 1]    # first, 18 in a row, the last two
    _drop_diagonals(plan, empty)
    c_st, c_len = plan.c_starts().cpu().numpy(), plan.c_lengths().cpu().numpy()
    zero = np.zeros(plan.info.c_nnz, bool)
    for k in empty:
        zero[c_st[k]: c_st[k] + c_len[k]] = True
    want = Cf.cpu().numpy().copy()
    want[zero] = 0.0
    for kernel in ("gather", "band", "astat"):
        Cv = torch.full((plan.info.c_nnz,), float("nan"), device=dev)
        plan.numeric(A.values, B.values, Cv, kernel=kernel)
        got = Cv.cpu().numpy()
        assert np.array_equal(got.view(np.int32), want.view(np.int32)), kernel


def test_plan_with_no_entries(dev):
    """A plan whose every C diagonal is empty: all of C is written as 0."""
    n = 3000
    A = workloads.hm_random(n, [-3, 0, 2], 61, dev)
    B = workloads.hm_random(n, [-1, 0, 4], 62, dev)
    plan = SpgemmPlan(A, B)
    _drop_diagonals(plan, range(plan.info.c_ndiag))
    assert plan.info.n_pairs == 0
    Cv = torch.full((plan.info.c_nnz,), float("nan"), device=dev)
    plan.numeric(A.values, B.values, Cv, kernel="gather")
    assert torch.equal(Cv, torch.zeros_like(Cv))


def test_wrappers_reject_short_or_strided_operands(dev):
    """The Python wrappers check operand sizes and layouts before any launch:
    a value tensor shorter than its plan's operand, a strided x, psi0 or
    out, or out aliasing psi0."""
    from diagpu_amd.krylov import expm_krylov
    from diagpu_amd.spmv import spmv_recon
    A = workloads.hm_random(4000, [-5, 0, 7], 71, dev)
    B = workloads.hm_random(4000, [-2, 0, 1], 72, dev)
    plan = SpgemmPlan(A, B)
    Cv = torch.empty(plan.info.c_nnz, device=dev)
    with pytest.raises(ValueError):
        plan.numeric(A.values[:-1], B.values, Cv)
    with pytest.raises(ValueError):
        plan.numeric(A.values, B.values[: B.values.numel() // 2], Cv)
    R = workloads.recon_random(1000, [-3, 0, 3], 73, dev)
    x2 = torch.randn(2000, device=dev)
    with pytest.raises(TypeError):
        spmv_recon(R.offsets, R.values, 1000, 1000, x2[::2])
    Rc = R.values.to(torch.complex64)
    psi = torch.randn(2000, device=dev, dtype=torch.complex64)
    with pytest.raises(TypeError):
        expm_krylov(R.offsets, Rc, 1000, psi[::2], 0.1, m=8)
    psi0 = psi[:1000].contiguous()
    with pytest.raises(TypeError):
        expm_krylov(R.offsets, Rc, 1000, psi0, 0.1, m=8, out=psi[::2])
    with pytest.raises(ValueError):
        expm_krylov(R.offsets, Rc, 1000, psi0, 0.1, m=8, out=psi0)


def test_band_lds_estimate_matches_prepare(dev):
    """The host's estimate of the band kernel's LDS footprint (used to skip
    the prepare step's sync for plans that cannot fit) equals what
    diagpu_spgemm_band_prepare reports, on narrow and wide operands."""
    for n, oa, ob in ((1 << 17, list(range(-10, 11)), list(range(-10, 11))),
                      (5000, [-300, -3, 0, 7, 250], [-1, 0, 1]),
                      (70001, list(range(-12, 13)), [-65000, -3, 0, 4, 65000])):
        A = workloads.hm_random(n, oa, 41, dev)
        B = workloads.hm_random(n, ob, 42, dev)
        plan = SpgemmPlan(A, B)
        assert A.host_offsets == sorted(oa)
        assert plan.band_lds_estimate() == plan.band_info()[1].lds_bytes


@pytest.mark.parametrize("n,offs_a,offs_b", [
    (4096, list(range(-10, 11)), list(range(-10, 11))),       # gemm_diag.cu:467-486 defaults
    (1 << 17, list(range(-10, 11)), list(range(-10, 11))),
    (70001, list(range(-12, 13)), list(range(-7, 8))),         # ragged last block
    (5000, [-10, -3, 0, 5, 9], [-8, -1, 0, 2, 7]),             # offsets with holes
    (37, [-10, -3, 0, 2, 10], [-9, -1, 0, 5, 7]),              # smaller than one block
    (300, [0], [0]),                                           # diagonal times diagonal
    (1, [0], [0]),                                             # a 1 x 1 matrix
    (3, [-2, -1, 0, 1, 2], [-2, 0, 1]),                        # every diagonal of 3 x 3
    (65537, list(range(-16, 17)), list(range(-8, 8))),         # widest A range, C span 47
    (20000, [-9, -4, 0, 3, 11], [-12, -2, 0, 1, 14]),          # holes, C span 46, ragged
])
def test_band_mfma_kernel(dev, oracle, n, offs_a, offs_b):
    """The MFMA band kernel: every C value within 1e-5 of its fp64 term sum
    (the same bound as the other kernels; not bit-identical: MFMA order), the
    reference's own 1e-1 (gemm_diag.cu:544) far inside, and the issued-block
    count matching the tile geometry."""
    A = workloads.hm_random(n, offs_a, 91, dev)
    B = workloads.hm_random(n, offs_b, 92, dev)
    plan = SpgemmPlan(A, B)
    _, info = plan.band_info()
    assert info.mfma_eligible and info.mfma_blocks > 0
    assert (info.b_off_min, info.b_off_max) == (min(offs_b), max(offs_b))
    Cm = torch.full((plan.info.c_nnz,), float("nan"), device=dev)
    plan.numeric(A.values, B.values, Cm, kernel="band_mfma")
    Cg = plan.multiply(A.values, B.values, kernel="gather")
    c_len, c_st = plan.c_lengths().cpu().numpy(), plan.c_starts().cpu().numpy()
    ptr, pairs = plan.pair_ptr().cpu().numpy(), plan.pairs_numpy()
    want, ab = oracle.spgemm_pairs_f64(A.values.cpu().numpy(), B.values.cpu().numpy(), c_len,
                                       c_st, ptr, pairs, 0, plan.info.c_ndiag)
    got = Cm.cpu().numpy()
    assert np.isfinite(got).all()
    check_values(got, want, ab)
    assert np.max(np.abs(got - Cg.cpu().numpy())) < 1e-1
    u = plan.mfma_utilisation()
    assert 0 < u <= 1


def test_band_mfma_refuses_wide_spans(dev):
    """Offset ranges beyond the MFMA kernel's tiles (config 4's +-16384) are
    refused with DIAGPU_ERR_CAPACITY before any launch."""
    A4, B4 = workloads.spgemm_config(4, seed=4, device=dev)
    p4 = SpgemmPlan(A4, B4)
    assert not p4.band_info()[1].mfma_eligible and p4.mfma_utilisation() is None
    Cv = torch.empty(p4.info.c_nnz, device=dev)
    with pytest.raises(_lib.DiagpuError) as e:
        p4.numeric(A4.values, B4.values, Cv, kernel="band_mfma")
    assert e.value.status == _lib.ERR_CAPACITY
