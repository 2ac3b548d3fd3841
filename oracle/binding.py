"""numpy/ctypes binding of oracle/liboracle.so -- TEST INFRASTRUCTURE ONLY.

Each wrapper names the C function (oracle/dia_oracle.c, dia_oracle_gen.cpp)
whose comment cites the reference lines it restates.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "liboracle.so"
REF_DIR = Path(__file__).resolve().parent / "_ref"

_lib: C.CDLL | None = None

GPAIR_DTYPE = np.dtype([("ab", "<u8"), ("bb", "<u8"), ("ash", "<i4"), ("bsh", "<i4"),
                        ("al", "<i4"), ("bl", "<i4")])


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} missing: build with `make -C oracle`")
        _lib = C.CDLL(str(LIB_PATH))
        _lib.orc_hval.restype = C.c_float
        _lib.orc_hval.argtypes = [C.c_int, C.c_int]
        _lib.orc_xval.restype = C.c_float
        _lib.orc_xval.argtypes = [C.c_int]
        _lib.orc_c_structure.restype = C.c_int
        _lib.orc_pairs_only.restype = C.c_int64
        _lib.orc_spmv_recon_omp_f32.restype = C.c_int
        _lib.orc_spmv_recon_omp_f64.restype = C.c_int
        _lib.orc_spgemm_pairs_omp_f32.restype = C.c_int
        _lib.orc_max_threads.restype = C.c_int
        _lib.orc_make_banded.restype = C.c_int
        _lib.orc_hval_band.restype = C.c_int64
    return _lib


def _p(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return C.c_void_p(a.ctypes.data)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def _i64(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int64)


# --------------------------------------------------------------------------
# generators
# --------------------------------------------------------------------------

def tc_spmv_case(N: int, offsets) -> tuple[np.ndarray, np.ndarray]:
    """Dense H and x of spmv/test/test_tc_spmv.cu:86-98 (orc_tc_spmv_case)."""
    offs = _i32(offsets)
    H = np.empty((N, N), dtype=np.float32)
    x = np.empty(N, dtype=np.float32)
    lib().orc_tc_spmv_case(N, _p(offs), len(offs), _p(H), _p(x))
    return H, x


def hval(r: int, d: int) -> float:
    return lib().orc_hval(r, d)


def xval(i: int) -> float:
    return lib().orc_xval(i)


def xval_array(N: int) -> np.ndarray:
    x = np.empty(N, dtype=np.float32)
    lib().orc_xval_fill(N, _p(x))
    return x


def hval_band(N: int, offsets) -> np.ndarray:
    """hval(r, d) for every entry of the N x N band, offset by offset (given
    order), rows ascending."""
    offs = _i32(offsets)
    out = np.empty(max(1, sum(N - abs(int(d)) for d in offs if abs(int(d)) < N)), np.float32)
    cnt = lib().orc_hval_band(N, _p(offs), len(offs), _p(out))
    return out[:cnt]


def hash_band_recon(N: int, offsets) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Recon (offsets descending, values) and x of spmv/bench/bench_cusparse.cu:84-144."""
    offs = _i32(offsets)
    K = len(offs)
    r_off = np.empty(K, dtype=np.int32)
    r_val = np.empty(K * N, dtype=np.float32)
    x = np.empty(N, dtype=np.float32)
    lib().orc_hash_band_recon(N, _p(offs), K, _p(r_off), _p(r_val), _p(x))
    return r_off, r_val, x


def make_banded(n: int, w: int, seed: int):
    """make_banded of spmspm/bench_spmspm.cu:89-106 (libstdc++ mt19937)."""
    m = 2 * w + 1
    offs = np.empty(m, dtype=np.int32)
    starts = np.empty(m, dtype=np.int64)
    lens = np.empty(m, dtype=np.int32)
    total = sum(max(0, n - abs(d)) for d in range(-w, w + 1))
    vals = np.empty(max(total, 1), dtype=np.float32)
    nd = lib().orc_make_banded(n, w, C.c_uint(seed), _p(offs), _p(starts), _p(lens), _p(vals))
    return offs[:nd].copy(), starts[:nd].copy(), lens[:nd].copy(), vals[:total].copy()


def pack_diag_matrix(n: int, offsets, seed: int) -> np.ndarray:
    """pack_diag_matrix of gemm_diag/gemm_diag.cu:362-382 (libstdc++ mt19937)."""
    offs = _i32(offsets)
    DA = np.empty((len(offs), n), dtype=np.float32)
    lib().orc_pack_diag_matrix(n, _p(offs), len(offs), C.c_uint(seed), _p(DA))
    return DA


# --------------------------------------------------------------------------
# SpMV
# --------------------------------------------------------------------------

def dense_to_dia(H: np.ndarray):
    """dense_to_dia of spmv/test/test_reconstruct.cpp:93-116."""
    H = np.ascontiguousarray(H, dtype=np.float32)
    rows, cols = H.shape
    nd = C.c_int(0)
    nv = C.c_int64(0)
    lib().orc_dense_to_dia_count(_p(H), rows, cols, C.byref(nd), C.byref(nv))
    offs = np.empty(nd.value, dtype=np.int32)
    starts = np.empty(nd.value, dtype=np.int64)
    lens = np.empty(nd.value, dtype=np.int32)
    vals = np.empty(max(nv.value, 1), dtype=np.float32)
    lib().orc_dense_to_dia(_p(H), rows, cols, _p(offs), _p(starts), _p(lens), _p(vals))
    return offs, starts, lens, vals[: nv.value]


def build_recon(rows: int, cols: int, offsets, starts, lengths, values):
    """build_recon of spmv/src/dia_reconstruct.cuh:77-107 -> (offsets desc, values K*cols)."""
    offs, st, ln = _i32(offsets), _i64(starts), _i32(lengths)
    K = len(offs)
    if np.asarray(values).dtype == np.float64:
        vals = np.ascontiguousarray(values, dtype=np.float64)
        out = np.empty(K * cols, dtype=np.float64)
        fn = lib().orc_build_recon_f64
    else:
        vals = np.ascontiguousarray(values, dtype=np.float32)
        out = np.empty(K * cols, dtype=np.float32)
        fn = lib().orc_build_recon_f32
    r_off = np.empty(K, dtype=np.int32)
    fn(rows, cols, K, _p(offs), _p(st), _p(ln), _p(vals), _p(r_off), _p(out))
    return r_off, out


def recon_to_dense(rows: int, cols: int, r_offsets, r_values) -> np.ndarray:
    offs = _i32(r_offsets)
    vals = np.ascontiguousarray(r_values, dtype=np.float32)
    H = np.empty((rows, cols), dtype=np.float32)
    lib().orc_recon_to_dense_f32(rows, cols, len(offs), _p(offs), _p(vals), _p(H))
    return H


def spmv_recon_f32(rows, cols, r_offsets, r_values, x) -> np.ndarray:
    """spmv_from_recon (serial fp32) of spmv/test/test_reconstruct.cpp:122-138."""
    offs = _i32(r_offsets)
    vals = np.ascontiguousarray(r_values, dtype=np.float32)
    xx = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(rows, dtype=np.float32)
    lib().orc_spmv_recon_f32(rows, cols, len(offs), _p(offs), _p(vals), _p(xx),
                             C.c_int64(len(xx)), _p(y))
    return y


def spmv_recon_ref64(rows, cols, r_offsets, r_values, x):
    """fp64 host result and sum of |terms| for Recon SpMV (fp32 or fp64 data)."""
    offs = _i32(r_offsets)
    vals = np.ascontiguousarray(r_values)
    y = np.empty(rows, dtype=np.float64)
    a = np.empty(rows, dtype=np.float64)
    if vals.dtype == np.float64:
        xx = np.ascontiguousarray(x, dtype=np.float64)
        lib().orc_spmv_recon_f64(rows, cols, len(offs), _p(offs), _p(vals), _p(xx),
                                 C.c_int64(len(xx)), _p(y), _p(a))
    else:
        vals = np.ascontiguousarray(vals, dtype=np.float32)
        xx = np.ascontiguousarray(x, dtype=np.float32)
        lib().orc_spmv_recon_f32_ref64(rows, cols, len(offs), _p(offs), _p(vals), _p(xx),
                                       C.c_int64(len(xx)), _p(y), _p(a))
    return y, a


def spmv_recon_complex_ref(rows, cols, r_offsets, r_values, x):
    """fp64 complex result (complex128 [rows]) and sum of |term parts| for a
    complex64 (or real float32) Recon matrix applied to a complex64 x."""
    offs = _i32(r_offsets)
    xx = np.ascontiguousarray(x, dtype=np.complex64)
    vals = np.ascontiguousarray(r_values)
    y = np.empty(rows, dtype=np.complex128)
    a = np.empty(rows, dtype=np.float64)
    if vals.dtype == np.complex64:
        fn = lib().orc_spmv_recon_c64_ref
    else:
        vals = np.ascontiguousarray(vals, dtype=np.float32)
        fn = lib().orc_spmv_recon_f32c64_ref
    fn(rows, cols, len(offs), _p(offs), _p(vals), _p(xx), C.c_int64(len(xx)), _p(y), _p(a))
    return y, a


def spmv_recon_omp(rows, cols, r_offsets, r_values, x, y) -> int:
    """OpenMP CPU baseline (orc_spmv_recon_omp_*); returns threads used."""
    offs = _i32(r_offsets)
    if r_values.dtype == np.float64:
        fn = lib().orc_spmv_recon_omp_f64
    else:
        fn = lib().orc_spmv_recon_omp_f32
    return fn(rows, cols, len(offs), _p(offs), _p(r_values), _p(x), C.c_int64(len(x)), _p(y))


def max_threads() -> int:
    return lib().orc_max_threads()


def set_threads(n: int) -> None:
    lib().orc_set_threads(n)


# --------------------------------------------------------------------------
# SpGEMM
# --------------------------------------------------------------------------

def c_structure(n: int, A_off, B_off):
    """make_c_structure of spmspm/bench_spmspm.cu:109-131 -> (C_off, C_len, C_starts, nnz)."""
    a, b = _i32(A_off), _i32(B_off)
    cap = max(1, min(len(a) * len(b), 2 * n - 1))
    off = np.empty(cap, dtype=np.int32)
    ln = np.empty(cap, dtype=np.int32)
    st = np.empty(cap, dtype=np.int64)
    nnz = C.c_int64(0)
    nc = lib().orc_c_structure(n, _p(a), len(a), _p(b), len(b), _p(off), _p(ln), _p(st),
                               C.byref(nnz))
    return off[:nc].copy(), ln[:nc].copy(), st[:nc].copy(), nnz.value


def c_lookup(n: int, C_off) -> np.ndarray:
    """build_c_diag_lookup of spmspm/paper_hm.cuh:121-130."""
    c = _i32(C_off)
    lk = np.empty(2 * n - 1, dtype=np.int32)
    lib().orc_c_lookup(n, _p(c), len(c), _p(lk))
    return lk


def pairs_only(n, A_off, A_len, A_starts, B_off, B_len, B_starts, C_off):
    """build_pairs_only of spmspm/gather_flat.cuh:231-255 -> (pair_ptr int64, pairs GPAIR)."""
    a, al, ast = _i32(A_off), _i32(A_len), _i64(A_starts)
    b, bl, bst = _i32(B_off), _i32(B_len), _i64(B_starts)
    c = _i32(C_off)
    ptr = np.empty(len(c) + 1, dtype=np.int64)
    np_total = lib().orc_pairs_only(n, _p(a), len(a), _p(al), _p(ast), _p(b), len(b), _p(bl),
                                    _p(bst), _p(c), len(c), _p(ptr), None)
    pairs = np.empty(max(1, np_total), dtype=GPAIR_DTYPE)
    lib().orc_pairs_only(n, _p(a), len(a), _p(al), _p(ast), _p(b), len(b), _p(bl), _p(bst),
                         _p(c), len(c), _p(ptr), _p(pairs))
    return ptr, pairs[:np_total]


def spgemm_gather_f64(n, A, B, Cs):
    """cpu_dia_spgemm loop (bench_spmspm.cu:376-408) in fp64 -> (C values, |term| sums).

    A, B: (off, len, starts, vals); Cs: (off, len, starts, nnz)."""
    A_off, A_len, A_st, A_v = A
    B_off, B_len, B_st, B_v = B
    C_off, C_len, C_st, nnz = Cs
    out = np.zeros(max(nnz, 1), dtype=np.float64)
    ab = np.zeros(max(nnz, 1), dtype=np.float64)
    arrs = [_i32(A_off), _i32(A_len), _i64(A_st), np.ascontiguousarray(A_v, np.float32),
            _i32(B_off), _i32(B_len), _i64(B_st), np.ascontiguousarray(B_v, np.float32),
            _i32(C_off), _i32(C_len), _i64(C_st)]
    lib().orc_spgemm_gather_f64(
        n, _p(arrs[0]), len(arrs[0]), _p(arrs[1]), _p(arrs[2]), _p(arrs[3]),
        _p(arrs[4]), len(arrs[4]), _p(arrs[5]), _p(arrs[6]), _p(arrs[7]),
        _p(arrs[8]), len(arrs[8]), _p(arrs[9]), _p(arrs[10]), _p(out), _p(ab))
    return out[:nnz], ab[:nnz]


def spgemm_pairs_f64(A_v, B_v, C_len, C_starts, pair_ptr, pairs, kbeg, kend):
    """Plan-driven fp64 numeric phase over C diagonals [kbeg, kend)."""
    C_len, C_starts = _i32(C_len), _i64(C_starts)
    pair_ptr = _i64(pair_ptr)
    pairs = np.ascontiguousarray(pairs, dtype=GPAIR_DTYPE)
    if kend <= kbeg:
        return np.zeros(0), np.zeros(0)
    total = int(C_starts[kend - 1] + C_len[kend - 1] - C_starts[kbeg])
    out = np.empty(max(total, 1), dtype=np.float64)
    ab = np.empty(max(total, 1), dtype=np.float64)
    lib().orc_spgemm_pairs_f64(_p(np.ascontiguousarray(A_v, np.float32)),
                               _p(np.ascontiguousarray(B_v, np.float32)), _p(C_len),
                               _p(C_starts), _p(pair_ptr), _p(pairs), kbeg, kend, _p(out), _p(ab))
    return out[:total], ab[:total]


def spgemm_pairs_complex(A_v, B_v, C_len, C_starts, pair_ptr, pairs, kbeg, kend):
    """Plan-driven complex numeric phase (complex64 data, fp64 accumulation)
    over C diagonals [kbeg, kend): complex128 values and the term bound."""
    C_len, C_starts = _i32(C_len), _i64(C_starts)
    pair_ptr = _i64(pair_ptr)
    pairs = np.ascontiguousarray(pairs, dtype=GPAIR_DTYPE)
    if kend <= kbeg:
        return np.zeros(0, np.complex128), np.zeros(0)
    total = int(C_starts[kend - 1] + C_len[kend - 1] - C_starts[kbeg])
    out = np.empty(max(total, 1), dtype=np.complex128)
    ab = np.empty(max(total, 1), dtype=np.float64)
    lib().orc_spgemm_pairs_c128(_p(np.ascontiguousarray(A_v, np.complex64)),
                                _p(np.ascontiguousarray(B_v, np.complex64)), _p(C_len),
                                _p(C_starts), _p(pair_ptr), _p(pairs), kbeg, kend, _p(out), _p(ab))
    return out[:total], ab[:total]


def spgemm_pairs_omp_f32(A_v, B_v, C_len, C_starts, pair_ptr, pairs, kbeg, kend, out) -> int:
    """OpenMP CPU baseline over C diagonals [kbeg, kend); returns threads used."""
    return lib().orc_spgemm_pairs_omp_f32(_p(A_v), _p(B_v), _p(C_len), _p(C_starts),
                                          _p(pair_ptr), _p(pairs), kbeg, kend, _p(out))


def spgemm_hm_atomic_f64(n, A, B, C_len, C_starts, C_lookup, nnz):
    """Haque atomic traversal (paper_hm_kernel.cu:31-93) sequentially in fp64."""
    A_off, A_len, A_st, A_v = A
    B_off, B_len, B_st, B_v = B
    arrs = [_i32(A_off), _i64(A_st), _i32(A_len), np.ascontiguousarray(A_v, np.float32),
            _i32(B_off), _i64(B_st), _i32(B_len), np.ascontiguousarray(B_v, np.float32),
            _i32(C_len), _i64(C_starts), _i32(C_lookup)]
    out = np.zeros(max(nnz, 1), dtype=np.float64)
    lib().orc_spgemm_hm_atomic_f64(
        n, _p(arrs[0]), len(arrs[0]), _p(arrs[1]), _p(arrs[2]), _p(arrs[3]),
        C.c_int64(len(arrs[3])), _p(arrs[4]), len(arrs[4]), _p(arrs[5]), _p(arrs[6]),
        _p(arrs[7]), _p(arrs[8]), _p(arrs[9]), _p(arrs[10]), _p(out))
    return out[:nnz]


def gemm_diag_f64(n, DA, off_A, DB, off_B, C_lookup, C_starts, nnz):
    """gemm_diag formula (gemm_diag.cu:9-15, :335-356) into the compact C layout, fp64."""
    DA = np.ascontiguousarray(DA, np.float32)
    DB = np.ascontiguousarray(DB, np.float32)
    oa, ob = _i32(off_A), _i32(off_B)
    lk, st = _i32(C_lookup), _i64(C_starts)
    out = np.zeros(max(nnz, 1), dtype=np.float64)
    ab = np.zeros(max(nnz, 1), dtype=np.float64)
    lib().orc_gemm_diag_f64(n, _p(DA), _p(oa), len(oa), _p(DB), _p(ob), len(ob), _p(lk),
                            _p(st), _p(out), _p(ab))
    return out[:nnz], ab[:nnz]


SCHED_ENTRY_DTYPE = np.dtype([("a_local", "<i4"), ("b_local", "<i4"), ("c_local", "<i4"),
                              ("a_shift", "<i4"), ("b_shift", "<i4")])


def build_schedule(n: int, A_off, B_off, C_off, T: int = 8, n_tile: int = 256) -> dict:
    """build_schedule of spmspm/bench_spmspm.cu:137-243 (orc_build_schedule):
    a dict with the Schedule's members (pairs as SCHED_ENTRY_DTYPE)."""
    a, b, c = _i32(A_off), _i32(B_off), _i32(C_off)
    sc = np.zeros(8, np.int32)
    lib().orc_build_schedule(n, _p(a), len(a), _p(b), len(b), _p(c), len(c), T, n_tile, _p(sc),
                             *([None] * 10))
    a_halo, b_halo, G, max_a, max_b, max_p, ntiles, nblocks = (int(v) for v in sc)
    out = {k: np.zeros(G, np.int32) for k in ("a_count", "b_count", "pair_count", "t_out")}
    out["a_globals"] = np.zeros(max(1, G * max_a), np.int32)
    out["b_globals"] = np.zeros(max(1, G * max_b), np.int32)
    out["c_globals"] = np.zeros(max(1, G * T), np.int32)
    out["pairs"] = np.zeros(max(1, G * max_p), SCHED_ENTRY_DTYPE)
    out["block_group"] = np.zeros(max(1, nblocks), np.int32)
    out["block_tile"] = np.zeros(max(1, nblocks), np.int32)
    lib().orc_build_schedule(n, _p(a), len(a), _p(b), len(b), _p(c), len(c), T, n_tile, _p(sc),
                             _p(out["a_count"]), _p(out["b_count"]), _p(out["pair_count"]),
                             _p(out["t_out"]), _p(out["a_globals"]), _p(out["b_globals"]),
                             _p(out["c_globals"]), _p(out["pairs"]), _p(out["block_group"]),
                             _p(out["block_tile"]))
    out["a_globals"] = out["a_globals"][: G * max_a]
    out["b_globals"] = out["b_globals"][: G * max_b]
    out["c_globals"] = out["c_globals"][: G * T]
    out["pairs"] = out["pairs"][: G * max_p]
    out["block_group"] = out["block_group"][:nblocks]
    out["block_tile"] = out["block_tile"][:nblocks]
    out.update(a_halo=a_halo, b_halo=b_halo, num_groups=G, max_a=max_a, max_b=max_b,
               max_pairs=max_p, num_ntiles=ntiles, num_blocks=nblocks)
    return out

