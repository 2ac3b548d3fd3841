"""ctypes binding of libdiagpu.so (the C ABI declared in include/diagpu.h).

The library is loaded from this package directory only; a missing library is
an error (there is no CPU fallback for any entry point).
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdiagpu.so"

OK = 0
ERR_ARG = 1
ERR_OFFSET = 2
ERR_DUPLICATE = 3
ERR_OVERFLOW = 4
ERR_CAPACITY = 5
ERR_HIP = 6


class DiagpuError(RuntimeError):
    """A libdiagpu entry point returned a non-zero status."""

    def __init__(self, status: int, name: str, message: str):
        super().__init__(f"{name}: {message}")
        self.status = status
        self.status_name = name


class ReconViewF32(C.Structure):
    _fields_ = [("rows", C.c_int32), ("cols", C.c_int32), ("num_diags", C.c_int32),
                ("diag_offsets", C.c_void_p), ("values", C.c_void_p)]


class ReconViewF64(C.Structure):
    _fields_ = [("rows", C.c_int32), ("cols", C.c_int32), ("num_diags", C.c_int32),
                ("diag_offsets", C.c_void_p), ("values", C.c_void_p)]


class ReconViewC64(C.Structure):
    _fields_ = [("rows", C.c_int32), ("cols", C.c_int32), ("num_diags", C.c_int32),
                ("diag_offsets", C.c_void_p), ("values", C.c_void_p)]


class Complex64(C.Structure):
    _fields_ = [("re", C.c_float), ("im", C.c_float)]


class KrylovInfo(C.Structure):
    _fields_ = [("steps", C.c_int32), ("breakdown", C.c_int32), ("psi0_norm", C.c_double),
                ("err_estimate", C.c_double)]


class GPair(C.Structure):
    _fields_ = [("ab", C.c_uint64), ("bb", C.c_uint64), ("ash", C.c_int32),
                ("bsh", C.c_int32), ("al", C.c_int32), ("bl", C.c_int32)]


class BandInfo(C.Structure):
    _fields_ = [("a_off_min", C.c_int32), ("a_off_max", C.c_int32),
                ("rows_per_block", C.c_int32), ("eligible", C.c_int32),
                ("lds_bytes", C.c_int64), ("n_pairs", C.c_int64),
                ("b_off_min", C.c_int32), ("b_off_max", C.c_int32),
                ("mfma_blocks", C.c_int32), ("mfma_eligible", C.c_int32),
                ("mfma_lds_bytes", C.c_int64)]


class SpgemmInfo(C.Structure):
    _fields_ = [("c_ndiag", C.c_int64), ("c_nnz", C.c_int64), ("n_pairs", C.c_int64),
                ("max_pairs", C.c_int64), ("useful_flops", C.c_int64), ("a_extent", C.c_int64),
                ("b_extent", C.c_int64)]


_vp, _i32, _i64, _sz = C.c_void_p, C.c_int32, C.c_int64, C.c_size_t

# name -> (restype, argtypes); every entry point declared in include/diagpu.h.
PROTOTYPES: dict[str, tuple] = {
    "diagpu_last_error": (C.c_char_p, []),
    "diagpu_status_name": (C.c_char_p, [C.c_int]),
    "diagpu_abi_version": (C.c_int, []),
    "diagpu_spmv_recon_f32": (C.c_int, [C.POINTER(ReconViewF32), _vp, _i64, _vp, _vp]),
    "diagpu_spmv_recon_f64": (C.c_int, [C.POINTER(ReconViewF64), _vp, _i64, _vp, _vp]),
    "diagpu_spmv_recon_c64": (C.c_int, [C.POINTER(ReconViewC64), _vp, _i64, _vp, _vp]),
    "diagpu_spmv_recon_f32_c64": (C.c_int, [C.POINTER(ReconViewF32), _vp, _i64, _vp, _vp]),
    "diagpu_expm_krylov_workspace": (C.c_int, [_i32, _i32, C.POINTER(_sz)]),
    "diagpu_expm_krylov_c64": (C.c_int, [C.POINTER(ReconViewC64), _vp, C.c_double, _i32, _vp,
                                         _vp, _sz, _vp, _vp, _vp, C.POINTER(KrylovInfo), _vp]),
    "diagpu_expm_krylov_f32": (C.c_int, [C.POINTER(ReconViewF32), _vp, C.c_double, _i32, _vp,
                                         _vp, _sz, _vp, _vp, _vp, C.POINTER(KrylovInfo), _vp]),
    "diagpu_spgemm_symbolic_workspace": (C.c_int, [_i32, _i32, _i32, C.POINTER(_sz)]),
    "diagpu_spgemm_symbolic": (C.c_int, [
        _i32,
        _vp, _vp, _vp, _i32,
        _vp, _vp, _vp, _i32,
        _vp, _vp, _vp, _i64,
        _vp, _vp, _i64,
        _vp,
        _vp, _sz,
        C.POINTER(SpgemmInfo), _vp]),
    "diagpu_spgemm_symbolic_astat": (C.c_int, [
        _i32,
        _vp, _vp, _vp, _i32,
        _vp, _vp, _vp, _i32,
        _vp, _vp, _vp, _i64,
        _vp, _vp, _i64,
        _vp,
        _vp, _sz,
        _vp, C.POINTER(_i32),
        C.POINTER(SpgemmInfo), _vp]),
    "diagpu_spgemm_symbolic_noalloc": (C.c_int, [
        _i32,
        _vp, _vp, _vp, _i32,
        _vp, _vp, _vp, _i32,
        _vp, _vp, _vp, _i64,
        _vp, _vp, _i64,
        _vp,
        C.POINTER(SpgemmInfo), _vp]),
    "diagpu_spgemm_numeric_f32": (C.c_int, [
        _i32, _vp, _vp,
        _vp, _vp, _vp, _i64,
        _vp, _vp, _i64,
        _vp, _vp]),
    "diagpu_spgemm_numeric_c64": (C.c_int, [
        _i32, _vp, _vp,
        _vp, _vp, _vp, _i64,
        _vp, _vp, _i64,
        _vp, _vp]),
    "diagpu_rowpacked_as_hm": (C.c_int, [_i32, _vp, _i32, _vp, _vp, _vp]),
    "diagpu_dia_axpby_f32": (C.c_int, [
        _i32, _vp, _vp, _i32, _vp, C.c_float,
        _vp, _vp, _i32, _vp, C.c_float,
        _vp, _vp, _i32, _vp, _vp]),
    "diagpu_dia_axpby_c64": (C.c_int, [
        _i32, _vp, _vp, _i32, _vp, Complex64,
        _vp, _vp, _i32, _vp, Complex64,
        _vp, _vp, _i32, _vp, _vp]),
    "diagpu_hm_to_recon_f32": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "diagpu_hm_to_recon_c64": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp]),
    "diagpu_promote_f32_c64": (C.c_int, [_i64, _vp, _vp, _vp]),
    "diagpu_spgemm_band_prepare": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _i64,
                                             _vp, C.POINTER(BandInfo), _vp]),
    "diagpu_spgemm_numeric_band_f32": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _vp, _i32, _vp,
                                                 _vp, _vp, _i64, _vp, _vp, C.POINTER(BandInfo),
                                                 _vp, _vp]),
    "diagpu_spgemm_numeric_band_mfma_f32": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _vp, _i32,
                                                      _vp, _vp, _vp, _i64, C.POINTER(BandInfo),
                                                      _vp, _vp]),
    "diagpu_spgemm_astat_prepare": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _i32, _vp, _vp,
                                                _i64, _vp, _i64, _vp, _vp]),
    "diagpu_spgemm_numeric_astat_f32": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp,
                                                  _i64, _vp, _vp, _i64, _vp, _vp]),
    "diagpu_spgemm_numeric_astat_c64": (C.c_int, [_i32, _vp, _vp, _i32, _vp, _vp, _vp, _vp, _vp,
                                                  _i64, _vp, _vp, _i64, _vp, _vp]),
    "diagpu_spgemm_numeric_astat_scaled_f32": (C.c_int, [
        _i32, _vp, _vp, _i32, _vp, C.c_float, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64,
        C.c_float, _vp, _vp]),
    "diagpu_spgemm_numeric_astat_scaled_c64": (C.c_int, [
        _i32, _vp, _vp, _i32, _vp, Complex64, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64,
        Complex64, _vp, _vp]),
}

# diagpu.h: DIAGPU_ASTAT_MAX_A, DIAGPU_ASTAT_MAX_A_C64, DIAGPU_SYMBOLIC_SCRATCH_BYTES
ASTAT_MAX_A = 142
ASTAT_MAX_A_C64 = 142
SYMBOLIC_SCRATCH_BYTES = 40 << 20

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load libdiagpu.so from the package directory (cached)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: the HIP library must be built first "
            "(python -m diagpu_amd.build, or __graft_entry__.build())")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in PROTOTYPES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            continue          # reported by missing_symbols() and the ABI test
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def missing_symbols() -> list[str]:
    lib = load()
    return [n for n in PROTOTYPES if not hasattr(lib, n)]


def check(status: int) -> None:
    if status != OK:
        lib = load()
        raise DiagpuError(status, lib.diagpu_status_name(status).decode(),
                          lib.diagpu_last_error().decode())


def call(name: str, *args) -> None:
    """Call entry point `name` and raise DiagpuError on a non-zero status."""
    check(getattr(load(), name)(*args))
