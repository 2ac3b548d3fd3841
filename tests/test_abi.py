"""C ABI of libdiagpu.so on the CPU: every symbol include/diagpu.h declares is
exported, and argument errors come back as status codes before any HIP call
(none of these calls reaches the GPU)."""
import ctypes as C
import re
from pathlib import Path

import pytest

from diagpu_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "diagpu.h").read_text()
    return sorted(set(re.findall(r"DIAGPU_API\s+[\w\s\*]+?\b(diagpu_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_symbols()
    assert len(names) >= 8
    for name in names:
        assert hasattr(lib, name), name
        assert name in _lib.PROTOTYPES, f"{name} has no ctypes prototype"
    assert set(_lib.PROTOTYPES) == set(names)


def test_status_names():
    lib = _lib.load()
    assert lib.diagpu_abi_version() >= 100
    for code, name in [(0, b"DIAGPU_OK"), (1, b"DIAGPU_ERR_ARG"), (5, b"DIAGPU_ERR_CAPACITY")]:
        assert lib.diagpu_status_name(code) == name


def _status(name, *args):
    return getattr(_lib.load(), name)(*args)


def test_spmv_argument_errors():
    V = _lib.ReconViewF32
    fake = C.c_void_p(0x1000)   # never dereferenced: validation fails first
    assert _status("diagpu_spmv_recon_f32", None, fake, 4, fake, None) == _lib.ERR_ARG
    assert b"R is NULL" in _lib.load().diagpu_last_error()
    v = V(-1, 4, 1, fake.value, fake.value)
    assert _status("diagpu_spmv_recon_f32", C.byref(v), fake, 4, fake, None) == _lib.ERR_ARG
    v = V(4, 4, 1, None, fake.value)
    assert _status("diagpu_spmv_recon_f32", C.byref(v), fake, 4, fake, None) == _lib.ERR_ARG
    v = V(4, 4, 1, fake.value, None)
    assert _status("diagpu_spmv_recon_f32", C.byref(v), fake, 4, fake, None) == _lib.ERR_ARG
    v = V(4, 4, 1, fake.value, fake.value)
    assert _status("diagpu_spmv_recon_f32", C.byref(v), None, 4, fake, None) == _lib.ERR_ARG
    assert _status("diagpu_spmv_recon_f32", C.byref(v), fake, 4, None, None) == _lib.ERR_ARG
    assert _status("diagpu_spmv_recon_f32", C.byref(v), fake, -1, fake, None) == _lib.ERR_ARG
    # rows == 0 is a successful no-op (tc_spmv_regdirect_kernel.cu:143)
    v = V(0, 4, 1, None, None)
    assert _status("diagpu_spmv_recon_f32", C.byref(v), None, 0, None, None) == _lib.OK
    w = _lib.ReconViewF64(0, 0, 0, None, None)
    assert _status("diagpu_spmv_recon_f64", C.byref(w), None, 0, None, None) == _lib.OK


def test_python_wrapper_rejects_bad_tensors():
    import torch
    from diagpu_amd.spmv import recon_view
    with pytest.raises(TypeError):
        recon_view(torch.zeros(2, dtype=torch.int32), torch.zeros(8), 4, 4)


def test_spgemm_argument_errors():
    lib = _lib.load()
    sz = C.c_size_t(0)
    assert lib.diagpu_spgemm_symbolic_workspace(0, 1, 1, C.byref(sz)) == _lib.ERR_ARG
    assert lib.diagpu_spgemm_symbolic_workspace(100, -1, 1, C.byref(sz)) == _lib.ERR_ARG
    assert lib.diagpu_spgemm_symbolic_workspace(100, 3, 4, None) == _lib.ERR_ARG
    assert lib.diagpu_spgemm_symbolic_workspace(1 << 20, 9, 7, C.byref(sz)) == _lib.OK
    # A lookup of 2n-1 int32 plus two bitmaps and a word prefix dominate
    assert sz.value >= 4 * (2 * (1 << 20) - 1) + 3 * 4 * ((2 * (1 << 20)) // 32)
    fake = C.c_void_p(0x1000)
    info = _lib.SpgemmInfo()
    args = [100, fake, fake, fake, 3, fake, fake, fake, 2, fake, fake, fake, 6, fake, fake, 6,
            None, fake, 1 << 20, C.byref(info), None]
    bad = list(args); bad[19] = None
    assert lib.diagpu_spgemm_symbolic(*bad) == _lib.ERR_ARG
    bad = list(args); bad[0] = 0
    assert lib.diagpu_spgemm_symbolic(*bad) == _lib.ERR_ARG
    bad = list(args); bad[1] = None
    assert lib.diagpu_spgemm_symbolic(*bad) == _lib.ERR_ARG
    bad = list(args); bad[13] = None
    assert lib.diagpu_spgemm_symbolic(*bad) == _lib.ERR_ARG
    bad = list(args); bad[18] = 16
    assert lib.diagpu_spgemm_symbolic(*bad) == _lib.ERR_CAPACITY
    assert b"workspace" in lib.diagpu_last_error()
    # the same call with the A-stationary records: both records pointers are
    # required, and the symbolic checks come before any HIP call
    rstat = C.c_int32(-1)
    fused = args[:19] + [fake, C.byref(rstat)] + args[19:]
    bad = list(fused); bad[19] = None
    assert lib.diagpu_spgemm_symbolic_astat(*bad) == _lib.ERR_ARG
    assert b"records" in lib.diagpu_last_error()
    bad = list(fused); bad[20] = None
    assert lib.diagpu_spgemm_symbolic_astat(*bad) == _lib.ERR_ARG
    assert b"records_status" in lib.diagpu_last_error()
    bad = list(fused); bad[18] = 16
    assert lib.diagpu_spgemm_symbolic_astat(*bad) == _lib.ERR_CAPACITY
    assert rstat.value == -1                  # untouched when the symbolic phase fails
    # numeric
    assert lib.diagpu_spgemm_numeric_f32(0, fake, fake, fake, fake, fake, 1, fake, fake, 1,
                                         fake, None) == _lib.ERR_ARG
    assert lib.diagpu_spgemm_numeric_f32(10, fake, fake, fake, fake, fake, 0, fake, fake, 0,
                                         fake, None) == _lib.OK      # no C diagonals: no-op
    assert lib.diagpu_spgemm_numeric_f32(10, fake, fake, None, fake, fake, 3, fake, fake, 1,
                                         fake, None) == _lib.ERR_ARG
    assert lib.diagpu_spgemm_numeric_f32(10, fake, fake, fake, fake, fake, 50, fake, fake, 1,
                                         fake, None) == _lib.ERR_ARG  # > 2n - 1 diagonals
    assert lib.diagpu_rowpacked_as_hm(0, fake, 1, fake, fake, None) == _lib.ERR_ARG
    assert lib.diagpu_rowpacked_as_hm(10, None, 1, fake, fake, None) == _lib.ERR_ARG
    assert lib.diagpu_rowpacked_as_hm(10, None, 0, None, None, None) == _lib.OK


def test_axpby_argument_errors():
    lib = _lib.load()
    fake = C.c_void_p(0x1000)
    args = [100, fake, fake, 2, fake, 1.0, fake, fake, 2, fake, 1.0, fake, fake, 3, fake, None]
    bad = list(args); bad[0] = 0
    assert lib.diagpu_dia_axpby_f32(*bad) == _lib.ERR_ARG
    bad = list(args); bad[13] = -1
    assert lib.diagpu_dia_axpby_f32(*bad) == _lib.ERR_ARG
    bad = list(args); bad[14] = None
    assert lib.diagpu_dia_axpby_f32(*bad) == _lib.ERR_ARG
    bad = list(args); bad[1] = None
    assert lib.diagpu_dia_axpby_f32(*bad) == _lib.ERR_ARG
    assert b"X arrays" in lib.diagpu_last_error()
    bad = list(args); bad[13] = 0
    assert lib.diagpu_dia_axpby_f32(*bad) == _lib.OK          # empty Z: no-op


def test_complex_and_krylov_argument_errors():
    fake = C.c_void_p(0x1000)   # never dereferenced: validation fails first
    V = _lib.ReconViewC64
    v = V(4, 4, 1, fake.value, fake.value)
    assert _status("diagpu_spmv_recon_c64", None, fake, 4, fake, None) == _lib.ERR_ARG
    assert _status("diagpu_spmv_recon_c64", C.byref(v), None, 4, fake, None) == _lib.ERR_ARG
    w = _lib.ReconViewF32(4, 4, 1, fake.value, fake.value)
    assert _status("diagpu_spmv_recon_f32_c64", C.byref(w), fake, 4, None, None) == _lib.ERR_ARG
    z = V(0, 0, 0, None, None)
    assert _status("diagpu_spmv_recon_c64", C.byref(z), None, 0, None, None) == _lib.OK

    b = C.c_size_t(0)
    assert _status("diagpu_expm_krylov_workspace", 100, 0, C.byref(b)) == _lib.ERR_ARG
    assert _status("diagpu_expm_krylov_workspace", 100, 65, C.byref(b)) == _lib.ERR_ARG
    assert _status("diagpu_expm_krylov_workspace", 0, 10, C.byref(b)) == _lib.ERR_ARG
    assert _status("diagpu_expm_krylov_workspace", 1000, 10, C.byref(b)) == _lib.OK
    assert b.value >= 10 * 1000 * 8
    info = _lib.KrylovInfo()
    sq = V(1000, 1000, 1, fake.value, fake.value)
    rect = V(1000, 999, 1, fake.value, fake.value)
    call = lambda view, m, ws_bytes, t=1.0: _status(
        "diagpu_expm_krylov_c64", C.byref(view), fake, t, m, fake, fake, ws_bytes, None, None,
        None, C.byref(info), None)
    assert call(rect, 10, b.value) == _lib.ERR_ARG                 # not square
    assert call(sq, 0, b.value) == _lib.ERR_ARG                    # m out of range
    assert call(sq, 10, b.value, float("nan")) == _lib.ERR_ARG     # t not finite
    assert call(sq, 10, b.value - 1) == _lib.ERR_CAPACITY          # workspace too small
    assert b"workspace" in _lib.load().diagpu_last_error()
    assert _status("diagpu_expm_krylov_f32", None, fake, 1.0, 10, fake, fake, b.value, None,
                   None, None, C.byref(info), None) == _lib.ERR_ARG
    assert _status("diagpu_promote_f32_c64", -1, fake, fake, None) == _lib.ERR_ARG
    assert _status("diagpu_promote_f32_c64", 5, None, fake, None) == _lib.ERR_ARG
    assert _status("diagpu_promote_f32_c64", 0, None, None, None) == _lib.OK
    band = _lib.BandInfo()
    assert _status("diagpu_spgemm_band_prepare", 0, fake, fake, 1, fake, fake, 1, fake, 1, fake,
                   C.byref(band), None) == _lib.ERR_ARG
    assert _status("diagpu_spgemm_band_prepare", 100, fake, fake, 70000, fake, fake, 1, fake, 1,
                   fake, C.byref(band), None) == _lib.ERR_ARG
    assert _status("diagpu_spgemm_band_prepare", 100, None, fake, 1, fake, fake, 1, fake, 1, fake,
                   C.byref(band), None) == _lib.ERR_ARG
    assert _status("diagpu_spgemm_band_prepare", 100, fake, fake, 1, None, fake, 1, fake, 1, fake,
                   C.byref(band), None) == _lib.ERR_ARG
    # numeric_band needs an eligible, consistent info (validated before any launch)
    band = _lib.BandInfo(0, 4, 256, 1, 4 * (3 * 256 + 2 * 260) + 16 * 7, 7)
    call = lambda nA, info: _status("diagpu_spgemm_numeric_band_f32", 100, fake, fake, nA, fake,
                                    fake, fake, 2, fake, fake, fake, 5, fake, fake, C.byref(info),
                                    fake, None)
    assert call(4, band) == _lib.ERR_CAPACITY    # lds_bytes does not match nA
    band.eligible = 0
    assert call(3, band) == _lib.ERR_CAPACITY
    # A-stationary kernel: argument checks before any HIP call or launch
    prep = lambda n, aoff, nA, nB, cptr, nC, npairs: _status(
        "diagpu_spgemm_astat_prepare", n, aoff, fake, nA, fake, fake, nB, fake, cptr, nC, fake,
        npairs, fake, None)
    assert prep(0, fake, 1, 1, fake, 1, 1) == _lib.ERR_ARG        # n < 1
    assert prep(10, fake, 0, 1, fake, 1, 1) == _lib.ERR_ARG       # no A diagonal
    assert prep(10, fake, 1, 0, fake, 1, 1) == _lib.ERR_ARG       # no B diagonal
    assert prep(10, None, 1, 1, fake, 1, 1) == _lib.ERR_ARG       # A offsets NULL
    assert prep(10, fake, 1, 1, None, 1, 1) == _lib.ERR_ARG       # pair_ptr NULL
    assert prep(10, fake, 1, 1, fake, 1, -1) == _lib.ERR_ARG      # negative entry count
    assert prep(10, fake, 1, 1, fake, 20, 1) == _lib.ERR_ARG      # c_ndiag > 2n - 1
    assert prep(10, fake, 1, 1, fake, 0, 1) == _lib.ERR_ARG       # entries without C
    astat = lambda nA, nC, n=100, npairs=1: _status("diagpu_spgemm_numeric_astat_f32", n, fake,
                                                    fake, nA, fake, fake, fake, fake, fake, nC,
                                                    fake, fake, npairs, fake, None)
    assert astat(0, 5) == _lib.ERR_ARG
    assert astat(3, 5, 1 << 30) == _lib.ERR_ARG     # n < 2^30 (C stores' 32-bit byte range)
    # the kernel reads metadata and records at 32-bit byte offsets
    assert astat(3, 1 << 29, 1 << 29) == _lib.ERR_ARG          # c_ndiag < 2^29
    assert astat(3, 5, 100, 1 << 28) == _lib.ERR_ARG           # n_pairs < 2^28
    assert astat(_lib.ASTAT_MAX_A + 1, 5) == _lib.ERR_CAPACITY
    assert astat(3, 200) == _lib.ERR_ARG           # c_ndiag > 2n - 1
    assert astat(3, 0) == _lib.OK                   # empty C: nothing to do
    astat_c = lambda nA, nC, n=100, npairs=1: _status("diagpu_spgemm_numeric_astat_c64", n, fake,
                                                      fake, nA, fake, fake, fake, fake, fake, nC,
                                                      fake, fake, npairs, fake, None)
    assert astat_c(0, 5) == _lib.ERR_ARG
    assert astat_c(3, 5, 1 << 30) == _lib.ERR_ARG
    assert astat_c(3, 1 << 29, 1 << 29) == _lib.ERR_ARG
    assert astat_c(3, 5, 100, 1 << 28) == _lib.ERR_ARG
    assert astat_c(_lib.ASTAT_MAX_A_C64 + 1, 5) == _lib.ERR_CAPACITY
    assert astat_c(3, 200) == _lib.ERR_ARG
    assert astat_c(3, 0) == _lib.OK
    # the fused (alpha A) B + sigma I entry points: the same checks, the same limits
    one = _lib.Complex64(1.0, 0.0)
    for name, a, s, cap in (("diagpu_spgemm_numeric_astat_scaled_f32", 2.0, 1.0, _lib.ASTAT_MAX_A),
                            ("diagpu_spgemm_numeric_astat_scaled_c64", one, one,
                             _lib.ASTAT_MAX_A_C64)):
        sc = lambda nA, nC, n=100, npairs=1: _status(name, n, fake, fake, nA, fake, a, fake,
                                                     fake, fake, fake, nC, fake, fake, npairs, s,
                                                     fake, None)
        assert sc(0, 5) == _lib.ERR_ARG
        assert sc(3, 5, 1 << 30) == _lib.ERR_ARG
        assert sc(3, 1 << 29, 1 << 29) == _lib.ERR_ARG
        assert sc(3, 5, 100, 1 << 28) == _lib.ERR_ARG
        assert sc(cap + 1, 5) == _lib.ERR_CAPACITY
        assert sc(3, 200) == _lib.ERR_ARG
        assert sc(3, 0) == _lib.OK
        bad = [100, fake, fake, 3, None, a, fake, fake, fake, fake, 5, fake, fake, 1, s, fake, None]
        assert _status(name, *bad) == _lib.ERR_ARG                # A values NULL


def test_astat_max_a_matches_header():
    """The Python constants mirror DIAGPU_ASTAT_MAX_A and _C64, and the
    staged rows of that many A diagonals (288 fp32; 144 complex64, the
    128-row blocks taken above 75 complex A diagonals) fit a workgroup's
    160 KiB of LDS, one more does not."""
    import re
    hdr = (Path(__file__).resolve().parents[1] / "include" / "diagpu.h").read_text()
    m = re.search(r"#define DIAGPU_ASTAT_MAX_A (\d+)", hdr)
    assert m and int(m.group(1)) == _lib.ASTAT_MAX_A
    assert 288 * _lib.ASTAT_MAX_A * 4 <= 160 * 1024 < 288 * (_lib.ASTAT_MAX_A + 1) * 4
    m = re.search(r"#define DIAGPU_ASTAT_MAX_A_C64 (\d+)", hdr)
    assert m and int(m.group(1)) == _lib.ASTAT_MAX_A_C64
    assert 144 * _lib.ASTAT_MAX_A_C64 * 8 <= 160 * 1024 < 144 * (_lib.ASTAT_MAX_A_C64 + 1) * 8


def test_symbolic_noalloc_rejects_beyond_scratch():
    """diagpu_spgemm_symbolic_noalloc: a workspace larger than the library's
    scratch array is DIAGPU_ERR_CAPACITY, reported before any HIP call (the
    fake pointers are never read)."""
    lib = _lib.load()
    n = 1 << 23
    ws = C.c_size_t(0)
    assert lib.diagpu_spgemm_symbolic_workspace(n, 3, 3, C.byref(ws)) == _lib.OK
    assert ws.value > _lib.SYMBOLIC_SCRATCH_BYTES
    fake = C.c_void_p(0x1000)
    info = _lib.SpgemmInfo()
    st = lib.diagpu_spgemm_symbolic_noalloc(n, fake, fake, fake, 3, fake, fake, fake, 3, fake,
                                            fake, fake, 9, fake, fake, 9, None, C.byref(info),
                                            None)
    assert st == _lib.ERR_CAPACITY
    assert b"scratch" in lib.diagpu_last_error()
    assert lib.diagpu_spgemm_symbolic_noalloc(n, fake, fake, fake, 3, fake, fake, fake, 3, fake,
                                              fake, fake, 9, fake, fake, 9, None, None,
                                              None) == _lib.ERR_ARG


def test_package_modules_import():
    """Every module of the package imports on a host without a GPU (the GPU
    tests would otherwise be the first to meet a broken module)."""
    import importlib

    import diagpu_amd
    names = [f.stem for f in Path(diagpu_amd.__file__).parent.glob("*.py") if f.stem != "__init__"]
    assert {"spgemm", "chain", "spmv", "krylov", "workloads", "_lib", "build"} <= set(names)
    for name in names:
        importlib.import_module(f"diagpu_amd.{name}")
