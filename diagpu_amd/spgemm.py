"""Host-side SpGEMM calls over device tensors: the symbolic plan
(diagpu_spgemm_symbolic) and the numeric phase (diagpu_spgemm_numeric_f32, or
_c64 for complex64 values)
for HM operands, and gemm_diag on row-packed operands
(diagpu_rowpacked_as_hm + the same two phases).

torch tensors only carry device memory and the stream.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from . import _lib
from .spmv import _stream_handle

GPAIR_BYTES = C.sizeof(_lib.GPair)
GPAIR_DTYPE = np.dtype([("ab", "<u8"), ("bb", "<u8"), ("ash", "<i4"), ("bsh", "<i4"),
                        ("al", "<i4"), ("bl", "<i4")])


def _check_dev(t: torch.Tensor, dtype, name: str):
    if not t.is_cuda or t.dtype != dtype or not t.is_contiguous():
        raise TypeError(f"{name} must be a contiguous {dtype} device tensor")


# The band kernel's row block and LDS budget (spgemm_band.hip: kRB,
# kLdsBudget), for telling on the host that a plan cannot fit.
BAND_ROWS = 256
BAND_LDS_BUDGET = 64 * 1024


class SpgemmPlan:
    """C = A * B for HM operands (objects with n, offsets, lengths, starts,
    int32/int32/int64 device tensors).  Builds the C structure and pair plan
    on construction (one stream sync); numeric() then fills C values."""

    def __init__(self, A, B, stream=None, want_lookup: bool = False):
        if A.n != B.n:
            raise ValueError("A and B must have the same dimension")
        for M, nm in ((A, "A"), (B, "B")):
            _check_dev(M.offsets, torch.int32, f"{nm}.offsets")
            _check_dev(M.lengths, torch.int32, f"{nm}.lengths")
            _check_dev(M.starts, torch.int64, f"{nm}.starts")
        self.A, self.B, self.n = A, B, A.n
        self.stream = stream
        dev = A.offsets.device
        na, nb = A.offsets.numel(), B.offsets.numel()
        self.c_cap = max(1, min(na * nb, 2 * self.n - 1))
        self.p_cap = max(1, na * nb)
        ws = C.c_size_t(0)
        _lib.call("diagpu_spgemm_symbolic_workspace", self.n, na, nb, C.byref(ws))
        # the workspace and every plan array in one allocation, 256-byte aligned parts
        parts = [("workspace", torch.uint8, ws.value), ("C_off", torch.int32, self.c_cap),
                 ("C_len", torch.int32, self.c_cap), ("C_starts", torch.int64, self.c_cap),
                 ("ptr", torch.int64, self.c_cap + 1),
                 ("pairs", torch.uint8, self.p_cap * GPAIR_BYTES)]
        if want_lookup:
            parts.append(("lookup", torch.int32, 2 * self.n - 1))
        # where the A-stationary kernel may take the plan, the symbolic call
        # also builds that kernel's records (diagpu_spgemm_symbolic_astat):
        # one stream sync for both
        self._fused = (4096 <= self.n < 1 << 30 and self.p_cap < 1 << 28
                       and na <= max(_lib.ASTAT_MAX_A, _lib.ASTAT_MAX_A_C64))
        if self._fused:
            parts.append(("records", torch.int32, 4 * self.p_cap + 4))
        esz = {torch.uint8: 1, torch.int32: 4, torch.int64: 8}
        sizes = [-(-cnt * esz[dt] // 256) * 256 for _, dt, cnt in parts]
        self._buf = torch.empty(sum(sizes), dtype=torch.uint8, device=dev)
        # the parts' tensor views are made on first use (C_off, ...); the
        # entry points take their addresses, base + byte offset
        self._parts, self._views, o = {}, {}, 0
        for (name, dt, cnt), sz in zip(parts, sizes):
            self._parts[name] = (o, dt, cnt, esz[dt])
            o += sz
        self._base = self._buf.data_ptr()
        self.info = _lib.SpgemmInfo()
        self._band = None
        self._astat = None
        self._rstat = C.c_int32(0)
        self._sym_fn = getattr(_lib.load(), "diagpu_spgemm_symbolic_astat" if self._fused
                               else "diagpu_spgemm_symbolic")
        self._sym_args, self._sym_caps, self._sym_ops = None, None, ()
        self.symbolic()

    def _view(self, name: str):
        v = self._views.get(name)
        if v is None:
            if name not in self._parts:
                return None                 # no lookup was asked for
            o, dt, cnt, e = self._parts[name]
            v = self._views[name] = self._buf[o: o + cnt * e].view(dt)
        return v

    def _addr(self, name: str):
        return self._base + self._parts[name][0] if name in self._parts else None

    C_off = property(lambda self: self._view("C_off"))
    C_len = property(lambda self: self._view("C_len"))
    C_starts = property(lambda self: self._view("C_starts"))
    ptr = property(lambda self: self._view("ptr"))
    pairs = property(lambda self: self._view("pairs"))
    lookup = property(lambda self: self._view("lookup"))
    workspace = property(lambda self: self._view("workspace"))

    def symbolic(self) -> None:
        """(Re)builds the C structure and pair plan from the operands'
        offsets, lengths and starts (diagpu_spgemm_symbolic, or
        diagpu_spgemm_symbolic_astat with the A-stationary records; one
        stream sync)."""
        self._band = None
        self._astat = None
        A, B = self.A, self.B
        ops = (A.offsets, A.lengths, A.starts, B.offsets, B.lengths, B.starts)
        if (self._sym_caps != (self.c_cap, self.p_cap)
                or any(t is not u for t, u in zip(ops, self._sym_ops))):
            # the call's arguments but the stream, kept while the capacities
            # and the operands' structure tensors stay the same objects (held
            # here, so the pointers in the arguments stay valid): one ctypes
            # call per symbolic() with nothing rebuilt
            self._sym_ops = ops
            self._sym_args = (self.n,
                              A.offsets.data_ptr(), A.lengths.data_ptr(), A.starts.data_ptr(),
                              A.offsets.numel(),
                              B.offsets.data_ptr(), B.lengths.data_ptr(), B.starts.data_ptr(),
                              B.offsets.numel(),
                              self._addr("C_off"), self._addr("C_len"), self._addr("C_starts"),
                              self.c_cap, self._addr("ptr"), self._addr("pairs"), self.p_cap,
                              self._addr("lookup"), self._addr("workspace"),
                              self._parts["workspace"][2])
            if self._fused:
                self._sym_args += (self._addr("records"), C.byref(self._rstat))
            self._sym_args += (C.byref(self.info),)
            self._sym_caps = (self.c_cap, self.p_cap)
        st = self._sym_fn(*self._sym_args, _stream_handle(self.stream))
        if st:
            _lib.check(st)
        if self._fused:
            rs = self._rstat.value
            if rs == _lib.OK:
                self._astat = True                # in the records part (viewed on demand)
            elif rs == _lib.ERR_CAPACITY:
                self._astat = False           # B indices beyond 2^30: not this kernel
            else:
                _lib.check(rs)

    # structure views (device tensors) --------------------------------------
    def c_offsets(self) -> torch.Tensor:
        return self.C_off[: self.info.c_ndiag]

    def c_lengths(self) -> torch.Tensor:
        return self.C_len[: self.info.c_ndiag]

    def c_starts(self) -> torch.Tensor:
        return self.C_starts[: self.info.c_ndiag]

    def pair_ptr(self) -> torch.Tensor:
        return self.ptr[: self.info.c_ndiag + 1]

    def pairs_numpy(self) -> np.ndarray:
        raw = self.pairs[: self.info.n_pairs * GPAIR_BYTES].cpu().numpy()
        return raw.view(GPAIR_DTYPE)

    # streams -----------------------------------------------------------------
    def prepare(self, dtype=torch.float32) -> str:
        """Runs now, on the plan's stream, the per-plan set-up of the kernel
        `numeric` takes by default for `dtype` (band or A-stationary
        prepare, each one stream sync), and returns that kernel's name."""
        return self.kernel_for(dtype)

    def hand_over(self, stream) -> None:
        """Continue the plan on `stream` (a torch stream): its buffers are
        marked in use there, so torch's allocator keeps them until the work
        queued on `stream` when they are freed has completed, and later
        launches (numeric, set-up) go there."""
        bufs = [self._buf]
        if self._band is not None:
            bufs.append(self._band[0])
        if isinstance(self._astat, torch.Tensor):
            bufs.append(self._astat)
        for t in bufs:
            t.record_stream(stream)
        self.stream = stream

    # numeric ---------------------------------------------------------------
    def band_info(self):
        """(entries, BandInfo) of diagpu_spgemm_band_prepare for this plan
        (computed once; one stream sync); entries int32 [4 n_pairs + 8]."""
        if self._band is None:
            A, B = self.A, self.B
            pab = torch.empty(4 * self.info.n_pairs + 8, dtype=torch.int32,
                              device=self.C_off.device)
            info = _lib.BandInfo()
            _lib.call("diagpu_spgemm_band_prepare", self.n, A.offsets.data_ptr(),
                      A.starts.data_ptr(), A.offsets.numel(), B.offsets.data_ptr(),
                      B.starts.data_ptr(), B.offsets.numel(), self.pairs.data_ptr(),
                      self.info.n_pairs, pab.data_ptr(), C.byref(info),
                      _stream_handle(self.stream))
            self._band = (pab, info)
        return self._band

    def uses_band(self, dtype=torch.float32) -> bool:
        """The automatic first choice: the LDS-staged band kernel for fp32
        plans whose staged operands fit, whose C diagonals average >= 3
        entries (each operand run then feeds several entries) and that have
        at least 1024 row blocks of 256 (below that the A-stationary kernel
        or the gather is faster: gemm_diag's band, interleaved rounds,
        A-stationary vs band 14.5 vs 20.0 us at n = 2^17, 32.0 vs 27.9 us at
        2^18; the 9-diagonal band's square 6.3 vs 8.2 and 11.7 vs 11.1 us)."""
        na, nb = self.A.offsets.numel(), self.B.offsets.numel()
        if (dtype != torch.float32 or self.info.c_ndiag == 0 or na > 65535 or nb > 32767
                or self.info.n_pairs < 3 * self.info.c_ndiag or self.n < 1024 * 256):
            return False
        est = self.band_lds_estimate()
        if est is not None and est > BAND_LDS_BUDGET:
            return False                          # known without the prepare step's sync
        return bool(self.band_info()[1].eligible)

    def band_lds_estimate(self) -> int | None:
        """The band kernel's LDS bytes per workgroup for this plan, as
        diagpu_spgemm_band_prepare reports them (4 (nA 256 + nB wb) +
        16 n_pairs, wb = 256 + A's offset span rounded up to a multiple of
        4), from A's host offsets when A carries them; else None."""
        ho = getattr(self.A, "host_offsets", None)
        if not ho:
            return None
        span = max(ho) - min(ho)
        wb = (BAND_ROWS + span + 3) & ~3
        return 4 * (len(ho) * BAND_ROWS + self.B.offsets.numel() * wb) + 16 * self.info.n_pairs

    def astat_records(self) -> torch.Tensor:
        """Records of diagpu_spgemm_astat_prepare for this plan; int32
        [4 n_pairs + 4].  Built by the symbolic call where the kernel may
        take the plan, else here, once (diagpu_spgemm_astat_prepare, one
        stream sync; also after `_astat` is reset to None, which makes it
        check the plan's entries again)."""
        if self._astat is True:
            self._astat = self._view("records")[: 4 * self.info.n_pairs + 4]
        if self._astat is None or self._astat is False:
            A = self.A
            rec = torch.empty(4 * self.info.n_pairs + 4, dtype=torch.int32,
                              device=self.C_off.device)
            B = self.B
            _lib.call("diagpu_spgemm_astat_prepare", self.n, A.offsets.data_ptr(),
                      A.starts.data_ptr(), A.offsets.numel(), B.offsets.data_ptr(),
                      B.starts.data_ptr(), B.offsets.numel(), self.C_off.data_ptr(),
                      self.ptr.data_ptr(), self.info.c_ndiag, self.pairs.data_ptr(),
                      self.info.n_pairs, rec.data_ptr(), _stream_handle(self.stream))
            self._astat = rec
        return self._astat

    def uses_astat(self, dtype=torch.float32) -> bool:
        """The automatic choice after the band kernel: the A-stationary kernel
        where A's diagonals fit its LDS (at most DIAGPU_ASTAT_MAX_A, or
        DIAGPU_ASTAT_MAX_A_C64 for complex values), 4096 <= n < 2^30, fewer
        than 2^29 C diagonals and 2^28 plan entries, B has fewer than 2^30
        values (the prepare step's bound), and

          fp32:      any plan, except one of fewer than 16 entries and at
                     least 1.5 per C diagonal at 2^19 <= n < 2^20;
          complex64: n >= 2^16, or >= 3 entries per A diagonal.

        fp32 thresholds from the gather and this kernel timed side by side
        in interleaved rounds over rotated operand sets (median of 10) on
        MI355X, 50 shapes from n = 4096 to 2^22: stencil, band and random
        products with 1 to 64 entries per A diagonal and 1 to 16 per C
        diagonal.  This kernel was faster on 48: by 30-60 % below n = 2^19
        (the gather's per-entry operand reads dominate small products),
        2-20 % above it, config 4 by 3 % (43.3 vs 44.7 us).  The gather was
        faster on the 9-entry square of the tridiagonal band at n = 2^20
        (11.4 vs 12.7 us: too little work per staged block) and tied on a
        36-entry random product at n = 2^20; from n = 2^22 this kernel's
        longer row blocks win again (tridiagonal square 42.5 vs 51.4 us).
        Thin plans (fewer than 16 entries) at 2^19 <= n <= 3 2^20, timed
        again after the scalar-cost changes with every product on operands
        no recent product touched (25 shapes x 2 runs): from n = 2^20 this
        kernel wins all of them, the tridiagonal square by 3-8 % (15.0 vs
        16.3 us at 2^20), plans of one entry per C diagonal by 5-21 %; at
        2^19 the gather wins the tridiagonal square (10.2 vs 13.4 us), random
        3 x 3 and 5-point x tridiagonal by 4-6 %.
        Complex values, timed the same way on 25 shapes from n = 4096 to
        2^22: this kernel was faster on 24, by 5-50 % (the complex gather
        re-reads the operand runs at its items' edges); the gather was
        faster (5.9 vs 6.3 us) on a 4096-row product with 2 entries per A
        diagonal."""
        na = self.A.offsets.numel()
        inf = self.info
        if (inf.c_ndiag == 0 or self.n < 4096 or self.n >= 1 << 30 or inf.c_ndiag >= 1 << 29
                or inf.n_pairs >= 1 << 28):
            return False
        if dtype == torch.float32:
            thin_mid = (inf.n_pairs < 16 and 2 * inf.n_pairs >= 3 * inf.c_ndiag
                        and 1 << 19 <= self.n < 1 << 20)
            ok = na <= _lib.ASTAT_MAX_A and not thin_mid
        elif dtype == torch.complex64:
            ok = na <= _lib.ASTAT_MAX_A_C64 and (self.n >= 1 << 16 or inf.n_pairs >= 3 * na)
        else:
            ok = False
        if not ok:
            return False
        if self._astat is False:                  # refused before: B indices beyond 2^30
            return False
        if self._astat is True:                   # built by the symbolic call
            return True
        try:
            self.astat_records()
        except _lib.DiagpuError as e:
            if e.status != _lib.ERR_CAPACITY:
                raise
            self._astat = False
            return False
        return True

    def mfma_utilisation(self) -> float | None:
        """Useful / issued flops of the MFMA band kernel on this plan (issued:
        2 * 16 * 16 * 4 per block, band_info().mfma_blocks blocks per 16-row
        tile, the four tiles of every 64-row slab), or None if it does not
        take the plan."""
        info = self.band_info()[1]
        if not info.mfma_eligible or info.mfma_blocks == 0:
            return None
        issued = 2 * 16 * 16 * 4 * info.mfma_blocks * 4 * -(-self.n // 64)
        return self.info.useful_flops / issued

    def kernel_for(self, dtype=torch.float32) -> str:
        """The kernel "auto" runs: "band", "astat" or "gather"."""
        if self.uses_band(dtype):
            return "band"
        if self.uses_astat(dtype):
            return "astat"
        return "gather"

    def numeric(self, A_vals: torch.Tensor, B_vals: torch.Tensor, C_vals: torch.Tensor,
                kernel: str = "auto") -> None:
        """C values for the plan's structure; float32 or complex64 (all three
        tensors the same dtype).  kernel: "auto" (kernel_for), "gather" (any
        plan), "band" (fp32, narrow bands) or "astat" (at most
        DIAGPU_ASTAT_MAX_A A diagonals, DIAGPU_ASTAT_MAX_A_C64 for complex
        values), which all return the same bits, or
        "band_mfma" (fp32, narrow bands on the matrix cores: the same values
        to rounding, finite operands)."""
        dt = A_vals.dtype
        name = {torch.float32: "diagpu_spgemm_numeric_f32",
                torch.complex64: "diagpu_spgemm_numeric_c64"}.get(dt)
        if name is None:
            raise TypeError(f"unsupported value dtype {dt}")
        if kernel not in ("auto", "gather", "band", "astat", "band_mfma"):
            raise ValueError(f"unknown kernel {kernel!r}")
        _check_dev(A_vals, dt, "A_vals")
        _check_dev(B_vals, dt, "B_vals")
        _check_dev(C_vals, dt, "C_vals")
        if A_vals.numel() < self.info.a_extent or B_vals.numel() < self.info.b_extent:
            raise ValueError(f"A_vals / B_vals hold {A_vals.numel()} / {B_vals.numel()} values; "
                             f"the plan's operands need {self.info.a_extent} / "
                             f"{self.info.b_extent}")
        if C_vals.numel() < self.info.c_nnz:
            raise ValueError(f"C_vals has {C_vals.numel()} elements, needs {self.info.c_nnz}")
        if kernel == "auto":
            kernel = self.kernel_for(dt)
        if kernel in ("band", "band_mfma") and dt != torch.float32:
            raise TypeError(f"the {kernel} kernel is fp32")
        if kernel == "band_mfma":
            _, info = self.band_info()
            A, B = self.A, self.B
            _lib.call("diagpu_spgemm_numeric_band_mfma_f32", self.n, A.offsets.data_ptr(),
                      A.starts.data_ptr(), A.offsets.numel(), A_vals.data_ptr(),
                      B.offsets.data_ptr(), B.starts.data_ptr(), B.offsets.numel(),
                      B_vals.data_ptr(), self.C_off.data_ptr(), self.C_starts.data_ptr(),
                      self.info.c_ndiag, C.byref(info), C_vals.data_ptr(),
                      _stream_handle(self.stream))
            return
        if kernel == "astat":
            rec = (self._addr("records") if self._astat is True
                   else self.astat_records().data_ptr())
            A = self.A
            _lib.call("diagpu_spgemm_numeric_astat_f32" if dt == torch.float32
                      else "diagpu_spgemm_numeric_astat_c64", self.n, A.offsets.data_ptr(),
                      A.starts.data_ptr(), A.offsets.numel(), A_vals.data_ptr(), B_vals.data_ptr(),
                      self.C_off.data_ptr(), self.C_len.data_ptr(), self.C_starts.data_ptr(),
                      self.info.c_ndiag, self.ptr.data_ptr(), rec, self.info.n_pairs,
                      C_vals.data_ptr(), _stream_handle(self.stream))
            return
        if kernel == "band":
            pab, info = self.band_info()
            A, B = self.A, self.B
            _lib.call("diagpu_spgemm_numeric_band_f32", self.n, A.offsets.data_ptr(),
                      A.starts.data_ptr(), A.offsets.numel(), A_vals.data_ptr(),
                      B.offsets.data_ptr(), B.starts.data_ptr(), B.offsets.numel(),
                      B_vals.data_ptr(), self.C_off.data_ptr(), self.C_starts.data_ptr(),
                      self.info.c_ndiag, self.ptr.data_ptr(), pab.data_ptr(), C.byref(info),
                      C_vals.data_ptr(), _stream_handle(self.stream))
            return
        st = getattr(_lib.load(), name)(
            self.n, A_vals.data_ptr(), B_vals.data_ptr(), self.C_off.data_ptr(),
            self.C_len.data_ptr(), self.C_starts.data_ptr(), self.info.c_ndiag,
            self.ptr.data_ptr(), self.pairs.data_ptr(), self.info.max_pairs,
            C_vals.data_ptr(), _stream_handle(self.stream))
        if st:
            _lib.check(st)

    def numeric_scaled(self, A_vals: torch.Tensor, B_vals: torch.Tensor, C_vals: torch.Tensor,
                       alpha, sigma=0.0) -> None:
        """C = (alpha A) B + sigma I in one pass on the A-stationary kernel
        (diagpu_spgemm_numeric_astat_scaled_f32 / _c64): A scaled in LDS,
        sigma added to C's main diagonal (none where C has no main
        diagonal).  fp32: the bits of numeric() on the operand fl(alpha A)
        plus fl(c + sigma) on the main diagonal.  For any plan that kernel
        takes (its limits, as numeric(kernel="astat"): at most
        DIAGPU_ASTAT_MAX_A A diagonals, or DIAGPU_ASTAT_MAX_A_C64 for complex
        values, 4096 <= n < 2^30, B indices below 2^30); ValueError
        otherwise."""
        dt = A_vals.dtype
        if dt not in (torch.float32, torch.complex64):
            raise TypeError(f"unsupported value dtype {dt}")
        for t, nm in ((A_vals, "A_vals"), (B_vals, "B_vals"), (C_vals, "C_vals")):
            _check_dev(t, dt, nm)
        inf = self.info
        if A_vals.numel() < inf.a_extent or B_vals.numel() < inf.b_extent:
            raise ValueError(f"A_vals / B_vals hold {A_vals.numel()} / {B_vals.numel()} values; "
                             f"the plan's operands need {inf.a_extent} / {inf.b_extent}")
        if C_vals.numel() < inf.c_nnz:
            raise ValueError(f"C_vals has {C_vals.numel()} elements, needs {inf.c_nnz}")
        cap = _lib.ASTAT_MAX_A if dt == torch.float32 else _lib.ASTAT_MAX_A_C64
        if (self.A.offsets.numel() > cap or not 4096 <= self.n < 1 << 30
                or inf.c_ndiag >= 1 << 29 or inf.n_pairs >= 1 << 28):
            raise ValueError("numeric_scaled: the A-stationary kernel does not take this plan")
        if self._astat is not True:
            try:
                self.astat_records()
            except _lib.DiagpuError as e:
                if e.status != _lib.ERR_CAPACITY:
                    raise
                self._astat = False
                raise ValueError("numeric_scaled: B indices beyond the A-stationary "
                                 "kernel's 2^30") from e
        rec = self._addr("records") if self._astat is True else self._astat.data_ptr()
        A = self.A
        if dt == torch.float32:
            name, a, s = "diagpu_spgemm_numeric_astat_scaled_f32", float(alpha), float(sigma)
        else:
            za, zs = complex(alpha), complex(sigma)
            name = "diagpu_spgemm_numeric_astat_scaled_c64"
            a, s = _lib.Complex64(za.real, za.imag), _lib.Complex64(zs.real, zs.imag)
        _lib.call(name, self.n, A.offsets.data_ptr(), A.starts.data_ptr(), A.offsets.numel(),
                  A_vals.data_ptr(), a, B_vals.data_ptr(), self._addr("C_off"),
                  self._addr("C_len"), self._addr("C_starts"), inf.c_ndiag, self._addr("ptr"),
                  rec, inf.n_pairs, s, C_vals.data_ptr(), _stream_handle(self.stream))

    def multiply(self, A_vals: torch.Tensor, B_vals: torch.Tensor,
                 kernel: str = "auto") -> torch.Tensor:
        Cv = torch.empty(max(1, self.info.c_nnz), dtype=A_vals.dtype, device=A_vals.device)
        self.numeric(A_vals, B_vals, Cv, kernel)
        return Cv[: self.info.c_nnz]


class RowPacked:
    """A P x n row-packed operand (gemm_diag layout) addressed as HM."""

    def __init__(self, n: int, offsets: torch.Tensor, DA: torch.Tensor, stream=None):
        _check_dev(offsets, torch.int32, "offsets")
        _check_dev(DA, torch.float32, "DA")
        if DA.numel() != offsets.numel() * n:
            raise ValueError("DA must hold ndiag * n values")
        self.n = n
        self.offsets = offsets
        self.values = DA
        self.starts = torch.empty(offsets.numel(), dtype=torch.int64, device=DA.device)
        self.lengths = torch.empty(offsets.numel(), dtype=torch.int32, device=DA.device)
        _lib.call("diagpu_rowpacked_as_hm", n, offsets.data_ptr(), offsets.numel(),
                  self.starts.data_ptr(), self.lengths.data_ptr(), _stream_handle(stream))


def gemm_diag(n: int, off_A: torch.Tensor, DA: torch.Tensor, off_B: torch.Tensor,
              DB: torch.Tensor, stream=None):
    """C = A * B for row-packed DA, DB (gemm_diag/gemm_diag.cu:9-15); returns
    (plan, C values in the compact C layout)."""
    A = RowPacked(n, off_A, DA, stream)
    B = RowPacked(n, off_B, DB, stream)
    plan = SpgemmPlan(A, B, stream=stream, want_lookup=True)
    return plan, plan.multiply(DA, DB)
