"""Matrix-power chain and truncated Taylor series on HM matrices: the caller
of the SpGEMM hot path that the reference describes but does not ship
(spmspm/gather_flat.cuh:13-14 "recurs each step of a matrix-power chain where
A grows"; :110-117 "fully on-device plan build").

Every product builds its C structure and pair plan on the GPU
(diagpu_spgemm_symbolic; one stream sync returns the counts) and fills C with
diagpu_spgemm_numeric_f32 (or _c64).  Sums and scalings use
diagpu_dia_axpby_f32 (or _c64) over the union of the operands' diagonals; the
union itself is a merge of two short sorted offset lists on the host.  A
Taylor step I + ((t/j) H) S whose plan the A-stationary kernel takes is one
fused product instead (diagpu_spgemm_numeric_astat_scaled_*: H scaled in
LDS, I added to the main diagonal's sums), with no scaling pass over H and
no identity pass over the product.  Values
are float32 or complex64; a complex factor or operand makes the result
complex (propagator(H, dt, order) builds exp(-i dt H), and to_recon hands it
to the SpMV path).

torch tensors only carry device memory; all arithmetic is in libdiagpu.
"""
from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib
from .spgemm import SpgemmPlan, _check_dev
from .spmv import _on_stream, _stream_handle
from .workloads import HM, hm_layout


def hm_structure(n: int, offsets, device, dtype=torch.float32) -> HM:
    """An HM matrix with the given (ascending, distinct) offsets and
    uninitialised values."""
    offs, lens, starts = hm_layout(n, offsets)
    if len(offs) != len(list(offsets)):
        raise ValueError("offsets must be distinct")
    if offs and (offs[0] <= -n or offs[-1] >= n):
        raise ValueError(f"offsets must satisfy |d| < n = {n}")
    return HM(n, torch.tensor(offs, dtype=torch.int32, device=device),
              torch.tensor(lens, dtype=torch.int32, device=device),
              torch.tensor(starts, dtype=torch.int64, device=device),
              torch.empty(max(1, int(sum(lens))), dtype=dtype, device=device)[: int(sum(lens))],
              offs)


def identity(n: int, device, dtype=torch.float32) -> HM:
    I = hm_structure(n, [0], device, dtype)
    I.values.fill_(1.0)
    return I


# Identities the chain reads (never writes), one per (n, device, dtype): a
# Taylor step adds I without building it again.  Each entry keeps the event
# recorded after its fill and the handles of the streams that have read it.
# A stream reading it for the first time waits for that event, and the
# entry's tensors are marked as used on that stream (record_stream), so
# dropping the cache never hands their memory to new work while a read on
# another stream is still queued.
_UNITS: dict = {}


def _unit(n: int, device, dtype) -> HM:
    """The cached identity, ready to be read on torch's current stream."""
    dev = torch.device(device)
    cur = torch.cuda.current_stream(dev)
    key = (n, str(dev), dtype)
    ent = _UNITS.get(key)
    if ent is None:
        if len(_UNITS) >= 8:
            _UNITS.clear()
        I = identity(n, dev, dtype)
        filled = torch.cuda.Event()
        filled.record(cur)
        ent = _UNITS[key] = (I, filled, {cur.cuda_stream})
    I, filled, readers = ent
    if cur.cuda_stream not in readers:
        cur.wait_event(filled)
        for t in (I.offsets, I.starts, I.values):
            t.record_stream(cur)
        readers.add(cur.cuda_stream)
    return I


def as_complex(M: HM, stream=None) -> HM:
    """The same matrix with complex64 values (a copy made on the device by
    diagpu_promote_f32_c64; M itself if already complex)."""
    if M.values.dtype == torch.complex64:
        return M
    _check_dev(M.values, torch.float32, "values")
    with _on_stream(stream):
        out = torch.empty(M.values.numel(), dtype=torch.complex64, device=M.values.device)
        _lib.call("diagpu_promote_f32_c64", M.values.numel(), M.values.data_ptr(),
                  out.data_ptr(), _stream_handle(stream))
    return HM(M.n, M.offsets, M.lengths, M.starts, out, M.host_offsets)


def _c64(z) -> "_lib.Complex64":
    z = complex(z)
    return _lib.Complex64(z.real, z.imag)


def _host_offsets(M: HM) -> list[int]:
    """M's offsets on the host: the copy M carries, else read from the device
    (a stream sync) and kept on M."""
    if M.host_offsets is None:
        M.host_offsets = M.offsets.cpu().tolist()
    return M.host_offsets


def _sumset(n: int, a: list[int], b: list[int]) -> list[int]:
    """The C offsets of A * B as the symbolic phase builds them: every sum
    da + db with |da + db| < n, ascending, once each."""
    s = np.unique(np.add.outer(np.asarray(a, dtype=np.int64), np.asarray(b, dtype=np.int64)))
    return s[(s > -n) & (s < n)].tolist()


def axpby(alpha, X: HM, beta, Y: HM | None, stream=None) -> HM:
    """Z = alpha * X + beta * Y on the union of the two diagonal sets (complex
    if either factor or operand is).  Every temporary and the kernel go on
    `stream` (torch's current stream when None)."""
    with _on_stream(stream):
        return _axpby(alpha, X, beta, Y, stream)


def _axpby(alpha, X: HM, beta, Y: HM | None, stream) -> HM:
    if Y is not None and Y.n != X.n:
        raise ValueError("X and Y must have the same dimension")
    cplx = (isinstance(alpha, complex) or isinstance(beta, complex)
            or X.values.dtype == torch.complex64
            or (Y is not None and Y.values.dtype == torch.complex64))
    if cplx:
        X = as_complex(X, stream)
        Y = as_complex(Y, stream) if Y is not None else None
    dt = torch.complex64 if cplx else torch.float32
    ox = _host_offsets(X)
    oy = _host_offsets(Y) if Y is not None else []
    for offs, nm in ((ox, "X"), (oy, "Y")):
        if any(b <= a for a, b in zip(offs, offs[1:])):
            raise ValueError(f"{nm} offsets must be ascending and distinct")
    if Y is None or oy == ox or set(oy) <= set(ox):
        # Z has X's diagonals: X's structure tensors, new values (no host
        # to device copies: I + t H for an H that holds the main diagonal)
        Z = HM(X.n, X.offsets, X.lengths, X.starts,
               torch.empty(X.values.numel(), dtype=dt, device=X.values.device), ox)
    elif set(ox) <= set(oy):
        Z = HM(Y.n, Y.offsets, Y.lengths, Y.starts,
               torch.empty(Y.values.numel(), dtype=dt, device=Y.values.device), oy)
    else:
        Z = hm_structure(X.n, sorted(set(ox) | set(oy)), X.values.device, dt)
    for M, nm in ((X, "X"), (Y, "Y")):
        if M is not None:
            _check_dev(M.values, dt, f"{nm}.values")
    ny = Y.ndiag if Y is not None else 0
    if cplx:
        a, b, name = _c64(alpha), _c64(beta), "diagpu_dia_axpby_c64"
    else:
        a, b, name = float(alpha), float(beta), "diagpu_dia_axpby_f32"
    _lib.call(name, X.n,
              X.offsets.data_ptr(), X.starts.data_ptr(), X.ndiag, X.values.data_ptr(), a,
              Y.offsets.data_ptr() if ny else None, Y.starts.data_ptr() if ny else None, ny,
              Y.values.data_ptr() if ny else None, b,
              Z.offsets.data_ptr(), Z.starts.data_ptr(), Z.ndiag, Z.values.data_ptr(),
              _stream_handle(stream))
    return Z


@dataclass
class ChainStats:
    """Wall-clock split of a chain (seconds, stream-synchronised per phase)."""
    symbolic: list[float] = field(default_factory=list)
    numeric: list[float] = field(default_factory=list)
    axpby: list[float] = field(default_factory=list)
    c_ndiag: list[int] = field(default_factory=list)
    n_pairs: list[int] = field(default_factory=list)
    useful_flops: list[int] = field(default_factory=list)


def _timed(stats_list, fn, *args, **kw):
    if stats_list is None:
        return fn(*args, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    out = fn(*args, **kw)
    torch.cuda.synchronize()
    stats_list.append(time.perf_counter() - t0)
    return out


def _c_values(nnz: int, like: torch.Tensor) -> torch.Tensor:
    """Uninitialised C values (at least one element allocated, nnz viewed)."""
    v = torch.empty(max(1, nnz), dtype=like.dtype, device=like.device)
    return v if nnz else v[:0]


def multiply(A: HM, B: HM, stats: ChainStats | None = None) -> HM:
    """C = A * B with its plan built on the device for this product (torch's
    current stream; one sync for the symbolic counts)."""
    if A.values.dtype != B.values.dtype:          # a complex operand makes both complex
        A, B = as_complex(A), as_complex(B)
    if stats is not None:
        torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan = SpgemmPlan(A, B)
    plan.prepare(A.values.dtype)      # the numeric kernel's set-up belongs to the plan
    inf = plan.info
    # C's structure arrays are views of the plan's buffer (kept alive by
    # them)
    C = HM(A.n, plan.c_offsets(), plan.c_lengths(), plan.c_starts(),
           _c_values(inf.c_nnz, A.values))
    if stats is not None:
        torch.cuda.synchronize()
    t1 = time.perf_counter()
    if inf.c_ndiag:
        plan.numeric(A.values, B.values, C.values)
    # C's host offsets follow from the operands' where both are known:
    # computed while the product runs
    if A.host_offsets is not None and B.host_offsets is not None:
        C.host_offsets = _sumset(A.n, A.host_offsets, B.host_offsets)
    if stats is not None:
        torch.cuda.synchronize()
        stats.symbolic.append(t1 - t0)
        stats.numeric.append(time.perf_counter() - t1)
        stats.c_ndiag.append(inf.c_ndiag)
        stats.n_pairs.append(inf.n_pairs)
        stats.useful_flops.append(inf.useful_flops)
    return C


def _narrow_first(X: HM) -> bool:
    """Whether a chain step multiplies the narrow factor X from the left: it
    is then the A operand, whose few diagonals the A-stationary kernel holds
    in LDS (the 7-point stencil's last Taylor step, (t H) * S_2 with 377 C
    diagonals: 0.97 ms against 1.24 for S_2 * (t H) on the gather; the
    complex propagator of the same stencil: 4.46 ms against 5.89).  Always
    for real values; for complex values where X fits the complex kernel
    (DIAGPU_ASTAT_MAX_A_C64 diagonals), else the gather takes the product,
    which is faster with the wide factor on the left."""
    return X.values.dtype == torch.float32 or X.ndiag <= _lib.ASTAT_MAX_A_C64


def power(H: HM, k: int, stats: ChainStats | None = None) -> HM:
    """H^k (k >= 1) by the chain P_j = H * P_{j-1} (P_{j-1} * H for complex
    values when H is too wide for the complex A-stationary kernel; the
    factors commute)."""
    if k < 1:
        raise ValueError("k must be >= 1")
    if stats is None:
        return _power_steps(H, k)
    P = H
    for _ in range(k - 1):
        P = multiply(H, P, stats) if _narrow_first(H) else multiply(P, H, stats)
    return P


def _power_steps(H: HM, k: int) -> HM:
    """power() with each product's plan built on the side stream while the
    previous product runs (as _taylor_steps): a plan needs only the
    operands' structure, and P_{j-1}'s is the previous plan's C arrays,
    complete once its symbolic phase has returned.  Products stay on the
    caller's stream, in order."""
    main = torch.cuda.current_stream(H.values.device)
    side = _side_stream(H.values.device)
    side.wait_stream(main)                      # H's structure
    narrow = _narrow_first(H)
    _host_offsets(H)
    P = H
    for _ in range(k - 1):
        with torch.cuda.stream(side):
            plan = SpgemmPlan(H, P, stream=side) if narrow else SpgemmPlan(P, H, stream=side)
            plan.prepare(H.values.dtype)
        plan.hand_over(main)
        inf = plan.info
        C = HM(H.n, plan.c_offsets(), plan.c_lengths(), plan.c_starts(),
               _c_values(inf.c_nnz, H.values))
        if inf.c_ndiag:
            if narrow:
                plan.numeric(H.values, P.values, C.values)
            else:
                plan.numeric(P.values, H.values, C.values)
        C.host_offsets = _sumset(H.n, _host_offsets(H), _host_offsets(P))   # while it runs
        P = C
    return P


def add_identity(S: HM, sigma=1.0, stream=None) -> HM:
    """S + sigma I: in place when S holds the main diagonal, else a new
    matrix on the union of the diagonal sets (on `stream`, like axpby)."""
    with _on_stream(stream):
        return _add_identity(S, sigma, stream)


def _add_identity(S: HM, sigma, stream) -> HM:
    offs = _host_offsets(S)
    dt = S.values.dtype
    I = _unit(S.n, S.values.device, dt)
    if 0 not in offs:
        return axpby(1.0, S, sigma, I, stream)
    i = offs.index(0)
    o4, s8 = S.offsets.element_size(), S.starts.element_size()
    if dt == torch.complex64:
        one, sg, name = _c64(1.0), _c64(sigma), "diagpu_dia_axpby_c64"
    else:
        one, sg, name = 1.0, float(sigma), "diagpu_dia_axpby_f32"
    # X = Z = S's main diagonal alone (one offset, its start), Y = I
    _lib.call(name, S.n,
              S.offsets.data_ptr() + i * o4, S.starts.data_ptr() + i * s8, 1,
              S.values.data_ptr(), one,
              I.offsets.data_ptr(), I.starts.data_ptr(), 1, I.values.data_ptr(), sg,
              S.offsets.data_ptr() + i * o4, S.starts.data_ptr() + i * s8, 1,
              S.values.data_ptr(), _stream_handle(stream))
    return S


def taylor_expm(H: HM, t, order: int, stats: ChainStats | None = None) -> HM:
    """S = sum_{k=0..order} (t H)^k / k! (t real or complex) in Horner form,

        S_order = I + (t/order) H,   S_j = I + S_{j+1} * ((t/j) H),   S = S_1,

    so each step is one device-planned SpGEMM of the wide S_{j+1} and the
    narrow (t/j) H (S_{j+1} is a polynomial in H, so the two commute; the
    narrow factor goes first where the A-stationary kernel holds it:
    _narrow_first), and an in-place add of I to the product's main
    diagonal (a full union pass only when the product lacks that diagonal).
    Where the A-stationary kernel takes a step's plan with H first, the
    scaling, the product and the add of I are one fused launch
    (SpgemmPlan.numeric_scaled); the values are those of the unfused step
    (fp32 bit for bit, complex to rounding)."""
    if order < 0:
        raise ValueError("order must be >= 0")
    dev = H.values.device
    if isinstance(t, complex):
        H = as_complex(H)
    if order == 0:
        return identity(H.n, dev, H.values.dtype)
    ax = stats.axpby if stats else None
    _host_offsets(H)                             # once: every product's offsets follow
    # everything queued before S_order: H's structure is complete once it is
    ready = torch.cuda.Event()
    ready.record(torch.cuda.current_stream(dev))
    S = _timed(ax, axpby, t / order, H, 1.0, _unit(H.n, dev, H.values.dtype))
    if stats is None:
        return _taylor_steps(H, t, order, S, ready)
    for j in range(order - 1, 0, -1):
        S = _horner_step_synced(H, t / j, S, stats)
    return S


def _has_main(H: HM, S: HM) -> bool:
    """Whether H S has a main diagonal: an offset of H has its negation in S."""
    hs = set(_host_offsets(S))
    return any(-d in hs for d in _host_offsets(H))


def _fused(plan: SpgemmPlan, H: HM) -> bool:
    """Whether a Horner step whose plan has H as its A operand runs as one
    fused product (SpgemmPlan.numeric_scaled): the A-stationary kernel takes
    the plan."""
    return plan.kernel_for(H.values.dtype) == "astat"


def _horner_step_synced(H: HM, alpha, S: HM, stats: ChainStats) -> HM:
    """I + (alpha H) S with each phase stream-synchronised into `stats`:
    the plan (symbolic), the product (numeric; fused with the scaling and
    the identity where _fused) and, unfused, the scaling and identity add
    (axpby)."""
    narrow = _narrow_first(H)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    plan = SpgemmPlan(H, S) if narrow else SpgemmPlan(S, H)
    fused = narrow and _fused(plan, H)   # the kernel's set-up belongs to the plan
    inf = plan.info
    C = HM(H.n, plan.c_offsets(), plan.c_lengths(), plan.c_starts(),
           _c_values(inf.c_nnz, H.values))
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    if fused:
        sigma = 1.0 if _has_main(H, S) else 0.0
        if inf.c_ndiag:
            plan.numeric_scaled(H.values, S.values, C.values, alpha, sigma)
        C.host_offsets = _sumset(H.n, _host_offsets(H), _host_offsets(S))   # while it runs
        torch.cuda.synchronize()
        stats.numeric.append(time.perf_counter() - t1)
        if not sigma:
            C = _timed(stats.axpby, add_identity, C)
    else:
        Hj = _timed(stats.axpby, axpby, alpha, H, 0.0, None)   # H's structure: the plan's
        torch.cuda.synchronize()
        t2 = time.perf_counter()
        if inf.c_ndiag:
            if narrow:
                plan.numeric(Hj.values, S.values, C.values)
            else:
                plan.numeric(S.values, Hj.values, C.values)
        C.host_offsets = _sumset(H.n, _host_offsets(H), _host_offsets(S))   # while it runs
        torch.cuda.synchronize()
        stats.numeric.append(time.perf_counter() - t2)
        C = _timed(stats.axpby, add_identity, C)
    stats.symbolic.append(t1 - t0)
    stats.c_ndiag.append(inf.c_ndiag)
    stats.n_pairs.append(inf.n_pairs)
    stats.useful_flops.append(inf.useful_flops)
    return C


# A stream per device for building plans beside the products (default
# priority, like every stream here).
_SIDE: dict = {}


def _side_stream(device) -> torch.cuda.Stream:
    key = str(torch.device(device))
    st = _SIDE.get(key)
    if st is None:
        st = _SIDE[key] = torch.cuda.Stream(device=device)
    return st


def _taylor_steps(H: HM, t, order: int, S: HM, ready: torch.cuda.Event) -> HM:
    """The Horner steps of taylor_expm with each product's plan built on a
    side stream while the previous product runs: a plan needs only its
    operands' structure (the previous plan's C arrays, complete once its
    symbolic phase has returned), so its one stream sync waits for its own
    symbolic phase, not for the product queued before it.  Products,
    scalings and identity adds stay on the caller's stream, in order.
    `ready`: recorded on the caller's stream before S was formed; where S
    shares H's structure, the first plan waits for it only, not for the
    pass that formed S's values."""
    main = torch.cuda.current_stream(H.values.device)
    side = _side_stream(H.values.device)
    if S.offsets is H.offsets and S.starts is H.starts and S.lengths is H.lengths:
        side.wait_event(ready)                  # H's structure
    else:
        side.wait_stream(main)                  # S's structure, formed on main
    narrow = _narrow_first(H)
    for j in range(order - 1, 0, -1):
        # the plan needs the operands' structure only: H's is (t/j) H's
        with torch.cuda.stream(side):
            plan = SpgemmPlan(H, S, stream=side) if narrow else SpgemmPlan(S, H, stream=side)
            fused = narrow and _fused(plan, H)   # the kernel's set-up, on the side stream
        plan.hand_over(main)
        inf = plan.info
        C = HM(H.n, plan.c_offsets(), plan.c_lengths(), plan.c_starts(),
               _c_values(inf.c_nnz, H.values))
        if fused:
            # one pass: (t/j) H scaled in LDS, I added to the main diagonal
            sigma = 1.0 if _has_main(H, S) else 0.0
            if inf.c_ndiag:
                plan.numeric_scaled(H.values, S.values, C.values, t / j, sigma)
        else:
            Hj = axpby(t / j, H, 0.0, None)
            if inf.c_ndiag:
                if narrow:
                    plan.numeric(Hj.values, S.values, C.values)
                else:
                    plan.numeric(S.values, Hj.values, C.values)
            sigma = 0.0
        C.host_offsets = _sumset(H.n, _host_offsets(H), _host_offsets(S))   # while the product runs
        S = C if sigma else add_identity(C)
        if S.offsets is not C.offsets:
            side.wait_stream(main)              # a new structure, written on main
    return S


def propagator(H: HM, dt: float, order: int, stats: ChainStats | None = None) -> HM:
    """U = sum_{k=0..order} (-i dt H)^k / k!, the truncated Taylor propagator
    exp(-i dt H) (complex64) built by the SpGEMM chain: the "build U once,
    apply it cheaply" side of slides/transcript.md:10-18."""
    return taylor_expm(H, complex(0.0, -dt), order, stats)


def to_recon(M: HM, stream=None) -> tuple[torch.Tensor, torch.Tensor]:
    """(offsets descending, values ndiag x n) of M in the Recon layout, built
    on the device (diagpu_hm_to_recon_f32 / _c64), for the SpMV path."""
    dt = M.values.dtype
    name = {torch.float32: "diagpu_hm_to_recon_f32",
            torch.complex64: "diagpu_hm_to_recon_c64"}.get(dt)
    if name is None:
        raise TypeError(f"unsupported value dtype {dt}")
    with _on_stream(stream):
        r_off = torch.empty(M.ndiag, dtype=torch.int32, device=M.values.device)
        r_val = torch.empty(M.ndiag * M.n, dtype=dt, device=M.values.device)
        _lib.call(name, M.n, M.offsets.data_ptr(), M.starts.data_ptr(), M.ndiag,
                  M.values.data_ptr(), r_off.data_ptr(), r_val.data_ptr(),
                  _stream_handle(stream))
    return r_off, r_val
