"""Krylov propagator psi(t) = exp(-i t H) psi_0 (Lanczos) over device
tensors: diagpu_expm_krylov_c64 (complex64 H) and diagpu_expm_krylov_f32
(real fp32 H applied to a complex state) in libdiagpu.so.

The matrix-free SpMV caller of slides/transcript.md:10-18 (one trajectory,
H applied to the state again and again); the reference ships no driver.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .spmv import _stream_handle, recon_view


@dataclass
class KrylovResult:
    psi: torch.Tensor          # complex64 [n], exp(-i t H) psi_0
    steps: int                 # Lanczos steps used
    breakdown: bool            # invariant subspace reached (result exact)
    psi0_norm: float
    err_estimate: float        # ||psi_0|| beta_m |[exp(-i t T_m)]_{m,1}|
    alpha: np.ndarray          # T_m diagonal (fp64, host)
    beta: np.ndarray           # T_m off-diagonal (fp64, host)


class KrylovWorkspace:
    """Device workspace for n x n operators and up to m steps (reusable), and
    the pinned host buffer (2m+1 doubles) that T_m's entries come back in."""

    def __init__(self, n: int, m: int, device="cuda"):
        b = C.c_size_t(0)
        _lib.call("diagpu_expm_krylov_workspace", n, m, C.byref(b))
        self.n, self.m = n, m
        self.buf = torch.empty(b.value, dtype=torch.uint8, device=device)
        self.host = torch.empty(2 * m + 1, dtype=torch.float64, pin_memory=True)


def expm_krylov(offsets: torch.Tensor, values: torch.Tensor, n: int, psi0: torch.Tensor,
                t: float, m: int = 30, out: torch.Tensor | None = None,
                workspace: KrylovWorkspace | None = None, stream=None) -> KrylovResult:
    """exp(-i t H) psi0 for the Hermitian n x n Recon matrix (offsets, values);
    values float32 (real symmetric H) or complex64; psi0 complex64 [n]."""
    if (psi0.dtype != torch.complex64 or not psi0.is_cuda or psi0.numel() != n
            or not psi0.is_contiguous()):
        raise TypeError("psi0 must be a contiguous complex64 device tensor of n elements")
    view = recon_view(offsets, values, n, n)
    name = {torch.complex64: "diagpu_expm_krylov_c64",
            torch.float32: "diagpu_expm_krylov_f32"}.get(values.dtype)
    if name is None:
        raise TypeError(f"unsupported matrix dtype {values.dtype}")
    if workspace is None or workspace.n != n or workspace.m < m:
        workspace = KrylovWorkspace(n, m, psi0.device)
    if out is None:
        out = torch.empty_like(psi0)
    if (out.dtype != torch.complex64 or not out.is_cuda or out.numel() != n
            or not out.is_contiguous()):
        raise TypeError("out must be a contiguous complex64 device tensor of n elements")
    if out.data_ptr() == psi0.data_ptr():
        raise ValueError("out must not overlap psi0")
    alpha = np.zeros(m, np.float64)
    beta = np.zeros(m, np.float64)
    info = _lib.KrylovInfo()
    _lib.call(name, C.byref(view), psi0.data_ptr(), float(t), int(m), out.data_ptr(),
              workspace.buf.data_ptr(), workspace.buf.numel(), workspace.host.data_ptr(),
              alpha.ctypes.data_as(C.c_void_p), beta.ctypes.data_as(C.c_void_p),
              C.byref(info), _stream_handle(stream))
    return KrylovResult(out, info.steps, bool(info.breakdown), info.psi0_norm,
                        info.err_estimate, alpha[: info.steps], beta[: info.steps])
