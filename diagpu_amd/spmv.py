"""Host-side SpMV call over device tensors (the Recon layout of
spmv/src/dia_reconstruct.cuh:61-118, the launcher of
spmv/src/tc_spmv_regdirect_kernel.cu:135-147).

torch tensors only carry device memory and the stream; the work is done by
diagpu_spmv_recon_f32 / _f64 / _c64 / _f32_c64 in libdiagpu.so.
"""
from __future__ import annotations

import contextlib
import ctypes as C

import torch

from . import _lib


def _on_stream(stream):
    """Context in which torch allocates and launches on `stream` (a
    torch.cuda.Stream, a raw HIP stream handle, or None for the current
    stream), so a wrapper's temporaries are ordered with its kernels."""
    if stream is None:
        return contextlib.nullcontext()
    if not isinstance(stream, torch.cuda.Stream):
        stream = torch.cuda.ExternalStream(int(stream))
    return torch.cuda.stream(stream)


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_handle(stream) -> int:
    if stream is None:
        if _raw_stream is not None:      # the current stream's handle, without a Stream object
            return _raw_stream(torch.cuda.current_device())
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


def recon_view(offsets: torch.Tensor, values: torch.Tensor, rows: int, cols: int):
    """ReconView over device tensors: offsets int32 [K], values [K * cols]."""
    if offsets.dtype != torch.int32 or not offsets.is_cuda:
        raise TypeError("offsets must be an int32 device tensor")
    if not values.is_cuda or not values.is_contiguous():
        raise TypeError("values must be a contiguous device tensor")
    K = offsets.numel()
    if values.numel() != K * cols:
        raise ValueError(f"values has {values.numel()} elements, expected K*cols = {K * cols}")
    cls = {torch.float32: _lib.ReconViewF32, torch.float64: _lib.ReconViewF64,
           torch.complex64: _lib.ReconViewC64}.get(values.dtype)
    if cls is None:
        raise TypeError(f"unsupported dtype {values.dtype}")
    return cls(rows, cols, K, offsets.data_ptr(), values.data_ptr())


# (matrix dtype, vector dtype) -> entry point
_SPMV = {
    (torch.float32, torch.float32): "diagpu_spmv_recon_f32",
    (torch.float64, torch.float64): "diagpu_spmv_recon_f64",
    (torch.complex64, torch.complex64): "diagpu_spmv_recon_c64",
    (torch.float32, torch.complex64): "diagpu_spmv_recon_f32_c64",
}


def spmv_recon(offsets: torch.Tensor, values: torch.Tensor, rows: int, cols: int,
               x: torch.Tensor, y: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """y = H x for the Recon matrix (offsets, values); y is overwritten.
    Values and x: float32/float32, float64/float64, complex64/complex64, or
    float32 values with a complex64 x (y takes x's dtype)."""
    view = recon_view(offsets, values, rows, cols)
    name = _SPMV.get((values.dtype, x.dtype))
    if name is None or not x.is_cuda or not x.is_contiguous():
        raise TypeError(f"unsupported (values, x) dtypes ({values.dtype}, {x.dtype}), "
                        "or x not a contiguous device tensor")
    if y is None:
        y = torch.empty(rows, dtype=x.dtype, device=values.device)
    if y.dtype != x.dtype or y.numel() < rows or not y.is_cuda or not y.is_contiguous():
        raise TypeError("y must be a contiguous device tensor of x's dtype with >= rows elements")
    _lib.call(name, C.byref(view), x.data_ptr(), x.numel(), y.data_ptr(), _stream_handle(stream))
    return y
