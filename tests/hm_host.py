"""Host (numpy) views of small HM matrices for the GPU tests: a dense float64
copy and a float64 matrix-vector product over the HM diagonals (layout of
spmspm/paper_hm.cuh:18-37).  Test helpers only."""
import numpy as np


def _offsets(M):
    return M.offsets.cpu().tolist()


def dense_of(M) -> np.ndarray:
    """Dense float64 (complex128) copy of a small HM matrix."""
    n = M.n
    offs = _offsets(M)
    starts = M.starts.cpu().numpy()
    v = M.values.cpu().numpy()
    vals = v.astype(np.complex128 if np.iscomplexobj(v) else np.float64)
    D = np.zeros((n, n), vals.dtype)
    for d, s in zip(offs, starts):
        ln = n - abs(d)
        r = np.arange(ln) + max(-d, 0)
        D[r, r + d] = vals[s: s + ln]
    return D


def matvec64(M, x: np.ndarray) -> np.ndarray:
    """y = M x in float64 (complex128 for complex M or x) over the HM
    diagonals."""
    n = M.n
    offs = _offsets(M)
    starts = M.starts.cpu().numpy()
    v = M.values.cpu().numpy()
    cplx = np.iscomplexobj(v) or np.iscomplexobj(x)
    vals = v.astype(np.complex128 if cplx else np.float64)
    y = np.zeros(n, np.complex128 if cplx else np.float64)
    for d, s in zip(offs, starts):
        ln = n - abs(d)
        r0 = max(-d, 0)
        y[r0: r0 + ln] += vals[s: s + ln] * x[r0 + d: r0 + d + ln]
    return y
