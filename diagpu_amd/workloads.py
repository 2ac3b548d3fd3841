"""Seeded synthetic inputs of the five benchmark configurations, built on the
device with torch (plain tensor fills: they are inputs, not the product).

Recon matrices follow spmv/src/dia_reconstruct.cuh:9-17 (column-indexed,
offsets descending, padding zero); HM matrices follow
spmspm/bench_spmspm.cu:74-86 (offsets ascending, position min(row, col),
int64 starts).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch


def _gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _uniform(shape, lo, hi, g, device, dtype):
    return torch.rand(shape, generator=g, device=device, dtype=dtype) * (hi - lo) + lo


@dataclass
class Recon:
    rows: int
    cols: int
    offsets: torch.Tensor      # int32 [K], descending
    values: torch.Tensor       # [K * cols]
    x: torch.Tensor            # [cols]

    @property
    def K(self) -> int:
        return self.offsets.numel()

    def useful_terms(self) -> int:
        """Number of in-range (row, diagonal) terms, sum_k len(d_k)."""
        o = self.offsets.cpu().numpy().astype(np.int64)
        lo = np.maximum(0, -o)
        hi = np.minimum(self.rows, self.cols - o)
        return int(np.maximum(0, hi - lo).sum())


def zero_recon_padding(offsets: torch.Tensor, values: torch.Tensor, rows: int, cols: int) -> None:
    """Zero Recon[k][c] where row c - d_k is outside [0, rows)."""
    K = offsets.numel()
    v = values.view(K, cols)
    c = torch.arange(cols, device=values.device, dtype=torch.int64)
    for k, d in enumerate(offsets.cpu().tolist()):
        r = c - d
        v[k].masked_fill_((r < 0) | (r >= rows), 0)


def recon_random(n: int, offsets, seed: int, device="cuda", dtype=torch.float32,
                 x_dist: str = "normal") -> Recon:
    """Values U[-1, 1] on every in-range entry, x ~ N(0, 1) or U[-1, 1]."""
    offs = sorted({int(d) for d in offsets}, reverse=True)
    g = _gen(device, seed)
    K = len(offs)
    vals = _uniform((K * n,), -1.0, 1.0, g, device, dtype)
    ot = torch.tensor(offs, dtype=torch.int32, device=device)
    zero_recon_padding(ot, vals, n, n)
    if x_dist == "normal":
        x = torch.randn(n, generator=g, device=device, dtype=dtype)
    else:
        x = _uniform((n,), -1.0, 1.0, g, device, dtype)
    return Recon(n, n, ot, vals, x)


def recon_poisson5(side: int, seed: int, device="cuda", dtype=torch.float32) -> Recon:
    """2-D 5-point Poisson stencil on a side x side grid (benchmark config 2):
    offsets {side, 1, 0, -1, -side}, diagonal 4, off-diagonals -1, the +-1
    entries that wrap across a grid row zeroed, x ~ N(0, 1)."""
    n = side * side
    offs = [side, 1, 0, -1, -side]
    vals = torch.full((5, n), -1.0, device=device, dtype=dtype)
    vals[2].fill_(4.0)
    c = torch.arange(n, device=device, dtype=torch.int64)
    vals[1].masked_fill_(c % side == 0, 0)          # H[r, r+1] with r % side == side-1
    vals[3].masked_fill_(c % side == side - 1, 0)   # H[r, r-1] with r % side == 0
    ot = torch.tensor(offs, dtype=torch.int32, device=device)
    vals = vals.reshape(-1).contiguous()
    zero_recon_padding(ot, vals, n, n)
    g = _gen(device, seed)
    x = torch.randn(n, generator=g, device=device, dtype=dtype)
    return Recon(n, n, ot, vals, x)


def random_band_offsets(count: int, half_width: int, seed: int) -> list[int]:
    """0 plus count-1 distinct offsets drawn uniformly from [-hw, hw] \\ {0}."""
    rng = np.random.default_rng(seed)
    pool = np.array([d for d in range(-half_width, half_width + 1) if d != 0])
    pick = rng.choice(pool, size=count - 1, replace=False)
    return sorted({0, *map(int, pick)})


_M32 = 0xFFFFFFFF


def _mul32(h: torch.Tensor, c: int) -> torch.Tensor:
    """(h * c) mod 2^32 for int64 h in [0, 2^32), in two 16-bit halves of c
    so that no int64 product overflows."""
    lo = h * (c & 0xFFFF)
    hi = (h * (c >> 16)) & 0xFFFF
    return (lo + (hi << 16)) & _M32


def _hash_unit(h: torch.Tensor) -> torch.Tensor:
    """Low 16 bits of h onto [-1, 1) in steps of 2^-15, in fp32 (exact)."""
    return (h & 0xFFFF).to(torch.float32) * (2.0 / 65536.0) - 1.0


def hval(r: torch.Tensor, d: int) -> torch.Tensor:
    """H[r, r + d] of the reference SpMV benchmark's band (integer hash of
    row and offset, spmv/bench/bench_cusparse.cu:70-76) for int64 rows r."""
    h = _mul32(r, 2654435761)
    h = h ^ (((d + 1024) * 40503) & _M32)
    h = h ^ (h >> 13)
    h = _mul32(h, 0x5BD1E995)
    h = h ^ (h >> 15)
    return _hash_unit(h)


def xval(i: torch.Tensor) -> torch.Tensor:
    """x[i] of the same benchmark (bench_cusparse.cu:78-82) for int64 i."""
    h = _mul32(i, 2246822519)
    h = h ^ (h >> 13)
    h = _mul32(h, 0x85EBCA6B)
    h = h ^ (h >> 16)
    return _hash_unit(h)


HASH_BAND_OFFSETS = [-9, -5, -2, -1, 0, 1, 2, 5, 9]   # bench_cusparse.cu:84-87


def hash_band(N: int = 1 << 20, offsets=HASH_BAND_OFFSETS, device="cuda") -> Recon:
    """The reference SpMV benchmark's matrix and x (bench_cusparse.cu:84-98,
    Recon fill :131-144): offsets descending, Recon[k][c] = hval(c - d_k,
    d_k) where row c - d_k exists, zero elsewhere; x[i] = xval(i).  Built
    on the device, value for value the reference's."""
    offs = sorted({int(d) for d in offsets}, reverse=True)
    c = torch.arange(N, device=device, dtype=torch.int64)
    vals = torch.zeros(len(offs), N, device=device, dtype=torch.float32)
    for k, d in enumerate(offs):
        r = c - d
        ok = (r >= 0) & (r < N)
        vals[k] = torch.where(ok, hval(r.clamp(0, N - 1), d), vals[k])
    return Recon(N, N, torch.tensor(offs, dtype=torch.int32, device=device),
                 vals.reshape(-1).contiguous(), xval(c).contiguous())


def spmv_config(cfg: int, seed: int = 0, device="cuda", dtype=torch.float32) -> Recon:
    """Benchmark SpMV configs 1-3: the tridiagonal n = 2^20 band, the
    2048 x 2048 Poisson stencil, and the random 64-diagonal band."""
    if cfg == 1:
        return recon_random(1 << 20, [-1, 0, 1], seed, device, dtype, x_dist="uniform")
    if cfg == 2:
        return recon_poisson5(2048, seed, device, dtype)
    if cfg == 3:
        return recon_random(4_194_304, random_band_offsets(64, 512, seed), seed, device, dtype)
    raise ValueError(f"no SpMV config {cfg}")


# --------------------------------------------------------------------------
# HM (compact) operands for SpGEMM
# --------------------------------------------------------------------------

@dataclass
class HM:
    n: int
    offsets: torch.Tensor      # int32 [D], ascending
    lengths: torch.Tensor      # int32 [D] = n - |d|
    starts: torch.Tensor       # int64 [D]
    values: torch.Tensor       # float32 [sum lengths]
    # a host copy of `offsets` where the builder knew it (None: not known;
    # read it from the device when needed)
    host_offsets: list | None = field(default=None, compare=False, repr=False)

    @property
    def ndiag(self) -> int:
        return self.offsets.numel()

    @property
    def nnz(self) -> int:
        return int(self.values.numel())


def hm_layout(n: int, offsets) -> tuple[list[int], list[int], list[int]]:
    offs = sorted({int(d) for d in offsets})
    lens = [n - abs(d) for d in offs]
    starts = np.concatenate([[0], np.cumsum(lens)[:-1]]).astype(np.int64).tolist() if offs else []
    return offs, lens, starts


def hm_from_values(n: int, offsets, values: torch.Tensor, device="cuda") -> HM:
    offs, lens, starts = hm_layout(n, offsets)
    return HM(n, torch.tensor(offs, dtype=torch.int32, device=device),
              torch.tensor(lens, dtype=torch.int32, device=device),
              torch.tensor(starts, dtype=torch.int64, device=device), values, offs)


def hm_random(n: int, offsets, seed: int, device="cuda") -> HM:
    offs, lens, _ = hm_layout(n, offsets)
    g = _gen(device, seed)
    vals = _uniform((sum(lens),), -1.0, 1.0, g, device, torch.float32)
    return hm_from_values(n, offs, vals, device)


def hm_stencil7(nx: int, ny: int, nz: int, device="cuda") -> HM:
    """3-D 7-point stencil on an nx x ny x nz grid (x fastest): offsets
    {0, +-1, +-nx, +-nx*ny}, diagonal 6, off-diagonals -1, entries whose
    neighbour wraps across a grid line or plane zeroed."""
    n = nx * ny * nz
    offs, lens, _ = hm_layout(n, [0, 1, -1, nx, -nx, nx * ny, -nx * ny])
    parts = []
    for d, ln in zip(offs, lens):
        v = torch.full((ln,), -1.0, device=device, dtype=torch.float32)
        if d == 0:
            v.fill_(6.0)
        else:
            # HM position p -> row i = p - min(d, 0); neighbour of row i is i + d.
            p = torch.arange(ln, device=device, dtype=torch.int64)
            i = p - min(d, 0)
            ad = abs(d)
            if ad == 1:
                bad = (i % nx == nx - 1) if d > 0 else (i % nx == 0)
            elif ad == nx:
                bad = ((i // nx) % ny == ny - 1) if d > 0 else ((i // nx) % ny == 0)
            else:
                bad = torch.zeros_like(i, dtype=torch.bool)   # z planes: padding covers it
            v.masked_fill_(bad, 0)
        parts.append(v)
    return hm_from_values(n, offs, torch.cat(parts), device)


def recon_to_hm(R: Recon) -> HM:
    """HM compact DIA of a square Recon matrix (the inverse of build_recon,
    spmv/src/dia_reconstruct.cuh:77-107): diagonal d, ascending, holds Recon
    row k's columns [max(d, 0), max(d, 0) + n - |d|).  Offsets must be
    distinct and inside (-n, n)."""
    if R.rows != R.cols:
        raise ValueError("recon_to_hm needs a square matrix")
    n = R.rows
    offs = R.offsets.cpu().tolist()
    if len(set(offs)) != len(offs) or any(abs(d) >= n for d in offs):
        raise ValueError("offsets must be distinct and inside (-n, n)")
    order = sorted(range(len(offs)), key=lambda k: offs[k])
    parts = [R.values[k * n + max(offs[k], 0): k * n + max(offs[k], 0) + n - abs(offs[k])]
             for k in order]
    vals = torch.cat(parts).contiguous() if parts else R.values.new_empty(0)
    return hm_from_values(n, [offs[k] for k in order], vals, R.values.device)


def mt19937_uniform(seed: int, count: int, a: float, b: float) -> np.ndarray:
    """count draws of std::uniform_real_distribution<float>(a, b) over
    std::mt19937(seed) as libstdc++ computes them: one 32-bit MT19937 output
    per value (numpy's RandomState is MT19937 with the same init_genrand
    seeding), generate_canonical<float, 24> = g / 2^32 in float (a result of
    1.0 replaced by the float just below it), then g * (b - a) + a in float."""
    raw = np.random.RandomState(seed).randint(0, 2 ** 32, size=count, dtype=np.uint32)
    g = raw.astype(np.float32) / np.float32(2.0 ** 32)
    g = np.where(g >= 1, np.nextafter(np.float32(1), np.float32(0)), g).astype(np.float32)
    return (g * (np.float32(b) - np.float32(a)) + np.float32(a)).astype(np.float32)


def make_banded(n: int, w: int, seed: int, device="cuda") -> HM:
    """make_banded of the reference SpGEMM benchmark
    (spmspm/bench_spmspm.cu:89-106): offsets -w..w (those with n - |d| > 0),
    each diagonal's n - |d| values drawn in order from U(-1, 1) with
    std::mt19937(seed), libstdc++'s mapping (mt19937_uniform)."""
    offs = [d for d in range(-w, w + 1) if n - abs(d) > 0]
    total = sum(n - abs(d) for d in offs)
    vals = torch.from_numpy(mt19937_uniform(seed, total, -1.0, 1.0)).to(device)
    return hm_from_values(n, offs, vals, device)


def spgemm_config(cfg: int, seed: int = 0, device="cuda") -> tuple[HM, HM]:
    """Benchmark SpGEMM configs 4 and 5; for configs 1-3 (SpMV matrices)
    the product H H of that config's matrix."""
    if cfg in (1, 2, 3):
        H = recon_to_hm(spmv_config(cfg, seed, device))
        return H, H
    if cfg == 4:
        n = 1 << 20
        A = hm_random(n, range(-4, 5), seed, device)
        B = hm_stencil7(128, 128, 64, device)     # offsets {0, +-1, +-128, +-16384}
        assert B.n == n
        return A, B
    if cfg == 5:
        n = 262_144
        rng = np.random.default_rng(seed)
        oa = rng.choice(np.arange(-4096, 4097), size=128, replace=False)
        ob = rng.choice(np.arange(-4096, 4097), size=128, replace=False)
        return hm_random(n, oa, seed, device), hm_random(n, ob, seed + 1, device)
    raise ValueError(f"no SpGEMM config {cfg}")
