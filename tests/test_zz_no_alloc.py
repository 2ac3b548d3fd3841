"""diagpu_spgemm_symbolic_noalloc against diagpu_spgemm_symbolic, through the
C ABI: the same C structure, lookup, pair plan and counts, bit for bit, on
calls in a row, each smaller than the one before (stale scratch contents
from the previous call would show), on the one-launch path (which keeps only
its state record in the scratch array) and on the multi-launch path (whose
A lookup, bitmaps and prefix sums live there); and from two host threads on
two streams at once, which the per-device lock serialises.  The size limit
is checked on the CPU (tests/test_abi.py)."""
import ctypes as C
import threading

import numpy as np
import pytest
import torch

from diagpu_amd import _lib, workloads

pytestmark = pytest.mark.gpu


def _outputs(n, na, nb, dev):
    c_cap = max(1, min(na * nb, 2 * n - 1))
    p_cap = max(1, na * nb)
    return {
        "C_off": torch.full((c_cap,), -7, dtype=torch.int32, device=dev),
        "C_len": torch.full((c_cap,), -7, dtype=torch.int32, device=dev),
        "C_starts": torch.full((c_cap,), -7, dtype=torch.int64, device=dev),
        "ptr": torch.full((c_cap + 1,), -7, dtype=torch.int64, device=dev),
        "pairs": torch.full((p_cap * C.sizeof(_lib.GPair),), 0xA5, dtype=torch.uint8,
                            device=dev),
        "lookup": torch.full((2 * n - 1,), -7, dtype=torch.int32, device=dev),
        "c_cap": c_cap, "p_cap": p_cap,
    }


def _symbolic(A, B, noalloc, stream=None):
    if stream is not None:      # outputs made, filled and read on `stream` too
        with torch.cuda.stream(stream):
            return _symbolic_on(A, B, noalloc, stream.cuda_stream)
    return _symbolic_on(A, B, noalloc, None)


def _symbolic_on(A, B, noalloc, sh):
    n, dev = A.n, A.offsets.device
    na, nb = A.offsets.numel(), B.offsets.numel()
    out = _outputs(n, na, nb, dev)
    info = _lib.SpgemmInfo()
    head = (n, A.offsets.data_ptr(), A.lengths.data_ptr(), A.starts.data_ptr(), na,
            B.offsets.data_ptr(), B.lengths.data_ptr(), B.starts.data_ptr(), nb,
            out["C_off"].data_ptr(), out["C_len"].data_ptr(), out["C_starts"].data_ptr(),
            out["c_cap"], out["ptr"].data_ptr(), out["pairs"].data_ptr(), out["p_cap"],
            out["lookup"].data_ptr())
    if noalloc:
        _lib.call("diagpu_spgemm_symbolic_noalloc", *head, C.byref(info), sh)
    else:
        ws = C.c_size_t(0)
        _lib.call("diagpu_spgemm_symbolic_workspace", n, na, nb, C.byref(ws))
        work = torch.empty(ws.value, dtype=torch.uint8, device=dev)
        _lib.call("diagpu_spgemm_symbolic", *head, work.data_ptr(), work.numel(),
                  C.byref(info), sh)
    torch.cuda.synchronize()
    nc, npair = info.c_ndiag, info.n_pairs
    res = {
        "C_off": out["C_off"][:nc].cpu().numpy(),
        "C_len": out["C_len"][:nc].cpu().numpy(),
        "C_starts": out["C_starts"][:nc].cpu().numpy(),
        "ptr": out["ptr"][:nc + 1].cpu().numpy(),
        "pairs": out["pairs"][:npair * C.sizeof(_lib.GPair)].cpu().numpy(),
        "lookup": out["lookup"].cpu().numpy(),
    }
    counts = (info.c_ndiag, info.c_nnz, info.n_pairs, info.max_pairs, info.useful_flops,
              info.a_extent, info.b_extent)
    return res, counts


def _operands(n, na, nb, span, seed, dev):
    rng = np.random.default_rng(seed)
    oa = rng.choice(np.arange(-span, span + 1), size=na, replace=False)
    ob = rng.choice(np.arange(-span, span + 1), size=nb, replace=False)
    return (workloads.hm_random(n, oa, seed=seed, device=dev),
            workloads.hm_random(n, ob, seed=seed + 1, device=dev))


def _equal(got, want):
    (g, gc), (w, wc) = got, want
    assert gc == wc, (gc, wc)
    assert wc[0] > 0 and wc[2] > 0
    for key in w:
        assert np.array_equal(g[key], w[key]), key


def _same(A, B):
    want = _symbolic(A, B, noalloc=False)
    _equal(_symbolic(A, B, noalloc=True), want)


def _wide(n, offs_a, offs_b, seed, dev):
    return (workloads.hm_random(n, offs_a, seed=seed, device=dev),
            workloads.hm_random(n, offs_b, seed=seed + 1, device=dev))


def _large_product(dev):
    """1100 x 1000 diagonals at n = 1200: more operand products than the
    one-launch path enumerates."""
    n = 1200
    rng = np.random.default_rng(17)
    oa = rng.choice(np.arange(-n + 1, n), size=1100, replace=False)
    ob = rng.choice(np.arange(-n + 1, n), size=1000, replace=False)
    return _wide(n, oa, ob, 83, dev)


def test_noalloc_matches_workspace_entry(dev):
    print("noalloc: config 4 operands, n = 2^20", flush=True)
    A, B = workloads.spgemm_config(4, seed=4, device=dev)
    _same(A, B)
    print("noalloc: smaller random product, n = 3001", flush=True)
    A2, B2 = _operands(3001, 40, 8, 2999, seed=7, dev=dev)
    _same(A2, B2)
    print("noalloc: n = 37 after the larger calls", flush=True)
    A3, B3 = _operands(37, 5, 4, 36, seed=8, dev=dev)
    _same(A3, B3)



def test_noalloc_multi_launch_path(dev):
    print("noalloc: wide spans, n = 600000 (multi-launch path)", flush=True)
    A, B = _wide(600_000, [-599_999, 0, 599_999], [-599_999, -1, 2, 599_999], 81, dev)
    _same(A, B)
    print("noalloc: 1100 x 1000 diagonals, n = 1200 (multi-launch path)", flush=True)
    A2, B2 = _large_product(dev)
    _same(A2, B2)
    print("noalloc: n = 37 after the multi-launch calls", flush=True)
    A3, B3 = _operands(37, 5, 4, 36, seed=8, dev=dev)
    _same(A3, B3)


def test_noalloc_two_threads(dev):
    """Two host threads, each on its own stream, call the no-alloc entry
    point at the same time, six times each (one thread on the multi-launch
    path, one on the one-launch path): every result equals its workspace
    twin bit for bit."""
    cases = [_wide(600_000, [-599_999, 0, 599_999], [-599_999, -1, 2, 599_999], 81, dev),
             workloads.spgemm_config(4, seed=4, device=dev)]
    want = [_symbolic(A, B, noalloc=False) for A, B in cases]
    torch.cuda.synchronize()
    results = [[], []]
    errors = []
    start = threading.Barrier(2)

    def work(i):
        try:
            s = torch.cuda.Stream(device=dev)
            start.wait()
            for _ in range(6):
                results[i].append(_symbolic(*cases[i], noalloc=True, stream=s))
        except Exception as e:          # reported by the main thread
            errors.append(e)

    print("noalloc: two threads, two streams", flush=True)
    threads = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    assert not errors, errors
    for i in range(2):
        assert len(results[i]) == 6
        for got in results[i]:
            _equal(got, want[i])
