"""Host logic of the workload builders (CPU): Recon -> HM is the inverse of
the reference's build_recon (spmv/src/dia_reconstruct.cuh:77-107)."""
import numpy as np
import pytest
import torch

from diagpu_amd import workloads


@pytest.mark.parametrize("n,offs", [(1000, [-999, -3, 0, 1, 64, 999]), (7, [0]), (50, [5, -5, 2])])
def test_recon_to_hm_inverts_build_recon(oracle, n, offs):
    R = workloads.recon_random(n, offs, seed=n, device="cpu")
    H = workloads.recon_to_hm(R)
    o = H.offsets.numpy()
    assert list(o) == sorted(offs)
    assert list(H.lengths.numpy()) == [n - abs(d) for d in o]
    r_off, r_val = oracle.build_recon(n, n, o, H.starts.numpy(), H.lengths.numpy(), H.values.numpy())
    # build_recon orders offsets descending, as the Recon builders do
    assert np.array_equal(r_off, R.offsets.numpy())
    assert np.array_equal(r_val, R.values.numpy())


def test_recon_to_hm_rejects():
    R = workloads.recon_random(10, [0, 1], seed=1, device="cpu")
    R2 = workloads.Recon(10, 10, torch.tensor([1, 1], dtype=torch.int32), R.values, R.x)
    with pytest.raises(ValueError):
        workloads.recon_to_hm(R2)
    R3 = workloads.Recon(10, 12, R.offsets, torch.zeros(24), torch.zeros(12))
    with pytest.raises(ValueError):
        workloads.recon_to_hm(R3)


# ---------------------------------------------------------------------------
# The reference benchmarks' own input generators in the package (used by
# bench.py to time those shapes), against the digests of the reference's
# source text run as written (tests/golden/generators.json).
# ---------------------------------------------------------------------------

import hashlib
import json
from pathlib import Path

GEN = json.loads((Path(__file__).resolve().parent / "golden" / "generators.json").read_text())


def _check(a, s):
    a = np.ascontiguousarray(a, np.float32)
    assert a.size == s["count"]
    if "bits" in s:
        assert a.view(np.uint32).tolist() == s["bits"]
    else:
        assert a[:64].view(np.uint32).tolist() == s["head_bits"]
    assert hashlib.sha256(a.tobytes()).hexdigest() == s["sha256"]


@pytest.mark.parametrize("idx", range(len(GEN["hval"])))
def test_hash_band_matches_reference(idx):
    """workloads.hash_band (torch integer hash) against bench_cusparse.cu:70-82,
    131-144 run as written: every band entry H[r, r + d], offset by offset
    in the fixture's order, rows ascending (N = 64 value for value, N = 2^20
    by digest); the padding of each Recon row is zero; x against xval."""
    f = GEN["hval"][idx]
    N = f["N"]
    R = workloads.hash_band(N, f["offsets"], device="cpu")
    assert R.offsets.tolist() == sorted(f["offsets"], reverse=True)
    V = R.values.view(R.K, N)
    k_of = {d: k for k, d in enumerate(R.offsets.tolist())}
    band, pad = [], []
    for d in f["offsets"]:
        c = np.arange(N)
        ok = (c - d >= 0) & (c - d < N)
        band.append(V[k_of[d]].numpy()[ok])     # column c = row c - d + d, rows ascending
        pad.append(V[k_of[d]].numpy()[~ok])
    _check(np.concatenate(band), f)
    assert not np.concatenate(pad).any()
    xs = [x for x in GEN["xval"] if x["N"] == N]
    for x in xs:
        _check(R.x.numpy(), x)


def test_xval_matches_reference():
    for f in GEN["xval"]:
        _check(workloads.xval(torch.arange(f["N"], dtype=torch.int64)).numpy(), f)


@pytest.mark.parametrize("idx", range(len(GEN["make_banded"])))
def test_make_banded_matches_reference(idx):
    """workloads.make_banded against spmspm/bench_spmspm.cu:89-106 run as
    written (libstdc++'s mt19937 and uniform_real_distribution): offsets,
    lengths, int64 starts and every value (small cases bit for bit, the
    bench's make_banded(100000, 16, 1234 / 5678) by digest)."""
    f = GEN["make_banded"][idx]
    M = workloads.make_banded(f["n"], f["w"], f["seed"], device="cpu")
    assert M.offsets.tolist() == f["offsets"]
    assert M.lengths.tolist() == f["lengths"]
    assert M.starts.tolist() == f["starts"]
    _check(M.values.numpy(), f["values"])
