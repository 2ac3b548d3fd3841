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
