"""The benchmark's device-side input generator (synthetic_fill_normal) against the oracle's
generator (oracle_fill_normal: splitmix64 + Box-Muller), so that a seed names the same
inputs in the GPU legs and in the CPU baseline."""

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("n,seed,std", [(1, 7, 1.0), (2, 8, 1.0), (100003, 12345, 0.5), (4096, 2**63 + 5, 0.02)])
def test_device_normal_matches_oracle_generator(gpu, f16, n, seed, std):
    """Same values as the oracle, odd lengths included; at most a last-bit difference
    where the device's double-precision log/cos/sin and glibc's round differently."""
    import cudaforge_amd as cf
    got = cf.DeviceBuffer.normal((n,), np.float16 if f16 else np.float32, seed, std).download()
    want = O.normal((n,), seed, 0.0, std)
    if f16:
        want = O.to_f16(want)
    assert got.shape == want.shape
    same = np.mean(got == want)
    assert same >= 0.999, f"only {same:.5f} identical"
    ulp = np.spacing(np.abs(want).astype(got.dtype))
    assert np.all(np.abs(got.astype(np.float64) - want.astype(np.float64)) <= ulp.astype(np.float64))
