"""The device generator of the large synthetic weights (synth.normal_torch on the GPU) against the host's
synth.normal: the same SplitMix64 stream and Box-Muller transform, so the same f32 values, bit for bit,
wherever the device's f64 log / sqrt / cos / sin round like the host's (checked here over 4M values)."""
import numpy as np
import pytest
import torch

from inference_amd.synth import normal, normal_torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("seed,n", [(4 * 1000003, 1 << 22), (71, (1 << 20) + 1)])
def test_device_weights_equal_host_generator(seed, n):
    a = normal(seed, (n,), 0.02)
    b = normal_torch(seed, (n,), 0.02, device=torch.device("cuda:0")).cpu().numpy()
    bad = np.flatnonzero(a.view(np.uint32) != b.view(np.uint32))
    assert bad.size == 0, (bad.size, bad[:5], a[bad[:5]], b[bad[:5]])
