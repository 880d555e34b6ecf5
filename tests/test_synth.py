"""The synthetic-input generator (inference_amd/synth.py): SplitMix64 as the reference's sampler defines it
(crates/llm/candle-llm/src/primitives/sampler.rs:27-52) feeding a Box-Muller transform in f64.

* the reference's known-answer test (sampler.rs:292-296): seed 0 yields 0xE220A8397B1DCDAF, then
  0x6E789E6AA1B965F4, and the counter-based form is the sequential generator's stream at every offset;
* normal() maps the stream to N(0, std^2) as stated: the first pair from the KAT values by hand, and the
  sample moments of a large draw;
* normal_torch() (the device generator of the large weights) equals normal() bit for bit here on the CPU,
  across chunk boundaries and odd lengths.
"""
import math

import numpy as np
import torch

from inference_amd.synth import normal, normal_torch, splitmix64


def sequential(seed, count):
    """The reference's SplitMix64::next_u64, one value at a time in Python integers."""
    m = (1 << 64) - 1
    state, out = seed, []
    for _ in range(count):
        state = (state + 0x9E3779B97F4A7C15) & m
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        out.append(z ^ (z >> 31))
    return out


def test_splitmix64_known_answers():
    assert [int(v) for v in splitmix64(0, 2)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]
    assert sequential(0, 2) == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4]


def test_counter_form_is_the_sequential_stream():
    for seed in (0, 1, 42, (1 << 63) + 12345):
        seq = sequential(seed, 200)
        assert [int(v) for v in splitmix64(seed, 200)] == seq
        assert [int(v) for v in splitmix64(seed, 50, 150)] == seq[150:]


def test_normal_first_pair_by_hand():
    r0, r1 = sequential(5, 2)
    u1 = ((r0 >> 11) + 1) / 2.0 ** 53
    u2 = (r1 >> 11) / 2.0 ** 53
    rad = math.sqrt(-2.0 * math.log(u1)) * 0.5
    want = np.array([rad * math.cos(2 * math.pi * u2), rad * math.sin(2 * math.pi * u2)], dtype=np.float32)
    assert np.array_equal(normal(5, (2,), 0.5), want)


def test_normal_moments():
    z = normal(3, (1 << 20,)).astype(np.float64)
    assert abs(z.mean()) < 5 / 1024  # 5 sigma of the mean of 2^20 draws
    assert abs(z.std() - 1.0) < 5e-3
    assert abs(np.mean(z ** 4) - 3.0) < 0.05  # Gaussian kurtosis


def test_device_generator_equals_host_generator():
    for seed, n, chunk in ((0, 1000, 1 << 25), (7, 12345, 1000), (2 ** 40 + 7, (1 << 20) + 3, 1 << 18)):
        a = normal(seed, (n,), 0.02)
        b = normal_torch(seed, (n,), 0.02, device="cpu", chunk=chunk).numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), seed
    assert normal_torch(1, (3, 5), device="cpu").shape == torch.Size([3, 5])
