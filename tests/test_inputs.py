"""The package's synthetic input generator (cuda_fused_attention_amd/inputs.py,
used by bench.py) against the oracle's C generator: both must give the same
bf16 bit patterns, so benchmark inputs and parity-test inputs are the same
tensors."""
import numpy as np
import pytest

import oracle
from cuda_fused_attention_amd import inputs


@pytest.mark.parametrize("shape,seed", [((1, 2, 128, 64), 11), ((3, 5, 7), 22), ((1, 1, 4099, 128), 33),
                                        ((2, 3, 17, 64), 0), ((5,), 2**63 + 12345)])
def test_uniform_matches_oracle(shape, seed):
    assert np.array_equal(inputs.fill_uniform(shape, seed), oracle.fill_uniform(shape, seed))


def test_uniform_chunking_is_seamless():
    shape = (3, 1000)
    assert np.array_equal(inputs.fill_uniform(shape, 7, chunk=257), inputs.fill_uniform(shape, 7))


def test_make_uniform_inputs_seeds():
    q, k, v = inputs.make_uniform_inputs(1, 2, 33, 64)
    oq, ok, ov = oracle.make_inputs(1, 2, 33, 64, "uniform")
    assert np.array_equal(q, oq) and np.array_equal(k, ok) and np.array_equal(v, ov)


def test_bf16_rounding_ties_to_even():
    # 1 + 2^-8 is halfway between bf16 1.0 and 1+2^-7: ties to even -> 1.0;
    # 1 + 3*2^-8 is halfway between 1+2^-7 and 1+2^-6: ties to even -> 1+2^-6.
    x = np.array([1 + 2**-8, 1 + 3 * 2**-8, -1 + 2**-24, 0.0], dtype=np.float32)
    got = inputs._f32_to_bf16_bits(x)
    assert list(got) == [0x3F80, 0x3F82, 0xBF80, 0x0000]
    for xi, gi in zip(x, got):
        assert gi == oracle.lib().fa_oracle_bf16_from_float(float(xi))


@pytest.mark.parametrize("shape,seed,sigma", [((1, 2, 128, 64), 11, 1.0), ((3, 5, 7), 22, 3.0),
                                              ((1, 1, 4099, 128), 33, 3.0), ((5,), 2**63 + 12345, 0.5)])
def test_normal_matches_oracle(shape, seed, sigma):
    assert np.array_equal(inputs.fill_normal(shape, seed, sigma), oracle.fill_normal(shape, seed, sigma))


def test_normal_chunking_is_seamless():
    shape = (3, 1000)
    assert np.array_equal(inputs.fill_normal(shape, 7, 3.0, chunk=257), inputs.fill_normal(shape, 7, 3.0))


def test_normal_moments():
    x = oracle.bf16_to_f32(inputs.fill_normal((1 << 18,), 5, 3.0)).astype(np.float64)
    assert abs(x.mean()) < 0.03 and abs(x.std() - 3.0) < 0.03


def test_make_stress_inputs_seeds():
    q, k, v = inputs.make_stress_inputs(1, 2, 33, 128)
    oq, ok, ov = oracle.make_inputs(1, 2, 33, 128, "stress")
    assert np.array_equal(q, oq) and np.array_equal(k, ok) and np.array_equal(v, ov)
