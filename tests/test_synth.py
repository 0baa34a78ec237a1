"""The product-side synthetic generator and quantisers agree with the pinned oracle."""
import numpy as np
import pytest

import oracle as O
from rust_trainer_amd import synth


@pytest.mark.parametrize("seed", [1, 2, 3, 9])
def test_rng_streams_match(seed):
    a, b = synth.Rng(seed), O.Rng(seed)
    assert [int(v) for v in a.next_u64(5)] == [b.next_u64() for _ in range(5)]
    a, b = synth.Rng(seed), O.Rng(seed)
    assert np.array_equal(a.uniform(9), np.array([b.uniform() for _ in range(9)], np.float32))
    n1 = synth.Rng(seed).vec_normal(5000, 0.02)
    n2 = O.Rng(seed).vec_normal(5000, 0.02)
    assert np.abs(n1 - n2).max() <= 2e-6 * 0.02 * 8  # last-ulp libm differences only


@pytest.mark.parametrize("wtype", [O.Q4_0, O.Q8_0, O.Q4_K, O.Q6_K])
def test_quantisers_bit_identical(wtype):
    w = O.Rng(1).vec_normal(37 * 512, 0.02).reshape(37, 512)
    w[0, :32] = 0.0
    w[1, :32] = np.float32(1e-7)
    w[2, :32] = np.array([127.0, 2.5, -2.5, 0.5, -0.5] + [0.0] * 27, np.float32)
    w[3, :256] = 0.0  # an all-zero super-block
    w[4, :256] = np.abs(w[4, :256])  # no negative values: min 0
    w[5, 256:] = -np.abs(w[5, 256:])  # no positive values
    assert np.array_equal(synth.QUANTIZERS[wtype](w), O.quantize(wtype, w))


def test_trainer_q8_0_packing_matches_oracle():
    # the product's FrozenWeight::q8_0 quantiser (rust_trainer_amd.pack_trainer_q8_0) against the
    # oracle's, bit for bit, including halves (x / d = m + 0.5) and all-zero blocks
    import rust_trainer_amd as rt

    for seed, (n, k) in enumerate([(64, 128), (33, 256), (5, 32)]):
        w = O.Rng(seed + 1).vec_normal(n * k, 0.02).reshape(n, k)
        w[0, :6] = [1.0, 0.5 / 127, -0.5 / 127, 1.5 / 127, -2.5 / 127, 0.0]
        w[1, :32] = 0.0
        assert np.array_equal(rt.pack_trainer_q8_0(w, n, k), O.quantize(O.TQ8_0, w))
