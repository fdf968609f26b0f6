"""The benchmark's seeded input generator draws the same tensors as the
oracle's, so a CPU check of a benchmark result can regenerate its inputs."""
import numpy as np

import oracle as O
from omnimatchdeeplearningtool_amd import synthetic as S


def test_generators_match_oracle():
    for shape, seed in (((7, 5), 11), ((2, 3, 9, 9), 900), ((1000,), 901)):
        assert np.array_equal(S.randn(shape, seed), O.randn(shape, seed))
        assert np.array_equal(S.randn(shape, seed, 0.1), O.randn(shape, seed, 0.1))
        assert np.array_equal(S.uniform(shape, seed, -0.5, 1.5), O.uniform(shape, seed, -0.5, 1.5))
    a = S.randn((4096,), 3)
    assert a.dtype == np.float32 and abs(float(a.mean())) < 0.1 and 0.9 < float(a.std()) < 1.1
