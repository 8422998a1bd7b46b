"""The product's synthetic-model generator (pq_synth_fill, host code of the
library) reproduces the oracle's generator bit for bit, so a model built by the
engine and one built by the oracle hold the same weights. CPU only."""
import numpy as np


def test_synth_matches_oracle(orc):
    from pulsar_amd.engine import synth_fill
    n = 100003
    assert np.array_equal(synth_fill(0, 11, n), orc.gen_codes(11, n))
    assert np.array_equal(synth_fill(1, 12, n).view(np.uint32), orc.gen_normal(12, n).view(np.uint32))
    assert np.array_equal(synth_fill(2, 13, n, 0.01), orc.gen_scales(13, n, 0.01))
    assert np.array_equal(synth_fill(3, 14, 5000, 4.0, 0.4).view(np.uint32),
                          orc.gen_affine(14, 5000, 4.0, 0.4).view(np.uint32))
    assert np.array_equal(synth_fill(4, 15, n), orc.gen_ternary(15, n))
    assert np.array_equal(synth_fill(5, 16, 256, 65536.0), orc.gen_tokens(16, 256, 65536))
