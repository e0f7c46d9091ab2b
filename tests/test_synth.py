"""The product package's host-side weight packers and generator, checked
against the oracle (CPU)."""
import numpy as np

from smq_pkg import synth


def test_normal_is_seeded_and_standard():
    a = synth.normal(1001, 200000)
    b = synth.normal(1001, 200000)
    assert np.array_equal(a, b)
    assert not np.array_equal(a, synth.normal(1002, 200000))
    assert abs(float(a.mean())) < 0.01 and abs(float(a.std()) - 1.0) < 0.01
    # a window of the stream equals the same slice of a longer draw
    assert np.array_equal(synth.normal(7, 10, start=5), synth.normal(7, 20)[10:20])


def test_q8_pack_matches_oracle(orc):
    for rows, cols, sigma in ((7, 896, 0.02), (3, 33, 1.0), (5, 4871, 3.0), (2, 7, 1e-30)):
        x = synth.normal(rows * 100 + cols, rows * cols, sigma).reshape(rows, cols)
        x[0, :5] = 0.0
        assert np.array_equal(synth.q8_pack(x).reshape(-1), orc.q8_weight_rows(x))


def test_q5_pack_matches_oracle(orc):
    for rows, cols, sigma in ((6, 896, 0.02), (3, 45, 1.0), (2, 1536, 5.0), (2, 64, 1e3)):
        x = synth.normal(rows * 7 + cols, rows * cols, sigma).reshape(rows, cols)
        x[1, 32:64] = 0.0
        assert np.array_equal(synth.q5_pack(x).reshape(-1), orc.quantize_q5_rows(x))
