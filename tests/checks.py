"""Comparison helpers shared by the GPU tests."""
import sys

import numpy as np


def say(*a):
    """Names the case on stdout before a GPU step (flushed)."""
    print(*a, flush=True)
    sys.stdout.flush()


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_same_f32(got, want, what=""):
    """Bit-identical f32 arrays; NaN positions must agree."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} vs {want.shape}"
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), f"{what}: NaN positions differ"
    bad = np.nonzero(bits(got[~nan]) != bits(want[~nan]))[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: " \
                          f"{got[~nan][bad[:5]]} vs {want[~nan][bad[:5]]}"


def q5_random(seed, rows, cols):
    """Q5 rows of random high-bit planes and nibbles under random finite f16 scales (every code and
    both signs of the scale; the kernels decode any bytes, so the 21-candidate rule is not needed)."""
    nb = (cols + 31) // 32
    rng = np.random.default_rng(seed)
    w = rng.integers(0, 256, (rows, nb, 22), dtype=np.uint8)
    scale = rng.uniform(-2e-3, 2e-3, (rows, nb)).astype(np.float16)
    w[:, :, 0:2] = scale.view(np.uint8).reshape(rows, nb, 2)
    return w.reshape(rows, nb * 22)
