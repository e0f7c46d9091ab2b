"""GPU parity of the Q5 weight conversion (smq_quantize_q5_row/_rows against
quantize_q5_row, src/kernels.c:1064-1117): every output byte equal to the
oracle's restatement, which is itself pinned byte for byte to the reference's
compiled quantize_q5_row (tests/test_oracle.py); where the reference is built
(oracle/_ref) the GPU bytes are also compared with it directly."""
import numpy as np
import pytest

from checks import say
from smq_pkg import smq, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert smq.init(0) == "gfx950"
    yield


def gpu_q5(x):
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    nb = (cols + 31) // 32
    xb = smq.DeviceBuffer.from_array(x)
    out = smq.DeviceBuffer(rows * nb * 22)
    out.fill(0xA5)  # every byte must be written
    smq.quantize_q5_rows(xb, rows, cols, out)
    return out.download(np.uint8).reshape(rows, nb * 22)


def check(orc, x, what, ref=None):
    got = gpu_q5(x)
    want = orc.quantize_q5_rows(x).reshape(got.shape)
    bad = np.nonzero(np.any(got != want, axis=1))[0]
    assert bad.size == 0, f"{what}: rows {bad[:5]} differ"
    if ref is not None:
        for r in range(min(x.shape[0], 4)):
            assert np.array_equal(got[r], ref.quantize_q5_row(x[r])), f"{what}: row {r} vs reference"


@pytest.mark.parametrize("rows,cols", [(8960, 1536), (1536, 8960)], ids=["c2-8960x1536", "c2-1536x8960"])
def test_config2_matrices(orc, rows, cols):
    """the Qwen2.5-1.5B-shaped matrices, N(0, 0.02)."""
    say("q5 convert", rows, cols)
    check(orc, synth.normal(6000 + rows, rows * cols, 0.02).reshape(rows, cols), f"{rows}x{cols}")


def edge_rows():
    rows = []
    z = np.zeros(96, np.float32)
    rows.append(z.copy())                                   # all zero: scale 0, codes 16
    r = z.copy(); r[40] = 3.0; rows.append(r)              # one nonzero element
    r = z.copy(); r[0], r[5] = 1.5, -1.5; rows.append(r)   # tie in |x|: the first wins (positive)
    r = z.copy(); r[0], r[5] = -1.5, 1.5; rows.append(r)   # tie: the first wins (negative)
    r = np.linspace(-1, 1, 96).astype(np.float32); rows.append(r)
    r = np.full(96, -2.0, np.float32); rows.append(r)       # constant block
    r = (np.arange(96) % 7 - 3).astype(np.float32) * 1e-3; rows.append(r)
    r = synth.normal(3, 96, 1e6); rows.append(r)            # extremes past f16 range for small k
    r = synth.normal(4, 96, 3e4); rows.append(r)            # near the f16 overflow boundary
    r = synth.normal(5, 96, 1e-6); rows.append(r)           # f16 subnormal scales
    r = synth.normal(6, 96, 1e-9); rows.append(r)           # every candidate rounds to 0
    r = synth.normal(7, 96, 1e-40); rows.append(r)          # f32 subnormal inputs
    r = synth.normal(8, 96, 1.0); r[::3] *= 40; rows.append(r)  # clipping at -16 / 15
    r = np.full(96, 65504.0 * 14.5, np.float32); rows.append(r)
    r = np.full(96, -0.0, np.float32); rows.append(r)       # negative zeros
    base = np.linspace(-1, 1, 96).astype(np.float32)
    r = base.copy(); r[3] = np.nan; rows.append(r)          # NaN: never the extreme, first candidate kept
    r = base.copy(); r[0] = np.nan; r[40] = np.nan; rows.append(r)
    r = np.full(96, np.nan, np.float32); rows.append(r)     # all NaN: zero blocks
    r = np.zeros(96, np.float32); r[9] = np.nan; rows.append(r)
    r = base.copy(); r[5] = np.inf; rows.append(r)          # infinite element: scale 0, codes 16
    r = base.copy(); r[33] = -np.inf; r[34] = np.nan; rows.append(r)
    r = base.copy(); r[31] = np.nan; r[30] = -3.0; rows.append(r)
    return np.stack(rows)


def test_edge_rows(orc, request):
    ref = None
    import oracle
    if oracle.Reference.available():
        ref = oracle.Reference()
    x = edge_rows()
    say("q5 convert edges", x.shape)
    check(orc, x, "edges", ref)
    for i in range(x.shape[0]):
        got = gpu_q5(x[i:i + 1])
        assert np.array_equal(got[0], orc.quantize_q5_rows(x[i:i + 1])), f"edge row {i}"
        if ref is not None:
            assert np.array_equal(got[0], ref.quantize_q5_row(x[i])), f"edge row {i} vs reference"


@pytest.mark.parametrize("cols", [1, 7, 31, 32, 33, 45, 63, 65, 1000])
def test_partial_blocks(orc, cols):
    """Widths with a partial last block: padding never enters the extreme or the error, codes 16."""
    x = synth.normal(900 + cols, 37 * cols, 0.5).reshape(37, cols)
    check(orc, x, f"cols={cols}")


def test_single_row_entry_point(orc):
    """smq_quantize_q5_row: the reference's own parameter list (kernels.h:205)."""
    cols = 1536
    x = synth.normal(77, cols, 0.02)
    xb = smq.DeviceBuffer.from_array(x)
    out = smq.DeviceBuffer(48 * 22)
    smq.quantize_q5_row(xb, cols, out)
    assert np.array_equal(out.download(np.uint8), orc.quantize_q5_rows(x.reshape(1, cols)).reshape(-1))


def test_round_trip_bound(orc):
    """The reference's property test (tests/test_kernels.c:71-87): dequantized values within one step of
    the block scale, also through the device dequantizer."""
    x = synth.normal(55, 4 * 256, 1.0).reshape(4, 256)
    q = gpu_q5(x)
    for r in range(4):
        out = smq.DeviceBuffer(256 * 4)
        smq.dequantize_q5_row(smq.DeviceBuffer.from_array(q[r]), 256, out)
        y = out.download(np.float32)
        scales = np.abs(q[r].reshape(8, 22)[:, :2].copy().view(np.float16).astype(np.float32)).repeat(32)
        assert np.all(np.abs(y - x[r]) <= scales * 1.0001 + 1e-7)
