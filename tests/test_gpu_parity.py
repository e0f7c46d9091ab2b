"""GPU parity: every entry point of the C ABI against the CPU oracle on the
same seeded inputs. Integer and f32 results must be bit-identical (the
contract is reproduced exactly); NaN results compare as NaN."""
import sys

import numpy as np
import pytest

from checks import q5_random
from patterns import LcgUniform
from smq_pkg import smq, synth

pytestmark = pytest.mark.gpu

Q8B, Q5B = 36, 22


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def gpu():
    arch = smq.init(0)
    assert arch == "gfx950"
    smq.kernels_set_fast(False)
    assert smq.kernels_select() == "gfx950"
    yield
    smq.kernels_set_fast(False)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def assert_same_f32(got, want, what=""):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, what
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan), what
    bad = np.nonzero(bits(got[~nan]) != bits(want[~nan]))[0]
    assert bad.size == 0, f"{what}: {bad.size} mismatches, first at {bad[:5]}: " \
                          f"{got[~nan][bad[:5]]} vs {want[~nan][bad[:5]]}"


def gpu_quantize(x):
    rows, n = x.shape
    nb = (n + 31) // 32
    xb = smq.DeviceBuffer.from_array(x)
    d = smq.DeviceBuffer(rows * nb * 4)
    q = smq.DeviceBuffer(rows * nb * 32)
    smq.quantize_q8_rows(xb, rows, n, d, q)
    smq.numeric_check()
    return d, q, d.download(np.float32).reshape(rows, nb), q.download(np.int8).reshape(rows, nb * 32)


# ------------------------------------------------------------------ quantize

@pytest.mark.parametrize("spread", [1.0, 50.0, 1e-30, 1e30, 1e-37, 1e-39])
def test_quantize_bit_exact(orc, spread):
    g = LcgUniform(101)
    for n in (1, 7, 31, 32, 33, 67, 896, 4864, 8960 + 5):
        x = g.uniform(-spread, spread, 3 * n).reshape(3, n)
        x[:, ::33] = 0.0
        say("quantize", spread, n)
        _, _, d, q = gpu_quantize(x)
        s, wd, wq = orc.quantize_q8(x)
        assert s == 0
        assert np.array_equal(bits(d), bits(wd)), (spread, n)
        assert np.array_equal(q, wq), (spread, n)


def test_quantize_single_and_nonfinite(orc):
    g = LcgUniform(5)
    x = g.uniform(-3, 3, 100)
    xb = smq.DeviceBuffer.from_array(x)
    d = smq.DeviceBuffer(4 * 4)
    q = smq.DeviceBuffer(4 * 32)
    assert smq.quantize_q8(xb, 100, d, q) == 0
    s, wd, wq = orc.quantize_q8(x)
    assert np.array_equal(bits(d.download(np.float32)), bits(wd[0]))
    assert np.array_equal(q.download(np.int8), wq[0])
    for at in (0, 7, 31, 40, 66):  # tests/test_kernels.c:400-410
        y = np.ones(67, np.float32)
        y[at] = np.nan if at % 2 else np.inf
        yb = smq.DeviceBuffer.from_array(y)
        assert smq.quantize_q8(yb, 67, d, q) == -1
    # the asynchronous row variant raises the sticky flag instead
    y = np.ones((2, 64), np.float32)
    y[1, 5] = -np.inf
    yb = smq.DeviceBuffer.from_array(y)
    smq.quantize_q8_rows(yb, 2, 64, d, q)
    with pytest.raises(smq.SmqError) as e:
        smq.numeric_check()
    assert e.value.status == smq.SM_ERR_NUMERIC
    smq.numeric_check()  # cleared


# ------------------------------------------------------------------ gemm / gemv

def run_gemm(w_host, row_bytes, x, nrows, ntok, nb, q5, stride=None, fast=False):
    stride = nrows if stride is None else stride
    dbuf, qbuf, xd, xq = gpu_quantize(x)
    wb = smq.DeviceBuffer.from_array(w_host)
    out = smq.DeviceBuffer(max(1, ntok * stride) * 4)
    out.fill(0xFF)
    smq.kernels_set_fast(fast)
    try:
        (smq.gemm_q5 if q5 else smq.gemm_q8)(wb, row_bytes, dbuf, qbuf, nrows, ntok, nb, out, stride)
        got = out.download(np.float32)[:ntok * stride]
    finally:
        smq.kernels_set_fast(False)
    return got, xd, xq


def weights(q5, seed, rows, cols, sigma=0.02):
    return (synth.q5_weights if q5 else synth.q8_weights)(seed, rows, cols, sigma).reshape(-1)


CONFIG_SHAPES = [  # (name, q5, rows, cols, ntok)
    ("c0", False, 896, 896, 1),
    ("c1-gate", False, 4864, 896, 1),
    ("c1-down", False, 896, 4864, 1),
    ("c2-up", True, 8960, 1536, 1),
    ("c2-down", True, 1536, 8960, 1),
    ("c1-gate-b128", False, 4864, 896, 128),
    ("c1-down-b128", False, 896, 4864, 128),
    ("c2-up-b64", True, 8960, 1536, 64),
    ("c2-down-b64", True, 1536, 8960, 64),
]


@pytest.mark.parametrize("name,q5,rows,cols,ntok", CONFIG_SHAPES)
def test_config_shapes_bit_exact(orc, name, q5, rows, cols, ntok):
    say("config", name)
    nb = (cols + 31) // 32
    w = weights(q5, 1000 + rows + cols, rows, cols)
    x = synth.activations(2000 + cols + ntok, ntok, cols)
    got, xd, xq = run_gemm(w, nb * (Q5B if q5 else Q8B), x, rows, ntok, nb, q5)
    want = orc.gemm(w, nb * (Q5B if q5 else Q8B), xd, xq, rows, ntok, nb, q5=q5)
    assert_same_f32(got, want, name)


@pytest.mark.parametrize("ntok", [1, 64])
def test_lm_head_bit_exact(orc, ntok):
    """c3: 151936 x 896 Q8 against RMSNorm-scaled activations; batch 64 is
    checked on every 16th row (the oracle is scalar)."""
    rows, cols, nb = 151936, 896, 28
    say("lm head", ntok)
    w = weights(False, 1003, rows, cols)
    raw = synth.activations(2003, ntok, cols)
    x = np.stack([orc.rmsnorm(r, np.ones(cols, np.float32), 1e-6)[1] for r in raw])
    got, xd, xq = run_gemm(w, nb * Q8B, x, rows, ntok, nb, False)
    got = got.reshape(ntok, rows)
    pick = np.arange(0, rows, 1 if ntok == 1 else 16)
    wsub = w.reshape(rows, nb * Q8B)[pick].reshape(-1)
    want = orc.gemm(wsub, nb * Q8B, xd, xq, len(pick), ntok, nb).reshape(ntok, len(pick))
    assert_same_f32(got[:, pick], want, "lm head")


class exact_kernel:
    """Which kernel the exact prefill GEMM takes inside the block (smq_set_exact_gemm), back to the
    choice by shape afterwards."""

    def __init__(self, mode):
        self.mode = mode

    def __enter__(self):
        smq.set_exact_gemm(self.mode)

    def __exit__(self, *exc):
        smq.set_exact_gemm(smq.EXACT_BY_SHAPE)


EXACT_MODES = [smq.EXACT_MFMA, smq.EXACT_VALU, smq.EXACT_MFMA_SPLIT, smq.EXACT_MFMA_SPLIT4]


@pytest.mark.parametrize("mode", EXACT_MODES)
@pytest.mark.parametrize("q5,fast", [(False, False), (True, False), (False, True), (True, True)])
def test_exact_gemm_16_token_tiles_ragged(orc, q5, fast, mode):
    """Both exact kernels on a shape with enough row tiles for 16-token (and 32-token) tiles: a ragged
    last row tile and token tile, an output stride wider than the rows, 30 blocks (a partial last K
    chunk), the fast contract."""
    rows, cols, ntok = 9723, 960, 37
    nb, stride = cols // 32, 9723 + 3
    say("exact 16-token tiles", q5, fast, mode)
    w = (q5_random(91, rows, cols) if q5 else synth.q8_weights(91, rows, cols)).reshape(-1)
    x = synth.activations(92, ntok, cols)
    with exact_kernel(mode):
        got, xd, xq = run_gemm(w, nb * (Q5B if q5 else Q8B), x, rows, ntok, nb, q5, stride, fast)
    want = orc.gemm(w, nb * (Q5B if q5 else Q8B), xd, xq, rows, ntok, nb, stride=stride, q5=q5, fast=fast)
    m = np.zeros(ntok * stride, bool)
    m.reshape(ntok, stride)[:, :rows] = True
    assert_same_f32(got[m], want[m], "16-token tiles")
    assert np.all(bits(got[~m]) == 0xFFFFFFFF), "wrote outside the output rows"


@pytest.mark.parametrize("mode", [smq.EXACT_BY_SHAPE, smq.EXACT_MFMA, smq.EXACT_MFMA_SPLIT, smq.EXACT_MFMA_SPLIT4])
def test_random_shapes_and_strides(orc, mode):
    """Ragged rows and tokens, odd widths (including odd Q5 widths, which take
    the generic kernel), output strides wider than the row count; then the
    same with every prefill shape on the MFMA lane-sum kernel."""
    g = LcgUniform(77)
    for trial in range(40):
        q5 = trial % 2 == 1
        nb = 1 + int(g.next(1)[0] % 40)
        rows = 1 + int(g.next(1)[0] % 70)
        ntok = 1 + int(g.next(1)[0] % 20)
        stride = rows + int(g.next(1)[0] % 3)
        cols = nb * 32 - int(g.next(1)[0] % 32)
        fast = trial % 5 == 4
        w = weights(q5, trial, rows, cols, 0.5)
        x = g.uniform(-30, 30, ntok * cols).reshape(ntok, cols)
        say("random", trial, q5, nb, rows, ntok, stride, fast, mode)
        with exact_kernel(mode):
            got, xd, xq = run_gemm(w, nb * (Q5B if q5 else Q8B), x, rows, ntok, nb, q5, stride, fast)
        want = orc.gemm(w, nb * (Q5B if q5 else Q8B), xd, xq, rows, ntok, nb, stride=stride, q5=q5, fast=fast)
        m = np.zeros(ntok * stride, bool)
        m.reshape(ntok, stride)[:, :rows] = True
        assert_same_f32(got[m], want[m], f"trial {trial}")
        assert np.all(bits(got[~m]) == 0xFFFFFFFF), "wrote outside the output rows"


@pytest.mark.parametrize("q5", [False, True])
@pytest.mark.parametrize("ntok", [20, 60, 90, 150, 220, 300, 410])
def test_by_shape_bands(orc, q5, ntok):
    """The by-shape choice at every band of the exact GEMM: 2043 ragged rows (64 tiles of 32) at 20-410
    tokens give 32, 128, 192, 320, 448, 640 and 832 tiles of 32 x 32, i.e. on 256 CUs the v_dot4 kernel,
    the four-wave split, the two-wave split for Q8 and the four-wave one for Q5, the two-wave split,
    32 x 32 workgroups, the two-wave split again (2 to 3 tiles per CU) and 32 x 32 workgroups; ragged
    widths and one FAST case."""
    rows, nb = 2043, 4
    cols = nb * 32 - 3
    fast = ntok == 300
    g = LcgUniform(300 + ntok)
    w = weights(q5, ntok, rows, cols, 0.5)
    x = g.uniform(-30, 30, ntok * cols).reshape(ntok, cols)
    say("bands", q5, rows, ntok, nb, fast)
    with exact_kernel(smq.EXACT_BY_SHAPE):
        got, xd, xq = run_gemm(w, nb * (Q5B if q5 else Q8B), x, rows, ntok, nb, q5, rows, fast)
    want = orc.gemm(w, nb * (Q5B if q5 else Q8B), xd, xq, rows, ntok, nb, stride=rows, q5=q5, fast=fast)
    assert_same_f32(got, want, f"bands q5={q5} ntok={ntok}")


def test_fma_probe_exact_and_fast():
    """tests/test_kernels.c:223-249: 0.0 with two roundings, 2^-12 with FMA."""
    w = np.zeros(2 * Q8B, np.uint8)
    w[0:4] = np.array([1.0], np.float32).view(np.uint8)
    w[Q8B:Q8B + 4] = np.array([1.0 + 1.0 / 4096], np.float32).view(np.uint8)
    w[4], w[5], w[Q8B + 4], w[Q8B + 5] = 127, 17, 127, 1
    xq = np.zeros(4 * 64, np.int8)
    for t in range(4):
        xq[t * 64 + 0], xq[t * 64 + 1], xq[t * 64 + 32], xq[t * 64 + 33] = -32, -2, 32, 33
    xd = np.ones(8, np.float32)
    wb, qb, db = (smq.DeviceBuffer.from_array(a) for a in (w, xq, xd))
    out = smq.DeviceBuffer(16 * 4)
    assert smq.dot_q8(wb, db, qb, 2) == 0.0
    smq.dot_q8_x4(wb, db, qb, 2, 2, out)
    assert np.all(out.download(np.float32, 4) == 0.0)
    smq.gemm_q8(wb, Q8B * 2, db, qb, 1, 4, 2, out, 1)
    assert np.all(out.download(np.float32, 4) == 0.0)
    smq.kernels_set_fast(True)
    try:
        assert smq.kernels_select() == "gfx950-fast"
        assert smq.dot_q8(wb, db, qb, 2) == 2.0 ** -12
        smq.gemm_q8(wb, Q8B * 2, db, qb, 1, 4, 2, out, 1)
        assert np.all(out.download(np.float32, 4) == 2.0 ** -12)
    finally:
        smq.kernels_set_fast(False)
    assert smq.kernels_select() == "gfx950"


def test_backend_edges(orc):
    """tests/test_kernels.c:251-278 edges through every GPU kernel shape."""
    import struct
    high = [0xFFFFFFFF, 0, 0xAAAAAAAA, 0x12345678]
    low = [0xF0, 0xFF, 0x5A, 0x0F]
    nb = 4
    w5 = np.zeros(nb * Q5B, np.uint8)
    w8 = np.zeros(nb * Q8B, np.uint8)
    xq = np.zeros(nb * 32, np.int8)
    j = np.arange(32)
    for b in range(nb):
        blk = w5[b * Q5B:(b + 1) * Q5B]
        blk[0], blk[1] = 0x00, 0x3C
        blk[2:6] = np.frombuffer(struct.pack("<I", high[b]), np.uint8)
        blk[6:] = low[b]
        w8[b * Q8B:b * Q8B + 4] = np.array([1.0], np.float32).view(np.uint8)
        w8[b * Q8B + 4:(b + 1) * Q8B] = np.where(j % 2 == 1, -128, 127).astype(np.int8).view(np.uint8)
        xq[b * 32:(b + 1) * 32] = np.where(b == 2, np.where(j % 3 != 0, 127, -127), -127)
    xd = np.array([1.0, 0.5, 2.0, 0.25], np.float32)
    for q5, w in ((True, w5), (False, w8)):
        rows = 9
        wrows = np.tile(w, rows)
        want = orc.gemm(wrows, len(w), xd, xq, rows, 1, nb, q5=q5)
        wb, qb, db = (smq.DeviceBuffer.from_array(a) for a in (wrows, xq, xd))
        out = smq.DeviceBuffer(rows * 4)
        (smq.gemm_q5 if q5 else smq.gemm_q8)(wb, len(w), db, qb, rows, 1, nb, out, rows)
        assert_same_f32(out.download(np.float32), want, f"edges q5={q5}")
        assert (smq.dot_q5 if q5 else smq.dot_q8)(wb, db, qb, nb) == want[0]


def test_dot_variants(orc):
    g = LcgUniform(12)
    for q5 in (False, True):
        nb = 28
        bb = Q5B if q5 else Q8B
        w = weights(q5, 5, 4, nb * 32, 1.0)
        x = g.uniform(-8, 8, 4 * nb * 32).reshape(4, -1)
        dbuf, qbuf, xd, xq = gpu_quantize(x)
        wb = smq.DeviceBuffer.from_array(w)
        out = smq.DeviceBuffer(4 * 4)
        (smq.dot_q5_x4 if q5 else smq.dot_q8_x4)(wb, dbuf, qbuf, nb, nb, out)
        want = [orc.dot(w[:nb * bb], xd[t], xq[t], nb, q5=q5) for t in range(4)]
        assert_same_f32(out.download(np.float32), want, "x4")
        (smq.dot_q5_r4 if q5 else smq.dot_q8_r4)(wb, nb * bb, dbuf, qbuf, nb, out)
        want = [orc.dot(w[r * nb * bb:(r + 1) * nb * bb], xd[0], xq[0], nb, q5=q5) for r in range(4)]
        assert_same_f32(out.download(np.float32), want, "r4")


def test_unaligned_weights_take_the_generic_kernel(orc):
    g = LcgUniform(3)
    nb, rows, ntok = 9, 13, 3
    for q5 in (False, True):
        bb = Q5B if q5 else Q8B
        w = weights(q5, 9, rows, nb * 32, 0.3)
        x = g.uniform(-4, 4, ntok * nb * 32).reshape(ntok, -1)
        dbuf, qbuf, xd, xq = gpu_quantize(x)
        wb = smq.DeviceBuffer(len(w) + 8)
        wb.upload(w, offset=1)
        out = smq.DeviceBuffer(ntok * rows * 4)
        (smq.gemm_q5 if q5 else smq.gemm_q8)(wb.at(1), nb * bb, dbuf, qbuf, rows, ntok, nb, out, rows)
        want = orc.gemm(w, nb * bb, xd, xq, rows, ntok, nb, q5=q5)
        assert_same_f32(out.download(np.float32), want, f"unaligned q5={q5}")


def test_empty_and_bad_arguments():
    wb = smq.DeviceBuffer(64)
    out = smq.DeviceBuffer(64)
    smq.gemm_q8(wb, 36, wb, wb, 0, 1, 1, out, 0)  # no rows: nothing to do
    smq.gemm_q8(wb, 36, wb, wb, 1, 0, 1, out, 1)  # no tokens
    with pytest.raises(smq.SmqError) as e:
        smq.gemm_q8(wb, 36, wb, wb, 4, 1, 1, out, 4)  # 4 rows of 36 B exceed the 64-byte allocation
    assert e.value.status == 4
    with pytest.raises(smq.SmqError):
        smq.gemm_q8(wb, 20, wb, wb, 1, 1, 1, out, 1)  # row_bytes < 36


# ------------------------------------------------------------------ matmul glue

@pytest.mark.parametrize("mode", EXACT_MODES)
def test_matmul_fused_items_bias_and_fault(orc, mode):
    """model.c:291-310: q/k/v share one input (896+128+128 rows), bias added,
    outputs checked finite; the prefill case on each exact kernel."""
    smq.set_exact_gemm(mode)
    try:
        matmul_fused_items_bias_and_fault(orc)
    finally:
        smq.set_exact_gemm(smq.EXACT_BY_SHAPE)


def matmul_fused_items_bias_and_fault(orc):
    g = LcgUniform(44)
    cols, nb = 896, 28
    shapes = [896, 128, 128]
    for ntok in (1, 5, 40):
        x = synth.activations(9 + ntok, ntok, cols)
        dbuf, qbuf, xd, xq = gpu_quantize(x)
        items, wants = [], []
        for i, rows in enumerate(shapes):
            w = weights(False, 50 + i, rows, cols)
            bias = g.uniform(-0.1, 0.1, rows)
            wb = smq.DeviceBuffer.from_array(w)
            bb = smq.DeviceBuffer.from_array(bias)
            yb = smq.DeviceBuffer(ntok * rows * 4)
            items.append((smq.QMat(wb, rows, cols), bb, yb))
            ok, y = orc.mat_item(w, nb * Q8B, rows, bias, xd, xq, ntok, nb)
            assert ok
            wants.append(y)
        smq.matmul(items, dbuf, qbuf, ntok)
        smq.numeric_check()
        for (_, _, yb), want in zip(items, wants):
            assert_same_f32(yb.download(np.float32), want, f"matmul ntok={ntok}")
    # an infinite weight scale makes a non-finite output: SM_ERR_NUMERIC
    w = weights(False, 7, 4, cols)
    w[0:4] = np.array([np.inf], np.float32).view(np.uint8)
    wb = smq.DeviceBuffer.from_array(w)
    yb = smq.DeviceBuffer(4 * 4)
    smq.matmul([(smq.QMat(wb, 4, cols), None, yb)], dbuf, qbuf, 1)
    with pytest.raises(smq.SmqError) as e:
        smq.numeric_check()
    assert e.value.status == smq.SM_ERR_NUMERIC
    # items of different widths are an internal error, as in the reference
    w2 = smq.DeviceBuffer.from_array(weights(False, 8, 4, 64))
    with pytest.raises(smq.SmqError) as e:
        smq.matmul([(smq.QMat(wb, 4, cols), None, yb), (smq.QMat(w2, 4, 64), None, yb)], dbuf, qbuf, 1)
    assert e.value.status == 7


@pytest.mark.parametrize("mode", [smq.EXACT_MFMA, smq.EXACT_MFMA_SPLIT, smq.EXACT_MFMA_SPLIT4])
@pytest.mark.parametrize("q5", [False, True])
def test_exact_mfma_items_bias_accumulate_nonfinite(orc, q5, mode):
    """The MFMA lane-sum kernel through smq_matmul: four items of ragged row counts (item edges inside
    and between 32-row tiles), bias on some, residual add on others, 70 tokens (a ragged 32-token tile);
    then an infinite weight scale flags SM_ERR_NUMERIC."""
    g = LcgUniform(45)
    cols, ntok = 1024, 70
    nb, bb = cols // 32, Q5B if q5 else Q8B
    x = synth.activations(46, ntok, cols)
    dbuf, qbuf, xd, xq = gpu_quantize(x)
    items, wants = [], []
    for i, rows in enumerate([33, 100, 7, 64]):
        w = (q5_random(60 + i, rows, cols) if q5 else synth.q8_weights(60 + i, rows, cols)).reshape(-1)
        bias = g.uniform(-0.1, 0.1, rows) if i % 2 == 0 else None
        acc = i % 3 == 1
        y0 = g.uniform(-1, 1, ntok * rows).astype(np.float32) if acc else np.zeros(ntok * rows, np.float32)
        ok, y = orc.mat_item(w, nb * bb, rows, bias, xd, xq, ntok, nb, q5=q5)
        assert ok
        wants.append(y0 + y if acc else y)
        items.append((smq.QMat(smq.DeviceBuffer.from_array(w), rows, cols, smq.DTYPE_Q5 if q5 else smq.DTYPE_Q8),
                      smq.DeviceBuffer.from_array(bias) if bias is not None else None,
                      smq.DeviceBuffer.from_array(y0), acc))
    say("exact mfma items", q5, mode)
    with exact_kernel(mode):
        smq.matmul(items, dbuf, qbuf, ntok)
        smq.numeric_check()
        for i, (it, want) in enumerate(zip(items, wants)):
            assert_same_f32(it[2].download(np.float32), want, f"item {i}")
        w = synth.q8_weights(7, 40, cols).reshape(-1)
        w[36 * nb * 3:36 * nb * 3 + 4] = np.array([np.inf], np.float32).view(np.uint8)  # row 3, block 0
        yb = smq.DeviceBuffer(ntok * 40 * 4)
        smq.matmul([(smq.QMat(smq.DeviceBuffer.from_array(w), 40, cols), None, yb)], dbuf, qbuf, ntok)
        with pytest.raises(smq.SmqError) as e:
            smq.numeric_check()
        assert e.value.status == smq.SM_ERR_NUMERIC


def test_exact_gemm_mode_refuses_other_values():
    for bad in (-1, 5, 7):
        with pytest.raises(smq.SmqError) as e:
            smq.set_exact_gemm(bad)
        assert e.value.status == smq.SM_ERR_RANGE
    smq.set_exact_gemm(smq.EXACT_BY_SHAPE)


def test_dequantize_rows(orc):
    for q5 in (False, True):
        for cols in (896, 45, 1):
            w = weights(q5, cols, 1, cols, 0.7)
            wb = smq.DeviceBuffer.from_array(w)
            out = smq.DeviceBuffer(cols * 4)
            (smq.dequantize_q5_row if q5 else smq.dequantize_q8_row)(wb, cols, out)
            assert_same_f32(out.download(np.float32), orc.dequantize_row(w, cols, q5=q5), "dequant")


def test_q5_scale_every_f16(orc):
    """Every one of the 65,536 f16 scale patterns through the Q5 row
    dequantization (q = 17, so each value is the scale itself): the device
    conversion against numpy's exact binary16 -> binary32 (finite values,
    subnormals and infinities bit for bit, NaN where NaN) and the oracle."""
    nblk = 1 << 16
    blocks = np.zeros((nblk, 22), np.uint8)
    blocks[:, 0:2] = np.arange(nblk, dtype=np.uint16).view(np.uint8).reshape(nblk, 2)
    blocks[:, 2:6] = 0xFF                       # high bit set for all 32 codes
    blocks[:, 6:22] = 0x11                      # low nibbles 1: q = 17, q - 16 = 1
    w = blocks.reshape(-1)
    cols = nblk * 32
    out = smq.DeviceBuffer(cols * 4)
    smq.dequantize_q5_row(smq.DeviceBuffer.from_array(w), cols, out)
    got = out.download(np.float32).reshape(nblk, 32)
    want = np.arange(nblk, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert_same_f32(got, np.repeat(want[:, None], 32, axis=1), "f16 scales")
    assert_same_f32(got.reshape(-1), orc.dequantize_row(w, cols, q5=True), "f16 scales vs oracle")


@pytest.mark.parametrize("rt", [1, 2, 4, 8, 16])
def test_every_gemv_tile_variant(orc, rt):
    """Forces each one-launch decode-GEMV tile shape (rows per workgroup)
    through the tuning call, exact and fast, with one- and multi-chunk widths."""
    g = LcgUniform(1000 + rt * 10)
    cases = [(False, 3, 37), (False, 28, 70), (False, 152, 9), (False, 300, 5), (True, 2, 41), (True, 48, 19),
             (True, 280, 6), (True, 600, 3)]
    smq.set_gemv_rows(rt)
    try:
        for q5, nb, rows in cases:
            for fast in (False, True):
                cols = nb * 32
                w = weights(q5, nb * 7 + rows, rows, cols, 0.3)
                x = g.uniform(-5, 5, cols).reshape(1, cols)
                say("variant", rt, q5, nb, rows, fast)
                got, xd, xq = run_gemm(w, nb * (Q5B if q5 else Q8B), x, rows, 1, nb, q5, fast=fast)
                want = orc.gemm(w, nb * (Q5B if q5 else Q8B), xd, xq, rows, 1, nb, q5=q5, fast=fast)
                assert_same_f32(got, want, f"rt={rt} q5={q5} nb={nb} fast={fast}")
    finally:
        smq.set_gemv_rows(0)


def test_gemv_rows_refuses_other_values():
    for bad in (-1, 3, 5, 32):
        with pytest.raises(smq.SmqError):
            smq.set_gemv_rows(bad)
    smq.set_gemv_rows(0)


# ------------------------------------------------------------------ MFMA prefill

def mfma_tolerance_ok(got, want, ntok, rows):
    """North-star tolerance for the relaxed-order path: per token,
    max_r |got - want| <= 1e-5 * max_r |want| (relative error in the max norm)."""
    g = got.reshape(ntok, -1)[:, :rows].astype(np.float64)
    w = want.reshape(ntok, -1)[:, :rows].astype(np.float64)
    err = np.abs(g - w).max(axis=1)
    scale = np.abs(w).max(axis=1)
    return bool(np.all(err <= 1e-5 * scale)), float((err / np.maximum(scale, 1e-30)).max())


MFMA_SHAPES = [("c1-gate-b128", False, 4864, 896, 128), ("c1-down-b128", False, 896, 4864, 128),
               ("c2-up-b64", True, 8960, 1536, 64), ("c2-down-b64", True, 1536, 8960, 64),
               ("ragged", False, 77, 416, 13), ("ragged-q5", True, 45, 64 * 5, 70), ("one-token", False, 33, 96, 1),
               ("c1-gateup-b128", False, 9728, 896, 128),   # 304 tiles: one slice
               ("split-ragged", False, 200, 4864, 70),      # K split over slices, a partial last chunk, ragged tiles
               ("two-tokens", False, 130, 224, 2),          # one K chunk of 7 blocks, two tokens
               ("lm-head-b64", False, 4096, 896, 64),
               ("q5-split-ragged", True, 200, 8960, 70),    # block-pair kernel, K over 10 slices, ragged tiles
               ("q5-split-partial", True, 100, 1984, 33)]   # 2 slices of 14-block chunks, the last chunk 6 blocks


@pytest.mark.parametrize("name,q5,rows,cols,ntok", MFMA_SHAPES)
def test_mfma_block_sums_exact_and_outputs_within_tolerance(orc, name, q5, rows, cols, ntok):
    say("mfma", name)
    nb = (cols + 31) // 32
    bb = Q5B if q5 else Q8B
    w = weights(q5, 3000 + rows, rows, cols)
    x = synth.activations(4000 + cols + ntok, ntok, cols)
    dbuf, qbuf, xd, xq = gpu_quantize(x)
    wb = smq.DeviceBuffer.from_array(w)
    # integer path: every per-block int32 sum bit-exact
    sums = smq.DeviceBuffer(ntok * rows * nb * 4)
    smq.block_sums(q5, wb, nb * bb, qbuf, rows, ntok, nb, sums)
    want_sums = orc.block_sums(w, nb * bb, xq, rows, ntok, nb, q5=q5)
    assert np.array_equal(sums.download(np.int32).reshape(ntok, rows, nb), want_sums), name
    # f32 outputs within 1e-5 of the exact contract
    out = smq.DeviceBuffer(ntok * rows * 4)
    (smq.gemm_q5_mfma if q5 else smq.gemm_q8_mfma)(wb, nb * bb, dbuf, qbuf, rows, ntok, nb, out, rows)
    want = orc.gemm(w, nb * bb, xd, xq, rows, ntok, nb, q5=q5)
    got = out.download(np.float32)
    ok, worst = mfma_tolerance_ok(got, want, ntok, rows)
    if not q5:
        exact = exact_outputs(orc, w, nb * bb, xd, xq, rows, ntok, nb)
        dist = per_output_errors(got[:ntok * rows], want, exact, ntok, rows)
        say(f"  normwise {worst:.3e}; per-output vs float64 (|out| >= 0.1 max): p99.9 {dist[2]:.2e} "
            f"max {dist[3]:.2e} (eight-lane contract max {dist[4]:.2e})")
        assert dist[3] <= 1e-5, (name, dist)
    else:
        say("  worst normwise relative error", worst)
    assert ok, (name, worst)


MFMA_WHOLE_K = [("f16-c1-gateup-b128", False, 9728, 896, 128),  # eight waves, one token tile
                ("f16-ragged-b70", False, 200, 896, 70),        # 13 subtiles, the last half full; 3 idle waves
                ("f16-b13", False, 77, 896, 13),                # four waves, one partial
                ("f16-b200", False, 300, 896, 200),             # two token tiles
                ("f16-b2", False, 33, 896, 2),
                ("f16-lm-b64", False, 4096, 896, 64),
                ("pair-q5-b64", True, 8960, 1536, 64),          # int8 block-pair kernel, K whole
                ("pair-q8-nb13", False, 4864, 416, 64)]


@pytest.mark.parametrize("name,q5,rows,cols,ntok", MFMA_WHOLE_K)
def test_mfma_whole_k_equals_blockwise_order(orc, name, q5, rows, cols, ntok):
    """The MFMA GEMMs that keep K whole (the f16 kernel with the activation in registers on 28-block
    Q8 rows, the int8 block-pair kernel otherwise) apply the blocks in order, acc = fma(ws * xs, S,
    acc): equal bit for bit to orc_gemm_blockwise, and within 1e-5 of the eight-lane contract."""
    say("mfma whole K", name)
    nb = (cols + 31) // 32
    bb = Q5B if q5 else Q8B
    w = weights(q5, 5000 + rows, rows, cols)
    x = synth.activations(5100 + cols + ntok, ntok, cols)
    dbuf, qbuf, xd, xq = gpu_quantize(x)
    wb = smq.DeviceBuffer.from_array(w)
    out = smq.DeviceBuffer(ntok * rows * 4)
    (smq.gemm_q5_mfma if q5 else smq.gemm_q8_mfma)(wb, nb * bb, dbuf, qbuf, rows, ntok, nb, out, rows)
    got = out.download(np.float32)
    assert_same_f32(got, orc.gemm_blockwise(w, nb * bb, xd, xq, rows, ntok, nb, q5=q5), name)
    ok, worst = mfma_tolerance_ok(got, orc.gemm(w, nb * bb, xd, xq, rows, ntok, nb, q5=q5), ntok, rows)
    assert ok, (name, worst)


def per_output_errors(got, want, exact, ntok, rows, floor=0.1):
    """Per-output relative error of `got` and of the eight-lane contract `want`, both against the
    float64 value of the block sums (exact), over outputs with |exact| >= floor * max|exact| of their
    token: (quantiles 0.5 / 0.99 / 0.999 / max of got, max of want, share of outputs kept)."""
    g = got.reshape(ntok, rows).astype(np.float64)
    w = want.reshape(ntok, rows).astype(np.float64)
    big = np.abs(exact) >= floor * np.abs(exact).max(axis=1, keepdims=True)
    rg = np.abs(g - exact)[big] / np.abs(exact[big])
    rw = np.abs(w - exact)[big] / np.abs(exact[big])
    return [float(v) for v in np.quantile(rg, [0.5, 0.99, 0.999])] + [float(rg.max()), float(rw.max()),
                                                                       float(big.mean())]


def exact_outputs(orc, w, row_bytes, xd, xq, rows, ntok, nb):
    """float64 sum over blocks of wscale * xscale * (exact int32 block sum): the value both block orders
    round towards."""
    sums = orc.block_sums(w, row_bytes, xq, rows, ntok, nb).astype(np.float64)  # [ntok, rows, nb]
    ws = w.reshape(rows, row_bytes)[:, :nb * Q8B].reshape(rows, nb, Q8B)[:, :, :4].copy().view(np.float32)
    xs = np.asarray(xd, np.float32).reshape(ntok, nb).astype(np.float64)
    return np.einsum("trb,rb,tb->tr", sums, ws[:, :, 0].astype(np.float64), xs)


# (name, rows, cols, ntok, row step of the check): the f16-MFMA GEMM's persistent loop at full size
MFMA_FULL = [("c3-lm-head-b64", 151936, 896, 64, 16),  # four waves, 9,496 subtiles over 512 workgroups (18-19 each)
             ("c1-gateup-b512", 9728, 896, 512, 2)]   # eight waves, four token tiles, 64 workgroups each (9-10 subtiles)


@pytest.mark.parametrize("name,rows,cols,ntok,step", MFMA_FULL, ids=[m[0] for m in MFMA_FULL])
def test_mfma_full_size_steady_state(orc, name, rows, cols, ntok, step):
    """The f16-MFMA prefill GEMM where every workgroup streams many 16-row subtiles through its two
    LDS buffers (the double-buffered loop, the two-subtile prefetch, buffer reuse): every `step`-th row
    bit for bit against orc_gemm_blockwise (the kernel's block order), within 1e-5 normwise of the
    eight-lane contract (src/kernels_x86.inc:206-249), and the per-output relative error against the
    float64 block-sum value reported beside the contract's own (outputs >= 0.1 of the token's largest)."""
    nb = cols // 32
    say("mfma full size", name)
    w = weights(False, 7000 + rows, rows, cols)
    raw = synth.activations(7100 + ntok, ntok, cols)
    if rows > 100000:  # configs[3]: RMSNorm-scaled activations
        raw = np.stack([orc.rmsnorm(r, np.ones(cols, np.float32), 1e-6)[1] for r in raw])
    dbuf, qbuf, xd, xq = gpu_quantize(raw)
    wb = smq.DeviceBuffer.from_array(w)
    out = smq.DeviceBuffer(ntok * rows * 4)
    out.fill(0xFF)
    smq.gemm_q8_mfma(wb, nb * Q8B, dbuf, qbuf, rows, ntok, nb, out, rows)
    got = out.download(np.float32).reshape(ntok, rows)
    del wb, out
    pick = np.arange(0, rows, step)
    wsub = w.reshape(rows, nb * Q8B)[pick].reshape(-1)
    got = np.ascontiguousarray(got[:, pick])
    assert_same_f32(got.reshape(-1), orc.gemm_blockwise(wsub, nb * Q8B, xd, xq, len(pick), ntok, nb), name)
    want = orc.gemm(wsub, nb * Q8B, xd, xq, len(pick), ntok, nb)
    ok, worst = mfma_tolerance_ok(got.reshape(-1), want, ntok, len(pick))
    exact = exact_outputs(orc, wsub, nb * Q8B, xd, xq, len(pick), ntok, nb)
    dist = per_output_errors(got, want, exact, ntok, len(pick))
    say(f"  normwise {worst:.3e}; per-output vs float64 (|out| >= 0.1 max, {dist[5]:.1%} of outputs): "
        f"median {dist[0]:.2e} p99 {dist[1]:.2e} p99.9 {dist[2]:.2e} max {dist[3]:.2e}; "
        f"eight-lane contract max {dist[4]:.2e}")
    assert ok, (name, worst)
    assert dist[3] <= 1e-5, (name, dist)


@pytest.mark.parametrize("rows,cols,ntok,q5", [(640, 896, 64, False), (200, 896, 100, False),
                                               (300, 4864, 96, False), (300, 8960, 64, True)])
def test_mfma_prefill_items_bias_accumulate(orc, rows, cols, ntok, q5):
    """smq_matmul on the MFMA GEMM with three items (bias, residual add; one K slice and several, on
    the 64x64 split-K kernel for Q8 and the block-pair kernel's K split for Q5): within 1e-5 of the
    exact contract, the prior added once."""
    nb = (cols + 31) // 32
    bb = Q5B if q5 else Q8B
    x = synth.activations(555 + rows, ntok, cols)
    dbuf, qbuf, xd, xq = gpu_quantize(x)
    items, wants = [], []
    for i, (r, with_bias, acc) in enumerate(((rows, True, False), (rows // 2 + 3, False, True), (64, True, True))):
        w = weights(q5, 600 + i, r, cols)
        bias = synth.normal(610 + i, r, 0.05) if with_bias else None
        prior = synth.normal(620 + i, ntok * r, 1.0)
        y = smq.DeviceBuffer.from_array(prior)
        items.append((smq.QMat(smq.DeviceBuffer.from_array(w), r, cols, smq.DTYPE_Q5 if q5 else smq.DTYPE_Q8),
                      smq.DeviceBuffer.from_array(bias) if bias is not None else None, y, acc))
        want = orc.mat_item(w, nb * bb, r, bias, xd, xq, ntok, nb, q5=q5)[1]
        wants.append((want + prior if acc else want, r))
    try:
        smq.set_prefill_mfma(True)
        smq.matmul(items, dbuf, qbuf, ntok)
        smq.numeric_check()
    finally:
        smq.set_prefill_mfma(False)
    for (_, _, y, _), (want, r) in zip(items, wants):
        ok, worst = mfma_tolerance_ok(y.download(np.float32), want, ntok, r)
        assert ok, worst


@pytest.mark.parametrize("ntok,with_bias", [(70, False), (40, True)])
def test_mfma_f16_small_items_and_nonfinite_flag(orc, ntok, with_bias):
    """The f16-MFMA GEMM (28-block Q8 rows) on items of fewer rows than a subtile and across a subtile
    edge (within 1e-5 of the exact contract), and its finiteness flag: clear for finite outputs, raised
    by an infinite weight scale (model.c:309's check), cleared by reading it."""
    cols, nb = 896, 28
    x = synth.activations(31 + ntok, ntok, cols)
    dbuf, qbuf, xd, xq = gpu_quantize(x)
    items, wants = [], []
    for i, rows in enumerate((5, 37)):
        w = weights(False, 70 + i, rows, cols)
        bias = synth.normal(80 + i, rows, 0.05) if with_bias else None
        items.append((smq.QMat(smq.DeviceBuffer.from_array(w), rows, cols),
                      smq.DeviceBuffer.from_array(bias) if bias is not None else None,
                      smq.DeviceBuffer(ntok * rows * 4)))
        wants.append((orc.mat_item(w, nb * Q8B, rows, bias, xd, xq, ntok, nb)[1], rows))
    try:
        smq.set_prefill_mfma(True)
        smq.matmul(items, dbuf, qbuf, ntok)
        smq.numeric_check()
        for (_, _, y), (want, r) in zip(items, wants):
            ok, worst = mfma_tolerance_ok(y.download(np.float32), want, ntok, r)
            assert ok, worst
        w = weights(False, 90, 20, cols)
        w[Q8B * 3:Q8B * 3 + 4] = np.array([np.inf], np.float32).view(np.uint8)  # row 0, block 3: scale inf
        yb = smq.DeviceBuffer(ntok * 20 * 4)
        smq.matmul([(smq.QMat(smq.DeviceBuffer.from_array(w), 20, cols), None, yb)], dbuf, qbuf, ntok)
        with pytest.raises(smq.SmqError) as e:
            smq.numeric_check()
        assert e.value.status == smq.SM_ERR_NUMERIC
        smq.numeric_check()  # cleared
    finally:
        smq.set_prefill_mfma(False)


def test_matmul_prefill_switch(orc):
    """smq_matmul with ntok > 1 takes the MFMA GEMM when selected (bias and
    finiteness still applied), the exact GEMM otherwise."""
    cols, nb, ntok = 896, 28, 32
    x = synth.activations(77, ntok, cols)
    dbuf, qbuf, xd, xq = gpu_quantize(x)
    items, wants = [], []
    for i, rows in enumerate((896, 128)):
        w = weights(False, 80 + i, rows, cols)
        bias = synth.normal(90 + i, rows, 0.05)
        items.append((smq.QMat(smq.DeviceBuffer.from_array(w), rows, cols), smq.DeviceBuffer.from_array(bias),
                      smq.DeviceBuffer(ntok * rows * 4)))
        wants.append(orc.mat_item(w, nb * Q8B, rows, bias, xd, xq, ntok, nb)[1])
    try:
        smq.set_prefill_mfma(True)
        smq.matmul(items, dbuf, qbuf, ntok)
        smq.numeric_check()
        for (wq, _, y), want in zip(items, wants):
            ok, worst = mfma_tolerance_ok(y.download(np.float32), want, ntok, wq.rows)
            assert ok, worst
    finally:
        smq.set_prefill_mfma(False)
    smq.matmul(items, dbuf, qbuf, ntok)
    for (_, _, y), want in zip(items, wants):
        assert_same_f32(y.download(np.float32), want, "exact prefill")


# ------------------------------------------------------------------ activation producers

@pytest.mark.parametrize("n", [896, 4864, 8960, 100, 1, 4096, 4097])
def test_norm_quantize_bit_exact(orc, n):
    """RMSNorm (sequential f32 sum) then Q8, against the oracle's row_work; 4096 and 4097 are the last row
    of the 256-thread workgroups and the first of the 1024-thread ones."""
    g = LcgUniform(300 + n)
    rows = 5
    x = g.uniform(-3, 3, rows * n)
    w = g.uniform(0.5, 1.5, n)
    nb = (n + 31) // 32
    xb, wb = smq.DeviceBuffer.from_array(x), smq.DeviceBuffer.from_array(w)
    y, d, q = smq.DeviceBuffer(rows * n * 4), smq.DeviceBuffer(rows * nb * 4), smq.DeviceBuffer(rows * nb * 32)
    smq.norm_quantize(xb, wb, 1e-6, rows, n, y, d, q)
    smq.numeric_check()
    ok, wy, wd, wq = orc.row_work(x, rows, n, norm=w, eps=1e-6)
    assert ok
    assert_same_f32(y.download(np.float32), wy, "rmsnorm y")
    assert_same_f32(d.download(np.float32), wd, "rmsnorm d")
    assert np.array_equal(q.download(np.int8), wq)


@pytest.mark.parametrize("gelu,n", [(False, 4864), (True, 4864), (False, 4096)])
def test_silu_quantize_bit_exact(orc, gelu, n):
    """SwiGLU / GeGLU with the binary64 exp, in place, then Q8; gate values
    cover the exp clamps, infinities and NaN-free extremes; 1024- and 256-thread rows."""
    g = LcgUniform(400 + gelu)
    rows = 3
    nb = n // 32
    up = g.uniform(-4, 4, rows * n)
    gate = g.uniform(-30, 30, rows * n)
    gate[::97] = np.array([88.7, 88.8, -88.7, -88.72, -88.8, -89.0, 103.0, 120.0, 1e-30, -1e-30, 0.0, -0.0, 200.0,
                           -200.0], np.float32)[np.arange(len(gate[::97])) % 14]
    ub, gb = smq.DeviceBuffer.from_array(up), smq.DeviceBuffer.from_array(gate)
    d, q = smq.DeviceBuffer(rows * nb * 4), smq.DeviceBuffer(rows * nb * 32)
    smq.silu_quantize(ub, gb, rows, n, d, q, gemma3=gelu)
    ok, wy, wd, wq = orc.row_work(up, rows, n, gate=gate, gelu=gelu)
    nonfinite = not ok
    if nonfinite:
        with pytest.raises(smq.SmqError):
            smq.numeric_check()
    else:
        smq.numeric_check()
    assert_same_f32(ub.download(np.float32), wy, "activation in place")
    if not nonfinite:
        assert_same_f32(d.download(np.float32), wd, "activation d")
        assert np.array_equal(q.download(np.int8), wq)


def test_row_quantize_flags_nonfinite(orc):
    rows, n = 2, 64
    x = np.ones(rows * n, np.float32)
    x[70] = np.inf
    xb = smq.DeviceBuffer.from_array(x)
    wb = smq.DeviceBuffer.from_array(np.ones(n, np.float32))
    d, q = smq.DeviceBuffer(rows * 2 * 4), smq.DeviceBuffer(rows * 64)
    smq.norm_quantize(xb, wb, 1e-6, rows, n, None, d, q)
    with pytest.raises(smq.SmqError) as e:
        smq.numeric_check()
    assert e.value.status == smq.SM_ERR_NUMERIC
    smq.row_quantize(xb, rows, n, d, q)  # plain quantize of an inf: also flagged
    with pytest.raises(smq.SmqError):
        smq.numeric_check()
    with pytest.raises(smq.SmqError) as e:
        smq.row_quantize(xb, rows, 20000, d, q)
    assert e.value.status == 4
