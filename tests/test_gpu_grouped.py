"""GPU parity of the streaming decode GEMV: grouped launches of independent
matrices with their own activations (smq_gemv_grouped) and single launches
large enough to take the persistent kernel (the LM head shape), against the
CPU oracle, bit for bit, in the exact and the fast (FMA) contract."""
import numpy as np
import pytest

from checks import assert_same_f32, q5_random, say
from smq_pkg import smq, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert smq.init(0) == "gfx950"
    smq.kernels_set_fast(False)
    smq.kernels_select()
    yield
    smq.kernels_set_fast(False)


def dev(a):
    return smq.DeviceBuffer.from_array(np.ascontiguousarray(a))


def quantized(seed, cols):
    x = synth.activations(seed, 1, cols)
    nb = (cols + 31) // 32
    xb = dev(x)
    d, q = smq.DeviceBuffer(nb * 4), smq.DeviceBuffer(nb * 32)
    smq.quantize_q8_rows(xb, 1, cols, d, q)
    return d, q, d.download(np.float32), q.download(np.int8)


GROUP_CASES = [
    # q5, cols, rows of each item, fast
    (False, 896, [4864, 4864, 896, 128, 7], False),   # FFN/QKV shapes and a ragged tail tile
    (False, 4864, [896, 896, 33], False),             # wide rows: several chunks per tile
    (False, 4864, [896, 50], True),                   # wide rows, fast contract
    (False, 16384, [40, 7], False),                   # the widest pinned activation (512 blocks)
    (True, 1536, [8960, 1536, 5], False),             # Q5 pairs
    (False, 896, [4864, 100], True),                  # fast contract (lane FMA)
    (True, 8960, [1536, 3], True),
    (False, 896, [1, 4864, 31, 4864, 33, 2000], False),  # item edges inside a workgroup's tile range
    (False, 2048, [3000, 17], True),                  # 64 blocks: the wide pinned activation
    (True, 2560, [3000, 9], False),                   # Q5, 80 blocks
    (False, 928, [4864, 4864], False),                # nb = 29 (odd)
    (False, 1024, [4864, 17], False),                 # nb = 32: the widest one-chunk (register) activation
    (False, 1000, [300, 2], True),                    # nb = 32 with a partial last block, fast
    (False, 1056, [500, 9], True),                    # nb = 33: the first two-chunk row
    (False, 20, [600, 3], False),                     # nb = 1: most threads of a tile idle
    (True, 2048, [700, 3], True),                     # Q5, 64 blocks (the widest pinned pair row), fast
    (True, 64, [100, 1], False),                      # Q5, one pair per row
    (True, 1472, [900, 5], False),                    # Q5, 46 blocks: one chunk, the last group of the chain half used
    (True, 4288, [700, 3], False),                    # Q5, 134 blocks: chunks of 68 and 66 (the last chunk's last
                                                      # group half used, its other slots written by the first chunk)
    (True, 4480, [500, 7], False),                    # Q5, 140 blocks: two chunks of 70
    # nb = 17: 30-row tiles whose last lane group's padded slots sit at the end of the product
    # buffer; enough rows for several tiles per workgroup, so both product buffers are used
    (False, 544, [100000], False),
    (False, 544, [60000, 7], True),
]
# items with neither bias nor residual add (the kernels then load no bias or prior output)
PLAIN_CASES = [
    (False, 896, [4864, 4864, 896, 7], False),
    (False, 896, [4864, 100], True),
    (False, 4864, [896, 896, 33], False),
    (False, 4864, [896, 5], True),
    (True, 1536, [8960, 5], False),
]


@pytest.mark.parametrize("q5,cols,rows,fast,plain", [c + (False,) for c in GROUP_CASES] +
                         [c + (True,) for c in PLAIN_CASES])
def test_grouped_gemv(orc, q5, cols, rows, fast, plain):
    say("grouped", q5, cols, rows, fast, plain)
    smq.kernels_set_fast(fast)
    nb = (cols + 31) // 32
    bb = 22 if q5 else 36
    items, want = [], []
    for i, r in enumerate(rows):
        w = (synth.q5_weights if q5 else synth.q8_weights)(100 + i, r, cols)
        bias = synth.normal(200 + i, r, 0.02) if i % 2 == 0 and not plain else None
        acc = i % 3 == 1 and not plain
        y0 = synth.normal(300 + i, r) if acc else np.zeros(r, np.float32)
        d, q, hd, hq = quantized(400 + i, cols)
        ok, prod = orc.mat_item(w, nb * bb, r, bias, hd, hq, 1, nb, q5=q5, fast=fast)
        assert ok
        want.append(y0 + prod if acc else prod)
        mat = smq.QMat(dev(w), r, cols, smq.DTYPE_Q5 if q5 else smq.DTYPE_Q8)
        items.append((mat, dev(bias) if bias is not None else None, dev(y0), acc, d, q))
    smq.gemv_grouped(items)
    smq.numeric_check()
    for i, (it, wnt) in enumerate(zip(items, want)):
        assert_same_f32(it[2].download(np.float32), wnt, f"item {i}")
    smq.kernels_set_fast(False)


@pytest.mark.parametrize("fast", [False, True])
def test_grouped_q5_configs2_down(orc, fast):
    """configs[2]'s 16 x 1536 x 8960 group as benched: 140 pairs a row, which the launcher cuts into
    7 chunks of 20 pairs (24-row tiles, two per workgroup); every item its own activation, some with
    a bias or a residual add."""
    say("grouped q5 configs2 down", fast)
    smq.kernels_set_fast(fast)
    rows, cols, n = 1536, 8960, 16
    nb = (cols + 31) // 32
    w = q5_random(77, rows, cols)
    wb = dev(w)  # one weight buffer shared by the items: the kernels read it as 16 matrices
    items, want = [], []
    for i in range(n):
        bias = synth.normal(500 + i, rows, 0.02) if i % 2 == 0 else None
        acc = i % 3 == 1
        y0 = synth.normal(600 + i, rows) if acc else np.zeros(rows, np.float32)
        d, q, hd, hq = quantized(700 + i, cols)
        ok, prod = orc.mat_item(w, nb * 22, rows, bias, hd, hq, 1, nb, q5=True, fast=fast)
        assert ok
        want.append(y0 + prod if acc else prod)
        items.append((smq.QMat(wb, rows, cols, smq.DTYPE_Q5), dev(bias) if bias is not None else None, dev(y0),
                      acc, d, q))
    smq.gemv_grouped(items)
    smq.numeric_check()
    for i, (it, wnt) in enumerate(zip(items, want)):
        assert_same_f32(it[2].download(np.float32), wnt, f"item {i}")
    smq.kernels_set_fast(False)


def test_grouped_rejects_mixed_widths():
    a = smq.QMat(dev(synth.q8_weights(1, 8, 64)), 8, 64)
    b = smq.QMat(dev(synth.q8_weights(2, 8, 96)), 8, 96)
    d, q, _, _ = quantized(3, 64)
    y = smq.DeviceBuffer(8 * 4)
    with pytest.raises(smq.SmqError) as e:
        smq.gemv_grouped([(a, None, y, False, d, q), (b, None, y, False, d, q)])
    assert e.value.status == smq.SM_ERR_STATE


@pytest.mark.parametrize("fast", [False, True])
def test_lm_head_streams(orc, fast):
    """151936 x 896: one matmul launch of 18992 tiles takes the persistent kernel."""
    say("lm head stream", fast)
    smq.kernels_set_fast(fast)
    rows, cols, nb = 151936, 896, 28
    w = synth.q8_weights(7, rows, cols)
    d, q, hd, hq = quantized(8, cols)
    y = smq.DeviceBuffer(rows * 4)
    smq.matmul([(smq.QMat(dev(w), rows, cols), None, y)], d, q, 1)
    smq.numeric_check()
    ok, want = orc.mat_item(w, nb * 36, rows, None, hd, hq, 1, nb, fast=fast)
    assert ok
    assert_same_f32(y.download(np.float32), want, "lm head")
    smq.kernels_set_fast(False)


def plan_items(orc, shapes, fast, plain=False, seed=500):
    """(items, wanted outputs) for Q8 matrices of the given (rows, cols) shapes, each with its own
    activation; odd items carry a bias, every third adds into its output (unless plain)."""
    items, want = [], []
    for i, (r, cols) in enumerate(shapes):
        nb = cols // 32
        w = synth.q8_weights(seed + i, r, cols)
        bias = synth.normal(seed + 1000 + i, r, 0.02) if i % 2 == 1 and not plain else None
        acc = i % 3 == 2 and not plain
        y0 = synth.normal(seed + 2000 + i, r) if acc else np.zeros(r, np.float32)
        d, q, hd, hq = quantized(seed + 3000 + i, cols)
        ok, prod = orc.mat_item(w, nb * 36, r, bias, hd, hq, 1, nb, fast=fast)
        assert ok
        want.append(y0 + prod if acc else prod)
        items.append((smq.QMat(dev(w), r, cols), dev(bias) if bias is not None else None, dev(y0), acc, d, q))
    return items, want


PLAN_CASES = [
    # (rows, cols) of the items, fast, plain
    ([(4864, 896), (896, 4864)] * 3, False, False),            # the FFN step's two widths in one launch
    ([(4864, 896), (896, 4864)] * 3, True, False),             # fast contract
    ([(896, 896)] * 60 + [(7, 896), (13, 4864)], False, True),  # more items than a grouped launch takes
    ([(5, 4864), (1, 896), (15, 4864), (9, 896)], False, False),  # items smaller than a tile
    ([(100000, 896), (30, 4864)], False, True),                # one item of many workgroups
]


@pytest.mark.parametrize("shapes,fast,plain", PLAN_CASES)
def test_gemv_plan(orc, shapes, fast, plain):
    """smq_gemv_plan: 28- and 152-block Q8 items in one launch, every output equal to the oracle's
    mat_item (bias, residual add) bit for bit."""
    say("gemv plan", len(shapes), shapes[:2], fast, plain)
    smq.kernels_set_fast(fast)
    items, want = plan_items(orc, shapes, fast, plain)
    plan = smq.GemvPlan(items)
    plan.launch()
    smq.numeric_check()
    for i, (it, wnt) in enumerate(zip(items, want)):
        assert_same_f32(it[2].download(np.float32), wnt, f"item {i}")
    plan.destroy()
    smq.kernels_set_fast(False)


def test_gemv_plan_in_a_graph(orc):
    """A plan launch captured once and replayed: each replay equals the oracle (items without a
    residual add, so every replay writes the same outputs)."""
    items, want = plan_items(orc, [(4864, 896), (896, 4864), (896, 896)] * 4, False, plain=True, seed=700)
    plan = smq.GemvPlan(items)
    g = smq.capture(plan.launch)
    for rep in range(3):
        say("gemv plan graph replay", rep)
        for it in items:
            it[2].fill(0)
        g.launch()
        smq.synchronize()
        smq.numeric_check()
        for i, (it, wnt) in enumerate(zip(items, want)):
            assert_same_f32(it[2].download(np.float32), wnt, f"replay {rep} item {i}")
    g.destroy()
    plan.destroy()


def test_gemv_plan_rejects_other_rows():
    d, q, _, _ = quantized(3, 1536)
    y = smq.DeviceBuffer(64 * 4)
    q8_48 = smq.QMat(dev(synth.q8_weights(1, 64, 1536)), 64, 1536)
    q5 = smq.QMat(dev(synth.q5_weights(2, 64, 896)), 64, 896, smq.DTYPE_Q5)
    d28, q28, _, _ = quantized(4, 896)
    for item in ((q8_48, None, y, False, d, q), (q5, None, y, False, d28, q28)):
        with pytest.raises(smq.SmqError) as e:
            smq.GemvPlan([item])
        assert e.value.status == smq.SM_ERR_RANGE
    with pytest.raises(smq.SmqError):
        smq.GemvPlan([])
