"""GPU parity of the fused decode matmuls (smq_matmul_act, smq_matmul_glu):
the activation producers of the reference's decode step (model.c:334-415,
vecmath.c:78-93) formed inside the matmul launch, against the CPU oracle's
row_work + mat_item composition and against the library's own unfused calls,
bit for bit. Shapes cover the fused kernel's tile sizes (1, 2, 4 and 8 rows
per workgroup), partial blocks, Q5 weights, bias and the residual add, the
widest fused RMSNorm row and the fallbacks (wider rows, mixed formats)."""
import numpy as np
import pytest

from checks import assert_same_f32, say
from smq_pkg import smq, synth

pytestmark = pytest.mark.gpu

Q8, Q5 = 1, 2


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert smq.init(0) == "gfx950"
    smq.kernels_set_fast(False)
    smq.kernels_select()
    yield


def dev(a):
    return smq.DeviceBuffer.from_array(np.ascontiguousarray(a))


def weights(seed, rows, cols, dtype):
    return synth.q5_weights(seed, rows, cols) if dtype == Q5 else synth.q8_weights(seed, rows, cols)


def row_bytes(cols, dtype):
    return (cols + 31) // 32 * (22 if dtype == Q5 else 36)


def expect_items(orc, mats, d, q, cols):
    """mat_item (bias, finiteness) of each (w, rows, dtype, bias, prior) on (d, q)."""
    nb = (cols + 31) // 32
    out = []
    for w, rows, dtype, bias, prior in mats:
        ok, y = orc.mat_item(w.reshape(-1), row_bytes(cols, dtype), rows, bias, d, q, 1, nb, q5=dtype == Q5)
        assert ok
        out.append(y if prior is None else prior + y)
    return out


@pytest.mark.parametrize("cols,rows,dtypes,with_bias,accumulate", [
    (896, [896, 128, 128], [Q8, Q8, Q8], True, False),    # Qwen2.5-0.5B q/k/v: 8 rows per workgroup
    (896, [896], [Q8], False, True),                      # an accumulating item (x += W a)
    (200, [77, 300], [Q8, Q8], True, False),              # partial block, ragged rows
    (1536, [1536, 256, 256], [Q8, Q8, Q8], True, False),  # 4 rows per workgroup
    (4864, [896], [Q8], False, True),                     # 1 row per workgroup, one chunk
    (8192, [64], [Q8], False, False),                     # the widest fused RMSNorm row (LDS past 64 KiB)
    (8200, [40], [Q8], False, False),                     # wider: the unfused fallback
    (896, [512, 128], [Q5, Q8], True, False),             # mixed formats: one fused launch per format
    (1536, [300], [Q5], False, True),                     # Q5: 2 rows per workgroup
])
def test_matmul_act_norm(orc, cols, rows, dtypes, with_bias, accumulate):
    say("matmul_act norm", cols, rows, dtypes, with_bias, accumulate)
    nb = (cols + 31) // 32
    x = synth.normal(501 + cols, cols)
    w = synth.normal(502 + cols, cols, 0.2) + 1.0
    eps = 1e-6
    ok, _, d, q = orc.row_work(x, 1, cols, norm=w, eps=eps)
    assert ok
    mats, items = [], []
    for i, (r, dt) in enumerate(zip(rows, dtypes)):
        wt = weights(510 + i, r, cols, dt)
        bias = synth.normal(520 + i, r, 0.02) if with_bias else None
        prior = synth.normal(530 + i, r) if accumulate else None
        y = dev(prior) if accumulate else smq.DeviceBuffer(r * 4)
        mats.append((wt, r, dt, bias, prior))
        items.append((smq.QMat(dev(wt), r, cols, dt), dev(bias) if with_bias else None, y, accumulate))
    xd_s, xq_s = smq.DeviceBuffer(nb * 4), smq.DeviceBuffer(nb * 32)
    smq.matmul_act(items, smq.act(smq.ACT_NORM, cols, x=dev(x), norm=dev(w), eps=eps, xd_scratch=xd_s,
                                  xq_scratch=xq_s))
    smq.numeric_check()
    for (m, it, want) in zip(mats, items, expect_items(orc, mats, d, q, cols)):
        assert_same_f32(it[2].download(np.float32), want, f"item rows {m[1]}")


@pytest.mark.parametrize("cols,rows,dtype", [(4864, 896, Q8), (896, 1000, Q8), (8960, 300, Q5), (100, 50, Q8)])
def test_matmul_act_f32(orc, cols, rows, dtype):
    """Q8 of an f32 row inside the launch (the down projection's input)."""
    say("matmul_act f32", cols, rows, dtype)
    nb = (cols + 31) // 32
    h = synth.normal(601 + cols, cols, 3.0)
    ok, _, d, q = orc.row_work(h, 1, cols)
    assert ok
    wt = weights(602, rows, cols, dtype)
    prior = synth.normal(603, rows)
    y = dev(prior)
    item = (smq.QMat(dev(wt), rows, cols, dtype), None, y, True)
    smq.matmul_act([item], smq.act(smq.ACT_F32, cols, x=dev(h), xd_scratch=smq.DeviceBuffer(nb * 4),
                                   xq_scratch=smq.DeviceBuffer(nb * 32)))
    smq.numeric_check()
    want = expect_items(orc, [(wt, rows, dtype, None, prior)], d, q, cols)[0]
    assert_same_f32(y.download(np.float32), want, "x + W q8(h)")


@pytest.mark.parametrize("cols,rows,dtype,gate_dtype", [
    (896, 4864, Q8, Q8),    # Qwen2.5-0.5B gate/up: 4 + 4 rows per workgroup
    (1536, 8960, Q5, Q5),   # 1.5B-shaped Q5: 1 + 1 rows per workgroup, two chunks
    (2048, 130, Q8, Q8),    # 2 + 2 rows per workgroup, ragged last tile
    (896, 200, Q8, Q5),     # mixed formats: the unfused fallback
])
def test_matmul_glu(orc, cols, rows, dtype, gate_dtype):
    """h = up * silu(gate) of the RMSNorm activation (model.c:636-640)."""
    say("matmul_glu", cols, rows, dtype, gate_dtype)
    nb = (cols + 31) // 32
    x = synth.normal(701 + cols, cols)
    w = synth.normal(702 + cols, cols, 0.2) + 1.0
    ok, _, d, q = orc.row_work(x, 1, cols, norm=w, eps=1e-6)
    assert ok
    wg = weights(703, rows, cols, gate_dtype)
    wu = weights(704, rows, cols, dtype)
    gate_mat = smq.QMat(dev(wg), rows, cols, gate_dtype)
    up_mat = smq.QMat(dev(wu), rows, cols, dtype)
    h = smq.DeviceBuffer(rows * 4)
    smq.matmul_glu(gate_mat, up_mat, smq.act(smq.ACT_NORM, cols, x=dev(x), norm=dev(w), eps=1e-6,
                                             xd_scratch=smq.DeviceBuffer(nb * 4), xq_scratch=smq.DeviceBuffer(nb * 32)),
                   1, h, gate_scratch=smq.DeviceBuffer(rows * 4))
    smq.numeric_check()
    g, u = expect_items(orc, [(wg, rows, gate_dtype, None, None), (wu, rows, dtype, None, None)], d, q, cols)
    assert_same_f32(h.download(np.float32), orc.act_mul(u, g), "h")


@pytest.mark.parametrize("cols,rows,glu,prologue", [
    (896, 4864, 1, "norm"),   # Qwen2.5-0.5B gate/up: 152 h blocks, one workgroup each
    (896, 4864, 2, "norm"),   # GeGLU
    (896, 200, 1, "norm"),    # a partial last h block (200 = 6*32 + 8)
    (880, 96, 1, "f32"),      # a partial last activation block, the f32 prologue
    (1536, 300, 1, "norm"),   # not a packed 28-block row: the unfused composition
])
def test_matmul_glu_q8(orc, cols, rows, glu, prologue):
    """h = up * act(gate) of the RMSNorm (or f32) activation and h's Q8 blocks
    (model.c:409-415, 636-640) in one call, against the oracle's row_work
    composition and the library's unfused smq_matmul_glu + smq_quantize_q8_rows."""
    say("matmul_glu_q8", cols, rows, glu, prologue)
    nb, nbh = (cols + 31) // 32, (rows + 31) // 32
    x = synth.normal(721 + cols, cols)
    w = synth.normal(722 + cols, cols, 0.2) + 1.0
    if prologue == "norm":
        ok, _, d, q = orc.row_work(x, 1, cols, norm=w, eps=1e-6)
        activation = lambda: smq.act(smq.ACT_NORM, cols, x=dev(x), norm=dev(w), eps=1e-6,  # noqa: E731
                                     xd_scratch=smq.DeviceBuffer(nb * 4), xq_scratch=smq.DeviceBuffer(nb * 32))
    else:
        ok, _, d, q = orc.row_work(x, 1, cols)
        activation = lambda: smq.act(smq.ACT_F32, cols, x=dev(x), xd_scratch=smq.DeviceBuffer(nb * 4),  # noqa: E731
                                     xq_scratch=smq.DeviceBuffer(nb * 32))
    assert ok
    wg, wu = weights(723, rows, cols, Q8), weights(724, rows, cols, Q8)
    gate_mat, up_mat = smq.QMat(dev(wg), rows, cols, Q8), smq.QMat(dev(wu), rows, cols, Q8)
    h, hd, hq = smq.DeviceBuffer(rows * 4), smq.DeviceBuffer(nbh * 4), smq.DeviceBuffer(nbh * 32)
    smq.matmul_glu_q8(gate_mat, up_mat, activation(), glu, h, hd, hq, gate_scratch=smq.DeviceBuffer(rows * 4))
    smq.numeric_check()
    g, u = expect_items(orc, [(wg, rows, Q8, None, None), (wu, rows, Q8, None, None)], d, q, cols)
    ok, want_h, want_d, want_q = orc.row_work(u, 1, rows, gate=g, gelu=glu == 2)
    assert ok
    assert_same_f32(h.download(np.float32), want_h, "h")
    assert_same_f32(hd.download(np.float32), want_d, "h scales")
    assert np.array_equal(hq.download(np.int8), want_q), "h blocks"
    # the unfused calls give the same bits
    h2, hd2, hq2 = smq.DeviceBuffer(rows * 4), smq.DeviceBuffer(nbh * 4), smq.DeviceBuffer(nbh * 32)
    smq.matmul_glu(gate_mat, up_mat, activation(), glu, h2, gate_scratch=smq.DeviceBuffer(rows * 4))
    smq.quantize_q8_rows(h2, 1, rows, hd2, hq2)
    smq.numeric_check()
    assert_same_f32(h2.download(np.float32), want_h, "h unfused")
    assert_same_f32(hd2.download(np.float32), want_d, "h scales unfused")
    assert np.array_equal(hq2.download(np.int8), want_q), "h blocks unfused"


def test_matmul_glu_q8_nonfinite_flag():
    cols, rows = 896, 64
    g = smq.QMat(dev(synth.q8_weights(931, rows, cols)), rows, cols)
    u = smq.QMat(dev(synth.q8_weights(932, rows, cols)), rows, cols)
    x = synth.normal(933, cols)
    x[17] = np.inf
    h, hd, hq = smq.DeviceBuffer(rows * 4), smq.DeviceBuffer(8), smq.DeviceBuffer(64)
    smq.matmul_glu_q8(g, u, smq.act(smq.ACT_NORM, cols, x=dev(x), norm=dev(np.ones(cols, np.float32))), 1, h, hd, hq)
    with pytest.raises(smq.SmqError) as e:
        smq.numeric_check()
    assert e.value.status == smq.SM_ERR_NUMERIC


def test_glu_chain_equals_unfused(orc):
    """One decode FFN (RMSNorm -> gate/up -> SwiGLU -> down, x += ...) through
    the fused calls and through the unfused ones: the same bits."""
    cols, hidden = 896, 4864
    nbc, nbh = cols // 32, hidden // 32
    x0 = synth.normal(801, cols)
    w = synth.normal(802, cols, 0.2) + 1.0
    gate = smq.QMat(dev(synth.q8_weights(803, hidden, cols)), hidden, cols)
    up = smq.QMat(dev(synth.q8_weights(804, hidden, cols)), hidden, cols)
    down = smq.QMat(dev(synth.q8_weights(805, cols, hidden)), cols, hidden)
    wb = dev(w)
    # fused
    xf = dev(x0)
    h = smq.DeviceBuffer(hidden * 4)
    smq.matmul_glu(gate, up, smq.act(smq.ACT_NORM, cols, x=xf, norm=wb, eps=1e-6), 1, h)
    smq.matmul_act([(down, None, xf, True)], smq.act(smq.ACT_F32, hidden, x=h, xd_scratch=smq.DeviceBuffer(nbh * 4),
                                                     xq_scratch=smq.DeviceBuffer(nbh * 32)))
    smq.numeric_check()
    # unfused
    xu = dev(x0)
    d, q = smq.DeviceBuffer(nbc * 4), smq.DeviceBuffer(nbc * 32)
    hd, hq = smq.DeviceBuffer(nbh * 4), smq.DeviceBuffer(nbh * 32)
    gb, ub = smq.DeviceBuffer(hidden * 4), smq.DeviceBuffer(hidden * 4)
    smq.norm_quantize(xu, wb, 1e-6, 1, cols, None, d, q)
    smq.matmul([(gate, None, gb), (up, None, ub)], d, q, 1)
    smq.silu_quantize(ub, gb, 1, hidden, hd, hq)
    smq.matmul([(down, None, xu, True)], hd, hq, 1)
    smq.numeric_check()
    assert_same_f32(h.download(np.float32), ub.download(np.float32), "h")
    assert_same_f32(xf.download(np.float32), xu.download(np.float32), "x")


def test_fused_nonfinite_flags():
    cols, rows = 896, 64
    wt = smq.QMat(dev(synth.q8_weights(901, rows, cols)), rows, cols)
    for bad in (np.inf, np.nan):
        x = synth.normal(902, cols)
        x[333] = bad
        y = smq.DeviceBuffer(rows * 4)
        say("fused nonfinite", bad)
        smq.matmul_act([(wt, None, y)], smq.act(smq.ACT_NORM, cols, x=dev(x), norm=dev(np.ones(cols, np.float32))))
        with pytest.raises(smq.SmqError) as e:
            smq.numeric_check()
        assert e.value.status == smq.SM_ERR_NUMERIC
        smq.matmul_act([(wt, None, y)], smq.act(smq.ACT_F32, cols, x=dev(x)))
        with pytest.raises(smq.SmqError):
            smq.numeric_check()


def test_fused_argument_errors():
    cols = 8200  # past the fused RMSNorm width: needs the scratch buffers
    wt = smq.QMat(dev(synth.q8_weights(911, 8, cols)), 8, cols)
    y = smq.DeviceBuffer(8 * 4)
    x = dev(synth.normal(912, cols))
    with pytest.raises(smq.SmqError) as e:
        smq.matmul_act([(wt, None, y)], smq.act(smq.ACT_NORM, cols, x=x, norm=x))
    assert e.value.status == smq.SM_ERR_RANGE
    with pytest.raises(smq.SmqError):  # column count of the activation differs
        smq.matmul_act([(wt, None, y)], smq.act(smq.ACT_F32, cols - 1, x=x))
    g = smq.QMat(dev(synth.q8_weights(913, 8, 64)), 8, 64)
    u = smq.QMat(dev(synth.q8_weights(914, 9, 64)), 9, 64)
    with pytest.raises(smq.SmqError):  # gate and up differ in rows
        smq.matmul_glu(g, u, smq.act(smq.ACT_NORM, 64, x=x, norm=x), 1, y)


@pytest.mark.parametrize("cols,heads,kv_heads,hd,pairs,dtype,context,pos,use_pos_dev", [
    (896, 14, 2, 64, 32, Q8, 64, 37, True),     # Qwen2.5-0.5B q/k/v: one fused launch, position on the device
    (896, 14, 2, 64, 32, Q8, 64, 63, False),    # the last cache slot, position by value
    (896, 4, 2, 64, 12, Q8, 40, 5, True),       # partial rotary: the tail of each head passes through
    (100, 2, 1, 32, 16, Q8, 16, 9, False),      # 4-block rows: the matmul, then RoPE and the store
    (896, 2, 1, 64, 32, Q5, 16, 3, True),       # Q5 weights: the same two calls
])
def test_matmul_act_rope(orc, cols, heads, kv_heads, hd, pairs, dtype, context, pos, use_pos_dev):
    """smq_matmul_act_rope == RMSNorm + Q8 (row_work), q/k/v mat_item with bias,
    then rope (model.c:442-450) and the cache store of k and v at the position
    (oracle), bit for bit; the other cache rows untouched."""
    say("matmul_act_rope", cols, heads, kv_heads, hd, pairs, dtype, context, pos, use_pos_dev)
    qd, kd = heads * hd, kv_heads * hd
    x = synth.normal(951 + cols, cols)
    nw = synth.normal(952 + cols, cols, 0.2) + 1.0
    ok, _, d, q = orc.row_work(x, 1, cols, norm=nw, eps=1e-6)
    assert ok
    mats, items = [], []
    for i, r in enumerate((qd, kd, kd)):
        wt = weights(953 + i, r, cols, dtype)
        bias = synth.normal(956 + i, r, 0.02)
        mats.append((wt, r, dtype, bias, None))
        items.append((smq.QMat(dev(wt), r, cols, dtype), dev(bias), smq.DeviceBuffer(r * 4), False))
    cs = synth.normal(960, context * pairs).reshape(context, pairs)
    sn = synth.normal(961, context * pairs).reshape(context, pairs)
    keys0 = synth.normal(962, context * kd).reshape(context, kd)
    values0 = synth.normal(963, context * kd).reshape(context, kd)
    keys, values = dev(keys0), dev(values0)
    shape = smq.attn_shape(heads, kv_heads, hd, pairs, 0, context)
    pos_dev = dev(np.array([pos], np.int32)) if use_pos_dev else None
    smq.matmul_act_rope(items, smq.act(smq.ACT_NORM, cols, x=dev(x), norm=dev(nw), eps=1e-6,
                                       xd_scratch=smq.DeviceBuffer((cols + 31) // 32 * 4),
                                       xq_scratch=smq.DeviceBuffer((cols + 31) // 32 * 32)),
                        shape, dev(cs), dev(sn), keys, values, 0 if use_pos_dev else pos, pos_dev)
    smq.numeric_check()
    wq, wk, wv = expect_items(orc, mats, d, q, cols)
    wq = orc.rope(wq, heads, hd, pairs, cs[pos], sn[pos])
    wk = orc.rope(wk, kv_heads, hd, pairs, cs[pos], sn[pos])
    want_keys, want_values = keys0.copy(), values0.copy()
    want_keys[pos], want_values[pos] = wk, wv
    assert_same_f32(items[0][2].download(np.float32), wq, "q")
    assert_same_f32(items[1][2].download(np.float32), wk, "k")
    assert_same_f32(items[2][2].download(np.float32), wv, "v")
    assert_same_f32(keys.download(np.float32).reshape(context, kd), want_keys, "keys")
    assert_same_f32(values.download(np.float32).reshape(context, kd), want_values, "values")


def test_matmul_act_rope_position_past_context():
    """A device position at the context: the numeric flag, and no cache row written."""
    cols, heads, kv_heads, hd, context = 896, 14, 2, 64, 8
    qd, kd = heads * hd, kv_heads * hd
    items = [(smq.QMat(dev(synth.q8_weights(970 + i, r, cols)), r, cols), None, smq.DeviceBuffer(r * 4), False)
             for i, r in enumerate((qd, kd, kd))]
    keys0 = synth.normal(975, context * kd)
    keys, values = dev(keys0), dev(keys0)
    table = dev(synth.normal(976, context * 32))
    x = dev(synth.normal(977, cols))
    smq.matmul_act_rope(items, smq.act(smq.ACT_NORM, cols, x=x, norm=x), smq.attn_shape(heads, kv_heads, hd, 32, 0,
                                                                                        context),
                        table, table, keys, values, 0, dev(np.array([context], np.int32)))
    with pytest.raises(smq.SmqError) as e:
        smq.numeric_check()
    assert e.value.status == smq.SM_ERR_NUMERIC
    assert_same_f32(keys.download(np.float32), keys0, "keys")
    assert_same_f32(values.download(np.float32), keys0, "values")
