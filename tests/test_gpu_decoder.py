"""GPU parity of the decoder pieces around the matmuls (src/model.c:425-542,
669-677; src/sampler.c:57-63; src/kernels.c:1119-1176): RoPE + KV store,
attention, greedy argmax, embedding rows, the residual-accumulating matmul and
the device decode bookkeeping, each against the CPU oracle, bit for bit."""
import numpy as np
import pytest

from checks import assert_same_f32, say
from smq_pkg import smq, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert smq.init(0) == "gfx950"
    smq.kernels_set_fast(False)
    smq.kernels_select()
    yield


def dev(a):
    return smq.DeviceBuffer.from_array(np.ascontiguousarray(a))


ROPE_CASES = [
    # heads, kv_heads, head_dim, pairs, context, ntok, pos0
    (14, 2, 64, 32, 48, 5, 7),   # Qwen2.5-0.5B heads
    (4, 4, 40, 12, 16, 3, 13),   # partial rotary, tail passes through, last slots
    (6, 3, 6, 3, 8, 8, 0),       # whole context in one batch
]


@pytest.mark.parametrize("heads,kv_heads,hd,pairs,context,ntok,pos0", ROPE_CASES)
@pytest.mark.parametrize("use_pos_dev", [False, True])
def test_rope_kv(orc, heads, kv_heads, hd, pairs, context, ntok, pos0, use_pos_dev):
    say("rope_kv", heads, kv_heads, hd, pairs, context, ntok, pos0, use_pos_dev)
    qd, kd = heads * hd, kv_heads * hd
    q = synth.normal(11, ntok * qd).reshape(ntok, qd)
    k = synth.normal(12, ntok * kd).reshape(ntok, kd)
    v = synth.normal(13, ntok * kd).reshape(ntok, kd)
    cs = synth.normal(14, context * pairs).reshape(context, pairs)
    sn = synth.normal(15, context * pairs).reshape(context, pairs)
    sentinel = synth.normal(16, context * kd).reshape(context, kd)
    qb, kb, vb, cb, sb = dev(q), dev(k), dev(v), dev(cs), dev(sn)
    keys, values = dev(sentinel), dev(sentinel)
    shape = smq.attn_shape(heads, kv_heads, hd, pairs, 0, context)
    pos_dev = dev(np.array([pos0], np.int32)) if use_pos_dev else None
    smq.rope_kv(qb, kb, vb, ntok, shape, cb, sb, keys, values, 0 if use_pos_dev else pos0, pos_dev)
    smq.numeric_check()
    want_q = np.stack([orc.rope(q[t], heads, hd, pairs, cs[pos0 + t], sn[pos0 + t]) for t in range(ntok)])
    want_k = np.stack([orc.rope(k[t], kv_heads, hd, pairs, cs[pos0 + t], sn[pos0 + t]) for t in range(ntok)])
    want_keys, want_values = sentinel.copy(), sentinel.copy()
    want_keys[pos0:pos0 + ntok] = want_k
    want_values[pos0:pos0 + ntok] = v
    assert_same_f32(qb.download(np.float32).reshape(ntok, qd), want_q, "q")
    assert_same_f32(kb.download(np.float32).reshape(ntok, kd), want_k, "k")
    assert_same_f32(keys.download(np.float32).reshape(context, kd), want_keys, "keys")
    assert_same_f32(values.download(np.float32).reshape(context, kd), want_values, "values")


def test_rope_kv_refuses_positions_past_context():
    shape = smq.attn_shape(2, 1, 8, 4, 0, 4)
    b = smq.DeviceBuffer(4 * 64)
    with pytest.raises(smq.SmqError) as e:
        smq.rope_kv(b, b, b, 3, shape, b, b, b, b, 2)
    assert e.value.status == smq.SM_ERR_RANGE
    with pytest.raises(smq.SmqError):
        smq.rope_kv(b, b, b, 1, smq.attn_shape(3, 2, 8, 4, 0, 4), b, b, b, b, 0)  # heads % kv_heads


def attend_expect(orc, q, keys, values, heads, kv_heads, hd, window, pos0, ntok):
    kd = kv_heads * hd
    flat_k, flat_v = keys.reshape(-1), values.reshape(-1)
    out = np.zeros((ntok, heads * hd), np.float32)
    for t in range(ntok):
        pos = pos0 + t
        start = pos - window + 1 if window and pos >= window else 0
        for h in range(heads):
            kh = h // (heads // kv_heads)
            out[t, h * hd:(h + 1) * hd] = orc.attend_f32(q[t, h * hd:(h + 1) * hd], flat_k[kh * hd:],
                                                         flat_v[kh * hd:], kd, hd, start, pos)
    return out


ATT_CASES = [
    # heads, kv_heads, hd, window, context, ntok, pos0, score scale
    (14, 2, 64, 0, 700, 1, 640, 1.0),    # Qwen decode at ~640 positions
    (14, 2, 64, 0, 96, 24, 0, 1.0),      # prefill batch from position 0
    (4, 2, 40, 5, 64, 6, 20, 1.0),       # sliding window, hd % 8 != 0
    (3, 1, 6, 0, 40, 4, 30, 1.0),        # hd < 8: tail only
    (2, 2, 64, 0, 300, 2, 290, 30.0),    # wide scores: exp underflows to 0
    (8, 8, 128, 3, 17, 17, 0, 1.0),      # every position, tiny window
    (2, 1, 64, 0, 8192, 1, 8000, 1.0),   # 63 value chunks through both buffers
    (4, 2, 128, 0, 2048, 2, 1500, 1.0),  # head_dim 128: 64-position chunks
    (2, 1, 256, 0, 600, 1, 590, 1.0),    # head_dim 256: four outputs per lane
    (16, 2, 64, 0, 1024, 3, 1021, 1.0),  # grouped prefill: eight heads per KV head, up to 1024 positions
    (6, 3, 64, 37, 200, 40, 100, 1.0),   # grouped prefill with a sliding window
    (7, 7, 64, 0, 33, 33, 0, 1.0),       # grouped prefill: one head per group, from position 0
]


@pytest.mark.parametrize("heads,kv_heads,hd,window,context,ntok,pos0,scale", ATT_CASES)
def test_attention(orc, heads, kv_heads, hd, window, context, ntok, pos0, scale):
    say("attention", heads, kv_heads, hd, window, context, ntok, pos0, scale)
    qd, kd = heads * hd, kv_heads * hd
    q = synth.normal(21, ntok * qd, scale).reshape(ntok, qd)
    keys = synth.normal(22, context * kd).reshape(context, kd)
    values = synth.normal(23, context * kd).reshape(context, kd)
    qb, kb, vb = dev(q), dev(keys), dev(values)
    att = smq.DeviceBuffer(ntok * qd * 4)
    shape = smq.attn_shape(heads, kv_heads, hd, hd // 2, window, context)
    smq.attention(qb, kb, vb, att, ntok, shape, pos0)
    smq.numeric_check()
    want = attend_expect(orc, q, keys, values, heads, kv_heads, hd, window, pos0, ntok)
    assert_same_f32(att.download(np.float32).reshape(ntok, qd), want, "att")


@pytest.mark.parametrize("heads,kv_heads,hd,window,context,ntok,pos0", [
    (14, 2, 64, 0, 1024, 1, 700),   # decode: one launch quantizes its head's blocks
    (4, 2, 96, 7, 300, 9, 100),     # head_dim 96: three blocks, the last lane group half used
    (3, 1, 40, 0, 64, 5, 20),       # head_dim % 32 != 0: attention, then a separate quantize
    (14, 2, 64, 0, 600, 20, 500),   # grouped prefill: two Q8 blocks per head
])
def test_attention_q8(orc, heads, kv_heads, hd, window, context, ntok, pos0):
    say("attention_q8", heads, kv_heads, hd, window, context, ntok, pos0)
    qd, kd = heads * hd, kv_heads * hd
    nb = (qd + 31) // 32
    q = synth.normal(24, ntok * qd).reshape(ntok, qd)
    keys = synth.normal(25, context * kd).reshape(context, kd)
    values = synth.normal(26, context * kd).reshape(context, kd)
    qb, kb, vb = dev(q), dev(keys), dev(values)
    att = smq.DeviceBuffer(ntok * qd * 4)
    xd, xq = smq.DeviceBuffer(ntok * nb * 4), smq.DeviceBuffer(ntok * nb * 32)
    shape = smq.attn_shape(heads, kv_heads, hd, hd // 2, window, context)
    smq.attention_q8(qb, kb, vb, att, ntok, shape, xd, xq, pos0)
    smq.numeric_check()
    want = attend_expect(orc, q, keys, values, heads, kv_heads, hd, window, pos0, ntok)
    assert_same_f32(att.download(np.float32).reshape(ntok, qd), want, "att")
    _, wd, wq = orc.quantize_q8(want)
    assert_same_f32(xd.download(np.float32).reshape(ntok, nb), wd.reshape(ntok, nb), "att scales")
    assert np.array_equal(xq.download(np.int8).reshape(ntok, nb * 32), wq.reshape(ntok, nb * 32))


@pytest.mark.parametrize("heads,kv_heads,hd,pairs,window,context,pos,use_pos_dev", [
    (14, 2, 64, 32, 0, 1024, 700, True),   # Qwen2.5-0.5B decode step: one launch
    (14, 2, 64, 32, 0, 1024, 700, False),
    (14, 2, 64, 32, 0, 64, 0, True),       # first position: the score row is the new key alone
    (4, 2, 64, 12, 9, 64, 30, False),      # partial rotary, sliding window
    (2, 1, 64, 32, 0, 2048, 1500, True),   # several score rounds and value passes
    (3, 1, 40, 20, 0, 64, 20, False),      # head_dim % 32 != 0: the two-call form
    (4, 2, 128, 64, 0, 300, 250, True),    # head_dim 128: the two-call form
])
def test_attention_rope_q8(orc, heads, kv_heads, hd, pairs, window, context, pos, use_pos_dev):
    """smq_attention_rope_q8 == smq_rope_kv then smq_attention_q8 (oracle): the
    attention row, its Q8 blocks and both caches, bit for bit."""
    say("attention_rope_q8", heads, kv_heads, hd, pairs, window, context, pos, use_pos_dev)
    qd, kd = heads * hd, kv_heads * hd
    nb = (qd + 31) // 32
    q = synth.normal(81, qd)
    k = synth.normal(82, kd)
    v = synth.normal(83, kd)
    cs = synth.normal(84, context * pairs).reshape(context, pairs)
    sn = synth.normal(85, context * pairs).reshape(context, pairs)
    keys0 = synth.normal(86, context * kd).reshape(context, kd)
    values0 = synth.normal(87, context * kd).reshape(context, kd)
    qb, kb, vb, cb, sb = dev(q), dev(k), dev(v), dev(cs), dev(sn)
    keys, values = dev(keys0), dev(values0)
    att = smq.DeviceBuffer(qd * 4)
    xd, xq = smq.DeviceBuffer(nb * 4), smq.DeviceBuffer(nb * 32)
    shape = smq.attn_shape(heads, kv_heads, hd, pairs, window, context)
    pos_dev = dev(np.array([pos], np.int32)) if use_pos_dev else None
    smq.attention_rope_q8(qb, kb, vb, shape, cb, sb, keys, values, att, xd, xq, 0 if use_pos_dev else pos, pos_dev)
    smq.numeric_check()
    want_q = orc.rope(q, heads, hd, pairs, cs[pos], sn[pos])
    want_k = orc.rope(k, kv_heads, hd, pairs, cs[pos], sn[pos])
    want_keys, want_values = keys0.copy(), values0.copy()
    want_keys[pos], want_values[pos] = want_k, v
    assert_same_f32(keys.download(np.float32).reshape(context, kd), want_keys, "keys")
    assert_same_f32(values.download(np.float32).reshape(context, kd), want_values, "values")
    want = attend_expect(orc, want_q.reshape(1, qd), want_keys, want_values, heads, kv_heads, hd, window, pos, 1)
    assert_same_f32(att.download(np.float32).reshape(1, qd), want, "att")
    _, wd, wq = orc.quantize_q8(want)
    assert_same_f32(xd.download(np.float32).reshape(1, nb), wd.reshape(1, nb), "att scales")
    assert np.array_equal(xq.download(np.int8).reshape(1, nb * 32), wq.reshape(1, nb * 32))


def test_attention_position_from_device(orc):
    heads, kv_heads, hd, context = 14, 2, 64, 128
    qd, kd = heads * hd, kv_heads * hd
    q = synth.normal(31, qd).reshape(1, qd)
    keys = synth.normal(32, context * kd).reshape(context, kd)
    values = synth.normal(33, context * kd).reshape(context, kd)
    qb, kb, vb = dev(q), dev(keys), dev(values)
    att = smq.DeviceBuffer(qd * 4)
    shape = smq.attn_shape(heads, kv_heads, hd, hd // 2, 0, context)
    for pos in (0, 1, 77, 127):
        say("attention pos_dev", pos)
        smq.attention(qb, kb, vb, att, 1, shape, 0, dev(np.array([pos], np.int32)))
        smq.numeric_check()
        want = attend_expect(orc, q, keys, values, heads, kv_heads, hd, 0, pos, 1)
        assert_same_f32(att.download(np.float32).reshape(1, qd), want, f"att pos {pos}")


def gpu_argmax(logits, banned=None):
    lb = dev(np.asarray(logits, np.float32))
    bb = dev(np.asarray(banned, np.uint8)) if banned is not None else None
    tok = smq.DeviceBuffer(4)
    smq.argmax(lb, len(logits), bb, tok)
    smq.synchronize()
    return int(tok.download(np.uint32)[0])


def test_argmax(orc):
    vocab = 151936
    logits = synth.normal(41, vocab)
    banned = np.zeros(vocab, np.uint8)
    banned[256] = 1
    say("argmax random")
    assert gpu_argmax(logits, banned) == orc.argmax(logits, banned)
    # ties: lowest id wins; the best banned id is skipped
    t = logits.copy()
    top = t.max() + 1
    t[[5000, 900, 120000]] = top
    banned2 = banned.copy()
    banned2[900] = 1
    say("argmax ties")
    assert gpu_argmax(t, banned2) == orc.argmax(t, banned2) == 5000
    # +0 and -0 compare equal
    z = np.full(1000, -1.0, np.float32)
    z[700] = 0.0
    z[300] = -0.0
    assert gpu_argmax(z) == orc.argmax(z) == 300
    # NaN: never wins later, but a NaN first candidate stays
    n = logits[:5000].copy()
    n[17] = np.nan
    assert gpu_argmax(n) == orc.argmax(n)
    n[0] = np.nan
    assert gpu_argmax(n) == orc.argmax(n) == 0
    b0 = np.zeros(5000, np.uint8)
    b0[0] = 1
    assert gpu_argmax(n, b0) == orc.argmax(n, b0)
    # every id banned
    assert gpu_argmax(logits[:64], np.ones(64, np.uint8)) == 0xFFFFFFFF


def test_argmax_partials(orc):
    """The two-stage argmax across workgroup spans: ties and the NaN rule
    where the deciding ids sit in different spans, and vocabularies large
    enough that each workgroup walks several passes."""
    for vocab in (1, 1023, 1025, 151936, 3 * 1024 * 1024 + 17):
        logits = synth.normal(43 + vocab % 97, vocab)
        say("argmax vocab", vocab)
        assert gpu_argmax(logits) == orc.argmax(logits)
        if vocab < 4096:
            continue
        t = logits.copy()
        top = t.max() + 1
        t[[vocab - 1, vocab // 2, 2048 + 5]] = top  # equal maxima in three spans: the lowest id wins
        assert gpu_argmax(t) == orc.argmax(t) == 2048 + 5
        b = np.zeros(vocab, np.uint8)
        b[:3000] = 1  # first candidate deep in a later span, and NaN
        t[3000] = np.nan
        assert gpu_argmax(t, b) == orc.argmax(t, b) == 3000
        t[3000] = -np.inf  # a finite maximum elsewhere wins over -inf
        assert gpu_argmax(t, b) == orc.argmax(t, b) == vocab // 2


def test_argmax_advance(orc):
    vocab = 151936
    pos = dev(np.array([100], np.int32))
    count = dev(np.array([1], np.uint32))
    hist = dev(np.full(4, 7, np.uint32))
    tok = smq.DeviceBuffer(4)
    want = []
    for i in range(5):
        logits = synth.normal(70 + i, vocab)
        banned = np.zeros(vocab, np.uint8)
        banned[256] = 1
        smq.argmax_advance(dev(logits), vocab, dev(banned), tok, pos, count, hist, 4)
        smq.synchronize()
        want.append(orc.argmax(logits, banned))
        assert int(tok.download(np.uint32)[0]) == want[-1]
    assert int(pos.download(np.int32)[0]) == 105
    assert int(count.download(np.uint32)[0]) == 6
    assert hist.download(np.uint32).tolist() == [7] + want[:3]  # capacity bounds the history


@pytest.mark.parametrize("q5", [False, True])
def test_argmax_advance_embed(orc, q5):
    """The pick, the bookkeeping and the chosen token's embedding row in one call."""
    vocab, cols = 300, 200  # partial last block
    say("argmax_advance_embed q5" if q5 else "argmax_advance_embed q8")
    w = synth.q5_weights(52, vocab, cols) if q5 else synth.q8_weights(52, vocab, cols)
    mat = smq.QMat(dev(w), vocab, cols, smq.DTYPE_Q5 if q5 else smq.DTYPE_Q8)
    pos = dev(np.array([10], np.int32))
    count = dev(np.array([0], np.uint32))
    hist = dev(np.zeros(8, np.uint32))
    tok, x = smq.DeviceBuffer(4), smq.DeviceBuffer(cols * 4)
    want = []
    for i in range(4):
        logits = synth.normal(90 + i, vocab)
        banned = np.zeros(vocab, np.uint8)
        banned[int(np.argmax(logits))] = i & 1  # every other call bans the plain maximum
        smq.argmax_advance_embed(dev(logits), vocab, dev(banned), tok, pos, count, hist, 8, mat, x)
        smq.numeric_check()
        want.append(orc.argmax(logits, banned))
        assert int(tok.download(np.uint32)[0]) == want[-1]
        assert_same_f32(x.download(np.float32), orc.dequantize_row(w[want[-1]], cols, q5=q5), "embedded row")
    assert int(pos.download(np.int32)[0]) == 14
    assert hist.download(np.uint32).tolist()[:4] == want
    # a token past the embedding's rows is no row: the numeric flag is raised and x keeps its contents
    logits = np.full(vocab + 10, -1.0, np.float32)
    logits[vocab + 5] = 1.0
    before = x.download(np.float32)
    smq.argmax_advance_embed(dev(logits), vocab + 10, None, tok, pos, count, hist, 8, mat, x)
    with pytest.raises(smq.SmqError):
        smq.numeric_check()
    assert int(tok.download(np.uint32)[0]) == vocab + 5
    assert np.array_equal(x.download(np.float32), before)


@pytest.mark.parametrize("q5", [False, True])
def test_embed(orc, q5):
    vocab, cols = 300, 200  # partial last block
    say("embed q5" if q5 else "embed q8")
    w = synth.q5_weights(51, vocab, cols) if q5 else synth.q8_weights(51, vocab, cols)
    tokens = np.array([0, 299, 17, 17, 256, 3], np.uint32)
    mat = smq.QMat(dev(w), vocab, cols, smq.DTYPE_Q5 if q5 else smq.DTYPE_Q8)
    x = smq.DeviceBuffer(len(tokens) * cols * 4)
    tb = dev(tokens)
    smq.embed(mat, tb, len(tokens), x)
    smq.numeric_check()
    want = np.stack([orc.dequantize_row(w[t], cols, q5=q5) for t in tokens])
    assert_same_f32(x.download(np.float32).reshape(len(tokens), cols), want, "embed")


@pytest.mark.parametrize("ntok", [1, 7])
def test_matmul_accumulate(orc, ntok):
    """x += W a (+ bias): the residual add fused into the matmul store."""
    rows, cols = 896, 4864
    nb = (cols + 31) // 32
    say("matmul accumulate", ntok)
    w = synth.q8_weights(61, rows, cols)
    bias = synth.normal(62, rows, 0.02)
    a = synth.activations(63, ntok, cols)
    x0 = synth.normal(64, ntok * rows).reshape(ntok, rows)
    ab = dev(a)
    d, q = smq.DeviceBuffer(ntok * nb * 4), smq.DeviceBuffer(ntok * nb * 32)
    smq.quantize_q8_rows(ab, ntok, cols, d, q)
    xd, xq = d.download(np.float32), q.download(np.int8)
    mat = smq.QMat(dev(w), rows, cols, smq.DTYPE_Q8)
    y = dev(x0)
    smq.matmul([(mat, dev(bias), y, True)], d, q, ntok)
    smq.numeric_check()
    prod = orc.gemm(w, nb * 36, xd, xq, rows, ntok, nb).reshape(ntok, rows)
    want = x0 + (prod + bias)
    assert_same_f32(y.download(np.float32).reshape(ntok, rows), want, "x + Wa + b")


def test_decode_advance():
    pos = dev(np.array([41], np.int32))
    count = dev(np.array([0], np.uint32))
    hist = dev(np.zeros(3, np.uint32))
    for i, t in enumerate([7, 9, 11, 13]):
        tok = dev(np.array([t], np.uint32))
        smq.decode_advance(pos, count, tok, hist, 3)
    smq.synchronize()
    assert int(pos.download(np.int32)[0]) == 45
    assert int(count.download(np.uint32)[0]) == 4
    assert hist.download(np.uint32).tolist() == [7, 9, 11]  # capacity bounds the history
