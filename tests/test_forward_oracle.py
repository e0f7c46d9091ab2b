"""The restated forward pass (oracle/smq_forward.c) against the reference's own
model layer (src/model.c built into oracle/_ref/libsmref_model.so) on
synthetic checkpoints: logits of batched prefill and single-token decode, the
KV cache and greedy tokens must be bit-identical. This pins the oracle that
the GPU forward is later compared with."""
import os

import numpy as np
import pytest

import oracle
from smq_pkg import smoe

TINY = {"architecture": "smolmoe_qwen2", "dim": 128, "hidden_dim": 320, "layers": 2, "heads": 4, "kv_heads": 2,
        "experts": 1, "top_k": 1, "vocab_size": 300, "max_context": 512, "shared_experts": 0, "bos_id": 256,
        "eos_id": 257, "rms_eps": "1e-06", "rope_theta": "1000000"}

VARIANTS = {
    "qwen2": dict(TINY),
    "v1_partial_rotary": dict(TINY, architecture="smolmoe_v1", rotary_dim=16, rope_attention_factor="1.25"),
    "llama3_window": dict(TINY, architecture="smolmoe_v1", heads=2, kv_heads=1, head_dim=40, sliding_window=5,
                          rope_theta="500000", rope_llama3_factor="8", rope_llama3_low_freq_factor="1",
                          rope_llama3_high_freq_factor="4", rope_llama3_original_context="64"),
    "q5_mixed": dict(TINY, dim=96, hidden_dim=200, heads=3, kv_heads=1),
}
Q5_NAMES = {"q5_mixed": ("l.0.q", "l.0.e.0.down", "l.1.e.0.up", "lm_head", "embed")}


def checkpoint(tmp_path, name, version=3, tie=True):
    cfg = VARIANTS[name]
    t = smoe.dense_tensors(cfg, seed=7, sigma=0.05, q5=Q5_NAMES.get(name, ()))
    path = str(tmp_path / f"{name}.smoe")
    text = smoe.config_text(cfg)
    if version == 3:
        smoe.write(path, t, version=3, config=text, tie_lm_head=tie and name != "q5_mixed")
    else:
        smoe.write(path, t, version=version, tie_lm_head=tie and version >= 2)
    cpath = str(tmp_path / f"{name}.ini")
    with open(cpath, "w") as f:
        f.write(text)
    if tie and version >= 2 and name != "q5_mixed":
        t["lm_head"] = t["embed"]
    return cfg, t, path, cpath


def prompt(n, vocab, seed=5):
    rng = np.random.default_rng(seed)
    return rng.integers(0, vocab, n).astype(np.uint32)


def bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


needs_ref = pytest.mark.skipif(not oracle.ReferenceModel.available(),
                               reason="reference model layer not built (oracle/_ref/libsmref_model.so)")


@needs_ref
@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_restated_forward_matches_reference(orc, tmp_path, name):
    cfg, t, path, _ = checkpoint(tmp_path, name)
    context, n = 48, 13
    ref = oracle.ReferenceModel(path, context=context, batch=8, logit_rows=8, threads=3)
    om = oracle.OracleModel(orc, cfg, t, context)
    toks = prompt(n, int(cfg["vocab_size"]))
    # every prompt row's logits, in two batches (the reference's batch is 8)
    assert ref.forward(toks[:8], 0, 2) == 0
    ok, want = om.forward(toks[:8], 0, 2)
    assert ok
    assert np.array_equal(bits(ref.logits(8)), bits(want))
    assert ref.forward(toks[8:], 8, 1) == 0
    ok, want = om.forward(toks[8:], 8, 1)
    assert ok and np.array_equal(bits(ref.logits(1)), bits(want))
    # KV caches after the prompt
    for layer in range(int(cfg["layers"])):
        for values in (False, True):
            got = ref.kv(layer, values, n, om.kv_dim)
            exp = (om.values if values else om.keys)[layer, :n]
            assert np.array_equal(bits(got), bits(exp)), (layer, values)
    # greedy decode, BOS banned
    banned = np.zeros(om.vocab, np.uint8)
    banned[256] = 1
    ref.set_banned(banned)
    got = ref.generate(n, 9)
    want = om.generate(n, 9, banned)
    assert got.tolist() == want.tolist()
    ref.close()


@needs_ref
def test_prefill_batch_size_does_not_change_logits(orc, tmp_path):
    """model.h:3-5: one code path for batched prefill and decode; outputs are
    identical either way (the reference with batch 1 vs the oracle at once)."""
    cfg, t, path, cpath = checkpoint(tmp_path, "qwen2", version=1, tie=False)
    toks = prompt(10, int(cfg["vocab_size"]), seed=9)
    ref = oracle.ReferenceModel(path, config_path=cpath, context=32, batch=1, logit_rows=1)
    ref.prefill(toks, 0, True)
    om = oracle.OracleModel(orc, cfg, t, 32)
    ok, want = om.forward(toks, 0, 1)
    assert ok and np.array_equal(bits(ref.logits(1)), bits(want))
    ref.close()


def test_restated_forward_is_batch_invariant(orc, tmp_path):
    """Without the reference: prefill in one batch == token by token."""
    cfg, t, _, _ = checkpoint(tmp_path, "v1_partial_rotary")
    toks = prompt(7, int(cfg["vocab_size"]), seed=3)
    a = oracle.OracleModel(orc, cfg, t, 16)
    ok, la = a.forward(toks, 0, 2)
    assert ok
    b = oracle.OracleModel(orc, cfg, t, 16)
    for i, tok in enumerate(toks):
        ok, lb = b.forward([tok], i, 1)
        assert ok and np.array_equal(bits(la[i]), bits(lb[0])), i
    assert np.array_equal(bits(a.keys), bits(b.keys))


def test_restated_forward_first_token_closed_form(orc, tmp_path):
    """At position 0 attention returns v exactly (softmax of one score is 1,
    so out = 0 + 1*v): one layer's first-token output reduces to
    x + O·q8(v) + FFN, computable from the oracle's separate pieces."""
    cfg = dict(TINY, layers=1)
    t = smoe.dense_tensors(cfg, seed=11, sigma=0.05)
    om = oracle.OracleModel(orc, cfg, t, 8)
    tok = 42
    dim, hidden = 128, 320
    x = orc.dequantize_row(t["embed"][3][tok], dim)
    okq, _, d, q = orc.row_work(x, 1, dim, norm=t["l.0.attn_norm"][3])
    nb = dim // 32
    v = orc.gemm(t["l.0.v"][3], nb * 36, d, q, 64, 1, nb) + t["l.0.v_bias"][3]
    # heads 0,1 read kv head 0; heads 2,3 read kv head 1 (head_dim 32)
    att = np.concatenate([v[:32], v[:32], v[32:], v[32:]]).astype(np.float32)
    _, ad, aq = orc.quantize_q8(att.reshape(1, -1))
    o = orc.gemm(t["l.0.o"][3], nb * 36, ad[0], aq[0], dim, 1, nb)
    x1 = (x + o).astype(np.float32)
    _, _, d2, q2 = orc.row_work(x1, 1, dim, norm=t["l.0.ffn_norm"][3])
    g = orc.gemm(t["l.0.e.0.gate"][3], nb * 36, d2, q2, hidden, 1, nb)
    u = orc.gemm(t["l.0.e.0.up"][3], nb * 36, d2, q2, hidden, 1, nb)
    _, _, hd_, hq = orc.row_work(u, 1, hidden, gate=g)
    nbh = hidden // 32
    dn = orc.gemm(t["l.0.e.0.down"][3], nbh * 36, hd_, hq, dim, 1, nbh)
    x2 = (x1 + dn).astype(np.float32)
    _, _, d3, q3 = orc.row_work(x2, 1, dim, norm=t["final_norm"][3])
    want = orc.gemm(t["lm_head"][3], nb * 36, d3, q3, 300, 1, nb)
    ok, got = om.forward([tok], 0, 1)
    assert ok and np.array_equal(bits(got[0]), bits(want))
