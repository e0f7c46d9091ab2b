"""GPU parity of the whole forward pass (include/smq_model.h): synthetic
checkpoints run through the C host forward on the gfx950 path must give the
restated oracle's logits, KV cache and greedy tokens bit for bit (the oracle
itself is pinned to the reference's model_forward in test_forward_oracle.py)."""
import numpy as np
import pytest

import oracle
from checks import assert_same_f32, say
from smq_pkg import smodel, smoe, smq
from test_forward_oracle import Q5_NAMES, TINY, VARIANTS, checkpoint, prompt

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert smq.init(0) == "gfx950"
    smq.kernels_set_fast(False)
    smq.kernels_select()
    smq.set_prefill_mfma(False)
    yield


@pytest.mark.parametrize("name", sorted(VARIANTS))
def test_forward_matches_oracle(orc, tmp_path, name):
    say("forward", name)
    cfg, t, path, _ = checkpoint(tmp_path, name)
    context, n = 48, 13
    m = smodel.Model(path, context=context, batch=8, logit_rows=8)
    om = oracle.OracleModel(orc, cfg, t, context)
    toks = prompt(n, int(cfg["vocab_size"]))
    m.forward(toks[:8], 0, smodel.LOGITS_ALL)
    ok, want = om.forward(toks[:8], 0, 2)
    assert ok
    assert_same_f32(m.logits(8), want, "prompt logits")
    m.forward(toks[8:], 8, smodel.LOGITS_LAST)
    ok, want = om.forward(toks[8:], 8, 1)
    assert_same_f32(m.logits(1), want, "last logits")
    for layer in range(int(cfg["layers"])):
        assert_same_f32(m.kv(layer, False, n), om.keys[layer, :n], f"keys {layer}")
        assert_same_f32(m.kv(layer, True, n), om.values[layer, :n], f"values {layer}")
    banned = np.zeros(om.vocab, np.uint8)
    banned[256] = 1
    m.set_banned(banned)
    say("generate", name)
    got = m.generate(n, 12)
    want = om.generate(n, 12, banned)
    assert got.tolist() == want.tolist()
    # the decode steps also left the same cache behind
    for layer in range(int(cfg["layers"])):
        assert_same_f32(m.kv(layer, False, n + 11), om.keys[layer, :n + 11], f"keys after decode {layer}")
    m.close()


def test_prefill_chunks_and_config_file(orc, tmp_path):
    """model_prefill in batch-sized chunks (batch 3), config from a file, a
    version-1 container with a separate lm_head."""
    say("prefill chunks")
    cfg, t, path, cpath = checkpoint(tmp_path, "qwen2", version=1, tie=False)
    toks = prompt(13, int(cfg["vocab_size"]), seed=21)
    m = smodel.Model(path, config_path=cpath, context=32, batch=3, logit_rows=1)
    m.prefill(toks, 0, True)
    om = oracle.OracleModel(orc, cfg, t, 32)
    ok, want = om.forward(toks, 0, 1)
    assert ok
    assert_same_f32(m.logits(1), want, "prefill logits")
    m.close()


def test_generate_twice_reuses_the_captured_step(orc, tmp_path):
    cfg, t, path, _ = checkpoint(tmp_path, "v1_partial_rotary")
    say("generate twice")
    m = smodel.Model(path, context=40, batch=8, logit_rows=1)
    om = oracle.OracleModel(orc, cfg, t, 40)
    toks = prompt(5, int(cfg["vocab_size"]), seed=2)
    m.forward(toks, 0, smodel.LOGITS_LAST)
    om.forward(toks, 0, 1)
    a = m.generate(5, 6)
    assert a.tolist() == om.generate(5, 6).tolist()
    # continue from where the first run stopped: feed its last token
    m.forward([int(a[-1])], 10, smodel.LOGITS_LAST)
    om.forward([int(a[-1])], 10, 1)
    b = m.generate(11, 4)
    assert b.tolist() == om.generate(11, 4).tolist()
    m.close()


def test_forward_errors(tmp_path):
    cfg, t, path, _ = checkpoint(tmp_path, "qwen2")
    m = smodel.Model(path, context=16, batch=4, logit_rows=1)
    with pytest.raises(smq.SmqError) as e:
        m.forward([1, 300], 0)  # vocab is 300
    assert e.value.status == smq.SM_ERR_RANGE and "out of vocabulary" in str(e.value)
    with pytest.raises(smq.SmqError) as e:
        m.forward([1, 2, 3], 14)  # past the context
    assert e.value.status == smq.SM_ERR_RANGE
    with pytest.raises(smq.SmqError) as e:
        m.forward([1] * 5, 0)  # more than the batch
    assert e.value.status == smq.SM_ERR_RANGE
    with pytest.raises(smq.SmqError):
        m.generate(10, 8)  # 10 + 7 decode positions > 16
    m.close()


@pytest.mark.parametrize("change", [dict(experts=2, top_k=1), dict(shared_experts=1),
                                    dict(architecture="smolmoe_gemma3")])
def test_unsupported_architectures_are_refused(tmp_path, change):
    cfg = dict(TINY, **change)
    path = str(tmp_path / "x.smoe")
    t = smoe.dense_tensors(dict(cfg, experts=1), seed=3)
    smoe.write(path, t, version=3, config=smoe.config_text(cfg), tie_lm_head=True)
    with pytest.raises(smq.SmqError) as e:
        smodel.Model(path, context=8, batch=2)
    assert e.value.status == smq.SM_ERR_FORMAT
