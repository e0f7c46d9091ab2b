"""BASELINE configs[4] at its real shape on the GPU: a random-init
Qwen2.5-0.5B checkpoint (24 layers, dim 896, SwiGLU 4864, GQA 14/2, head_dim
64, vocab 151936, tied embeddings, Q8), a 512-token prefill in one batch, then
greedy decode steps, against the reference's own model layer (src/model.c
model_forward, src/sampler.c:57-63, compiled from its sources into
oracle/_ref) on the same file. Compared bit for bit: the prompt's last logits,
the KV cache of every layer, teacher-forced logits at eight further positions,
and the greedy tokens of the decode loop (HIP-graph replays) with the caches
they leave behind: 128 steps after the teacher-forced positions (to position
647, past the 640 value rows the decode attention takes in one pass), and
BASELINE's own sequence, a fresh 512-token prefill and then 128 greedy steps
(src/main.c:571-600, src/sampler.c:57-63), whose decode step is captured again
after that prefill."""
import os

import numpy as np
import pytest

import oracle
from checks import assert_same_f32, say
from smq_pkg import smodel, smoe, smq

pytestmark = pytest.mark.gpu

PROMPT, EXTRA, DECODE, CONTEXT = 512, 8, 128, 1024


@pytest.fixture(scope="module")
def qwen05(tmp_path_factory):
    if not oracle.ReferenceModel.available():
        pytest.skip("needs the reference's model layer (make -C oracle ref: oracle/_ref/libsmref_model.so)")
    assert smq.init(0) == "gfx950"
    smq.kernels_set_fast(False)
    smq.kernels_select()
    smq.set_prefill_mfma(False)
    path = str(tmp_path_factory.mktemp("qwen05") / "qwen05.smoe")
    threads = min(16, len(os.sched_getaffinity(0)))
    say("qwen05: writing checkpoint")
    smodel.synth_checkpoint(path, smoe.config_text(smoe.QWEN05), seed=4000, sigma=0.02, tied=True, threads=threads)
    say("qwen05: opening the reference model")
    ref = oracle.ReferenceModel(path, context=CONTEXT, batch=PROMPT, logit_rows=EXTRA, threads=threads)
    say("qwen05: opening the GPU model")
    m = smodel.Model(path, context=CONTEXT, batch=PROMPT, logit_rows=EXTRA)
    yield m, ref
    m.close()
    ref.close()
    os.remove(path)


def test_qwen05_prefill_decode_bit_exact(qwen05):
    m, ref = qwen05
    vocab, layers, kv_dim = 151936, 24, 128
    rng = np.random.default_rng(3000)
    prompt = rng.integers(0, vocab, PROMPT).astype(np.uint32)
    banned = np.zeros(vocab, np.uint8)
    banned[256] = 1  # BOS (docs/FORMAT.md:81-82)
    m.set_banned(banned)
    ref.set_banned(banned)

    say("qwen05: prefill 512")
    m.forward(prompt, 0, smodel.LOGITS_LAST)
    ref.prefill(prompt, 0, True)
    assert_same_f32(m.logits(1), ref.logits(1), "prompt logits")
    for layer in range(layers):
        assert_same_f32(m.kv(layer, False, PROMPT), ref.kv(layer, False, PROMPT, kv_dim), f"keys {layer}")
        assert_same_f32(m.kv(layer, True, PROMPT), ref.kv(layer, True, PROMPT, kv_dim), f"values {layer}")

    say("qwen05: teacher-forced logits at 8 positions")
    extra = rng.integers(0, vocab, EXTRA).astype(np.uint32)
    m.forward(extra, PROMPT, smodel.LOGITS_ALL)
    assert ref.forward(extra, PROMPT, smodel.LOGITS_ALL) == 0
    assert_same_f32(m.logits(EXTRA), ref.logits(EXTRA), "teacher-forced logits")

    say(f"qwen05: {DECODE} greedy decode steps")
    pos = PROMPT + EXTRA
    # both continue from the last row of the teacher-forced batch: re-run that token with LOGITS_LAST
    m.forward(extra[-1:], pos - 1, smodel.LOGITS_LAST)
    assert ref.forward(extra[-1:], pos - 1, smodel.LOGITS_LAST) == 0
    got = m.generate(pos, DECODE)
    want = ref.generate(pos, DECODE)
    assert got.tolist() == want.tolist()
    n = pos + DECODE - 1
    for layer in range(layers):
        assert_same_f32(m.kv(layer, False, n), ref.kv(layer, False, n, kv_dim), f"keys after decode {layer}")
        assert_same_f32(m.kv(layer, True, n), ref.kv(layer, True, n, kv_dim), f"values after decode {layer}")


def test_qwen05_baseline_sequence_bit_exact(qwen05):
    """configs[4] as BASELINE states it: prefill 512 random ids, then 128 greedy decode steps from
    position 512; tokens and every layer's caches (positions 0..638) against the reference."""
    m, ref = qwen05
    vocab, layers, kv_dim = 151936, 24, 128
    prompt = np.random.default_rng(3001).integers(0, vocab, PROMPT).astype(np.uint32)
    banned = np.zeros(vocab, np.uint8)
    banned[256] = 1
    m.set_banned(banned)
    ref.set_banned(banned)
    say("qwen05 baseline: prefill 512")
    m.forward(prompt, 0, smodel.LOGITS_LAST)
    ref.prefill(prompt, 0, True)
    assert_same_f32(m.logits(1), ref.logits(1), "prompt logits")
    say("qwen05 baseline: 128 greedy decode steps")
    got = m.generate(PROMPT, 128)
    want = ref.generate(PROMPT, 128)
    assert got.tolist() == want.tolist()
    n = PROMPT + 128 - 1
    for layer in range(layers):
        assert_same_f32(m.kv(layer, False, n), ref.kv(layer, False, n, kv_dim), f"keys {layer}")
        assert_same_f32(m.kv(layer, True, n), ref.kv(layer, True, n, kv_dim), f"values {layer}")
