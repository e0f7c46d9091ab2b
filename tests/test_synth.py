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


def _mix(z):
    m = (1 << 64) - 1
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
    return z ^ (z >> 31)


def _name_seed(seed, name):
    h = 1469598103934665603  # FNV-1a over the tensor name
    for ch in name.encode():
        h = ((h ^ ch) * 1099511628211) & ((1 << 64) - 1)
    return _mix(seed ^ h)


def _draws(s, n, sigma32):
    """f32(N(0,1) * double(sigma)) of stream s, Box-Muller in double with libm (math) as the C writer."""
    import math
    gold, m = 0x9E3779B97F4A7C15, (1 << 64) - 1
    out = np.empty(n, np.float32)
    sig = float(np.float32(sigma32))
    for e in range(n):
        p = e // 2
        u1 = 1.0 - (_mix((s + (2 * p + 1) * gold) & m) >> 11) * (1.0 / 9007199254740992.0)
        u2 = (_mix((s + (2 * p + 2) * gold) & m) >> 11) * (1.0 / 9007199254740992.0)
        r, a = math.sqrt(-2.0 * math.log(u1)), 2.0 * 3.14159265358979323846 * u2
        out[e] = np.float32((r * math.sin(a) if e & 1 else r * math.cos(a)) * sig)
    return out


def test_checkpoint_writer_follows_the_q8_rule(orc, tmp_path):
    """smq_synth_checkpoint (host C) against the q8pack rule (tools/q8pack.c:38-44, via the oracle pinned to
    the reference's SHA-256 goldens): every quantized tensor is the rule applied to the writer's documented
    draws, norm weights are 1, Qwen2 biases are the draws themselves, lm_head aliases embed."""
    from smq_pkg import smoe, smodel
    cfg = {"architecture": "smolmoe_qwen2", "dim": 64, "hidden_dim": 96, "layers": 1, "heads": 2, "kv_heads": 1,
           "experts": 1, "top_k": 1, "vocab_size": 300, "max_context": 64, "shared_experts": 0, "bos_id": 256,
           "eos_id": 257, "rms_eps": "1e-06", "rope_theta": "10000"}
    path = str(tmp_path / "w.smoe")
    seed, sigma = 77, 0.05
    smodel.synth_checkpoint(path, smoe.config_text(cfg), seed=seed, sigma=sigma, tied=True, threads=3)
    version, t = smoe.read(path)
    assert version == 3 and t["lm_head"][3] == 1
    checked = 0
    for name, (dtype, rows, cols, alias, view) in t.items():
        if alias or dtype == smoe.BLOB:
            continue
        if dtype == smoe.Q8:
            x = _draws(_name_seed(seed, name), rows * cols, sigma).reshape(rows, cols)
            assert np.array_equal(np.asarray(view), orc.q8_weight_rows(x)), name
        elif name.endswith("_norm"):
            assert np.all(np.asarray(view) == 1.0), name
        else:
            assert np.array_equal(np.asarray(view), _draws(_name_seed(seed, name), rows * cols, sigma)), name
        checked += 1
    assert checked >= 12
