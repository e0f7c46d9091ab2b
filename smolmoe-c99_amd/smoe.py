"""SMOEQ8 checkpoint container and config text, in Python.

The reference's on-disk format (docs/FORMAT.md "Checkpoint container"; parsed
by src/modelfile.c:47-100): a 16-byte header (``SMOEQ8``, NUL, version byte,
u32 tensor count, u32 zero), then one 72-byte record per tensor (name[40],
rows, cols, dtype, alias/reserved, u64 offset, u64 byte count), sorted by
name, then the payloads. Version 2 allows ``lm_head`` to alias ``embed``'s
extent; version 3 adds opaque blobs (dtype 3) such as ``__config__``.

Used by the tests and the benchmark to build synthetic checkpoints that the
GPU forward (include/smq_model.h), the CPU oracle and the reference's own
loader all read.
"""
import struct

import numpy as np

from . import synth

MAGIC = b"SMOEQ8\0"
HEADER_BYTES, RECORD_BYTES, NAME_BYTES = 16, 72, 40
F32, Q8, Q5, BLOB = 0, 1, 2, 3

# src/config.c:63-68, in file order
CONFIG_KEYS = ("architecture", "dim", "hidden_dim", "layers", "heads", "kv_heads", "experts", "top_k", "vocab_size",
               "max_context", "shared_experts", "bos_id", "eos_id", "rms_eps", "rope_theta", "rotary_dim",
               "rope_attention_factor", "head_dim", "sliding_window", "rope_local_theta", "rope_llama3_factor",
               "rope_llama3_low_freq_factor", "rope_llama3_high_freq_factor", "rope_llama3_original_context")

# Qwen2.5-0.5B (config 4 of the benchmark): 24 layers, dim 896, GQA 14/2,
# head_dim 64, SwiGLU 4864, eps 1e-6, theta 1e6, vocab 151936, tied head.
QWEN05 = {"architecture": "smolmoe_qwen2", "dim": 896, "hidden_dim": 4864, "layers": 24, "heads": 14,
          "kv_heads": 2, "experts": 1, "top_k": 1, "vocab_size": 151936, "max_context": 32768,
          "shared_experts": 0, "bos_id": 256, "eos_id": 257, "rms_eps": "1e-06", "rope_theta": "1000000"}


def config_text(cfg):
    """key=value lines (src/config.c grammar) for a dict of config keys."""
    lines = []
    for k in CONFIG_KEYS:
        if k in cfg:
            lines.append(f"{k}={cfg[k]}")
    unknown = set(cfg) - set(CONFIG_KEYS)
    if unknown:
        raise KeyError(f"unknown config keys {sorted(unknown)}")
    return "\n".join(lines) + "\n"


def _payload_bytes(dtype, rows, cols):
    if dtype == F32:
        return rows * cols * 4
    nb = (cols + 31) // 32
    return rows * nb * (36 if dtype == Q8 else 22)


def write(path, tensors, version=1, config=None, tie_lm_head=False, align=32):
    """tensors: {name: (dtype, rows, cols, payload)}; payload is a numpy array
    (float32 for F32, uint8 rows for Q8/Q5). tie_lm_head writes lm_head as an
    alias of embed (needs version >= 2); config (text) embeds a __config__ blob
    (needs version 3)."""
    entries = dict(tensors)
    if config is not None:
        if version < 3:
            raise ValueError("an embedded config needs version 3")
        entries["__config__"] = (BLOB, 1, 1, np.frombuffer(config.encode(), np.uint8))
    if tie_lm_head:
        if version < 2:
            raise ValueError("a tied lm_head needs version >= 2")
        entries.pop("lm_head", None)
    names = sorted(list(entries) + (["lm_head"] if tie_lm_head else []))
    offset = HEADER_BYTES + RECORD_BYTES * len(names)
    records, payloads, placed = [], [], {}
    for name in names:
        if tie_lm_head and name == "lm_head":
            continue
        dtype, rows, cols, data = entries[name]
        raw = np.ascontiguousarray(data).tobytes()
        if dtype != BLOB and len(raw) != _payload_bytes(dtype, rows, cols):
            raise ValueError(f"{name}: {len(raw)} payload bytes for {rows}x{cols} dtype {dtype}")
        offset = (offset + align - 1) // align * align
        placed[name] = (offset, len(raw))
        payloads.append((offset, raw))
        offset += len(raw)
    for name in names:
        if tie_lm_head and name == "lm_head":
            dtype, rows, cols, _ = entries["embed"]
            off, nbytes = placed["embed"]
            alias = 1
        else:
            dtype, rows, cols, _ = entries[name]
            off, nbytes = placed[name]
            alias = 0
        enc = name.encode()
        if len(enc) >= NAME_BYTES:
            raise ValueError(f"tensor name too long: {name}")
        records.append(enc.ljust(NAME_BYTES, b"\0") + struct.pack("<IIIIQQ", rows, cols, dtype, alias, off, nbytes))
    with open(path, "wb") as f:
        f.write(MAGIC + bytes([version]) + struct.pack("<II", len(names), 0))
        for r in records:
            f.write(r)
        for off, raw in payloads:
            f.seek(off)
            f.write(raw)
    return path


def read(path):
    """-> (version, {name: (dtype, rows, cols, alias, numpy view)}); no
    validation beyond the header (the loaders under test do that)."""
    data = np.memmap(path, np.uint8, mode="r")
    if bytes(data[:7]) != MAGIC:
        raise ValueError("not a SMOEQ8 file")
    version = int(data[7])
    count = struct.unpack("<I", bytes(data[8:12]))[0]
    out = {}
    for i in range(count):
        rec = bytes(data[HEADER_BYTES + i * RECORD_BYTES:HEADER_BYTES + (i + 1) * RECORD_BYTES])
        name = rec[:NAME_BYTES].split(b"\0", 1)[0].decode()
        rows, cols, dtype, alias, off, nbytes = struct.unpack("<IIIIQQ", rec[NAME_BYTES:])
        view = data[off:off + nbytes]
        if dtype == F32:
            view = view.view(np.float32)
        out[name] = (dtype, rows, cols, alias, view)
    return version, out


def dense_tensors(cfg, seed=1, sigma=0.02, q5=(), norm_spread=0.1):
    """Seeded synthetic tensors for a one-expert checkpoint of config dict
    `cfg` (names and shapes of docs/FORMAT.md "Tensor names"): Q8 matrices
    (Q5 for names in `q5`) from N(0, sigma), norms 1 + N(0, norm_spread),
    Qwen2 biases N(0, sigma). Each tensor has its own seed stream."""
    dim, hidden, layers = int(cfg["dim"]), int(cfg["hidden_dim"]), int(cfg["layers"])
    heads, kv_heads, vocab = int(cfg["heads"]), int(cfg["kv_heads"]), int(cfg["vocab_size"])
    hd = int(cfg.get("head_dim", dim // heads))
    qd, kd = heads * hd, kv_heads * hd
    experts = int(cfg.get("experts", 1))
    t = {}
    counter = [seed * 1000003]

    def mat(name, rows, cols):
        counter[0] += 1
        if name in q5:
            t[name] = (Q5, rows, cols, synth.q5_weights(counter[0], rows, cols, sigma))
        else:
            t[name] = (Q8, rows, cols, synth.q8_weights(counter[0], rows, cols, sigma))

    def vec(name, n, base, spread):
        counter[0] += 1
        t[name] = (F32, 1, n, (base + synth.normal(counter[0], n, spread)).astype(np.float32))

    mat("embed", vocab, dim)
    mat("lm_head", vocab, dim)
    vec("final_norm", dim, 1.0, norm_spread)
    for layer in range(layers):
        p = f"l.{layer}."
        vec(p + "attn_norm", dim, 1.0, norm_spread)
        vec(p + "ffn_norm", dim, 1.0, norm_spread)
        mat(p + "q", qd, dim)
        mat(p + "k", kd, dim)
        mat(p + "v", kd, dim)
        mat(p + "o", dim, qd)
        mat(p + "router", experts, dim)
        if cfg.get("architecture") == "smolmoe_qwen2":
            vec(p + "q_bias", qd, 0.0, sigma)
            vec(p + "k_bias", kd, 0.0, sigma)
            vec(p + "v_bias", kd, 0.0, sigma)
        mat(p + "e.0.gate", hidden, dim)
        mat(p + "e.0.up", hidden, dim)
        mat(p + "e.0.down", dim, hidden)
    return t
