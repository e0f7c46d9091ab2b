"""Seeded synthetic inputs and the offline weight rules, in numpy.

Generator: splitmix64 streams (one per seed) turned into N(0, sigma) by
Box-Muller in float64, rounded once to float32. CPU and GPU consume the same
host arrays, so the generator choice cannot affect parity.

Weight packers (the converters' rules, run on the host before upload):
  * ``q8_pack``: tools/q8pack.c:38-44 — scale = f32(max|v| / 127),
    q = clamp(nearbyint(double(v) / double(scale)), -127, 127), 0 for a zero
    scale, zero padding; 36-byte blocks.
  * ``q5_pack``: src/kernels.c:1064-1117 — signed extreme (first largest |v|),
    21 candidates f16(extreme / -(14.5 + 0.1k)), squared error in double
    summed in element order, first minimum wins; 22-byte blocks.
"""
import numpy as np

QK = 32
_GOLD = np.uint64(0x9E3779B97F4A7C15)


def splitmix64(seed, n, start=0):
    """Outputs start..start+n-1 of the splitmix64 stream seeded with `seed`."""
    i = np.arange(start + 1, start + n + 1, dtype=np.uint64)
    with np.errstate(over="ignore"):
        z = np.uint64(seed) + i * _GOLD
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return z ^ (z >> np.uint64(31))


def normal(seed, n, sigma=1.0, start=0):
    """n float32 draws of N(0, sigma^2): pairs of uniforms -> Box-Muller."""
    pairs = (n + 1) // 2
    z = splitmix64(seed, 2 * pairs, 2 * start)
    u = (z >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    out = np.empty(2 * pairs, np.float64)
    out[0::2] = r * np.cos(2.0 * np.pi * u2)
    out[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (out[:n] * sigma).astype(np.float32)


def _blocks(x):
    rows, cols = x.shape
    nb = (cols + QK - 1) // QK
    pad = np.zeros((rows, nb * QK), np.float32)
    pad[:, :cols] = x
    return pad.reshape(rows, nb, QK), nb


def q8_pack(x):
    """float32 [rows, cols] -> uint8 [rows, nb*36] (tools/q8pack.c:38-44)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    blk, nb = _blocks(x)
    high = np.abs(blk).max(axis=2)
    scale = (high / np.float32(127.0)).astype(np.float32)
    safe = np.where(scale != 0, scale, np.float32(1)).astype(np.float64)
    q = np.rint(blk.astype(np.float64) / safe[:, :, None])
    q = np.where(scale[:, :, None] != 0, q, 0)
    q = np.clip(q, -127, 127).astype(np.int8)
    out = np.zeros((rows, nb, 36), np.uint8)
    out[:, :, :4] = scale.view(np.uint8).reshape(rows, nb, 4)
    out[:, :, 4:] = q.view(np.uint8)
    return out.reshape(rows, nb * 36)


def _q5_level(x, inv):
    return np.clip(np.rint((x * inv).astype(np.float32)), -16, 15)


def q5_pack(x):
    """float32 [rows, cols] -> uint8 [rows, nb*22] (src/kernels.c:1083-1117)."""
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.shape
    blk, nb = _blocks(x)
    flat = blk.reshape(-1, QK)
    nblk = flat.shape[0]
    idx = np.argmax(np.abs(flat), axis=1)  # first largest |x|
    ext = flat[np.arange(nblk), idx]
    best_err = np.full(nblk, np.inf)
    best_h = np.zeros(nblk, np.uint16)
    best_d = np.zeros(nblk, np.float32)
    xd64 = flat.astype(np.float64)
    for k in range(21):
        div = -(np.float32(14.5) + np.float32(0.1) * np.float32(k))
        with np.errstate(over="ignore", divide="ignore", invalid="ignore"):
            h = (ext / div).astype(np.float32).astype(np.float16)
            d = h.astype(np.float32)
            ok = (d != 0) & np.isfinite(d) & (ext != 0)
            inv = np.where(ok, np.float32(1.0) / np.where(ok, d, np.float32(1)), np.float32(0)).astype(np.float32)
        lv = _q5_level(flat, inv[:, None]).astype(np.float64)
        e = xd64 - lv * d.astype(np.float64)[:, None]
        err = np.zeros(nblk)
        for j in range(QK):  # sequential sum, element order
            err = err + e[:, j] * e[:, j]
        better = ok & (err < best_err)
        best_err = np.where(better, err, best_err)
        best_h = np.where(better, h.view(np.uint16), best_h)
        best_d = np.where(better, d, best_d)
    with np.errstate(divide="ignore"):
        inv = np.where(best_d != 0, np.float32(1.0) / np.where(best_d != 0, best_d, 1), 0).astype(np.float32)
    lv = np.where(best_d[:, None] != 0, _q5_level(flat, inv[:, None]), 0).astype(np.int64)
    # padding of a partial last block quantizes to 0 (code 16)
    valid = np.ones((rows, nb, QK), bool)
    valid.reshape(rows, nb * QK)[:, cols:] = False
    lv = np.where(valid.reshape(-1, QK), lv, 0)
    u = (lv + 16).astype(np.uint32)
    high = ((u >> 4) & 1) << np.arange(QK, dtype=np.uint32)
    high = np.bitwise_or.reduce(high, axis=1).astype(np.uint32)
    nib = ((u[:, :16] & 15) | ((u[:, 16:] & 15) << 4)).astype(np.uint8)
    out = np.zeros((nblk, 22), np.uint8)
    out[:, 0:2] = best_h.astype(np.uint16).view(np.uint8).reshape(nblk, 2)
    out[:, 2:6] = high.view(np.uint8).reshape(nblk, 4)
    out[:, 6:] = nib
    return out.reshape(rows, nb * 22)


def q8_weights(seed, rows, cols, sigma=0.02):
    """Seeded N(0, sigma) weights packed to Q8 (rows x nb*36 bytes)."""
    return q8_pack(normal(seed, rows * cols, sigma).reshape(rows, cols))


def q5_weights(seed, rows, cols, sigma=0.02):
    return q5_pack(normal(seed, rows * cols, sigma).reshape(rows, cols))


def activations(seed, ntok, cols, sigma=1.0):
    return normal(seed, ntok * cols, sigma).reshape(ntok, cols)
