"""Seeded input generators shared by the tests.

``lcg_stream`` and ``bf16_patterns`` restate the generator that produced the
reference's Q8 goldens (tests/convert-quant.test.ts:28-49 in the reference):
an LCG x = x*1664525 + 1013904223 (mod 2^32) feeding six kinds of finite
bf16 patterns, one kind per row (row % 6). ``lcg_uniform`` restates the unit
tests' generator (tests/test_kernels.c:28-35): next = x >> 8, scaled by 2^-24.
"""
import numpy as np

A, C, M = 1664525, 1013904223, 1 << 32


def lcg_stream(seed, count):
    """The next `count` LCG states after `seed` (uint64 array, each < 2^32)."""
    out = np.empty(count, np.uint64)
    k = 1024
    first = np.empty(k, np.uint64)
    x = seed & 0xFFFFFFFF
    for i in range(k):
        x = (x * A + C) % M
        first[i] = x
    # leapfrog: x_{n+k} = Ak x_n + Ck (mod 2^32)
    ak, ck = 1, 0
    for _ in range(k):
        ak, ck = (ak * A) % M, (ck * A + C) % M
    cur = first.copy()
    pos = 0
    ak64, ck64, mask = np.uint64(ak), np.uint64(ck), np.uint64(0xFFFFFFFF)
    while pos < count:
        n = min(k, count - pos)
        out[pos:pos + n] = cur[:n]
        pos += n
        # 64-bit products of 32-bit values can overflow uint64 only above 2^64: split ak.
        lo, hi = ak64 & np.uint64(0xFFFF), ak64 >> np.uint64(16)
        cur = ((cur * lo) + (((cur * hi) & mask) << np.uint64(16)) + ck64) & mask
    return out


class _Stream:
    def __init__(self, seed):
        self.seed = seed & 0xFFFFFFFF
        self.buf = np.empty(0, np.uint64)
        self.pos = 0

    def take(self, n):
        if self.pos + n > self.buf.shape[0]:
            more = max(n, 1 << 16)
            start = int(self.buf[-1]) if self.buf.shape[0] else self.seed
            self.buf = np.concatenate([self.buf[self.pos:], lcg_stream(start, more)])
            self.pos = 0
        v = self.buf[self.pos:self.pos + n]
        self.pos += n
        return v.astype(np.uint64)

    def peek(self, n):
        v = self.take(n)
        self.pos -= n
        return v


def bf16_patterns(rows, cols, seed):
    """uint16 bf16 bit patterns, rows x cols, as the reference's golden generator."""
    s = _Stream(seed)
    out = np.empty((rows, cols), np.uint16)
    j = np.arange(cols)
    for r in range(rows):
        mode = r % 6
        if mode == 0:  # any finite pattern: reject exponent 0xff
            need = cols
            acc = []
            while need:
                cand = s.peek(max(2 * need, 64))
                u = cand & np.uint64(0xFFFF)
                ok = ((u >> np.uint64(7)) & np.uint64(0xFF)) != 0xFF
                idx = np.nonzero(ok)[0]
                if idx.shape[0] >= need:
                    last = idx[need - 1]
                    acc.append(u[idx[:need]])
                    s.take(int(last) + 1)
                    need = 0
                else:
                    acc.append(u[idx])
                    s.take(cand.shape[0])
                    need -= idx.shape[0]
            out[r] = np.concatenate(acc).astype(np.uint16)
        elif mode in (1, 5):  # exp draw, sign draw, mantissa draw per element
            v = s.take(3 * cols).reshape(cols, 3)
            if mode == 1:
                e = np.uint64(0x78) + v[:, 0] % np.uint64(6)
            else:
                e = np.uint64(0xF0) + v[:, 0] % np.uint64(0xE)
            out[r] = (((v[:, 1] & np.uint64(1)) << np.uint64(15)) | (e << np.uint64(7)) |
                      (v[:, 2] & np.uint64(0x7F))).astype(np.uint16)
        elif mode == 2:  # sign, tiny exponent (0..2), mantissa
            v = s.take(3 * cols).reshape(cols, 3)
            out[r] = (((v[:, 0] & np.uint64(1)) << np.uint64(15)) | ((v[:, 1] % np.uint64(3)) << np.uint64(7)) |
                      (v[:, 2] & np.uint64(0x7F))).astype(np.uint16)
        elif mode == 3:  # 127.0 at each block start, else exact .5 ties
            drawn = j % 32 != 0
            v = s.take(int(drawn.sum()))
            ties = ((v % np.uint64(254)).astype(np.int64) - 127).astype(np.float32) + np.float32(0.5)
            row = np.full(cols, 0x42FE, np.uint16)
            row[drawn] = (ties.view(np.uint32) >> 16).astype(np.uint16)
            out[r] = row
        else:  # signed zeros
            v = s.take(cols)
            out[r] = np.where((v & np.uint64(1)) != 0, 0x8000, 0).astype(np.uint16)
    return out


def bf16_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


class LcgUniform:
    """tests/test_kernels.c:28-35: x = x*1664525 + 1013904223; next = x >> 8."""

    def __init__(self, seed=12345):
        self.s = _Stream(seed)

    def next(self, n):
        return (self.s.take(n) >> np.uint64(8)).astype(np.uint64)

    def uniform(self, lo, hi, n):
        u = self.next(n).astype(np.float32)
        lo, hi = np.float32(lo), np.float32(hi)
        return (lo + (hi - lo) * u / np.float32(16777216.0)).astype(np.float32)
