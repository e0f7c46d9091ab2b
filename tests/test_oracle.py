"""Pins the CPU oracle (oracle/smq_oracle.c) before anything is checked
against it: known answers from the reference's own tests and goldens, library
routines (numpy's IEEE half conversion), closed forms, exact-integer brute
force, and the reference's kernels compiled from its sources (oracle/_ref)."""
import hashlib
import json
import os
import struct

import numpy as np
import pytest

from patterns import LcgUniform, bf16_patterns, bf16_to_f32

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
Q8B, Q5B = 36, 22


def f32_bits(x):
    return np.asarray(x, np.float32).view(np.uint32)


# ---------------------------------------------------------------- binary16

def test_f16_to_f32_matches_numpy_all_halves(orc):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([orc.f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(f32_bits(got[~nan]), f32_bits(want[~nan]))


def test_f16_round_trip_and_constants(orc):
    # tests/test_kernels.c:51-61 and tests/convert-quant.test.ts:117-132
    for h in range(0, 65536, 7):
        f = orc.f16_to_f32(h)
        if f != f:
            continue
        assert orc.f32_to_f16(f) == h
    cases = [(1.0, 0x3C00), (-2.0, 0xC000), (65504.0, 0x7BFF), (65520.0, 0x7C00), (1e-8, 0x0000),
             (5.960464477539063e-8, 0x0001), (1 + 2 ** -11, 0x3C00), (1 + 3 * 2 ** -11, 0x3C02),
             (float("inf"), 0x7C00), (-0.0, 0x8000)]
    for x, h in cases:
        assert orc.f32_to_f16(x) == h, (x, hex(h))


def test_f32_to_f16_matches_numpy_random(orc):
    rng = np.random.default_rng(5)
    bits = rng.integers(0, 2 ** 32, 20000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    # concentrate on the half range, subnormals and rounding ties too
    extra = (rng.standard_normal(20000) * np.exp2(rng.integers(-26, 17, 20000))).astype(np.float32)
    ties = (np.arange(-3000, 3000) * 2.0 ** -11 + 2.0 ** -12).astype(np.float32)
    for arr in (x, extra, ties):
        want = arr.astype(np.float16).view(np.uint16)
        got = np.array([orc.f32_to_f16(float(v)) for v in arr], np.uint16)
        assert np.array_equal(got, want)


# ---------------------------------------------------------------- quantize_q8

def numpy_quantize_q8(x):
    """Vectorised restatement used only to cross-check the C oracle."""
    n = x.shape[0]
    nb = (n + 31) // 32
    pad = np.zeros(nb * 32, np.float32)
    pad[:n] = x
    blocks = pad.reshape(nb, 32)
    amax = np.abs(blocks).max(axis=1)
    scale = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(scale >= np.finfo(np.float32).tiny, np.float32(1.0) / np.where(scale > 0, scale, 1),
                   0).astype(np.float32)
    q = np.rint((blocks * inv[:, None]).astype(np.float32))
    q = np.clip(q, -127, 127).astype(np.int8).reshape(-1)
    q[n:] = 0
    return scale, q


def test_quantize_properties(orc):
    # tests/test_kernels.c:89-107
    g = LcgUniform()
    x = g.uniform(-3.0, 3.0, 100)
    s, d, q = orc.quantize_q8(x)
    d, q = d[0], q[0]
    assert s == 0
    back = d[np.arange(100) // 32] * q[:100].astype(np.float32)
    assert np.all(np.abs(back - x) <= d[np.arange(100) // 32] * 0.5 + 1e-6)
    assert np.all(np.abs(q) <= 127)
    assert np.all(q[100:] == 0)
    s, d, q = orc.quantize_q8(np.zeros(32, np.float32))
    assert s == 0 and d[0, 0] == 0 and np.all(q == 0)
    for bad in (np.inf, -np.inf, np.nan):
        z = np.zeros(32, np.float32)
        z[3] = bad
        assert orc.quantize_q8(z)[0] == -1


@pytest.mark.parametrize("spread", [50.0, 1e-30, 1e30, 1e-37, 1e-39, 3.0])
def test_quantize_matches_numpy(orc, spread):
    g = LcgUniform(77)
    for n in (1, 31, 32, 33, 100, 896, 4864 + 7):
        x = g.uniform(-spread, spread, n)
        x[::33] = 0.0
        s, d, q = orc.quantize_q8(x)
        wd, wq = numpy_quantize_q8(x)
        assert s == 0
        assert np.array_equal(f32_bits(d[0]), f32_bits(wd))
        assert np.array_equal(q[0], wq)


def test_quantize_matches_reference(orc, ref):
    g = LcgUniform(9)
    for trial in range(200):
        n = 1 + int(g.next(1)[0] % (64 * 32 + 7))
        spread = [1e-30, 1e30, 1e-37, 1e-39, 50.0, 7.0][trial % 6]
        x = g.uniform(-spread, spread, n)
        s, d, q = orc.quantize_q8(x)
        for avx2 in (False, True):
            rs, rd, rq = ref.quantize_q8(x, avx2=avx2)
            assert rs == s
            assert np.array_equal(f32_bits(d[0]), f32_bits(rd)) and np.array_equal(q[0], rq)
    for at in (0, 7, 31, 40, 66):  # tests/test_kernels.c:400-410
        x = np.ones(67, np.float32)
        x[at] = np.nan if at % 2 else np.inf
        assert orc.quantize_q8(x)[0] == -1 and ref.quantize_q8(x)[0] == -1


# ---------------------------------------------------------------- dot contract

def random_q8_weights(g, nb, extremes=False):
    """tests/test_kernels.c:37-49: scales U(0, 0.05), q uniform in [-127, 127]
    (plus -128/127 at every 7th lane when extremes)."""
    w = np.zeros((nb, Q8B), np.uint8)
    scales = g.uniform(0.0, 0.05, nb)
    q = (g.next(nb * 32) % np.uint64(255)).astype(np.int64) - 127
    q = q.reshape(nb, 32)
    if extremes:
        j = np.arange(32)
        q[:, j % 7 == 0] = np.where(j[j % 7 == 0] % 2 == 1, -128, 127)
    w[:, :4] = scales.view(np.uint8).reshape(nb, 4)
    w[:, 4:] = q.astype(np.int8).view(np.uint8)
    return w.reshape(-1)


def exact_dot(w, xd, xq, nb, q5, orc):
    """float64 value of sum_b wscale*xscale*sum_j wq*xq, and the exact integer lanes."""
    tot = 0.0
    lanes = []
    for b in range(nb):
        if q5:
            blk = w[b * Q5B:(b + 1) * Q5B]
            ws = np.frombuffer(blk[:2].tobytes(), np.float16)[0].astype(np.float64)
            wq = unpack_q5_numpy(blk)
        else:
            blk = w[b * Q8B:(b + 1) * Q8B]
            ws = float(np.frombuffer(blk[:4].tobytes(), np.float32)[0])
            wq = blk[4:].view(np.int8).astype(np.int64)
        prods = wq * xq[b * 32:(b + 1) * 32].astype(np.int64)
        lanes.append(prods.reshape(8, 4).sum(axis=1))
        tot += ws * float(xd[b]) * float(prods.sum())
    return tot, np.array(lanes)


def unpack_q5_numpy(blk):
    high = int.from_bytes(blk[2:6].tobytes(), "little")
    nib = blk[6:22]
    lo = np.concatenate([nib & 15, nib >> 4]).astype(np.int64)
    hi = np.array([(high >> j) & 1 for j in range(32)], np.int64)
    return (lo | (hi << 4)) - 16


def test_dot_closed_form(orc):
    # tests/test_kernels.c:109-127
    g = LcgUniform(12345)
    for nb in range(1, 65):
        w = random_q8_weights(g, nb)
        x = g.uniform(-2.0, 2.0, nb * 32)
        _, xd, xq = orc.quantize_q8(x)
        exact, _ = exact_dot(w, xd[0], xq[0], nb, False, orc)
        got = orc.dot(w, xd[0], xq[0], nb)
        assert abs(got - exact) <= 1e-4 * (1 + abs(exact)), nb


def test_dot_lane_order_by_hand(orc):
    """Builds the dot from exact integer lanes with numpy float32 scalars in
    the contract's order; a dropped lane, a swapped reduction pair or a fused
    multiply-add fails this on random data."""
    g = LcgUniform(3)
    for nb in (1, 2, 5, 28):
        w = random_q8_weights(g, nb, extremes=True)
        x = g.uniform(-20, 20, nb * 32)
        _, xd, xq = orc.quantize_q8(x)
        _, lanes = exact_dot(w, xd[0], xq[0], nb, False, orc)
        acc = [np.float32(0)] * 8
        for b in range(nb):
            ws = np.frombuffer(w[b * Q8B:b * Q8B + 4].tobytes(), np.float32)[0]
            d = np.float32(ws * xd[0][b])
            for l in range(8):
                acc[l] = np.float32(acc[l] + np.float32(d * np.float32(lanes[b][l])))
        want = np.float32(np.float32(np.float32(acc[0] + acc[4]) + np.float32(acc[2] + acc[6])) +
                          np.float32(np.float32(acc[1] + acc[5]) + np.float32(acc[3] + acc[7])))
        assert f32_bits(orc.dot(w, xd[0], xq[0], nb)) == f32_bits(want)


def fma_probe_inputs():
    # tests/test_kernels.c:223-249, 531-550
    w = np.zeros(2 * Q8B, np.uint8)
    w[0:4] = np.array([1.0], np.float32).view(np.uint8)
    w[Q8B:Q8B + 4] = np.array([1.0 + 1.0 / 4096], np.float32).view(np.uint8)
    w[4], w[5] = 127, 17
    w[Q8B + 4], w[Q8B + 5] = 127, 1
    xq = np.zeros(64, np.int8)
    xq[0], xq[1], xq[32], xq[33] = -32, -2, 32, 33
    xd = np.ones(2, np.float32)
    return w, xd, xq


def test_fma_probe(orc):
    w, xd, xq = fma_probe_inputs()
    assert orc.dot(w, xd, xq, 2) == 0.0
    assert orc.dot(w, xd, xq, 2, fast=True) == 2.0 ** -12


def test_backend_edges(orc):
    """tests/test_kernels.c:251-278: Q5 high planes all / none / alternating,
    Q8 weights -128/127 against activations of -127 — checked against exact
    integer lanes in float64."""
    high = [0xFFFFFFFF, 0, 0xAAAAAAAA]
    low = [0xF0, 0xFF, 0x5A]
    w5 = np.zeros(3 * Q5B, np.uint8)
    w8 = np.zeros(3 * Q8B, np.uint8)
    xq = np.zeros(96, np.int8)
    for b in range(3):
        blk = w5[b * Q5B:(b + 1) * Q5B]
        blk[0], blk[1] = 0x00, 0x3C
        blk[2:6] = np.frombuffer(struct.pack("<I", high[b]), np.uint8)
        blk[6:] = low[b]
        w8[b * Q8B:b * Q8B + 4] = np.array([1.0], np.float32).view(np.uint8)
        j = np.arange(32)
        w8[b * Q8B + 4:(b + 1) * Q8B] = np.where(j % 2 == 1, -128, 127).astype(np.int8).view(np.uint8)
        xq[b * 32:(b + 1) * 32] = np.where(b == 2, np.where(j % 3 != 0, 127, -127), -127)
    xd = np.array([1.0, 0.5, 2.0], np.float32)
    for q5, w in ((True, w5), (False, w8)):
        exact, _ = exact_dot(w, xd, xq, 3, q5, orc)
        got = orc.dot(w, xd, xq, 3, q5=q5)
        # all partial sums here are integers times powers of two below 2^24: exact
        assert got == exact


def random_q5_weights(orc, g, nb, spread):
    x = g.uniform(-spread, spread, nb * 32)
    return orc.quantize_q5_rows(x.reshape(1, -1))


def test_dots_match_reference(orc, ref):
    g = LcgUniform(11)
    for trial in range(120):
        nb = 1 + int(g.next(1)[0] % 64)
        q5 = trial % 2 == 1
        ntok = 1 + int(g.next(1)[0] % 9)
        nrows = 1 + int(g.next(1)[0] % 7)
        if q5:
            w = random_q5_weights(orc, g, nb * nrows, 0.5 + trial % 7)
        else:
            w = random_q8_weights(g, nb * nrows, extremes=trial % 3 == 0)
        x = g.uniform(-50, 50, ntok * nb * 32).reshape(ntok, nb * 32)
        _, xd, xq = orc.quantize_q8(x)
        rb = nb * (Q5B if q5 else Q8B)
        for fast in (False, True):
            got = orc.gemm(w, rb, xd, xq, nrows, ntok, nb, q5=q5, fast=fast)
            want = ref.gemm(w, rb, xd, xq, nrows, ntok, nb, q5=q5, variant="scalar_fast" if fast else "scalar")
            assert np.array_equal(f32_bits(got), f32_bits(want)), (trial, fast)
        want = ref.gemm(w, rb, xd, xq, nrows, ntok, nb, q5=q5, variant="avx2")
        assert np.array_equal(f32_bits(orc.gemm(w, rb, xd, xq, nrows, ntok, nb, q5=q5)), f32_bits(want))


def test_gemm_wide_repack_matches_reference(orc, ref):
    # tests/test_kernels.c:632-670: rows over 16 KiB take the repack in the AVX2 kernel
    g = LcgUniform(21)
    nb, nrows, ntok = 480, 3, 9
    for q5 in (False, True):
        if q5:
            w = np.concatenate([random_q5_weights(orc, g, nb, 1.0) for _ in range(nrows)])
        else:
            w = random_q8_weights(g, nb * nrows, extremes=True)
        _, xd, xq = orc.quantize_q8(g.uniform(-2, 2, ntok * nb * 32).reshape(ntok, -1))
        rb = nb * (Q5B if q5 else Q8B)
        got = orc.gemm(w, rb, xd, xq, nrows, ntok, nb, stride=5, q5=q5)
        want = ref.gemm(w, rb, xd, xq, nrows, ntok, nb, stride=5, q5=q5, variant="avx2")
        assert np.array_equal(f32_bits(got), f32_bits(want))


def test_block_sums_brute_force(orc):
    g = LcgUniform(4)
    for q5 in (False, True):
        nb, nrows, ntok = 5, 3, 2
        w = random_q5_weights(orc, g, nb * nrows, 2.0) if q5 else random_q8_weights(g, nb * nrows, True)
        _, xd, xq = orc.quantize_q8(g.uniform(-9, 9, ntok * nb * 32).reshape(ntok, -1))
        bb = Q5B if q5 else Q8B
        sums = orc.block_sums(w, nb * bb, xq, nrows, ntok, nb, q5=q5)
        for t in range(ntok):
            for r in range(nrows):
                for b in range(nb):
                    blk = w[(r * nb + b) * bb:(r * nb + b + 1) * bb]
                    wq = unpack_q5_numpy(blk) if q5 else blk[4:].view(np.int8).astype(np.int64)
                    assert sums[t, r, b] == int((wq * xq[t, b * 32:(b + 1) * 32].astype(np.int64)).sum())


def test_gemm_blockwise_exact_and_close(orc):
    """orc_gemm_blockwise (the MFMA kernels' order): with power-of-two scales every product and sum
    is exact, so it equals the float64 sum; with random scales it stays within 1e-5 (normwise, per
    token) of the eight-lane contract orc_gemm."""
    g = LcgUniform(11)
    nb, nrows, ntok = 6, 7, 3
    # exact case: scales 2^-k and 2^-m (k < 3, m < 2), |S| < 2^16: every partial sum fits 24 bits
    w = random_q8_weights(g, nb * nrows, True)
    blocks = w.reshape(nb * nrows, Q8B)
    exps = (np.arange(nb * nrows) % 3).astype(np.float32)
    blocks[:, :4] = np.ascontiguousarray((2.0 ** -exps).astype("<f4")).view(np.uint8).reshape(-1, 4)
    xq = (np.arange(ntok * nb * 32) % 23 - 11).astype(np.int8)
    xd = (2.0 ** -(np.arange(ntok * nb) % 2)).astype(np.float32)
    got = orc.gemm_blockwise(w, nb * Q8B, xd, xq, nrows, ntok, nb)
    ws = blocks[:, :4].copy().view("<f4").reshape(nrows, nb).astype(np.float64)
    wq = blocks[:, 4:].view(np.int8).reshape(nrows, nb, 32).astype(np.int64)
    xqb = xq.reshape(ntok, nb, 32).astype(np.int64)
    S = np.einsum("rbk,tbk->trb", wq, xqb).astype(np.float64)
    want = (S * ws[None] * xd.reshape(ntok, 1, nb).astype(np.float64)).sum(axis=2)
    assert np.array_equal(got.reshape(ntok, nrows).astype(np.float64), want)
    # random scales: close to the exact contract
    nb, nrows, ntok = 28, 40, 5
    for q5 in (False, True):
        w = random_q5_weights(orc, g, nb * nrows, 2.0) if q5 else random_q8_weights(g, nb * nrows, False)
        _, xd, xq = orc.quantize_q8(g.uniform(-3, 3, ntok * nb * 32).reshape(ntok, -1))
        rb = nb * (Q5B if q5 else Q8B)
        got = orc.gemm_blockwise(w, rb, xd, xq, nrows, ntok, nb, q5=q5).reshape(ntok, nrows).astype(np.float64)
        want = orc.gemm(w, rb, xd, xq, nrows, ntok, nb, q5=q5).reshape(ntok, nrows).astype(np.float64)
        err = np.abs(got - want).max(axis=1)
        assert np.all(err <= 1e-5 * np.abs(want).max(axis=1)), err


# ---------------------------------------------------------------- offline weight rules

def test_q8_weight_rule_goldens(orc):
    """tests/goldens/convert-q8.json: SHA-256 of q8pack.c's output on the
    bf16 pattern generator — a known-answer test of the weight rule."""
    with open(os.path.join(GOLDEN, "convert-q8.json")) as f:
        cases = json.load(f)["cases"]
    for c in cases:
        x = bf16_to_f32(bf16_patterns(c["rows"], c["cols"], c["seed"]))
        out = orc.q8_weight_rows(x)
        assert out.nbytes == c["bytes"]
        if "firstRowHex" in c:
            nb = (c["cols"] + 31) // 32
            assert out[:nb * Q8B].tobytes().hex() == c["firstRowHex"]
        assert hashlib.sha256(out.tobytes()).hexdigest() == c["sha256"], c


def test_q8_weight_rule_small_cases(orc):
    # tests/convert-quant.test.ts:75-103
    out = orc.q8_weight_rows(np.array([[1, -2, 0.5, 4, -4]], np.float32))
    assert np.frombuffer(out[:4].tobytes(), np.float32)[0] == np.float32(4) / np.float32(127)
    assert list(out[4:9].view(np.int8)) == [32, -64, 16, 127, -127]
    assert np.all(out[9:] == 0)
    out = orc.q8_weight_rows(np.array([[-0.0, -0.0, -0.0]], np.float32))
    assert out[:4].view(np.uint32)[0] == 0
    assert np.all(orc.q8_weight_rows(np.zeros((1, 896), np.float32)) == 0)


def q5_errors_float64(x, d):
    inv = np.float32(1.0) / np.float32(d)
    lv = np.clip(np.rint((x * inv).astype(np.float32)), -16, 15)
    return float(((x.astype(np.float64) - lv.astype(np.float64) * float(d)) ** 2).sum())


def test_q5_rule_is_first_minimum_of_candidates(orc):
    """The chosen scale must be the first of the 21 f16-rounded candidates
    with the least squared error, recomputed here in numpy."""
    g = LcgUniform(8)
    for trial in range(40):
        cols = 1 + int(g.next(1)[0] % 100)
        x = g.uniform(-3, 3, cols)
        if trial % 5 == 0:
            x[int(g.next(1)[0] % cols)] = -7.5
        out = orc.quantize_q5_rows(x.reshape(1, -1))
        for b in range((cols + 31) // 32):
            xb = x[b * 32:(b + 1) * 32]
            ext = xb[np.argmax(np.abs(xb))]
            best, best_h = None, 0
            for k in range(21):
                div = -(np.float32(14.5) + np.float32(0.1) * np.float32(k))
                h = np.float32(ext / div).astype(np.float16)
                d = h.astype(np.float32)
                if d == 0 or not np.isfinite(d):
                    continue
                e = q5_errors_float64(xb, d)
                if best is None or e < best:
                    best, best_h = e, int(h.view(np.uint16))
            blk = out[b * Q5B:(b + 1) * Q5B]
            assert int(blk[0]) | (int(blk[1]) << 8) == best_h
            back = orc.dequantize_row(blk, len(xb), q5=True)
            d = np.uint16(best_h).view(np.float16).astype(np.float32)
            inv = np.float32(1) / d
            lv = np.clip(np.rint((xb * inv).astype(np.float32)), -16, 15).astype(np.float32)
            assert np.array_equal(back, (d * lv).astype(np.float32))


def q5_nonfinite_rows():
    """Blocks with NaN and infinite elements (the public Q5 converter takes any floats)."""
    rows = []
    base = np.linspace(-1, 1, 64).astype(np.float32)
    r = base.copy(); r[3] = np.nan; rows.append(r)                     # one NaN, finite extreme
    r = base.copy(); r[0] = np.nan; r[40] = np.nan; rows.append(r)     # NaN first in its block
    r = np.full(64, np.nan, np.float32); rows.append(r)                # all NaN: extreme 0, zero block
    r = np.zeros(64, np.float32); r[9] = np.nan; rows.append(r)        # NaN among zeros
    r = base.copy(); r[5] = np.inf; rows.append(r)                     # +inf: non-finite candidates
    r = base.copy(); r[33] = -np.inf; r[34] = np.nan; rows.append(r)   # -inf and NaN in one block
    r = base.copy(); r[31] = np.nan; r[31 - 1] = -3.0; rows.append(r)  # NaN next to the extreme
    return np.stack(rows)


def test_q5_rule_nonfinite_closed_form(orc):
    """A NaN is never the extreme (fabsf(NaN) > m is false, kernels.c:1090-1091); with a NaN in the
    block every candidate's error is NaN, so the first kept candidate (k = 0 here) stays
    (kernels.c:1099), and the NaN element's code is 0 (x86-64 lrintf gives LONG_MIN, clamped to -16);
    an infinite element makes every candidate non-finite: scale 0, every code 16."""
    x = q5_nonfinite_rows()
    out = orc.quantize_q5_rows(x).reshape(x.shape[0], 2, Q5B)
    for r in range(x.shape[0]):
        for b in range(2):
            xb = x[r, b * 32:(b + 1) * 32]
            blk = out[r, b]
            h = int(blk[0]) | (int(blk[1]) << 8)
            codes = [((blk[6 + (j % 16)] >> (4 * (j // 16))) & 15) | (((int.from_bytes(bytes(blk[2:6]), "little") >> j)
                                                                     & 1) << 4) for j in range(32)]
            if np.any(np.isinf(xb)) or not np.any(np.abs(np.nan_to_num(xb, nan=0.0)) > 0):
                assert h == 0 and codes == [16] * 32, (r, b)
                continue
            finite = np.where(np.isnan(xb), 0.0, xb)
            ext = xb[int(np.argmax(np.abs(finite)))]
            if np.any(np.isnan(xb)):
                want_h = int(np.float32(ext / -np.float32(14.5)).astype(np.float16).view(np.uint16))
                assert h == want_h, (r, b)
                d = np.uint16(h).view(np.float16).astype(np.float32)
                inv = np.float32(1) / d
                for j in range(32):
                    want = 0 if np.isnan(xb[j]) else int(np.clip(np.rint(np.float32(xb[j] * inv)), -16, 15)) + 16
                    assert codes[j] == want, (r, b, j)


def test_q5_rule_nonfinite_matches_reference(orc, ref):
    x = q5_nonfinite_rows()
    for r in range(x.shape[0]):
        assert np.array_equal(orc.quantize_q5_rows(x[r:r + 1]), ref.quantize_q5_row(x[r])), r


def test_q5_round_trip_bound(orc):
    # tests/test_kernels.c:71-87
    g = LcgUniform(12345)
    x = g.uniform(-1, 1, 100)
    x[7] = 3.0
    out = orc.quantize_q5_rows(x.reshape(1, -1))
    back = orc.dequantize_row(out, 100, q5=True)
    amax = np.where(np.arange(100) < 32, 3.0, 1.0)
    assert np.all(np.abs(back - x) <= amax / 15.0)
    z = orc.quantize_q5_rows(np.zeros((1, 32), np.float32))
    assert np.all(orc.dequantize_row(z, 32, q5=True) == 0)


def test_q5_rule_and_dequant_match_reference(orc, ref):
    g = LcgUniform(31)
    for trial in range(60):
        cols = 1 + int(g.next(1)[0] % 300)
        x = g.uniform(-(0.1 + trial), 0.1 + trial, cols)
        mine = orc.quantize_q5_rows(x.reshape(1, -1))
        theirs = ref.quantize_q5_row(x)
        assert np.array_equal(mine, theirs), trial
        assert np.array_equal(f32_bits(orc.dequantize_row(mine, cols, q5=True)),
                              f32_bits(ref.dequantize_row(theirs, cols, q5=True)))
        w8 = orc.q8_weight_rows(x.reshape(1, -1))
        assert np.array_equal(f32_bits(orc.dequantize_row(w8, cols)), f32_bits(ref.dequantize_row(w8, cols)))


# ---------------------------------------------------------------- caller glue

def test_split_range_coverage(orc):
    # tests/test_kernels.c:514-529
    for total in range(50):
        for count in range(1, 9):
            prev = 0
            covered = 0
            for i in range(count):
                b, e = orc.split_range(total, i, count)
                assert b == prev and b <= e
                covered += e - b
                prev = e
            assert covered == total


def test_mat_item_bias_and_finiteness(orc):
    g = LcgUniform(6)
    nb, rows, ntok = 4, 5, 3
    w = random_q8_weights(g, nb * rows)
    _, xd, xq = orc.quantize_q8(g.uniform(-4, 4, ntok * nb * 32).reshape(ntok, -1))
    bias = g.uniform(-1, 1, rows)
    ok, y = orc.mat_item(w, nb * Q8B, rows, bias, xd, xq, ntok, nb)
    base = orc.gemm(w, nb * Q8B, xd, xq, rows, ntok, nb)
    assert ok
    assert np.array_equal(f32_bits(y), f32_bits((base.reshape(ntok, rows) + bias).astype(np.float32).reshape(-1)))
    w2 = w.copy()
    w2[0:4] = np.array([np.inf], np.float32).view(np.uint8)
    ok, _ = orc.mat_item(w2, nb * Q8B, rows, None, xd, xq, ntok, nb)
    assert not ok


def test_rmsnorm_sequential(orc):
    g = LcgUniform(2)
    x = g.uniform(-3, 3, 896)
    w = g.uniform(0.5, 1.5, 896)
    s, y = orc.rmsnorm(x, w, 1e-6)
    sq = np.float32(0)
    for v in x:
        sq = np.float32(sq + np.float32(v * v))
    inv = np.float32(1) / np.sqrt(np.float32(sq / np.float32(896) + np.float32(1e-6)))
    assert s == 0
    assert np.array_equal(f32_bits(y), f32_bits(((x * inv).astype(np.float32) * w).astype(np.float32)))


# ---------------------------------------------------------------- exp_det and gated activations

def test_exp_table_is_the_mathematics(orc):
    """The oracle's exp_det table equals 2^(j/32) correctly rounded (computed
    independently in 60-digit decimal), minus j << 47."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("gen_exp_table", os.path.join(
        os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "oracle", "gen_exp_table.py"))
    gen = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(gen)
    assert orc.exp2_table() == gen.exp2_table()


def test_exp_det_accuracy_and_specials(orc):
    """tests/test_kernels.c:330-357: at most 1 ulp from the correctly rounded
    e^x, at most 1 in 10^4 not correctly rounded; clamps and NaN."""
    xs = (-103.5 + 192.2 * np.arange(200001) / 200000.0).astype(np.float32)
    got = np.array([orc.exp_det(float(v)) for v in xs], np.float32)
    want = np.exp(xs.astype(np.float64)).astype(np.float32)
    gi, wi = got.view(np.int32).astype(np.int64), want.view(np.int32).astype(np.int64)
    d = np.abs(gi - wi)
    assert d.max() <= 1
    assert (d != 0).sum() <= len(xs) // 10000
    assert orc.exp_det(0.0) == 1.0
    assert orc.exp_det(89.0) == np.inf and orc.exp_det(np.inf) == np.inf
    assert orc.exp_det(-110.0) == 0.0 and orc.exp_det(-np.inf) == 0.0
    assert orc.exp_det(-100.0) > 0.0
    assert np.isnan(orc.exp_det(np.nan))


def test_exp_det_and_activations_match_reference(orc, ref):
    g = LcgUniform(17)
    xs = np.concatenate([g.uniform(-110, 95, 20000), np.array([0.0, -0.0, 88.7, 88.8, -88.7, -88.72, -88.8, -89.0,
                                                               103.0, 120.0, 1e-30, -1e-30, np.inf, -np.inf,
                                                               np.nan], np.float32)])
    a = np.array([orc.exp_det(float(v)) for v in xs], np.float32)
    b = np.array([ref.exp_det(float(v)) for v in xs], np.float32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    gate = np.concatenate([g.uniform(-30, 30, 3000), xs[-15:]]).astype(np.float32)
    up = g.uniform(-4, 4, gate.shape[0])
    for gelu in (False, True):
        mine, theirs = orc.act_mul(up, gate, gelu), ref.act_mul(up, gate, gelu)
        nan = np.isnan(theirs)
        assert np.array_equal(np.isnan(mine), nan)
        assert np.array_equal(mine[~nan].view(np.uint32), theirs[~nan].view(np.uint32))


def test_silu_against_float64(orc):
    # tests/test_kernels.c:372-381
    g = LcgUniform(23)
    gate = g.uniform(-30, 30, 2000)
    up = g.uniform(-4, 4, 2000)
    got = orc.act_mul(up, gate)
    want = up.astype(np.float64) * (gate / (1.0 + np.exp(-gate.astype(np.float64))))
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-30)


def test_row_work_composes(orc):
    g = LcgUniform(29)
    rows, n = 3, 100
    src = g.uniform(-3, 3, rows * n)
    norm = g.uniform(0.5, 1.5, n)
    ok, y, d, q = orc.row_work(src, rows, n, norm=norm, eps=1e-6)
    assert ok
    for r in range(rows):
        s, yr = orc.rmsnorm(src[r * n:(r + 1) * n], norm, 1e-6)
        assert np.array_equal(y[r * n:(r + 1) * n].view(np.uint32), yr.view(np.uint32))
        st, dr, qr = orc.quantize_q8(yr)
        assert np.array_equal(d[r * 4:(r + 1) * 4].view(np.uint32), dr[0].view(np.uint32))
    gate = g.uniform(-5, 5, rows * n)
    ok, y2, d2, q2 = orc.row_work(src, rows, n, gate=gate)
    assert ok and np.array_equal(y2.view(np.uint32), orc.act_mul(src, gate).view(np.uint32))
    bad = src.copy()
    bad[5] = np.inf
    assert not orc.row_work(bad, rows, n, norm=norm)[0]


# ---------------------------------------------------------------- attention pieces

def test_dot_f32_and_attention_match_reference(orc, ref):
    """kernels.c:1119-1176 and tests/test_kernels.c:458-484: strided KV, every
    head size 2..24, start offsets, a -0.0 key."""
    g = LcgUniform(41)
    for trial in range(60):
        hd = 2 + int(g.next(1)[0] % 70)
        npos = 1 + int(g.next(1)[0] % 90)
        start = int(g.next(1)[0] % npos)
        stride = hd + int(g.next(1)[0] % 9)
        q = g.uniform(-4, 4, hd)
        keys = g.uniform(-3, 3, npos * stride)
        values = g.uniform(-3, 3, npos * stride)
        keys[0] = -0.0
        assert np.array_equal(f32_bits(orc.dot_f32(q, keys[:hd])), f32_bits(ref.dot_f32(q, keys[:hd])))
        a = orc.attend_f32(q, keys, values, stride, hd, start, npos - 1)
        b = ref.attend_f32(q, keys, values, stride, hd, start, npos - 1)
        assert np.array_equal(f32_bits(a), f32_bits(b)), trial


def test_attention_closed_form(orc):
    g = LcgUniform(43)
    hd, npos = 64, 40
    q = g.uniform(-1, 1, hd)
    keys = g.uniform(-1, 1, npos * hd).reshape(npos, hd)
    values = g.uniform(-1, 1, npos * hd).reshape(npos, hd)
    s = keys.astype(np.float64) @ q.astype(np.float64) / np.sqrt(hd)
    p = np.exp(s - s.max())
    want = (p / p.sum()) @ values.astype(np.float64)
    got = orc.attend_f32(q, keys.reshape(-1), values.reshape(-1), hd, hd, 0, npos - 1)
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_rope_closed_form(orc):
    g = LcgUniform(47)
    heads, hd, pairs = 3, 16, 6
    x = g.uniform(-2, 2, heads * hd)
    ang = g.uniform(-3, 3, pairs)
    cs, sn = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    y = orc.rope(x, heads, hd, pairs, cs, sn)
    xr = x.reshape(heads, hd).astype(np.float64)
    yr = y.reshape(heads, hd)
    for i in range(pairs):
        a, b = xr[:, 2 * i], xr[:, 2 * i + 1]
        assert np.allclose(yr[:, 2 * i], a * cs[i] - b * sn[i], atol=1e-6)
        assert np.allclose(yr[:, 2 * i + 1], a * sn[i] + b * cs[i], atol=1e-6)
    assert np.array_equal(yr[:, 2 * pairs:], x.reshape(heads, hd)[:, 2 * pairs:])


def test_argmax_semantics(orc):
    """sampler.c:57-63 by brute force: lowest id on ties, banned skipped, a
    NaN only wins as the first candidate."""
    def brute(l, banned):
        best = None
        for i, v in enumerate(l):
            if banned is not None and banned[i]:
                continue
            if best is None or v > l[best]:
                best = i
        return 0xFFFFFFFF if best is None else best
    g = LcgUniform(53)
    for trial in range(200):
        n = 1 + int(g.next(1)[0] % 300)
        l = np.round(g.uniform(-3, 3, n) * 2) / 2  # many ties
        banned = (g.next(n) % np.uint64(5) == 0).astype(np.uint8) if trial % 2 else None
        if trial % 7 == 0:
            l[int(g.next(1)[0] % n)] = np.nan
        if trial % 11 == 0:
            l[0] = np.nan
        assert orc.argmax(l, banned) == brute(l, banned), trial
    assert orc.argmax(np.zeros(3, np.float32), np.ones(3, np.uint8)) == 0xFFFFFFFF
