"""The allocation-free argmax (smq_argmax_noalloc: partials in the library's
static device array) against smq_argmax (its allocated workspace), through
the C ABI: two calls in a row, the second with a smaller vocabulary, then
ties, banned ids, a NaN first candidate and the size limit."""
import numpy as np
import pytest

from checks import say
from smq_pkg import smq, synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert smq.init(0) == "gfx950"
    yield


def both(logits, banned=None):
    n = logits.size
    lb = smq.DeviceBuffer.from_array(np.ascontiguousarray(logits, np.float32))
    bb = smq.DeviceBuffer.from_array(np.ascontiguousarray(banned, np.uint8)) if banned is not None else None
    t1, t2 = smq.DeviceBuffer(4), smq.DeviceBuffer(4)
    t1.fill(0xFF)
    t2.fill(0x00)
    smq.argmax(lb, n, bb, t1)
    smq.argmax_noalloc(lb, n, bb, t2)
    smq.synchronize()
    return int(t1.download(np.uint32)[0]), int(t2.download(np.uint32)[0])


def test_noalloc_matches_allocated_twice_then_smaller():
    say("noalloc argmax 151936 then 50000")
    big = synth.normal(11, 151936, 3.0)
    a, b = both(big)
    assert a == b == int(np.argmax(big))
    small = synth.normal(12, 50000, 3.0)  # second call, smaller input: stale partials must not leak in
    small[:] = np.minimum(small, 1.0)
    small[777] = 2.0
    a, b = both(small)
    assert a == b == 777


def test_noalloc_edge_cases():
    say("noalloc argmax edges")
    v = np.zeros(4096, np.float32)
    v[100] = v[3000] = 5.0  # tie: the lowest id
    assert both(v) == (100, 100)
    banned = np.zeros(4096, np.uint8)
    banned[100] = 1
    assert both(v, banned) == (3000, 3000)
    w = synth.normal(13, 1048576, 1.0)  # the largest vocabulary the static partials serve
    w[1048575] = 50.0
    assert both(w) == (1048575, 1048575)
    x = synth.normal(14, 300, 1.0)
    x[0] = np.nan  # a NaN first candidate wins (nothing compares greater)
    assert both(x) == (0, 0)
    allb = np.ones(300, np.uint8)
    assert both(x, allb) == (0xFFFFFFFF, 0xFFFFFFFF)


def test_noalloc_refuses_past_its_scratch():
    lb = smq.DeviceBuffer(4 * 1048577)
    t = smq.DeviceBuffer(4)
    with pytest.raises(smq.SmqError) as e:
        smq.argmax_noalloc(lb, 1048577, None, t)
    assert e.value.status == smq.SM_ERR_RANGE and "static scratch" in str(e.value)
