"""The measurement anchors bench.py reports beside the GEMVs: the HBM stream
kernels move or read exactly the bytes asked for, and the grid barrier probe
passes its barriers (no workgroup gives up a wait) for every kind, refusing
grids that could not all be resident."""
import numpy as np
import pytest

from checks import say
from smq_pkg import smq

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def gpu():
    assert smq.init(0) == "gfx950"
    yield


@pytest.mark.parametrize("nbytes,wgs,threads,nt", [(1 << 20, 256, 256, True), ((1 << 20) + 48, 7, 64, False),
                                                   (16, 1, 64, True)])
def test_stream_copy_moves_every_byte(nbytes, wgs, threads, nt):
    say("stream_copy", nbytes, wgs, threads, nt)
    src = np.random.default_rng(5).integers(0, 256, nbytes, dtype=np.uint8)
    a = smq.DeviceBuffer.from_array(src)
    b = smq.DeviceBuffer(nbytes + 64)
    b.upload(np.full(nbytes + 64, 0xAB, np.uint8))
    smq.stream_copy(b, a, nbytes, wgs, threads, nt)
    smq.synchronize()
    got = b.download(np.uint8)
    assert np.array_equal(got[:nbytes], src)
    assert np.all(got[nbytes:] == 0xAB)  # nothing past the range


def test_stream_read_writes_nothing():
    say("stream_read")
    a = smq.DeviceBuffer.from_array(np.zeros(1 << 20, np.uint8))
    sink = smq.DeviceBuffer.from_array(np.array([7], np.uint32))
    smq.stream_read(a, 1 << 20, 512, 256, True, sink)
    smq.synchronize()
    assert sink.download(np.uint32)[0] == 7


def test_stream_anchor_argument_errors():
    a = smq.DeviceBuffer(4096)
    with pytest.raises(smq.SmqError):
        smq.stream_read(a, 4008, 1, 64, True, a)  # size not a multiple of 16
    with pytest.raises(smq.SmqError):
        smq.stream_copy(a, a, 4096, 1, 96, True)  # threads not a multiple of 64


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("wgs", [1, 9, 64, 256])
def test_grid_barrier_probe_passes(kind, wgs):
    say("grid_barrier_probe", kind, wgs)
    ms0 = smq.grid_barrier_probe(wgs, 0, kind)
    ms = smq.grid_barrier_probe(wgs, 50, kind)
    assert 0.0 < ms0 and 0.0 < ms < 1000.0


def test_grid_barrier_probe_refuses_oversized_grids():
    with pytest.raises(smq.SmqError):
        smq.grid_barrier_probe(257, 1, 0)  # more workgroups than the 256 CUs
    with pytest.raises(smq.SmqError):
        smq.grid_barrier_probe(0, 1, 0)
    with pytest.raises(smq.SmqError):
        smq.grid_barrier_probe(8, 1, 3)
