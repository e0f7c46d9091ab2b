"""CPU checks of the C-ABI libraries: they load, export every entry point
that include/smq.h and include/smq_model.h declare, and report a missing GPU
as a status (no compute)."""
import ctypes
import os
import re

import pytest

from smq_pkg import smodel, smq

INCLUDE = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include")
HEADER = os.path.join(INCLUDE, "smq.h")
MODEL_HEADER = os.path.join(INCLUDE, "smq_model.h")


def declared(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(smq_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(smq.LIB_PATH):
        pytest.fail("libsmq_gfx950.so is not built: run __graft_entry__.build()")
    return ctypes.CDLL(smq.LIB_PATH)


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_the_header():
    assert set(declared()) == set(smq.exported_symbols())


def test_code_object_targets_gfx950_only():
    data = open(smq.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data
    for other in (b"--gfx90a", b"--gfx942", b"--gfx1100"):
        assert other not in data


def test_calls_without_init_report_state_error(lib):
    smq.load()
    l = smq.load()
    l.smq_clear_error()
    assert l.smq_quantize_q8(None, 32, None, None) == -1
    assert l.smq_last_status() == 7  # SM_ERR_STATE
    assert b"smq_init" in l.smq_last_error()
    l.smq_clear_error()


def test_model_library_exports_its_header():
    if not os.path.exists(smodel.MODEL_LIB):
        pytest.fail("libsmq_model.so is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(smodel.MODEL_LIB)
    names = declared(MODEL_HEADER)
    assert len(names) >= 15
    assert not [n for n in names if not hasattr(lib, n)]
    assert set(names) == set(smodel.exported_symbols())


def test_model_open_without_init_reports_state_error(tmp_path):
    smodel.load_model_lib()
    path = tmp_path / "empty.smoe"
    path.write_bytes(b"SMOEQ8\0\x01" + b"\0" * 8)
    with pytest.raises(smq.SmqError):
        smodel.Model(str(path), context=8, batch=1)
