"""ctypes binding of the C host forward pass (include/smq_model.h,
libsmq_model.so): the reference's Config / ModelFile / Model API
(src/config.h, src/modelfile.h, src/model.h) on the gfx950 path."""
import ctypes
import os

import numpy as np

from . import HERE, SmqError, _check, load

MODEL_LIB = os.path.join(HERE, "libsmq_model.so")
LOGITS_NONE, LOGITS_LAST, LOGITS_ALL = 0, 1, 2

_u32, _vp = ctypes.c_uint32, ctypes.c_void_p


class Config(ctypes.Structure):
    """smq_config = src/config.h:13-28."""
    _fields_ = [(n, _u32) for n in ("dim", "hidden", "layers", "heads", "kv_heads", "experts", "top_k", "vocab",
                                    "max_context", "shared", "bos", "eos", "qkv_bias", "gemma3", "head_dim",
                                    "rotary_dim", "sliding_window")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float), ("local_theta", ctypes.c_float),
                ("rope_factor", ctypes.c_double), ("llama3_rope", _u32), ("llama3_original", _u32),
                ("llama3_factor", ctypes.c_double), ("llama3_low", ctypes.c_double),
                ("llama3_high", ctypes.c_double)]


class _Tensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 40), ("rows", _u32), ("cols", _u32), ("dtype", _u32), ("alias", _u32),
                ("offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64), ("data", _vp)]


class _ModelFile(ctypes.Structure):
    _fields_ = [("base", _vp), ("size", ctypes.c_uint64), ("version", _u32), ("count", _u32), ("blobs", _u32),
                ("tensors", ctypes.POINTER(_Tensor))]


_SIGS = {
    "smq_config_parse": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(Config)]),
    "smq_config_read": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(Config)]),
    "smq_modelfile_parse": (ctypes.c_int, [ctypes.POINTER(_ModelFile), _vp, ctypes.c_uint64]),
    "smq_modelfile_verify_payload": (ctypes.c_int, [ctypes.POINTER(_ModelFile)]),
    "smq_modelfile_find": (ctypes.POINTER(_Tensor), [ctypes.POINTER(_ModelFile), ctypes.c_char_p, _u32, _u32, _u32]),
    "smq_modelfile_blob": (ctypes.POINTER(_Tensor), [ctypes.POINTER(_ModelFile), ctypes.c_char_p]),
    "smq_modelfile_release": (None, [ctypes.POINTER(_ModelFile)]),
    "smq_model_open": (_vp, [ctypes.c_char_p, ctypes.c_char_p, _u32, _u32, _u32]),
    "smq_model_open_bytes": (_vp, [_vp, ctypes.c_uint64, ctypes.POINTER(Config), _u32, _u32, _u32]),
    "smq_model_close": (None, [_vp]),
    "smq_model_config": (ctypes.POINTER(Config), [_vp]),
    "smq_model_device_bytes": (ctypes.c_size_t, [_vp]),
    "smq_model_forward": (ctypes.c_int, [_vp, _vp, _u32, _u32, ctypes.c_int]),
    "smq_model_prefill": (ctypes.c_int, [_vp, _vp, _u32, _u32, ctypes.c_int]),
    "smq_model_logits": (ctypes.c_int, [_vp, _vp, _u32]),
    "smq_model_logits_device": (_vp, [_vp]),
    "smq_model_kv_layer": (_vp, [_vp, _u32, ctypes.c_int]),
    "smq_model_set_banned": (ctypes.c_int, [_vp, _vp]),
    "smq_model_generate": (ctypes.c_int, [_vp, _u32, _u32, _vp]),
    "smq_model_prepare_decode": (ctypes.c_int, [_vp]),
    "smq_synth_checkpoint": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_uint64, ctypes.c_float,
                                            ctypes.c_int, _u32]),
}

_mlib = None


def load_model_lib():
    """Loads libsmq_model.so (and libsmq_gfx950.so); raises if not built."""
    global _mlib
    if _mlib is None:
        load()
        if not os.path.exists(MODEL_LIB):
            raise SmqError(7, f"{MODEL_LIB} is missing: run __graft_entry__.build()")
        lib = ctypes.CDLL(MODEL_LIB)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _mlib = lib
    return _mlib


def exported_symbols():
    return sorted(_SIGS)


def config_parse(text):
    c = Config()
    raw = text.encode() if isinstance(text, str) else bytes(text)
    _check(load_model_lib().smq_config_parse(raw, len(raw), ctypes.byref(c)))
    return c


def config_read(path):
    c = Config()
    _check(load_model_lib().smq_config_read(path.encode(), ctypes.byref(c)))
    return c


def synth_checkpoint(path, config_text, seed=1, sigma=0.02, tied=True, threads=8):
    """Writes a synthetic one-expert checkpoint (smq_synth_checkpoint)."""
    _check(load_model_lib().smq_synth_checkpoint(path.encode(), config_text.encode(), seed, sigma, int(bool(tied)),
                                                 threads))
    return path


class ModelFile:
    """smq_modelfile_parse over bytes held by this object (host only)."""

    def __init__(self, data):
        self._buf = np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray) else data
        self._mf = _ModelFile()
        lib = load_model_lib()
        _check(lib.smq_modelfile_parse(ctypes.byref(self._mf), self._buf.ctypes.data, self._buf.nbytes))

    def verify(self):
        _check(load_model_lib().smq_modelfile_verify_payload(ctypes.byref(self._mf)))

    @property
    def version(self):
        return self._mf.version

    @property
    def count(self):
        return self._mf.count

    @property
    def blobs(self):
        return self._mf.blobs

    def find(self, name, rows, cols, dtype):
        p = load_model_lib().smq_modelfile_find(ctypes.byref(self._mf), name.encode(), rows, cols, dtype)
        if not p:
            _check()
        t = p.contents
        return t.name.decode(), t.rows, t.cols, t.dtype, t.alias, t.offset, t.bytes

    def __del__(self):
        if _mlib is not None and getattr(self, "_mf", None) is not None:
            _mlib.smq_modelfile_release(ctypes.byref(self._mf))


class Model:
    """A checkpoint on the GPU (smq_model_open). smq.init must run first."""

    def __init__(self, path, config_path=None, context=1024, batch=64, logit_rows=1):
        lib = load_model_lib()
        self._m = lib.smq_model_open(path.encode(), config_path.encode() if config_path else None, context, batch,
                                     logit_rows)
        if not self._m:
            _check()
            raise SmqError(1, "smq_model_open failed")
        c = lib.smq_model_config(self._m).contents
        self.vocab, self.dim, self.layers = c.vocab, c.dim, c.layers
        self.kv_dim = c.kv_heads * c.head_dim
        self.context, self.logit_rows = context, logit_rows

    def close(self):
        if self._m:
            load_model_lib().smq_model_close(self._m)
            self._m = None

    def __del__(self):
        if _mlib is not None and getattr(self, "_m", None):
            _mlib.smq_model_close(self._m)
            self._m = None

    @property
    def device_bytes(self):
        return load_model_lib().smq_model_device_bytes(self._m)

    def forward(self, tokens, pos0, mode=LOGITS_LAST):
        t = np.ascontiguousarray(tokens, np.uint32)
        _check(load_model_lib().smq_model_forward(self._m, t.ctypes.data, t.size, pos0, mode))

    def prefill(self, tokens, pos0=0, last_logits=True):
        t = np.ascontiguousarray(tokens, np.uint32)
        _check(load_model_lib().smq_model_prefill(self._m, t.ctypes.data, t.size, pos0, int(bool(last_logits))))

    def logits(self, rows=1):
        out = np.empty((rows, self.vocab), np.float32)
        _check(load_model_lib().smq_model_logits(self._m, out.ctypes.data, rows))
        return out

    def kv(self, layer, values=False, positions=None):
        """Host copy of one layer's keys or values: [positions, kv_dim] f32."""
        n = self.context if positions is None else positions
        p = load_model_lib().smq_model_kv_layer(self._m, layer, int(bool(values)))
        if not p:
            raise SmqError(4, "kv_layer: layer out of range")
        out = np.empty((n, self.kv_dim), np.float32)
        _check(load().smq_memcpy_dtoh(out.ctypes.data, p, out.nbytes))
        return out

    def set_banned(self, banned=None):
        if banned is None:
            _check(load_model_lib().smq_model_set_banned(self._m, None))
        else:
            b = np.ascontiguousarray(banned, np.uint8)
            assert b.size == self.vocab
            _check(load_model_lib().smq_model_set_banned(self._m, b.ctypes.data))

    def generate(self, pos, ntokens):
        out = np.zeros(ntokens, np.uint32)
        _check(load_model_lib().smq_model_generate(self._m, pos, ntokens, out.ctypes.data))
        return out

    def prepare_decode(self):
        """Captures the decode step now (a batch forward drops it), so a timed generate only replays."""
        _check(load_model_lib().smq_model_prepare_decode(self._m))
