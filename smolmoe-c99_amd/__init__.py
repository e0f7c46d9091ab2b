"""Python host mirror of the gfx950 quantized matrix-product path.

Binds include/smq.h (libsmq_gfx950.so, built in this directory by build.py)
with ctypes and mirrors the reference's kernel seam by name and meaning
(src/kernels.h:49-87, 183-196 and the matmul glue of src/model.c:236-310):
``kernels_select``, ``kernels_set_fast``, ``quantize_q8``, ``dot_q8``,
``dot_q8_x4``, ``dot_q8_r4``, ``gemm_q8``, ``gemm_q5``, ``matmul``, ...

Array arguments are ``DeviceBuffer`` objects (device memory owned by the
library). There is no CPU fallback: importing works anywhere, but every call
needs the compiled library and a gfx950 GPU and raises ``SmqError``
otherwise.

The directory name is not a Python identifier; import it with
``importlib.import_module("smolmoe-c99_amd")``.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsmq_gfx950.so")
QK = 32
Q8_BLOCK_BYTES = 36
Q5_BLOCK_BYTES = 22
DTYPE_Q8, DTYPE_Q5 = 1, 2

# src/util.h:28-37
STATUS = {0: "SM_OK", 1: "SM_ERR", 2: "SM_ERR_IO", 3: "SM_ERR_FORMAT", 4: "SM_ERR_RANGE", 5: "SM_ERR_NUMERIC",
          6: "SM_ERR_NOMEM", 7: "SM_ERR_STATE"}
SM_ERR_FORMAT, SM_ERR_RANGE, SM_ERR_NUMERIC, SM_ERR_STATE = 3, 4, 5, 7


class SmqError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status


_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_sz = ctypes.c_size_t


class _QMat(ctypes.Structure):
    _fields_ = [("data", _vp), ("rows", _u32), ("cols", _u32), ("nb", _u32), ("dtype", _u32), ("row_bytes", _sz)]


class _MatItem(ctypes.Structure):
    _fields_ = [("w", ctypes.POINTER(_QMat)), ("bias", _vp), ("y", _vp), ("accumulate", ctypes.c_int)]


class _GroupItem(ctypes.Structure):
    _fields_ = [("w", ctypes.POINTER(_QMat)), ("bias", _vp), ("y", _vp), ("accumulate", ctypes.c_int),
                ("xd", _vp), ("xq", _vp)]


class _Act(ctypes.Structure):
    _fields_ = [("kind", ctypes.c_int), ("cols", _u32), ("x", _vp), ("norm", _vp), ("eps", ctypes.c_float),
                ("xd", _vp), ("xq", _vp), ("xd_scratch", _vp), ("xq_scratch", _vp)]


class _AttnShape(ctypes.Structure):
    _fields_ = [("heads", _u32), ("kv_heads", _u32), ("head_dim", _u32), ("rotary_pairs", _u32), ("window", _u32),
                ("context", _u32)]


_SIGS = {
    "smq_last_status": (ctypes.c_int, []),
    "smq_last_error": (ctypes.c_char_p, []),
    "smq_clear_error": (None, []),
    "smq_set_error": (ctypes.c_int, [ctypes.c_int, ctypes.c_char_p]),
    "smq_init": (ctypes.c_int, [ctypes.c_int]),
    "smq_shutdown": (None, []),
    "smq_stream": (_vp, []),
    "smq_set_stream": (ctypes.c_int, [_vp]),
    "smq_synchronize": (ctypes.c_int, []),
    "smq_device_arch": (ctypes.c_char_p, []),
    "smq_kernels_select": (ctypes.c_char_p, [ctypes.c_int]),
    "smq_kernels_set_fast": (None, [ctypes.c_int]),
    "smq_kernels_fast": (ctypes.c_int, []),
    "smq_gemm_scratch_bytes": (_sz, [_u32]),
    "smq_set_checks": (None, [ctypes.c_int]),
    "smq_quantize_q8": (ctypes.c_int, [_vp, _u32, _vp, _vp]),
    "smq_quantize_q8_rows": (ctypes.c_int, [_vp, _u32, _u32, _vp, _vp]),
    "smq_row_quantize": (ctypes.c_int, [_vp, _vp, ctypes.c_float, _vp, ctypes.c_int, _u32, _u32, _vp, _vp, _vp]),
    "smq_norm_quantize": (ctypes.c_int, [_vp, _vp, ctypes.c_float, _u32, _u32, _vp, _vp, _vp]),
    "smq_silu_quantize": (ctypes.c_int, [_vp, _vp, ctypes.c_int, _u32, _u32, _vp, _vp]),
    "smq_dot_q8": (ctypes.c_float, [_vp, _vp, _vp, _u32]),
    "smq_dot_q5": (ctypes.c_float, [_vp, _vp, _vp, _u32]),
    "smq_dot_q8_x4": (None, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "smq_dot_q5_x4": (None, [_vp, _vp, _vp, _u32, _u32, _vp]),
    "smq_dot_q8_r4": (None, [_vp, _sz, _vp, _vp, _u32, _vp]),
    "smq_dot_q5_r4": (None, [_vp, _sz, _vp, _vp, _u32, _vp]),
    "smq_gemm_q8": (None, [_vp, _sz, _vp, _vp, _u32, _u32, _u32, _vp, _sz, _vp]),
    "smq_gemm_q5": (None, [_vp, _sz, _vp, _vp, _u32, _u32, _u32, _vp, _sz, _vp]),
    "smq_gemm_q8_mfma": (None, [_vp, _sz, _vp, _vp, _u32, _u32, _u32, _vp, _sz, _vp]),
    "smq_gemm_q5_mfma": (None, [_vp, _sz, _vp, _vp, _u32, _u32, _u32, _vp, _sz, _vp]),
    "smq_block_sums": (None, [ctypes.c_int, _vp, _sz, _vp, _u32, _u32, _u32, _vp]),
    "smq_set_prefill_mfma": (None, [ctypes.c_int]),
    "smq_set_gemv_rows": (ctypes.c_int, [ctypes.c_int]),
    "smq_set_exact_gemm": (ctypes.c_int, [ctypes.c_int]),
    "smq_matmul": (ctypes.c_int, [ctypes.POINTER(_MatItem), _u32, _vp, _vp, _u32]),
    "smq_numeric_check": (ctypes.c_int, []),
    "smq_matmul_act": (ctypes.c_int, [ctypes.POINTER(_MatItem), _u32, ctypes.POINTER(_Act)]),
    "smq_matmul_act_rope": (ctypes.c_int, [ctypes.POINTER(_MatItem), ctypes.POINTER(_Act), ctypes.POINTER(_AttnShape),
                                           _vp, _vp, _vp, _vp, _u32, _vp]),
    "smq_matmul_glu": (ctypes.c_int, [ctypes.POINTER(_QMat), ctypes.POINTER(_QMat), ctypes.POINTER(_Act), ctypes.c_int,
                                      _vp, _vp]),
    "smq_matmul_glu_q8": (ctypes.c_int, [ctypes.POINTER(_QMat), ctypes.POINTER(_QMat), ctypes.POINTER(_Act),
                                         ctypes.c_int, _vp, _vp, _vp, _vp]),
    "smq_gemv_grouped": (ctypes.c_int, [ctypes.POINTER(_GroupItem), _u32]),
    "smq_gemv_plan_create": (ctypes.c_int, [ctypes.POINTER(_GroupItem), _u32, ctypes.POINTER(ctypes.c_void_p)]),
    "smq_gemv_plan_launch": (ctypes.c_int, [_vp]),
    "smq_gemv_plan_destroy": (None, [_vp]),
    "smq_rope_kv": (ctypes.c_int, [_vp, _vp, _vp, _u32, ctypes.POINTER(_AttnShape), _vp, _vp, _vp, _vp, _u32, _vp]),
    "smq_attention": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, ctypes.POINTER(_AttnShape), _u32, _vp]),
    "smq_attention_q8": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32, ctypes.POINTER(_AttnShape), _u32, _vp, _vp, _vp]),
    "smq_argmax": (ctypes.c_int, [_vp, _u32, _vp, _vp]),
    "smq_argmax_noalloc": (ctypes.c_int, [_vp, _u32, _vp, _vp]),
    "smq_embed": (ctypes.c_int, [ctypes.POINTER(_QMat), _vp, _u32, _vp]),
    "smq_decode_advance": (ctypes.c_int, [_vp, _vp, _vp, _vp, _u32]),
    "smq_attention_rope_q8": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _u32, _vp, _vp, _vp]),
    "smq_argmax_advance": (ctypes.c_int, [_vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32]),
    "smq_argmax_advance_embed": (ctypes.c_int, [_vp, _u32, _vp, _vp, _vp, _vp, _vp, _u32, ctypes.POINTER(_QMat),
                                                _vp]),
    "smq_quantize_q5_row": (None, [_vp, _u32, _vp]),
    "smq_quantize_q5_rows": (ctypes.c_int, [_vp, _u32, _u32, _vp]),
    "smq_dequantize_q8_row": (None, [_vp, _u32, _vp]),
    "smq_dequantize_q5_row": (None, [_vp, _u32, _vp]),
    "smq_malloc": (_vp, [_sz]),
    "smq_free": (None, [_vp]),
    "smq_memcpy_htod": (ctypes.c_int, [_vp, _vp, _sz]),
    "smq_memcpy_dtoh": (ctypes.c_int, [_vp, _vp, _sz]),
    "smq_memcpy_dtod": (ctypes.c_int, [_vp, _vp, _sz]),
    "smq_memset": (ctypes.c_int, [_vp, ctypes.c_int, _sz]),
    "smq_capture_begin": (ctypes.c_int, []),
    "smq_capture_end": (_vp, []),
    "smq_graph_launch": (ctypes.c_int, [_vp]),
    "smq_graph_destroy": (None, [_vp]),
    "smq_timer_start": (ctypes.c_int, []),
    "smq_timer_stop": (ctypes.c_double, []),
    "smq_stream_read": (ctypes.c_int, [_vp, _sz, _u32, _u32, ctypes.c_int, _vp]),
    "smq_stream_copy": (ctypes.c_int, [_vp, _vp, _sz, _u32, _u32, ctypes.c_int]),
    "smq_grid_barrier_probe": (ctypes.c_int, [_u32, _u32, _u32, ctypes.POINTER(ctypes.c_double)]),
}

_lib = None


def load():
    """Loads libsmq_gfx950.so; raises if it was not built (no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise SmqError(7, f"{LIB_PATH} is missing: run __graft_entry__.build() (hipcc, gfx950)")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def exported_symbols():
    return sorted(_SIGS)


def _check(status=None):
    lib = load()
    st = lib.smq_last_status() if status is None else status
    if st != 0:
        msg = lib.smq_last_error().decode()
        lib.smq_clear_error()
        raise SmqError(st, msg)


def init(device=0):
    lib = load()
    _check(lib.smq_init(device))
    return lib.smq_device_arch().decode()


def shutdown():
    load().smq_shutdown()


def synchronize():
    _check(load().smq_synchronize())


def set_checks(on):
    load().smq_set_checks(int(bool(on)))


class DeviceBuffer:
    """Device memory from smq_malloc, with numpy upload/download."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        self.ptr = load().smq_malloc(max(1, self.nbytes))
        if not self.ptr:
            _check()
            raise SmqError(6, "smq_malloc returned NULL")

    @classmethod
    def from_array(cls, arr):
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr, offset=0):
        arr = np.ascontiguousarray(arr)
        if offset + arr.nbytes > self.nbytes:
            raise ValueError("upload exceeds buffer")
        _check(load().smq_memcpy_htod(self.ptr + offset, arr.ctypes.data, arr.nbytes))

    def download(self, dtype, count=None, offset=0):
        dtype = np.dtype(dtype)
        count = (self.nbytes - offset) // dtype.itemsize if count is None else count
        out = np.empty(count, dtype)
        if count:
            _check(load().smq_memcpy_dtoh(out.ctypes.data, self.ptr + offset, out.nbytes))
        return out

    def copy_from(self, other, nbytes=None):
        n = other.nbytes if nbytes is None else nbytes
        _check(load().smq_memcpy_dtod(self.ptr, other.ptr, n))

    def fill(self, value=0):
        _check(load().smq_memset(self.ptr, value, self.nbytes))

    def at(self, offset):
        return self.ptr + offset

    def free(self):
        if self.ptr:
            load().smq_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _p(x, offset=0):
    if x is None:
        return None
    if isinstance(x, DeviceBuffer):
        return x.ptr + offset
    return int(x) + offset


# ---- src/kernels.h:72-87
def kernels_select(force_exact=False):
    name = load().smq_kernels_select(int(bool(force_exact))).decode()
    _check()
    return name


def kernels_set_fast(fast):
    load().smq_kernels_set_fast(int(bool(fast)))


def kernels_fast():
    return bool(load().smq_kernels_fast())


def gemm_scratch_bytes(nb):
    return load().smq_gemm_scratch_bytes(nb)


# ---- src/kernels.h:183-187
def quantize_q8(x, n, d, q):
    """QuantizeQ8 on device buffers: returns 0, or -1 for a non-finite input."""
    r = load().smq_quantize_q8(_p(x), n, _p(d), _p(q))
    if r != 0 and load().smq_last_status() != 0:
        _check()
    return r


def quantize_q8_rows(x, rows, n, d, q):
    _check(load().smq_quantize_q8_rows(_p(x), rows, n, _p(d), _p(q)))


# ---- src/model.c:347-415
def row_quantize(src, rows, n, d, q, norm=None, eps=1e-6, gate=None, act=0, y=None):
    _check(load().smq_row_quantize(_p(src), _p(norm), eps, _p(gate), act, rows, n, _p(y), _p(d), _p(q)))


def norm_quantize(src, norm, eps, rows, n, y, d, q):
    _check(load().smq_norm_quantize(_p(src), _p(norm), eps, rows, n, _p(y), _p(d), _p(q)))


def silu_quantize(up, gate, rows, n, d, q, gemma3=False):
    _check(load().smq_silu_quantize(_p(up), _p(gate), int(bool(gemma3)), rows, n, _p(d), _p(q)))


# ---- src/kernels.h:49-70
def dot_q8(w, xd, xq, nb):
    v = load().smq_dot_q8(_p(w), _p(xd), _p(xq), nb)
    _check()
    return v


def dot_q5(w, xd, xq, nb):
    v = load().smq_dot_q5(_p(w), _p(xd), _p(xq), nb)
    _check()
    return v


def dot_q8_x4(w, xd, xq, nb, stride, out):
    load().smq_dot_q8_x4(_p(w), _p(xd), _p(xq), nb, stride, _p(out))
    _check()


def dot_q5_x4(w, xd, xq, nb, stride, out):
    load().smq_dot_q5_x4(_p(w), _p(xd), _p(xq), nb, stride, _p(out))
    _check()


def dot_q8_r4(w, row_bytes, xd, xq, nb, out):
    load().smq_dot_q8_r4(_p(w), row_bytes, _p(xd), _p(xq), nb, _p(out))
    _check()


def dot_q5_r4(w, row_bytes, xd, xq, nb, out):
    load().smq_dot_q5_r4(_p(w), row_bytes, _p(xd), _p(xq), nb, _p(out))
    _check()


def gemm_q8(w, row_bytes, xd, xq, nrows, ntok, nb, out, stride, scratch=None):
    load().smq_gemm_q8(_p(w), row_bytes, _p(xd), _p(xq), nrows, ntok, nb, _p(out), stride, _p(scratch))
    _check()


def gemm_q5(w, row_bytes, xd, xq, nrows, ntok, nb, out, stride, scratch=None):
    load().smq_gemm_q5(_p(w), row_bytes, _p(xd), _p(xq), nrows, ntok, nb, _p(out), stride, _p(scratch))
    _check()


def gemm_q8_mfma(w, row_bytes, xd, xq, nrows, ntok, nb, out, stride, scratch=None):
    load().smq_gemm_q8_mfma(_p(w), row_bytes, _p(xd), _p(xq), nrows, ntok, nb, _p(out), stride, _p(scratch))
    _check()


def gemm_q5_mfma(w, row_bytes, xd, xq, nrows, ntok, nb, out, stride, scratch=None):
    load().smq_gemm_q5_mfma(_p(w), row_bytes, _p(xd), _p(xq), nrows, ntok, nb, _p(out), stride, _p(scratch))
    _check()


def block_sums(q5, w, row_bytes, xq, nrows, ntok, nb, sums):
    load().smq_block_sums(int(bool(q5)), _p(w), row_bytes, _p(xq), nrows, ntok, nb, _p(sums))
    _check()


def set_prefill_mfma(on):
    load().smq_set_prefill_mfma(int(bool(on)))


def set_gemv_rows(rows):
    """Rows per workgroup of the one-launch decode GEMV (1, 2, 4, 8, 16), or 0 for the default choice."""
    _check(load().smq_set_gemv_rows(int(rows)))


EXACT_BY_SHAPE, EXACT_MFMA, EXACT_VALU, EXACT_MFMA_SPLIT, EXACT_MFMA_SPLIT4 = 0, 1, 2, 3, 4


def set_exact_gemm(mode):
    """Kernel of the exact prefill GEMM: EXACT_BY_SHAPE (default), EXACT_MFMA (lane sums on the matrix
    cores), EXACT_VALU (lane sums as v_dot4), EXACT_MFMA_SPLIT or EXACT_MFMA_SPLIT4 (matrix cores, each tile's
    lane sums over two or four waves); the outputs are the same bit for bit."""
    _check(load().smq_set_exact_gemm(int(mode)))


# ---- src/model.c:236-310
class QMat:
    """model.h:15-19: a quantized matrix in device memory."""

    def __init__(self, data, rows, cols, dtype=DTYPE_Q8, offset=0):
        self.buf = data
        self.offset = offset
        self.rows, self.cols, self.dtype = rows, cols, dtype
        self.nb = (cols + QK - 1) // QK
        self.row_bytes = self.nb * (Q5_BLOCK_BYTES if dtype == DTYPE_Q5 else Q8_BLOCK_BYTES)

    def _c(self):
        return _QMat(_p(self.buf, self.offset), self.rows, self.cols, self.nb, self.dtype, self.row_bytes)


def matmul(items, xd, xq, ntok):
    """items: sequence of (QMat, bias DeviceBuffer or None, y DeviceBuffer[,
    accumulate]); accumulate adds the result into y (the residual add)."""
    cm = [it[0]._c() for it in items]
    arr = (_MatItem * len(items))()
    for i, it in enumerate(items):
        arr[i].w = ctypes.pointer(cm[i])
        arr[i].bias = _p(it[1])
        arr[i].y = _p(it[2])
        arr[i].accumulate = int(bool(it[3])) if len(it) > 3 else 0
    _check(load().smq_matmul(arr, len(items), _p(xd), _p(xq), ntok))


ACT_Q8, ACT_NORM, ACT_F32 = 0, 1, 2


def act(kind, cols, x=None, norm=None, eps=1e-6, xd=None, xq=None, xd_scratch=None, xq_scratch=None):
    """The activation of a fused decode matmul (smq_act); holds its buffers."""
    a = _Act(kind, cols, _p(x), _p(norm), eps, _p(xd), _p(xq), _p(xd_scratch), _p(xq_scratch))
    a._keep = (x, norm, xd, xq, xd_scratch, xq_scratch)  # the device buffers live as long as the descriptor
    return a


def _items(items):
    cm = [it[0]._c() for it in items]
    arr = (_MatItem * len(items))()
    for i, it in enumerate(items):
        arr[i].w = ctypes.pointer(cm[i])
        arr[i].bias = _p(it[1])
        arr[i].y = _p(it[2])
        arr[i].accumulate = int(bool(it[3])) if len(it) > 3 else 0
    return arr, cm


def matmul_act(items, activation):
    """smq_matmul_act: one token, the activation formed in the matmul's launch."""
    arr, _keep = _items(items)
    _check(load().smq_matmul_act(arr, len(items), ctypes.byref(activation)))


def matmul_act_rope(items, activation, shape, cos_table, sin_table, keys, values, pos0=0, pos_dev=None):
    """smq_matmul_act_rope: the q, k, v matmuls of one token, then RoPE and the cache store."""
    arr, _keep = _items(items)
    _check(load().smq_matmul_act_rope(arr, ctypes.byref(activation), ctypes.byref(shape), _p(cos_table),
                                      _p(sin_table), _p(keys), _p(values), pos0, _p(pos_dev)))


def matmul_glu(gate, up, activation, glu, h, gate_scratch=None):
    """smq_matmul_glu: h = up * act(gate) of one token (glu 1 SwiGLU, 2 GeGLU)."""
    g, u = gate._c(), up._c()
    _check(load().smq_matmul_glu(ctypes.byref(g), ctypes.byref(u), ctypes.byref(activation), glu, _p(h),
                                 _p(gate_scratch)))


def matmul_glu_q8(gate, up, activation, glu, h, hd, hq, gate_scratch=None):
    """smq_matmul_glu_q8: h = up * act(gate) and h's Q8 blocks (hd, hq) of one token."""
    g, u = gate._c(), up._c()
    _check(load().smq_matmul_glu_q8(ctypes.byref(g), ctypes.byref(u), ctypes.byref(activation), glu, _p(h), _p(hd),
                                    _p(hq), _p(gate_scratch)))


def _group_items(items):
    cm = [it[0]._c() for it in items]
    arr = (_GroupItem * len(items))()
    for i, it in enumerate(items):
        arr[i].w = ctypes.pointer(cm[i])
        arr[i].bias = _p(it[1])
        arr[i].y = _p(it[2])
        arr[i].accumulate = int(bool(it[3]))
        arr[i].xd = _p(it[4])
        arr[i].xq = _p(it[5])
    return arr, cm


def gemv_grouped(items):
    """items: sequence of (QMat, bias or None, y, accumulate, xd, xq): independent
    one-token GEMVs with their own activations, one launch."""
    arr, _keep = _group_items(items)
    _check(load().smq_gemv_grouped(arr, len(items)))


class GemvPlan:
    """smq_gemv_plan: items as for gemv_grouped (Q8 rows of 28 or 152 blocks, any number up to
    4096), split over workgroups once; launch() is one launch (capturable)."""

    def __init__(self, items):
        arr, _keep = _group_items(items)
        self._items = items  # the buffers the plan points at live as long as the plan
        h = ctypes.c_void_p()
        _check(load().smq_gemv_plan_create(arr, len(items), ctypes.byref(h)))
        self.handle = h.value

    def launch(self):
        _check(load().smq_gemv_plan_launch(self.handle))

    def destroy(self):
        if self.handle:
            load().smq_gemv_plan_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


# ---- decoder pieces (src/model.c:425-542, 669-677; src/sampler.c:57-63)
def attn_shape(heads, kv_heads, head_dim, rotary_pairs, window, context):
    return _AttnShape(heads, kv_heads, head_dim, rotary_pairs, window, context)


def rope_kv(q, k, v, ntok, shape, cos_table, sin_table, keys, values, pos0=0, pos_dev=None):
    _check(load().smq_rope_kv(_p(q), _p(k), _p(v), ntok, ctypes.byref(shape), _p(cos_table), _p(sin_table),
                              _p(keys), _p(values), pos0, _p(pos_dev)))


def attention(q, keys, values, att, ntok, shape, pos0=0, pos_dev=None):
    _check(load().smq_attention(_p(q), _p(keys), _p(values), _p(att), ntok, ctypes.byref(shape), pos0, _p(pos_dev)))


def attention_q8(q, keys, values, att, ntok, shape, xd, xq, pos0=0, pos_dev=None):
    _check(load().smq_attention_q8(_p(q), _p(keys), _p(values), _p(att), ntok, ctypes.byref(shape), pos0,
                                   _p(pos_dev), _p(xd), _p(xq)))


def attention_rope_q8(q, k, v, shape, cos_table, sin_table, keys, values, att, xd, xq, pos0=0, pos_dev=None):
    _check(load().smq_attention_rope_q8(_p(q), _p(k), _p(v), ctypes.byref(shape), _p(cos_table), _p(sin_table),
                                        _p(keys), _p(values), _p(att), pos0, _p(pos_dev), _p(xd), _p(xq)))


def argmax(logits, vocab, banned, token):
    _check(load().smq_argmax(_p(logits), vocab, _p(banned), _p(token)))


def argmax_noalloc(logits, vocab, banned, token):
    """smq_argmax_noalloc: smq_argmax with its partials in the library's static device array."""
    _check(load().smq_argmax_noalloc(_p(logits), vocab, _p(banned), _p(token)))


def embed(w, tokens, ntok, x):
    c = w._c()
    _check(load().smq_embed(ctypes.byref(c), _p(tokens), ntok, _p(x)))


def decode_advance(pos, count, token, history, capacity):
    _check(load().smq_decode_advance(_p(pos), _p(count), _p(token), _p(history), capacity))


def argmax_advance(logits, vocab, banned, token, pos, count, history, capacity):
    _check(load().smq_argmax_advance(_p(logits), vocab, _p(banned), _p(token), _p(pos), _p(count), _p(history),
                                     capacity))


def argmax_advance_embed(logits, vocab, banned, token, pos, count, history, capacity, embed, x):
    """smq_argmax_advance, then x = the embedding row (QMat `embed`) of the chosen token."""
    e = embed._c()
    _check(load().smq_argmax_advance_embed(_p(logits), vocab, _p(banned), _p(token), _p(pos), _p(count),
                                           _p(history), capacity, ctypes.byref(e), _p(x)))


def numeric_check():
    """Raises SmqError(SM_ERR_NUMERIC) if a non-finite value was seen."""
    _check(load().smq_numeric_check())


# ---- src/kernels.h:193-196
def quantize_q5_row(x, cols, out):
    """quantize_q5_row (kernels.h:205) on device buffers."""
    load().smq_quantize_q5_row(_p(x), cols, _p(out))
    _check()


def quantize_q5_rows(x, rows, cols, out):
    _check(load().smq_quantize_q5_rows(_p(x), rows, cols, _p(out)))


def dequantize_q8_row(w, cols, out):
    load().smq_dequantize_q8_row(_p(w), cols, _p(out))
    _check()


def dequantize_q5_row(w, cols, out):
    load().smq_dequantize_q5_row(_p(w), cols, _p(out))
    _check()


# ---- graphs
class Graph:
    """A captured sequence of launches on the library stream (HIP graph)."""

    def __init__(self, handle):
        self.handle = handle

    def launch(self):
        _check(load().smq_graph_launch(self.handle))

    def destroy(self):
        if self.handle:
            load().smq_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


def capture(fn):
    """Runs fn() under stream capture and returns the replayable Graph."""
    lib = load()
    _check(lib.smq_capture_begin())
    try:
        fn()
    finally:
        handle = lib.smq_capture_end()
    if not handle:
        _check()
    return Graph(handle)


# ---- timing
def timer_start():
    _check(load().smq_timer_start())


def timer_stop():
    ms = load().smq_timer_stop()
    _check()
    return ms


def stream_read(buf, nbytes, workgroups, threads, nontemporal, sink):
    """smq_stream_read: the HBM read anchor (coalesced 16-byte loads, nothing written)."""
    _check(load().smq_stream_read(_p(buf), nbytes, workgroups, threads, int(bool(nontemporal)), _p(sink)))


def grid_barrier_probe(workgroups, episodes, kind):
    """smq_grid_barrier_probe: milliseconds of one launch of `workgroups` resident workgroups passing
    `episodes` grid barriers (kind 0 one counter, 1 per-XCD counters, 2 per-workgroup flags)."""
    ms = ctypes.c_double()
    _check(load().smq_grid_barrier_probe(workgroups, episodes, kind, ctypes.byref(ms)))
    return ms.value


def stream_copy(dst, src, nbytes, workgroups, threads, nontemporal):
    """smq_stream_copy: the HBM copy anchor."""
    _check(load().smq_stream_copy(_p(dst), _p(src), nbytes, workgroups, threads, int(bool(nontemporal))))
