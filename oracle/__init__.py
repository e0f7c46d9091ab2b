"""ctypes binding of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The GPU
product never imports it.

``Oracle`` wraps ``liboracle.so`` (the C restatement, ``smq_oracle.c``).
``Reference`` wraps ``_ref/libsmref.so``: the reference's own kernel sources
compiled where they lie (``oracle/Makefile``), present when it was built.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
Q8_BLOCK = 36
Q5_BLOCK = 22

_u8p = ctypes.POINTER(ctypes.c_uint8)
_f32p = ctypes.POINTER(ctypes.c_float)
_i8p = ctypes.POINTER(ctypes.c_int8)
_i32p = ctypes.POINTER(ctypes.c_int32)
_u32 = ctypes.c_uint32
_sz = ctypes.c_size_t

GEMM_FN = ctypes.CFUNCTYPE(None, _u8p, _sz, _f32p, _i8p, _u32, _u32, _u32, _f32p, _sz, _u8p)


def _ptr(a, t):
    return a.ctypes.data_as(t)


def build():
    """Compile the oracle (and the reference library when its tree exists)."""
    import subprocess
    targets = ["all"]
    if os.path.isdir("/root/reference/src"):
        targets.append("ref")
    subprocess.run(["make", "-s", "-B", "-C", HERE] + targets, check=True)


class Oracle:
    """The C restatement of the reference's quantized matrix-product path."""

    def __init__(self, path=None):
        path = path or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run make -C oracle")
        lib = ctypes.CDLL(path)
        self.lib = lib
        lib.orc_f16_to_f32.restype = ctypes.c_float
        lib.orc_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.orc_f32_to_f16.restype = ctypes.c_uint16
        lib.orc_f32_to_f16.argtypes = [ctypes.c_float]
        lib.orc_quantize_q8.restype = ctypes.c_int
        lib.orc_quantize_q8.argtypes = [_f32p, _u32, _f32p, _i8p]
        for name in ("orc_dot_q8", "orc_dot_q5", "orc_dot_q8_fast", "orc_dot_q5_fast"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_float
            fn.argtypes = [_u8p, _f32p, _i8p, _u32]
        lib.orc_dot_x4.argtypes = [ctypes.c_int, ctypes.c_int, _u8p, _f32p, _i8p, _u32, _u32, _f32p]
        lib.orc_dot_r4.argtypes = [ctypes.c_int, ctypes.c_int, _u8p, _sz, _f32p, _i8p, _u32, _f32p]
        lib.orc_gemm.argtypes = [ctypes.c_int, ctypes.c_int, _u8p, _sz, _f32p, _i8p, _u32, _u32, _u32, _f32p, _sz]
        lib.orc_block_sums.argtypes = [ctypes.c_int, _u8p, _sz, _i8p, _u32, _u32, _u32, _i32p]
        lib.orc_split_range.argtypes = [_u32, _u32, _u32, ctypes.POINTER(_u32), ctypes.POINTER(_u32)]
        lib.orc_mat_item.restype = ctypes.c_int
        lib.orc_mat_item.argtypes = [ctypes.c_int, ctypes.c_int, _u8p, _sz, _u32, _f32p, _f32p, _i8p, _u32, _u32,
                                     _f32p]
        lib.orc_rmsnorm.restype = ctypes.c_int
        lib.orc_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _u32, ctypes.c_float]
        lib.orc_q8_weight_rows.argtypes = [_f32p, _u32, _u32, _u8p]
        lib.orc_quantize_q5_row.argtypes = [_f32p, _u32, _u8p]
        lib.orc_dequantize_row.argtypes = [ctypes.c_int, _u8p, _u32, _f32p]
        lib.orc_exp2_table.restype = ctypes.POINTER(ctypes.c_uint64)
        lib.orc_exp_det.restype = ctypes.c_float
        lib.orc_exp_det.argtypes = [ctypes.c_float]
        lib.orc_silu_mul.argtypes = [_f32p, _f32p, _sz]
        lib.orc_gelu_mul.argtypes = [_f32p, _f32p, _sz]
        lib.orc_row_work.restype = ctypes.c_int
        lib.orc_row_work.argtypes = [_f32p, _f32p, ctypes.c_float, _f32p, ctypes.c_int, _u32, _u32, _f32p, _f32p,
                                     _i8p]
        lib.orc_dot_f32.restype = ctypes.c_float
        lib.orc_dot_f32.argtypes = [_f32p, _f32p, _u32]
        lib.orc_rope.argtypes = [_f32p, _u32, _u32, _u32, _f32p, _f32p]
        lib.orc_attend_f32.argtypes = [_f32p, _f32p, _f32p, _u32, _u32, _u32, _u32, _f32p, _f32p]
        lib.orc_argmax.restype = _u32
        lib.orc_argmax.argtypes = [_f32p, _u32, _u8p]
        lib.orc_time_gemm_pass.restype = ctypes.c_double
        lib.orc_time_gemm_pass.argtypes = [ctypes.c_void_p, ctypes.POINTER(_u8p), ctypes.POINTER(_u32),
                                           ctypes.POINTER(_u32), ctypes.POINTER(_f32p), ctypes.POINTER(_i8p), _u32,
                                           _u32, _u32, _f32p, _u32, _u32, _sz]

    # -- binary16
    def f16_to_f32(self, h):
        return self.lib.orc_f16_to_f32(int(h))

    def f32_to_f16(self, f):
        return self.lib.orc_f32_to_f16(float(f))

    # -- activation quantizer: rows of n floats -> (status, d[rows, nb], q[rows, nb*32])
    def quantize_q8(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        rows, n = (1, x.shape[0]) if x.ndim == 1 else x.shape
        nb = (n + 31) // 32
        d = np.zeros((rows, nb), np.float32)
        q = np.zeros((rows, nb * 32), np.int8)
        status = 0
        x2 = x.reshape(rows, n)
        for r in range(rows):
            xr = np.ascontiguousarray(x2[r])
            dr = np.zeros(nb, np.float32)
            qr = np.zeros(nb * 32, np.int8)
            s = self.lib.orc_quantize_q8(_ptr(xr, _f32p), n, _ptr(dr, _f32p), _ptr(qr, _i8p))
            status = status or s
            d[r], q[r] = dr, qr
        return status, d, q

    # -- dots
    def dot(self, w, xd, xq, nb, q5=False, fast=False):
        name = "orc_dot_q5" if q5 else "orc_dot_q8"
        if fast:
            name += "_fast"
        w = np.ascontiguousarray(w, np.uint8)
        xd = np.ascontiguousarray(xd, np.float32)
        xq = np.ascontiguousarray(xq, np.int8)
        return getattr(self.lib, name)(_ptr(w, _u8p), _ptr(xd, _f32p), _ptr(xq, _i8p), nb)

    def gemm(self, w, row_bytes, xd, xq, nrows, ntok, nb, stride=None, q5=False, fast=False):
        stride = nrows if stride is None else stride
        w = np.ascontiguousarray(w, np.uint8)
        xd = np.ascontiguousarray(xd, np.float32)
        xq = np.ascontiguousarray(xq, np.int8)
        out = np.zeros(max(1, ntok * stride), np.float32)
        self.lib.orc_gemm(int(q5), int(fast), _ptr(w, _u8p), row_bytes, _ptr(xd, _f32p), _ptr(xq, _i8p), nrows,
                          ntok, nb, _ptr(out, _f32p), stride)
        return out[:ntok * stride]

    def block_sums(self, w, row_bytes, xq, nrows, ntok, nb, q5=False):
        w = np.ascontiguousarray(w, np.uint8)
        xq = np.ascontiguousarray(xq, np.int8)
        sums = np.zeros(max(1, ntok * nrows * nb), np.int32)
        self.lib.orc_block_sums(int(q5), _ptr(w, _u8p), row_bytes, _ptr(xq, _i8p), nrows, ntok, nb,
                                _ptr(sums, _i32p))
        return sums[:ntok * nrows * nb].reshape(ntok, nrows, nb)

    def mat_item(self, w, row_bytes, rows, bias, xd, xq, ntok, nb, q5=False, fast=False):
        w = np.ascontiguousarray(w, np.uint8)
        xd = np.ascontiguousarray(xd, np.float32)
        xq = np.ascontiguousarray(xq, np.int8)
        y = np.zeros(max(1, ntok * rows), np.float32)
        bp = None
        if bias is not None:
            bias = np.ascontiguousarray(bias, np.float32)
            bp = _ptr(bias, _f32p)
        ok = self.lib.orc_mat_item(int(q5), int(fast), _ptr(w, _u8p), row_bytes, rows, bp, _ptr(xd, _f32p),
                                   _ptr(xq, _i8p), ntok, nb, _ptr(y, _f32p))
        return bool(ok), y[:ntok * rows]

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = np.ascontiguousarray(w, np.float32)
        y = np.zeros_like(x)
        s = self.lib.orc_rmsnorm(_ptr(x, _f32p), _ptr(w, _f32p), _ptr(y, _f32p), x.shape[0], eps)
        return s, y

    def split_range(self, total, index, count):
        b, e = _u32(), _u32()
        self.lib.orc_split_range(total, index, count, ctypes.byref(b), ctypes.byref(e))
        return b.value, e.value

    # -- deterministic exp and gated activations
    def exp2_table(self):
        t = self.lib.orc_exp2_table()
        return [t[i] for i in range(32)]

    def exp_det(self, x):
        return self.lib.orc_exp_det(float(x))

    def act_mul(self, up, gate, gelu=False):
        up = np.array(up, np.float32, copy=True)
        gate = np.ascontiguousarray(gate, np.float32)
        fn = self.lib.orc_gelu_mul if gelu else self.lib.orc_silu_mul
        fn(_ptr(up, _f32p), _ptr(gate, _f32p), up.shape[0])
        return up

    def row_work(self, src, rows, n, norm=None, eps=1e-6, gate=None, gelu=False):
        """model.c:354-362 over `rows` rows: (ok, y, d, q)."""
        src = np.ascontiguousarray(src, np.float32)
        nb = (n + 31) // 32
        y = np.zeros(rows * n, np.float32)
        d = np.zeros(rows * nb, np.float32)
        q = np.zeros(rows * nb * 32, np.int8)
        np_ = None if norm is None else np.ascontiguousarray(norm, np.float32)
        gp = None if gate is None else np.ascontiguousarray(gate, np.float32)
        ok = self.lib.orc_row_work(_ptr(src, _f32p), None if np_ is None else _ptr(np_, _f32p), eps,
                                   None if gp is None else _ptr(gp, _f32p), int(gelu), rows, n, _ptr(y, _f32p),
                                   _ptr(d, _f32p), _ptr(q, _i8p))
        return bool(ok), y, d, q

    # -- attention pieces
    def dot_f32(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        return self.lib.orc_dot_f32(_ptr(a, _f32p), _ptr(b, _f32p), a.shape[0])

    def rope(self, x, heads, hd, pairs, cs, sn):
        x = np.array(x, np.float32, copy=True)
        cs = np.ascontiguousarray(cs, np.float32)
        sn = np.ascontiguousarray(sn, np.float32)
        self.lib.orc_rope(_ptr(x, _f32p), heads, hd, pairs, _ptr(cs, _f32p), _ptr(sn, _f32p))
        return x

    def attend_f32(self, q, keys, values, stride, hd, start, pos):
        q = np.ascontiguousarray(q, np.float32)
        keys = np.ascontiguousarray(keys, np.float32)
        values = np.ascontiguousarray(values, np.float32)
        scores = np.zeros(pos + 1, np.float32)
        out = np.zeros(hd, np.float32)
        self.lib.orc_attend_f32(_ptr(q, _f32p), _ptr(keys, _f32p), _ptr(values, _f32p), stride, hd, start, pos,
                                _ptr(scores, _f32p), _ptr(out, _f32p))
        return out

    def argmax(self, logits, banned=None):
        logits = np.ascontiguousarray(logits, np.float32)
        bp = None
        if banned is not None:
            banned = np.ascontiguousarray(banned, np.uint8)
            bp = _ptr(banned, _u8p)
        return self.lib.orc_argmax(_ptr(logits, _f32p), logits.shape[0], bp)

    # -- offline weight rules
    def q8_weight_rows(self, x):
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        nb = (cols + 31) // 32
        out = np.zeros(rows * nb * Q8_BLOCK, np.uint8)
        self.lib.orc_q8_weight_rows(_ptr(x, _f32p), rows, cols, _ptr(out, _u8p))
        return out

    def quantize_q5_rows(self, x):
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        nb = (cols + 31) // 32
        out = np.zeros((rows, nb * Q5_BLOCK), np.uint8)
        for r in range(rows):
            xr = np.ascontiguousarray(x[r])
            orow = np.zeros(nb * Q5_BLOCK, np.uint8)
            self.lib.orc_quantize_q5_row(_ptr(xr, _f32p), cols, _ptr(orow, _u8p))
            out[r] = orow
        return out.reshape(-1)

    def dequantize_row(self, w, cols, q5=False):
        w = np.ascontiguousarray(w, np.uint8)
        out = np.zeros(cols, np.float32)
        self.lib.orc_dequantize_row(int(q5), _ptr(w, _u8p), cols, _ptr(out, _f32p))
        return out

    # -- CPU baseline timing
    def time_gemm_pass(self, fn_addr, mats, rows, nbs, xds, xqs, ntok, block_bytes, threads, reps,
                       scratch_bytes=0):
        """Best wall time (s) of one pass over `mats` with a GemmQ8-shaped
        function at address `fn_addr`, rows split over `threads`."""
        n = len(mats)
        mp = (_u8p * n)(*[_ptr(m, _u8p) for m in mats])
        rp = (_u32 * n)(*rows)
        bp = (_u32 * n)(*nbs)
        dp = (_f32p * n)(*[_ptr(d, _f32p) for d in xds])
        qp = (_i8p * n)(*[_ptr(q, _i8p) for q in xqs])
        out = np.zeros(max(rows) * ntok, np.float32)
        return self.lib.orc_time_gemm_pass(ctypes.c_void_p(fn_addr), mp, rp, bp, dp, qp, n, ntok, block_bytes,
                                           _ptr(out, _f32p), threads, reps, scratch_bytes)

    def gemm_fn_addr(self, q5=False):
        fn = self.lib.orc_gemm_q5_fn if q5 else self.lib.orc_gemm_q8_fn
        return ctypes.cast(fn, ctypes.c_void_p).value


class Reference:
    """The reference's own kernels (kernels.c, kernels_x86.c, vecmath.c),
    compiled from its sources by oracle/Makefile into _ref/libsmref.so."""

    PATH = os.path.join(HERE, "_ref", "libsmref.so")

    @classmethod
    def available(cls):
        return os.path.exists(cls.PATH)

    def __init__(self):
        lib = ctypes.CDLL(self.PATH)
        self.lib = lib
        lib.quantize_q8_scalar.restype = ctypes.c_int
        lib.quantize_q8_scalar.argtypes = [_f32p, _u32, _f32p, _i8p]
        lib.quantize_q8_avx2.restype = ctypes.c_int
        lib.quantize_q8_avx2.argtypes = [_f32p, _u32, _f32p, _i8p]
        for name in ("dot_q8_scalar", "dot_q5_scalar", "dot_q8_scalar_fast", "dot_q5_scalar_fast"):
            fn = getattr(lib, name)
            fn.restype = ctypes.c_float
            fn.argtypes = [_u8p, _f32p, _i8p, _u32]
        for name in ("gemm_q8_scalar", "gemm_q5_scalar", "gemm_q8_avx2", "gemm_q5_avx2", "gemm_q8_scalar_fast",
                     "gemm_q5_scalar_fast"):
            getattr(lib, name).argtypes = [_u8p, _sz, _f32p, _i8p, _u32, _u32, _u32, _f32p, _sz, _u8p]
        lib.quantize_q5_row.argtypes = [_f32p, _u32, _u8p]
        lib.dequantize_q8_row.argtypes = [_u8p, _u32, _f32p]
        lib.dequantize_q5_row.argtypes = [_u8p, _u32, _f32p]
        lib.gemm_scratch_bytes.restype = _sz
        lib.gemm_scratch_bytes.argtypes = [_u32]
        lib.exp_det.restype = ctypes.c_float
        lib.exp_det.argtypes = [ctypes.c_float]
        lib.silu_mul_scalar.argtypes = [_f32p, _f32p, _sz]
        lib.dot_f32.restype = ctypes.c_float
        lib.dot_f32.argtypes = [_f32p, _f32p, _u32]
        lib.attend_f32_scalar.argtypes = [_f32p, _f32p, _f32p, _u32, _u32, _u32, _u32, _f32p, _f32p]
        lib.gelu_mul_scalar.argtypes = [_f32p, _f32p, _sz]

    def quantize_q8(self, x, avx2=False):
        x = np.ascontiguousarray(x, np.float32)
        n = x.shape[0]
        nb = (n + 31) // 32
        d = np.zeros(nb, np.float32)
        q = np.zeros(nb * 32, np.int8)
        fn = self.lib.quantize_q8_avx2 if avx2 else self.lib.quantize_q8_scalar
        s = fn(_ptr(x, _f32p), n, _ptr(d, _f32p), _ptr(q, _i8p))
        return s, d, q

    def gemm(self, w, row_bytes, xd, xq, nrows, ntok, nb, stride=None, q5=False, variant="scalar"):
        stride = nrows if stride is None else stride
        fn = getattr(self.lib, f"gemm_{'q5' if q5 else 'q8'}_{variant}")
        w = np.ascontiguousarray(w, np.uint8)
        xd = np.ascontiguousarray(xd, np.float32)
        xq = np.ascontiguousarray(xq, np.int8)
        out = np.zeros(max(1, ntok * stride), np.float32)
        scratch = np.zeros(self.lib.gemm_scratch_bytes(nb), np.uint8)
        fn(_ptr(w, _u8p), row_bytes, _ptr(xd, _f32p), _ptr(xq, _i8p), nrows, ntok, nb, _ptr(out, _f32p), stride,
           _ptr(scratch, _u8p))
        return out[:ntok * stride]

    def quantize_q5_row(self, x):
        x = np.ascontiguousarray(x, np.float32)
        nb = (x.shape[0] + 31) // 32
        out = np.zeros(nb * Q5_BLOCK, np.uint8)
        self.lib.quantize_q5_row(_ptr(x, _f32p), x.shape[0], _ptr(out, _u8p))
        return out

    def dequantize_row(self, w, cols, q5=False):
        w = np.ascontiguousarray(w, np.uint8)
        out = np.zeros(cols, np.float32)
        fn = self.lib.dequantize_q5_row if q5 else self.lib.dequantize_q8_row
        fn(_ptr(w, _u8p), cols, _ptr(out, _f32p))
        return out

    def exp_det(self, x):
        return self.lib.exp_det(float(x))

    def act_mul(self, up, gate, gelu=False):
        up = np.array(up, np.float32, copy=True)
        gate = np.ascontiguousarray(gate, np.float32)
        fn = self.lib.gelu_mul_scalar if gelu else self.lib.silu_mul_scalar
        fn(_ptr(up, _f32p), _ptr(gate, _f32p), up.shape[0])
        return up

    def dot_f32(self, a, b):
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        return self.lib.dot_f32(_ptr(a, _f32p), _ptr(b, _f32p), a.shape[0])

    def attend_f32(self, q, keys, values, stride, hd, start, pos):
        q = np.ascontiguousarray(q, np.float32)
        keys = np.ascontiguousarray(keys, np.float32)
        values = np.ascontiguousarray(values, np.float32)
        scores = np.zeros(pos + 1, np.float32)
        out = np.zeros(hd, np.float32)
        self.lib.attend_f32_scalar(_ptr(q, _f32p), _ptr(keys, _f32p), _ptr(values, _f32p), stride, hd, start, pos,
                                   _ptr(scores, _f32p), _ptr(out, _f32p))
        return out

    def fn_addr(self, name):
        return ctypes.cast(getattr(self.lib, name), ctypes.c_void_p).value
