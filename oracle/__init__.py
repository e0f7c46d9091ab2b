"""ctypes binding of the CPU oracle (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker. The GPU
product never imports it.

``Oracle`` wraps ``liboracle.so`` (the C restatement, ``smq_oracle.c``);
``OracleModel`` runs its restated forward pass (``smq_forward.c``) over a
checkpoint's tensors. ``Reference`` wraps ``_ref/libsmref.so``: the
reference's own kernel sources compiled where they lie (``oracle/Makefile``),
present when it was built; ``ReferenceModel`` wraps ``_ref/libsmref_model.so``,
the reference's own model layer behind a small driver (``ref_model.c``).
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


class _OrcLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "ffn_norm", "q_bias", "k_bias", "v_bias", "q", "k", "v",
                                               "o", "gate", "up", "down")] + \
               [(n + "_dtype", _u32) for n in ("q", "k", "v", "o", "gate", "up", "down")]


class _OrcModel(ctypes.Structure):
    _fields_ = [(n, _u32) for n in ("dim", "hidden", "layers", "heads", "kv_heads", "head_dim", "vocab", "rotary_dim",
                                    "window", "context", "llama3_rope", "llama3_original")] + \
               [("eps", ctypes.c_float), ("theta", ctypes.c_float), ("local_theta", ctypes.c_float),
                ("rope_factor", ctypes.c_double),
                ("llama3_factor", ctypes.c_double), ("llama3_low", ctypes.c_double),
                ("llama3_high", ctypes.c_double), ("embed", ctypes.c_void_p), ("head", ctypes.c_void_p),
                ("embed_dtype", _u32), ("head_dtype", _u32), ("final_norm", ctypes.c_void_p),
                ("layer", ctypes.POINTER(_OrcLayer)), ("keys", ctypes.c_void_p), ("values", ctypes.c_void_p)]


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
        lib.orc_gemm_blockwise.argtypes = [ctypes.c_int, _u8p, _sz, _f32p, _i8p, _u32, _u32, _u32, _f32p, _sz]
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
        lib.orc_forward.restype = ctypes.c_int
        lib.orc_forward.argtypes = [ctypes.POINTER(_OrcModel), ctypes.POINTER(_u32), _u32, _u32, ctypes.c_int,
                                    _f32p]
        lib.orc_time_gemm_pass.restype = ctypes.c_double
        lib.orc_time_gemm_pass.argtypes = [ctypes.c_void_p, ctypes.POINTER(_u8p), ctypes.POINTER(_u32),
                                           ctypes.POINTER(_u32), ctypes.POINTER(_f32p), ctypes.POINTER(_i8p), _u32,
                                           _u32, _u32, _f32p, _u32, _u32, _sz, ctypes.c_void_p]

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

    def gemm_blockwise(self, w, row_bytes, xd, xq, nrows, ntok, nb, stride=None, q5=False):
        """The relaxed-order (MFMA) contract: blocks in order, acc = fmaf(ws * xs, S, acc)."""
        stride = nrows if stride is None else stride
        w = np.ascontiguousarray(w, np.uint8)
        xd = np.ascontiguousarray(xd, np.float32)
        xq = np.ascontiguousarray(xq, np.int8)
        out = np.zeros(max(1, ntok * stride), np.float32)
        self.lib.orc_gemm_blockwise(int(q5), _ptr(w, _u8p), row_bytes, _ptr(xd, _f32p), _ptr(xq, _i8p), nrows,
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
        """(best, median) wall time (s) of one pass over `mats` with a
        GemmQ8-shaped function at address `fn_addr`, rows split over
        `threads`, over `reps` passes."""
        n = len(mats)
        mp = (_u8p * n)(*[_ptr(m, _u8p) for m in mats])
        rp = (_u32 * n)(*rows)
        bp = (_u32 * n)(*nbs)
        dp = (_f32p * n)(*[_ptr(d, _f32p) for d in xds])
        qp = (_i8p * n)(*[_ptr(q, _i8p) for q in xqs])
        out = np.zeros(max(rows) * ntok, np.float32)
        times = np.zeros(max(reps, 1), np.float64)
        best = self.lib.orc_time_gemm_pass(ctypes.c_void_p(fn_addr), mp, rp, bp, dp, qp, n, ntok, block_bytes,
                                           _ptr(out, _f32p), threads, reps, scratch_bytes, times.ctypes.data)
        return best, float(np.median(times[:reps])) if reps else best

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


class OracleModel:
    """The restated forward pass (smq_forward.c) over one-expert checkpoint
    tensors. `cfg` is the config as key=value pairs (the text's keys);
    `tensors` maps names to (dtype, rows, cols, ..., array) with the array
    last (uint8 rows for Q8/Q5, float32 for F32). The KV cache lives here."""

    def __init__(self, orc, cfg, tensors, context):
        dim, heads = int(cfg["dim"]), int(cfg["heads"])
        hd = int(cfg.get("head_dim", dim // heads))
        self.orc, self.context = orc, context
        self.vocab = int(cfg["vocab_size"])
        self.layers = int(cfg["layers"])
        self.kv_dim = int(cfg["kv_heads"]) * hd
        self._keep = []

        def arr(name, dtype):
            t = tensors[name]
            a = np.ascontiguousarray(t[-1], dtype)
            self._keep.append(a)
            return a.ctypes.data, int(t[0])

        m = _OrcModel()
        m.dim, m.hidden, m.layers, m.heads = dim, int(cfg["hidden_dim"]), self.layers, heads
        m.kv_heads, m.head_dim, m.vocab = int(cfg["kv_heads"]), hd, self.vocab
        m.rotary_dim = int(cfg.get("rotary_dim", hd))
        m.window = int(cfg.get("sliding_window", 0))
        m.context = context
        # config.c parses reals with strtod and narrows eps and theta to float
        m.eps = float(np.float32(float(cfg["rms_eps"])))
        m.theta = float(np.float32(float(cfg["rope_theta"])))
        m.local_theta = float(np.float32(float(cfg.get("rope_local_theta", cfg["rope_theta"]))))
        m.rope_factor = float(cfg.get("rope_attention_factor", 1.0))
        l3 = "rope_llama3_factor" in cfg
        m.llama3_rope = int(l3)
        if l3:
            m.llama3_factor = float(cfg["rope_llama3_factor"])
            m.llama3_low = float(cfg["rope_llama3_low_freq_factor"])
            m.llama3_high = float(cfg["rope_llama3_high_freq_factor"])
            m.llama3_original = int(cfg["rope_llama3_original_context"])
        m.embed, m.embed_dtype = arr("embed", np.uint8)
        m.head, m.head_dtype = arr("lm_head" if "lm_head" in tensors else "embed", np.uint8)
        m.final_norm, _ = arr("final_norm", np.float32)
        layers = (_OrcLayer * self.layers)()
        qwen = cfg.get("architecture") == "smolmoe_qwen2"
        for i in range(self.layers):
            p, L = f"l.{i}.", layers[i]
            L.attn_norm, _ = arr(p + "attn_norm", np.float32)
            L.ffn_norm, _ = arr(p + "ffn_norm", np.float32)
            if qwen:
                L.q_bias, _ = arr(p + "q_bias", np.float32)
                L.k_bias, _ = arr(p + "k_bias", np.float32)
                L.v_bias, _ = arr(p + "v_bias", np.float32)
            for n, key in (("q", "q"), ("k", "k"), ("v", "v"), ("o", "o"), ("gate", "e.0.gate"), ("up", "e.0.up"),
                           ("down", "e.0.down")):
                ptr, dt = arr(p + key, np.uint8)
                setattr(L, n, ptr)
                setattr(L, n + "_dtype", dt)
        self.keys = np.zeros((self.layers, context, self.kv_dim), np.float32)
        self.values = np.zeros((self.layers, context, self.kv_dim), np.float32)
        m.layer = layers
        m.keys, m.values = self.keys.ctypes.data, self.values.ctypes.data
        self._layers, self._m = layers, m

    def forward(self, tokens, pos0, mode=1):
        """-> (ok, logits [rows, vocab]); ok False where the reference fails
        with SM_ERR_NUMERIC."""
        t = np.ascontiguousarray(tokens, np.uint32)
        rows = 0 if mode == 0 else (t.size if mode == 2 else 1)
        logits = np.zeros((max(rows, 1), self.vocab), np.float32)
        ok = self.orc.lib.orc_forward(ctypes.byref(self._m), _ptr(t, ctypes.POINTER(_u32)), t.size, pos0, mode,
                                      _ptr(logits, _f32p))
        if ok < 0:
            raise MemoryError("orc_forward allocation failed")
        self.last_logits = logits[rows - 1] if rows else None
        return bool(ok), logits[:rows]

    def generate(self, pos, ntokens, banned=None):
        """main.c:580-597 with temperature 0: out[0] from the last logits."""
        out = []
        for i in range(ntokens):
            out.append(self.orc.argmax(self.last_logits, banned))
            if i + 1 < ntokens:
                ok, _ = self.forward([out[-1]], pos + i, 1)
                assert ok
        return np.array(out, np.uint32)


class ReferenceModel:
    """The reference's own model layer (model.c, modelfile.c, config.c,
    sampler.c, ...) compiled from its sources with ref_model.c as driver."""

    PATH = os.path.join(HERE, "_ref", "libsmref_model.so")

    @classmethod
    def available(cls):
        return os.path.exists(cls.PATH)

    _lib = None

    @classmethod
    def _load(cls):
        if cls._lib is None:
            lib = ctypes.CDLL(cls.PATH)
            vp = ctypes.c_void_p
            lib.ref_last_error.restype = ctypes.c_char_p
            lib.ref_backend.restype = ctypes.c_char_p
            lib.ref_backend.argtypes = [ctypes.c_int, ctypes.c_int]
            lib.ref_backend_avx2.restype = ctypes.c_char_p
            lib.ref_backend_avx2.argtypes = []
            lib.ref_model_open.restype = vp
            lib.ref_model_open.argtypes = [ctypes.c_char_p, ctypes.c_char_p, _u32, _u32, _u32, _u32]
            lib.ref_model_close.argtypes = [vp]
            lib.ref_model_forward.argtypes = [vp, vp, _u32, _u32, ctypes.c_int]
            lib.ref_model_prefill.argtypes = [vp, vp, _u32, _u32, ctypes.c_int]
            lib.ref_model_logits.restype = vp
            lib.ref_model_logits.argtypes = [vp]
            lib.ref_model_kv.restype = vp
            lib.ref_model_kv.argtypes = [vp, _u32, ctypes.c_int]
            lib.ref_model_vocab.restype = _u32
            lib.ref_model_vocab.argtypes = [vp]
            lib.ref_model_set_banned.argtypes = [vp, vp]
            lib.ref_model_generate.argtypes = [vp, _u32, _u32, vp]
            lib.ref_modelfile_check.argtypes = [vp, ctypes.c_uint64, _u32]
            cls._lib = lib
        return cls._lib

    @classmethod
    def check_file(cls, data, threads=2):
        """The reference's modelfile_parse + modelfile_verify_payload over checkpoint bytes:
        (status, message)."""
        lib = cls._load()
        buf = np.frombuffer(bytes(data), np.uint8).copy()
        st = lib.ref_modelfile_check(buf.ctypes.data, buf.nbytes, threads)
        return st, (lib.ref_last_error().decode() if st else "")

    def __init__(self, path, config_path=None, context=256, batch=64, logit_rows=1, threads=1, scalar=False,
                 avx2=False):
        """avx2=True: the kernels kernels_select picks on an AVX2+F16C host without VNNI
        (RuntimeError where this CPU has no AVX2)."""
        lib = self._load()
        if avx2 and not scalar:
            b = lib.ref_backend_avx2()
            if not b:
                raise RuntimeError("this CPU has no AVX2+F16C")
            self.backend = b.decode()
        else:
            self.backend = lib.ref_backend(int(scalar), 0).decode()
        self._h = lib.ref_model_open(path.encode(), config_path.encode() if config_path else None, context, batch,
                                     logit_rows, threads)
        if not self._h:
            raise RuntimeError(lib.ref_last_error().decode())
        self.vocab = lib.ref_model_vocab(self._h)
        self.context, self.logit_rows = context, logit_rows

    def close(self):
        if self._h:
            self._lib.ref_model_close(self._h)
            self._h = None

    def _status(self, st):
        if st != 0:
            raise RuntimeError(f"status {st}: {self._lib.ref_last_error().decode()}")

    def forward(self, tokens, pos0, mode=1):
        t = np.ascontiguousarray(tokens, np.uint32)
        return self._lib.ref_model_forward(self._h, t.ctypes.data, t.size, pos0, mode)

    def prefill(self, tokens, pos0=0, last_logits=True):
        t = np.ascontiguousarray(tokens, np.uint32)
        self._status(self._lib.ref_model_prefill(self._h, t.ctypes.data, t.size, pos0, int(bool(last_logits))))

    def logits(self, rows=1):
        p = self._lib.ref_model_logits(self._h)
        return np.ctypeslib.as_array(ctypes.cast(p, _f32p), (rows, self.vocab)).copy()

    def kv(self, layer, values, positions, kv_dim):
        p = self._lib.ref_model_kv(self._h, layer, int(bool(values)))
        return np.ctypeslib.as_array(ctypes.cast(p, _f32p), (positions, kv_dim)).copy()

    def set_banned(self, banned=None):
        if banned is None:
            self._lib.ref_model_set_banned(self._h, None)
        else:
            b = np.ascontiguousarray(banned, np.uint8)
            self._lib.ref_model_set_banned(self._h, b.ctypes.data)

    def generate(self, pos, ntokens):
        out = np.zeros(ntokens, np.uint32)
        self._status(self._lib.ref_model_generate(self._h, pos, ntokens, out.ctypes.data))
        return out
