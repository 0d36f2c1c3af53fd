"""TEST INFRASTRUCTURE ONLY: ctypes front end of the CPU oracle.

Two libraries live under ``oracle/``:

* ``liboracle.so`` -- the clean-room C restatement (``edgexpu_oracle.c``) of the
  reference quantized-weight path (src/gguf_quant.c, src/gguf_dot_q8.c,
  src/cpu_kernel.c).  Always built by ``make -C oracle``.
* ``_ref/libedgexpu_ref.so`` -- the reference's own three source files compiled
  from source (only where the reference tree is present; the built library
  travels with the working tree).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's CPU-baseline leg import
this module, and only as a checker or baseline, never as the product.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libedgexpu_ref.so")

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 8, 12, 13, 14
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)
_i32p = C.POINTER(C.c_int32)


def _p(a, t):
    return a.ctypes.data_as(t) if a is not None else None


def row_bytes(qtype: int, n: int) -> int:
    bs, bb = BLOCK[qtype]
    assert n % bs == 0
    return n // bs * bb


class _Lib:
    """Common wrapper: the oracle and the reference build share call shapes."""

    def __init__(self, path: str, prefix: str):
        self.path = path
        self.lib = C.CDLL(path)
        self.prefix = prefix

    def fn(self, name, restype, argtypes):
        f = getattr(self.lib, name)
        f.restype = restype
        f.argtypes = argtypes
        return f


def _ew_setup(obj, rms, silu, mul, add):
    """Binds the elementwise layer ops (same signatures in both libraries)."""
    L = obj.fn
    obj._rms = L(rms, None, [_f32p, _f32p, _f32p, C.c_int, C.c_float])
    obj._silu = L(silu, None, [_f32p, _f32p, C.c_int])
    obj._mul = L(mul, None, [_f32p, _f32p, _f32p, C.c_int])
    obj._add = L(add, None, [_f32p, _f32p, _f32p, C.c_int])


def _sample_setup(obj, softmax, sample):
    obj._softmax = obj.fn(softmax, None, [_f32p, C.c_int])
    obj._sample = obj.fn(sample, C.c_int, [_f32p, C.c_int, C.c_float, C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)])

    def softmax_(x):
        io = np.array(x, dtype=np.float32, copy=True)
        obj._softmax(_p(io, _f32p), io.size)
        return io

    def sample_softmax(logits, top_p, rng):
        """(token, probabilities, new rng state)."""
        io = np.array(logits, dtype=np.float32, copy=True)
        st = C.c_uint64(rng)
        out = C.c_uint32(0)
        assert obj._sample(_p(io, _f32p), io.size, C.c_float(top_p), C.byref(st), C.byref(out)) == 1
        return int(out.value), io, int(st.value)

    obj.softmax = softmax_
    obj.sample_softmax = sample_softmax


class _Elementwise:
    """rmsnorm / silu / mul / add over float32 vectors (one row at a time)."""

    def rmsnorm(self, x, w, eps):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty_like(x)
        for t in range(x.shape[0] if x.ndim == 2 else 1):
            xr = x[t] if x.ndim == 2 else x
            orow = out[t] if x.ndim == 2 else out
            self._rms(_p(orow, _f32p), _p(xr, _f32p), _p(w, _f32p), xr.size, eps)
        return out

    def silu(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        self._silu(_p(out, _f32p), _p(x, _f32p), x.size)
        return out

    def mul(self, a, b):
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        out = np.empty_like(a)
        self._mul(_p(out, _f32p), _p(a, _f32p), _p(b, _f32p), a.size)
        return out

    def add(self, a, b):
        a = np.ascontiguousarray(a, dtype=np.float32)
        b = np.ascontiguousarray(b, dtype=np.float32)
        out = np.empty_like(a)
        self._add(_p(out, _f32p), _p(a, _f32p), _p(b, _f32p), a.size)
        return out


class Oracle(_Lib, _Elementwise):
    """The clean-room restatement (``ora_*`` symbols)."""

    def __init__(self, path: str = ORACLE_SO):
        super().__init__(path, "ora_")
        L = self.fn
        self._deq = L("ora_dequantize", C.c_int, [_u8p, C.c_uint32, C.c_uint64, _f32p])
        self._q80 = L("ora_quantize_q8_0", C.c_int, [_f32p, C.c_int, _u8p])
        self._q8k = L("ora_quantize_q8_k", C.c_int, [_f32p, C.c_int, _u8p])
        self._dq8 = L("ora_dot_q8", C.c_float, [C.c_uint32, _u8p, _u8p, C.c_int])
        self._dq8k = L("ora_dot_q8k", C.c_float, [C.c_uint32, _u8p, _u8p, C.c_int])
        self._df32 = L("ora_dot_f32", C.c_float, [C.c_uint32, _u8p, _f32p, C.c_int])
        self._lin = L("ora_linear_quant_batch", C.c_int,
                      [_f32p, _f32p, _u8p, C.c_uint32, _f32p, C.c_int, C.c_int, C.c_int])
        self._logits = L("ora_logits", C.c_uint32,
                         [_f32p, _f32p, _u8p, C.c_uint32, _f32p, C.c_int, C.c_int, C.c_size_t])
        self._l80 = L("ora_q8_0_block_lanes", None, [_u8p, _u8p, _i32p])
        self._l4k = L("ora_q4_k_block_lanes", None, [_u8p, _u8p, _i32p, _i32p])
        self._l6k = L("ora_q6_k_block_lanes", None, [_u8p, _u8p, _i32p])
        self._l40 = L("ora_q4_0_block_lanes", None, [_u8p, _u8p, _i32p])
        self._l50 = L("ora_q5_0_block_lanes", None, [_u8p, _u8p, _i32p])
        self._l5k = L("ora_q5_k_block_lanes", None, [_u8p, _u8p, _i32p, _i32p])
        self._h2f = L("ora_fp16_to_fp32", C.c_float, [C.c_uint16])
        self._f2h = L("ora_fp32_to_fp16", C.c_uint16, [C.c_float])
        self._self = L("ora_selftest", C.c_int, [C.c_char_p, C.c_size_t])
        _ew_setup(self, "ora_rmsnorm", "ora_silu", "ora_mul", "ora_add")
        _sample_setup(self, "ora_softmax", "ora_sample_softmax")

    # -- codecs
    def fp16_to_fp32(self, h: int) -> float:
        return self._h2f(h)

    def fp32_to_fp16(self, f: float) -> int:
        return self._f2h(f)

    def dequantize(self, src: np.ndarray, qtype: int, n: int) -> np.ndarray:
        src = np.ascontiguousarray(src, dtype=np.uint8)
        out = np.empty(n, dtype=np.float32)
        if not self._deq(_p(src, _u8p), qtype, n, _p(out, _f32p)):
            raise ValueError("oracle dequantize rejected the arguments")
        return out

    def quantize_q8_0(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.empty(x.size // 32 * 34, dtype=np.uint8)
        if not self._q80(_p(x, _f32p), x.size, _p(out, _u8p)):
            raise ValueError("bad q8_0 input")
        return out

    def quantize_q8_k(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.empty(x.size // 256 * 292, dtype=np.uint8)
        if not self._q8k(_p(x, _f32p), x.size, _p(out, _u8p)):
            raise ValueError("bad q8_k input")
        return out

    # -- block integers
    def block_lanes(self, qtype: int, wblk: np.ndarray, xblk: np.ndarray):
        wblk = np.ascontiguousarray(wblk, dtype=np.uint8)
        xblk = np.ascontiguousarray(xblk, dtype=np.uint8)
        lanes = np.zeros(8, dtype=np.int32)
        mins = np.zeros(4, dtype=np.int32)
        if qtype == Q8_0:
            self._l80(_p(wblk, _u8p), _p(xblk, _u8p), _p(lanes, _i32p))
        elif qtype == Q4_K:
            self._l4k(_p(wblk, _u8p), _p(xblk, _u8p), _p(lanes, _i32p), _p(mins, _i32p))
        elif qtype == Q6_K:
            self._l6k(_p(wblk, _u8p), _p(xblk, _u8p), _p(lanes, _i32p))
        elif qtype == Q4_0:
            self._l40(_p(wblk, _u8p), _p(xblk, _u8p), _p(lanes, _i32p))
        elif qtype == Q5_0:
            self._l50(_p(wblk, _u8p), _p(xblk, _u8p), _p(lanes, _i32p))
        elif qtype == Q5_K:
            self._l5k(_p(wblk, _u8p), _p(xblk, _u8p), _p(lanes, _i32p), _p(mins, _i32p))
        else:
            raise ValueError(qtype)
        return lanes, mins

    # -- dots
    def dot_q8(self, qtype, wrow, xq, n):
        return self._dq8(qtype, _p(wrow, _u8p), _p(xq, _u8p), n)

    def dot_q8k(self, qtype, wrow, xq, n):
        return self._dq8k(qtype, _p(wrow, _u8p), _p(xq, _u8p), n)

    def dot_f32(self, qtype, wrow, x, n):
        x = np.ascontiguousarray(x, dtype=np.float32)
        return self._df32(qtype, _p(wrow, _u8p), _p(x, _f32p), n)

    def linear_quant_batch(self, x, w, qtype, bias, m, n_out, n_in):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        out = np.zeros((m, n_out), dtype=np.float32)
        if not self._lin(_p(out, _f32p), _p(x, _f32p), _p(w, _u8p), qtype, _p(b, _f32p), m, n_out, n_in):
            raise ValueError("oracle linear_quant_batch rejected the arguments")
        return out

    def logits(self, hidden, w, qtype, bias, vocab, n_embd, chunk_rows=0):
        hidden = np.ascontiguousarray(hidden, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        scores = np.zeros(vocab, dtype=np.float32)
        best = self._logits(_p(scores, _f32p), _p(hidden, _f32p), _p(w, _u8p), qtype, _p(b, _f32p),
                            vocab, n_embd, chunk_rows)
        return scores, int(best)

    def selftest(self):
        buf = C.create_string_buffer(256)
        ok = self._self(buf, 256)
        return bool(ok), buf.value.decode()


class Reference(_Lib, _Elementwise):
    """The reference's own kernels, compiled from source into oracle/_ref."""

    def __init__(self, path: str = REF_SO):
        super().__init__(path, "edgexpu_")
        L = self.fn
        self._deq = L("edgexpu_gguf_dequantize", C.c_int,
                      [_u8p, C.c_uint32, C.c_uint64, _f32p, C.c_char_p, C.c_size_t])
        self._q80 = L("edgexpu_gguf_quantize_q8_0", C.c_int, [_f32p, C.c_int, _u8p])
        self._q8k = L("edgexpu_gguf_quantize_q8_k", C.c_int, [_f32p, C.c_int, _u8p])
        self._dq8 = L("edgexpu_gguf_dot_quant_q8", C.c_float, [C.c_uint32, _u8p, _u8p, C.c_int])
        self._dq8k = L("edgexpu_gguf_dot_quant_q8k", C.c_float, [C.c_uint32, _u8p, _u8p, C.c_int])
        self._df32 = L("edgexpu_gguf_dot_quant", C.c_float, [C.c_uint32, _u8p, _f32p, C.c_int])
        self._lin = L("edgexpu_cpu_linear_quant_batch", None,
                      [_f32p, _f32p, _u8p, C.c_uint32, _f32p, C.c_int, C.c_int, C.c_int])
        # oracle/ref_logits.c: src/native.c's greedy logits loop over the row kernels above
        self._logits = L("edgexpu_refdrv_logits", C.c_uint32,
                         [_f32p, _f32p, _u8p, C.c_uint32, _f32p, C.c_int, C.c_int, C.c_size_t])
        self._self = L("edgexpu_gguf_quant_selftest", C.c_int, [C.c_char_p, C.c_size_t])
        _ew_setup(self, "edgexpu_cpu_rmsnorm", "edgexpu_cpu_silu", "edgexpu_cpu_mul", "edgexpu_cpu_add")
        _sample_setup(self, "edgexpu_cpu_softmax", "edgexpu_cpu_sample_softmax")

    def dequantize(self, src, qtype, n):
        src = np.ascontiguousarray(src, dtype=np.uint8)
        out = np.empty(n, dtype=np.float32)
        err = C.create_string_buffer(256)
        if not self._deq(_p(src, _u8p), qtype, n, _p(out, _f32p), err, 256):
            raise ValueError(err.value.decode(errors="replace"))
        return out

    def quantize_q8_0(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.empty(x.size // 32 * 34, dtype=np.uint8)
        assert self._q80(_p(x, _f32p), x.size, _p(out, _u8p))
        return out

    def quantize_q8_k(self, x):
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
        out = np.empty(x.size // 256 * 292, dtype=np.uint8)
        assert self._q8k(_p(x, _f32p), x.size, _p(out, _u8p))
        return out

    def dot_q8(self, qtype, wrow, xq, n):
        return self._dq8(qtype, _p(wrow, _u8p), _p(xq, _u8p), n)

    def dot_q8k(self, qtype, wrow, xq, n):
        return self._dq8k(qtype, _p(wrow, _u8p), _p(xq, _u8p), n)

    def dot_f32(self, qtype, wrow, x, n):
        x = np.ascontiguousarray(x, dtype=np.float32)
        return self._df32(qtype, _p(wrow, _u8p), _p(x, _f32p), n)

    def linear_quant_batch(self, x, w, qtype, bias, m, n_out, n_in):
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        out = np.zeros((m, n_out), dtype=np.float32)
        self._lin(_p(out, _f32p), _p(x, _f32p), _p(w, _u8p), qtype, _p(b, _f32p), m, n_out, n_in)
        return out

    def logits(self, hidden, w, qtype, bias, vocab, n_embd, chunk_rows=0):
        hidden = np.ascontiguousarray(hidden, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.uint8)
        b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
        scores = np.zeros(vocab, dtype=np.float32)
        best = self._logits(_p(scores, _f32p), _p(hidden, _f32p), _p(w, _u8p), qtype, _p(b, _f32p),
                            vocab, n_embd, chunk_rows)
        return scores, int(best)

    def selftest(self):
        buf = C.create_string_buffer(256)
        ok = self._self(buf, 256)
        return bool(ok), buf.value.decode(errors="replace")


def load_oracle() -> Oracle:
    if not os.path.exists(ORACLE_SO):
        raise FileNotFoundError(f"{ORACLE_SO} missing: run `make -C oracle`")
    return Oracle()


def load_reference():
    """The reference build, or None where it was never built."""
    return Reference() if os.path.exists(REF_SO) else None
