"""Python front end of the MI355X quantized-weight path.

Thin ctypes bindings over the C-ABI of ``lib/libedgexpu_hip.so`` (declared in
``include/edgexpu_hip.h``) and ``lib/libedgexpu_kernels.so`` (the reference-named
drop-in set, ``include/edgexpu_kernels.h``).  torch supplies device memory and
streams only; every computation is a HIP kernel of the shared library.  When the
library is missing this module raises instead of falling back to anything.
"""
from __future__ import annotations

import ctypes as C
import os

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
HIP_SO = os.path.join(LIB_DIR, "libedgexpu_hip.so")
KERNELS_SO = os.path.join(LIB_DIR, "libedgexpu_kernels.so")

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 8, 12, 13, 14
# (elements per block, bytes per block); Q8_K is the activation format
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q5_0: (32, 22), Q8_0: (32, 34),
         Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}
Q8_K_BLOCK = (256, 292)
TYPE_NAMES = {F32: "f32", F16: "f16", Q4_0: "q4_0", Q5_0: "q5_0", Q8_0: "q8_0", Q4_K: "q4_k",
              Q5_K: "q5_k", Q6_K: "q6_k"}


class HipError(RuntimeError):
    pass


def row_bytes(qtype: int, n: int) -> int:
    bs, bb = BLOCK[qtype]
    if n % bs:
        raise ValueError(f"n={n} not a multiple of {bs}")
    return n // bs * bb


_vp = C.c_void_p
_u8p = C.POINTER(C.c_uint8)
_f32p = C.POINTER(C.c_float)


def _sig(lib, name, restype, argtypes):
    f = getattr(lib, name)
    f.restype = restype
    f.argtypes = argtypes
    return f


class HipLib:
    """Bindings of include/edgexpu_hip.h."""

    def __init__(self, path: str = HIP_SO):
        if not os.path.exists(path):
            raise HipError(f"{path} is missing: build it with `make -C edgexpu-llm_amd` "
                           "(or __graft_entry__.build()); there is no fallback path")
        self.path = path
        self.lib = C.CDLL(path)
        L = self.lib
        self.init = _sig(L, "edgexpu_hip_init", C.c_int, [C.c_int])
        self.shutdown = _sig(L, "edgexpu_hip_shutdown", None, [])
        self._last_error = _sig(L, "edgexpu_hip_last_error", C.c_int, [C.c_char_p, C.c_size_t])
        self.clear_error = _sig(L, "edgexpu_hip_clear_error", None, [])
        self.supports_type = _sig(L, "edgexpu_hip_supports_type", C.c_int, [C.c_uint32])
        self.set_prefill_mode = _sig(L, "edgexpu_hip_set_prefill_mode", C.c_int, [C.c_int])
        self.prefill_mode = _sig(L, "edgexpu_hip_prefill_mode", C.c_int, [])
        self.set_gemv_mode = _sig(L, "edgexpu_hip_set_gemv_mode", C.c_int, [C.c_int])
        self.gemv_mode = _sig(L, "edgexpu_hip_gemv_mode", C.c_int, [])
        self.synchronize = _sig(L, "edgexpu_hip_synchronize", C.c_int, [])
        self.stream = _sig(L, "edgexpu_hip_stream", _vp, [])
        self.row_bytes = _sig(L, "edgexpu_hip_row_bytes", C.c_size_t, [C.c_uint32, C.c_int])
        self.weight_upload = _sig(L, "edgexpu_hip_weight_upload", _vp, [_vp, C.c_uint32, C.c_int, C.c_int, _vp])
        self.weight_wrap = _sig(L, "edgexpu_hip_weight_wrap", _vp, [_vp, C.c_uint32, C.c_int, C.c_int, _vp])
        self.weight_free = _sig(L, "edgexpu_hip_weight_free", None, [_vp])
        self.upload_bytes = _sig(L, "edgexpu_hip_upload_bytes", _vp, [_vp, C.c_size_t])
        self.download_bytes = _sig(L, "edgexpu_hip_download_bytes", C.c_int, [_vp, _vp, C.c_size_t])
        self.free_bytes = _sig(L, "edgexpu_hip_free_bytes", None, [_vp])
        self.linear_dev = _sig(L, "edgexpu_hip_linear_quant_batch_dev", C.c_int,
                               [_vp, _vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int, C.c_int, _vp])
        self.linear_group_dev = _sig(L, "edgexpu_hip_linear_quant_group_dev", C.c_int,
                                     [C.c_int, _vp, _vp, _vp, C.c_uint32, _vp, _vp, C.c_int, C.c_int, _vp])
        self.gemv_q8_dev = _sig(L, "edgexpu_hip_gemv_q8_dev", C.c_int,
                                [_vp, _vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int, C.c_int, _vp])
        self.logits_dev = _sig(L, "edgexpu_hip_logits_dev", C.c_int,
                               [_vp, _vp, _vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp])
        self.logits_noalloc_dev = _sig(L, "edgexpu_hip_logits_noalloc_dev", C.c_int,
                                       [_vp, _vp, _vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int, C.c_int, C.c_int, _vp])
        self.dequant_dev = _sig(L, "edgexpu_hip_dequantize_dev", C.c_int, [_vp, C.c_uint32, C.c_uint64, _vp, _vp])
        self.embed_rows_dev = _sig(L, "edgexpu_hip_embed_rows_dev", C.c_int,
                                   [_vp, _vp, C.c_uint32, C.c_longlong, C.c_int, _vp, C.c_int, _vp, _vp])
        self.sample_dev = _sig(L, "edgexpu_hip_sample_softmax_dev", C.c_int,
                               [_vp, C.c_int, C.c_float, C.POINTER(C.c_uint64), _vp, _vp])
        self.softmax_dev = _sig(L, "edgexpu_hip_softmax_dev", C.c_int, [_vp, C.c_int, _vp])
        self.div_scalar_dev = _sig(L, "edgexpu_hip_div_scalar_dev", C.c_int, [_vp, C.c_longlong, C.c_float, _vp])
        self.sample_host = _sig(L, "edgexpu_hip_sample_softmax", C.c_int,
                                [_vp, C.c_int, C.c_float, C.POINTER(C.c_uint64), C.POINTER(C.c_uint32)])
        self.softmax_host = _sig(L, "edgexpu_hip_softmax", C.c_int, [_vp, C.c_int])
        self.q80_dev = _sig(L, "edgexpu_hip_quantize_q8_0_dev", C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp])
        self.q8k_dev = _sig(L, "edgexpu_hip_quantize_q8_k_dev", C.c_int, [_vp, C.c_int, C.c_int, _vp, _vp])
        self.linear_host_w = _sig(L, "edgexpu_hip_linear_quant_batch", C.c_int, [_vp, _vp, _vp, C.c_int])
        self.linear_host = _sig(L, "edgexpu_hip_linear_quant_batch_host", C.c_int,
                                [_vp, _vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int, C.c_int])
        self.logits_host = _sig(L, "edgexpu_hip_logits", C.c_int, [_vp, C.POINTER(C.c_uint32), _vp, _vp, C.c_int])
        self.dequant_host = _sig(L, "edgexpu_hip_dequantize", C.c_int, [_vp, C.c_uint32, C.c_uint64, _vp])
        self.q80_host = _sig(L, "edgexpu_hip_quantize_q8_0", C.c_int, [_vp, C.c_int, _vp])
        self.q8k_host = _sig(L, "edgexpu_hip_quantize_q8_k", C.c_int, [_vp, C.c_int, _vp])
        self.dot_f32_rows = _sig(L, "edgexpu_hip_dot_f32_rows", C.c_int,
                                 [_vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int])
        self.dot_q8_rows = _sig(L, "edgexpu_hip_dot_q8_rows", C.c_int,
                                [_vp, _vp, C.c_uint32, _vp, C.c_int, C.c_int])
        self.rmsnorm_dev = _sig(L, "edgexpu_hip_rmsnorm_dev", C.c_int,
                                [_vp, _vp, _vp, C.c_int, C.c_int, C.c_float, _vp])
        self.silu_dev = _sig(L, "edgexpu_hip_silu_dev", C.c_int, [_vp, _vp, C.c_longlong, _vp])
        self.mul_dev = _sig(L, "edgexpu_hip_mul_dev", C.c_int, [_vp, _vp, _vp, C.c_longlong, _vp])
        self.add_dev = _sig(L, "edgexpu_hip_add_dev", C.c_int, [_vp, _vp, _vp, C.c_longlong, _vp])
        self.silu_mul_dev = _sig(L, "edgexpu_hip_silu_mul_dev", C.c_int, [_vp, _vp, _vp, C.c_longlong, _vp])
        self.gate_up_silu_dev = _sig(L, "edgexpu_hip_gate_up_silu_dev", C.c_int,
                                     [_vp, _vp, _vp, C.c_float, _vp, _vp, C.c_uint32, _vp, _vp, C.c_int, C.c_int,
                                      C.c_int, _vp])
        self.layer_linear_dev = _sig(L, "edgexpu_hip_layer_linear_dev", C.c_int,
                                     [C.c_int, _vp, _vp, _vp, _vp, C.c_float, _vp, C.c_uint32, _vp, _vp, _vp,
                                      C.c_int, C.c_int, _vp])

    def last_error(self) -> tuple[int, str]:
        buf = C.create_string_buffer(512)
        code = self._last_error(buf, 512)
        return code, buf.value.decode(errors="replace")

    def check(self, ok: int, what: str):
        if not ok:
            code, msg = self.last_error()
            self.clear_error()
            raise HipError(f"{what} failed (code {code}): {msg}")


_HIP: HipLib | None = None


def hip() -> HipLib:
    global _HIP
    if _HIP is None:
        _HIP = HipLib()
    return _HIP


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream():
    import torch

    return torch.cuda.current_stream().cuda_stream


# ---------------------------------------------------------------- device API


def linear_quant_batch(w, qtype: int, x, n_out: int, n_in: int, bias=None, out=None):
    """out[m, n_out] = bias + W · q8(x) on the GPU (edgexpu_hip_linear_quant_batch_dev).

    ``w`` is a uint8 device tensor of n_out GGUF rows, ``x`` a float32 [m, n_in]
    device tensor.  Work is queued on torch's current stream.
    """
    import torch

    m = x.shape[0]
    if out is None:
        out = torch.empty((m, n_out), dtype=torch.float32, device=x.device)
    L = hip()
    L.check(L.linear_dev(_ptr(out), _ptr(x), _ptr(w), qtype, _ptr(bias), m, n_out, n_in, _stream()),
            "linear_quant_batch")
    return out


def linear_quant_group(ws, qtype: int, x, n_outs, n_in: int, biases=None, outs=None):
    """Several projections of one input in one launch (edgexpu_hip_linear_quant_group_dev)."""
    import torch

    m = x.shape[0]
    nmat = len(ws)
    if outs is None:
        outs = [torch.empty((m, n), dtype=torch.float32, device=x.device) for n in n_outs]
    arr_p = C.c_void_p * nmat
    out_a = arr_p(*[o.data_ptr() for o in outs])
    w_a = arr_p(*[w.data_ptr() for w in ws])
    b_a = None if biases is None else arr_p(*[None if b is None else b.data_ptr() for b in biases])
    n_a = (C.c_int * nmat)(*n_outs)
    L = hip()
    L.check(L.linear_group_dev(nmat, out_a, _ptr(x), w_a, qtype, b_a, n_a, m, n_in, _stream()), "linear_quant_group")
    return outs


def gemv_q8(w, qtype: int, xq, m: int, n_out: int, n_in: int, bias=None, out=None):
    """GEMV against activations already in Q8_0 / Q8_K block bytes (edgexpu_hip_gemv_q8_dev)."""
    import torch

    if out is None:
        out = torch.empty((m, n_out), dtype=torch.float32, device=xq.device)
    L = hip()
    L.check(L.gemv_q8_dev(_ptr(out), _ptr(xq), _ptr(w), qtype, _ptr(bias), m, n_out, n_in, _stream()), "gemv_q8")
    return out


def logits(w, qtype: int, hidden, vocab: int, n_embd: int, bias=None, chunk_rows: int = 0, scores=None,
           want_best: bool = True):
    """Logits product + greedy argmax (edgexpu_hip_logits_dev); hidden is [m, n_embd]."""
    import torch

    m = hidden.shape[0] if hidden.dim() == 2 else 1
    if scores is None:
        scores = torch.empty((m, vocab), dtype=torch.float32, device=hidden.device)
    best = torch.empty(m, dtype=torch.int32, device=hidden.device) if want_best else None
    L = hip()
    L.check(L.logits_dev(_ptr(scores), _ptr(best), _ptr(hidden), _ptr(w), qtype, _ptr(bias), m, vocab, n_embd,
                         chunk_rows, _stream()), "logits")
    return scores, best


def dequantize(src, qtype: int, n: int, dst=None):
    import torch

    if dst is None:
        dst = torch.empty(n, dtype=torch.float32, device=src.device)
    L = hip()
    L.check(L.dequant_dev(_ptr(src), qtype, n, _ptr(dst), _stream()), "dequantize")
    return dst


def embed_rows(table, qtype: int, n_rows: int, n_embd: int, ids, bad=None, out=None):
    """out[len(ids), n_embd] = rows ids of the GGUF matrix `table` dequantized
    (edgexpu_hip_embed_rows_dev); ids is an int32 device tensor, bad an optional
    int32 device tensor of one element set to 1 for an index out of range."""
    import torch

    n = ids.numel()
    if out is None:
        out = torch.empty((n, n_embd), dtype=torch.float32, device=ids.device)
    L = hip()
    L.check(L.embed_rows_dev(_ptr(out), _ptr(table), qtype, n_rows, n_embd, _ptr(ids), n, _ptr(bad), _stream()),
            "embed_rows")
    return out


def sample_softmax(logits, top_p: float, rng: int, out=None):
    """Softmax of the f32 device tensor `logits` in place, then one draw
    (edgexpu_hip_sample_softmax_dev; the reference's edgexpu_cpu_sample_softmax,
    src/cpu_kernel.c:762-849).  Returns (token tensor [1] int32 on the device,
    the advanced rng state)."""
    import ctypes as C

    import torch

    if out is None:
        out = torch.empty(1, dtype=torch.int32, device=logits.device)
    state = C.c_uint64(rng)
    L = hip()
    L.check(L.sample_dev(_ptr(logits), logits.numel(), top_p, C.byref(state), _ptr(out), _stream()), "sample_softmax")
    return out, state.value


def div_scalar(io, d: float):
    """io /= d in place on the device (edgexpu_hip_div_scalar_dev: the
    temperature scaling of src/native.c:2339)."""
    L = hip()
    L.check(L.div_scalar_dev(_ptr(io), io.numel(), d, _stream()), "div_scalar")
    return io


def softmax(io):
    """Softmax of the f32 device tensor `io` in place (edgexpu_hip_softmax_dev;
    the reference's edgexpu_cpu_softmax, src/cpu_kernel.c:328-353)."""
    L = hip()
    L.check(L.softmax_dev(_ptr(io), io.numel(), _stream()), "softmax")
    return io


def quantize_q8_0(x):
    import torch

    m, n = (x.shape[0], x.shape[1]) if x.dim() == 2 else (1, x.shape[0])
    dst = torch.empty(m * (n // 32) * 34, dtype=torch.uint8, device=x.device)
    L = hip()
    L.check(L.q80_dev(_ptr(x), m, n, _ptr(dst), _stream()), "quantize_q8_0")
    return dst


def quantize_q8_k(x):
    import torch

    m, n = (x.shape[0], x.shape[1]) if x.dim() == 2 else (1, x.shape[0])
    dst = torch.empty(m * (n // 256) * 292, dtype=torch.uint8, device=x.device)
    L = hip()
    L.check(L.q8k_dev(_ptr(x), m, n, _ptr(dst), _stream()), "quantize_q8_k")
    return dst


# ------------------------------------------------------ layer elementwise ops


def rmsnorm(x, weight, eps: float, out=None):
    """RMSNorm of each row of a float32 [m, n] device tensor (edgexpu_hip_rmsnorm_dev)."""
    import torch

    m, n = x.shape
    if out is None:
        out = torch.empty_like(x)
    L = hip()
    L.check(L.rmsnorm_dev(out.data_ptr(), x.data_ptr(), weight.data_ptr(), m, n, eps, _stream()), "rmsnorm")
    return out


def _ew(fn, what, a, b=None, out=None):
    import torch

    if out is None:
        out = torch.empty_like(a)
    L = hip()
    args = [out.data_ptr(), a.data_ptr()] + ([] if b is None else [b.data_ptr()]) + [a.numel(), _stream()]
    L.check(getattr(L, fn)(*args), what)
    return out


def silu(x, out=None):
    return _ew("silu_dev", "silu", x, out=out)


def mul(a, b, out=None):
    return _ew("mul_dev", "mul", a, b, out=out)


def add(a, b, out=None):
    return _ew("add_dev", "add", a, b, out=out)


def silu_mul(gate, up, out=None):
    return _ew("silu_mul_dev", "silu_mul", gate, up, out=out)


def layer_linear(ws, qtype: int, x, n_outs, n_in: int, x2=None, norm_weight=None, eps: float = 1e-5,
                 biases=None, residuals=None, outs=None):
    """outs[z] = residuals[z] + (biases[z] + W[z] . q8(act)), act = rmsnorm(x)
    (norm_weight), silu(x) * x2 (x2) or x (edgexpu_hip_layer_linear_dev)."""
    import torch

    m = x.shape[0]
    k = len(ws)
    if outs is None:
        outs = [torch.empty((m, n), dtype=torch.float32, device=x.device) for n in n_outs]
    arr = C.c_void_p * 4
    b = None if biases is None else arr(*[_ptr(t) for t in biases])
    r = None if residuals is None else arr(*[_ptr(t) for t in residuals])
    L = hip()
    L.check(L.layer_linear_dev(k, arr(*[o.data_ptr() for o in outs]), x.data_ptr(), _ptr(x2), _ptr(norm_weight),
                               eps, arr(*[t.data_ptr() for t in ws]), qtype, b, r, (C.c_int * 4)(*n_outs), m, n_in,
                               _stream()), "layer_linear")
    return outs


def gate_up_silu(w_gate, w_up, qtype: int, x, n_ff: int, n_in: int, norm_weight=None, eps: float = 1e-5,
                 b_gate=None, b_up=None, out=None):
    """act = silu(gate(a)) * up(a), a = rmsnorm(x) or x (edgexpu_hip_gate_up_silu_dev)."""
    import torch

    m = x.shape[0]
    if out is None:
        out = torch.empty((m, n_ff), dtype=torch.float32, device=x.device)
    L = hip()
    L.check(L.gate_up_silu_dev(out.data_ptr(), x.data_ptr(), _ptr(norm_weight), eps, w_gate.data_ptr(),
                               w_up.data_ptr(), qtype, _ptr(b_gate), _ptr(b_up), m, n_ff, n_in, _stream()),
            "gate_up_silu")
    return out


# ---------------------------------------------------------------- GGUF upload


class GgufTensor(C.Structure):
    """edgexpu_gguf_up_tensor (include/edgexpu_gguf_upload.h)."""
    _fields_ = [("name", C.c_char * 96), ("n_dims", C.c_uint32), ("type", C.c_uint32),
                ("dims", C.c_uint64 * 4), ("offset", C.c_uint64), ("nbytes", C.c_uint64)]


class GgufTable(C.Structure):
    """edgexpu_gguf_up_table."""
    _fields_ = [("version", C.c_uint32), ("alignment", C.c_uint32), ("tensor_count", C.c_uint64),
                ("kv_count", C.c_uint64), ("data_offset", C.c_uint64), ("file_size", C.c_uint64),
                ("n_tensors", C.c_uint32), ("tensors", C.POINTER(GgufTensor))]


class Gguf:
    """Bindings of include/edgexpu_gguf_upload.h (libedgexpu_kernels.so)."""

    def __init__(self, path: str = KERNELS_SO):
        if not os.path.exists(path):
            raise HipError(f"{path} is missing: build it with `make -C edgexpu-llm_amd`")
        L = C.CDLL(path)
        self._read = _sig(L, "edgexpu_gguf_up_read_table", C.c_int,
                          [C.c_char_p, C.POINTER(GgufTable), C.c_char_p, C.c_size_t])
        self._free_table = _sig(L, "edgexpu_gguf_up_table_free", None, [C.POINTER(GgufTable)])
        self._upload = _sig(L, "edgexpu_gguf_device_upload", _vp, [C.c_char_p, C.c_char_p, C.c_size_t])
        self._dtable = _sig(L, "edgexpu_gguf_device_table", C.POINTER(GgufTable), [_vp])
        self._dtensor = _sig(L, "edgexpu_gguf_device_tensor", _vp, [_vp, C.c_char_p])
        self._dweight = _sig(L, "edgexpu_gguf_device_weight", _vp,
                             [_vp, C.c_char_p, C.c_int, C.c_int, C.c_char_p, C.c_size_t])
        self._dfree = _sig(L, "edgexpu_gguf_device_free", None, [_vp])

    @staticmethod
    def _table_dict(t: GgufTable) -> dict:
        tensors = []
        for i in range(t.n_tensors):
            e = t.tensors[i]
            tensors.append({"name": e.name.decode(errors="replace"), "n_dims": e.n_dims, "type": e.type,
                            "dims": list(e.dims)[:e.n_dims], "offset": e.offset, "nbytes": e.nbytes})
        return {"version": t.version, "alignment": t.alignment, "tensor_count": t.tensor_count,
                "kv_count": t.kv_count, "data_offset": t.data_offset, "file_size": t.file_size,
                "tensors": tensors}

    def read_table(self, path: str) -> dict:
        """The tensor table of a GGUF v3 file; raises ValueError with the library's message."""
        t = GgufTable()
        err = C.create_string_buffer(256)
        if not self._read(path.encode(), C.byref(t), err, 256):
            raise ValueError(err.value.decode(errors="replace"))
        try:
            return self._table_dict(t)
        finally:
            self._free_table(C.byref(t))

    def upload(self, path: str) -> int:
        """The file's data section on the GPU (an opaque model handle)."""
        err = C.create_string_buffer(256)
        h = self._upload(path.encode(), err, 256)
        if not h:
            raise ValueError(err.value.decode(errors="replace"))
        return h

    def device_table(self, h: int) -> dict:
        return self._table_dict(self._dtable(h).contents)

    def device_tensor(self, h: int, name: str) -> int | None:
        return self._dtensor(h, name.encode())

    def device_weight(self, h: int, name: str, n_out: int, n_in: int) -> int:
        err = C.create_string_buffer(256)
        w = self._dweight(h, name.encode(), n_out, n_in, err, 256)
        if not w:
            raise ValueError(err.value.decode(errors="replace"))
        return w

    def free(self, h: int):
        self._dfree(h)
