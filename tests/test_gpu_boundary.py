"""GPU tests of the boundary's handle-based entry points: the drop-in weight
registry of libedgexpu_kernels.so (edgexpu_kernels_register_weight / lookup /
unregister and the registry hit inside edgexpu_cpu_linear_quant_batch), the
weight handles of libedgexpu_hip.so (edgexpu_hip_weight_upload / _wrap with
edgexpu_hip_linear_quant_batch) and the host-buffer logits entry
(edgexpu_hip_logits), each against the oracle.

Bars: fp32 outputs within TOL of the row's conditioning scale S (the sum of
|block terms| for quantized activations, sum |w x| for F32 rows) plus |bias|;
the argmax equal to the oracle's when its top two scores are further apart
than the bound.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import npref
import edgexpu_amd as E
from edgexpu_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
DEV = "cuda:0"
F32, Q8_0, Q4_K, Q6_K = 0, 8, 12, 14
_f32p = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)


def _p(a, t):
    return None if a is None else a.ctypes.data_as(t)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def scales(qt, w, x, f32_act=False):
    """S[t, i]: block-term scale of the quantized-activation dot, or sum |w x|
    for the f32-activation one (F32 rows; every logits row but Q8_0's)."""
    m = x.shape[0]
    S = np.zeros((m, w.shape[0]))
    for t in range(m):
        if qt == F32 or f32_act:
            S[t] = [npref.f32_dot_f64(qt, w[i], x[t])[1] for i in range(w.shape[0])]
            continue
        xq = npref.quantize_q8_0(x[t]) if qt == Q8_0 else npref.quantize_q8_k(x[t])
        S[t] = [npref.q8_dot_f64(qt, w[i], xq)[1] for i in range(w.shape[0])]
    return S


def assert_tol(got, want, S, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = err > TOL * S + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} outside tolerance"


@pytest.fixture(scope="module")
def kern(hipdev):
    k = C.CDLL(E.KERNELS_SO)
    k.edgexpu_cpu_linear_quant_batch.restype = None
    k.edgexpu_cpu_linear_quant_batch.argtypes = [_f32p, _f32p, _u8p, C.c_uint32, _f32p, C.c_int, C.c_int, C.c_int]
    k.edgexpu_kernels_register_weight.restype = C.c_int
    k.edgexpu_kernels_register_weight.argtypes = [_u8p, C.c_uint32, C.c_int, C.c_int, _f32p]
    k.edgexpu_kernels_unregister_weight.restype = C.c_int
    k.edgexpu_kernels_unregister_weight.argtypes = [_u8p]
    k.edgexpu_kernels_lookup_weight.restype = C.c_void_p
    k.edgexpu_kernels_lookup_weight.argtypes = [_u8p]
    return k


def _dropin(kern, w, x, qt, bias, m, n_out, n_in):
    out = np.full((m, n_out), np.nan, np.float32)
    kern.edgexpu_cpu_linear_quant_batch(_p(out, _f32p), _p(x, _f32p), _p(w, _u8p), qt, _p(bias, _f32p), m, n_out,
                                        n_in)
    return out


@pytest.mark.parametrize("qt,n_in,n_out,m", [(Q4_K, 4096, 96, 1), (Q6_K, 2560, 70, 3), (Q8_0, 576, 65, 2),
                                             (F32, 1000, 40, 1)])
def test_registry_uses_the_device_copy(kern, ora, qt, n_in, n_out, m):
    """A registered weight is served from its device copy: after the host
    bytes change, a call with the registered shape and bias pointer still
    gives the product of the bytes as registered.  A call with another bias
    pointer or another shape is no registry hit and uploads the current bytes.
    Unregistering drops the copy; NULL and duplicate registrations are refused."""
    rng = np.random.default_rng(7100 + qt + m)
    w = np.ascontiguousarray(synth.np_weights(qt, n_out, n_in, rng))
    x = np.ascontiguousarray(synth.np_activations(m, n_in, rng))
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    w0 = w.copy()
    assert kern.edgexpu_kernels_register_weight(_p(w, _u8p), qt, n_out, n_in, _p(bias, _f32p)) == 1
    try:
        assert kern.edgexpu_kernels_lookup_weight(_p(w, _u8p)) is not None
        assert kern.edgexpu_kernels_register_weight(_p(w, _u8p), qt, n_out, n_in, _p(bias, _f32p)) == 0
        assert kern.edgexpu_kernels_register_weight(None, qt, n_out, n_in, None) == 0
        # other bytes under the registered pointer: the device copy answers
        w[:] = np.ascontiguousarray(synth.np_weights(qt, n_out, n_in, rng))
        S0 = scales(qt, w0, x) + np.abs(bias)[None, :]
        want0 = ora.linear_quant_batch(x, w0, qt, bias, m, n_out, n_in)
        assert_tol(_dropin(kern, w, x, qt, bias, m, n_out, n_in), want0, S0, "registry hit")
        # another bias pointer (same values): uploaded per call, current bytes
        S1 = scales(qt, w, x) + np.abs(bias)[None, :]
        want1 = ora.linear_quant_batch(x, w, qt, bias, m, n_out, n_in)
        assert_tol(_dropin(kern, w, x, qt, bias.copy(), m, n_out, n_in), want1, S1, "other bias pointer")
        # another shape (fewer rows): uploaded per call
        want2 = ora.linear_quant_batch(x, w[: n_out - 1], qt, bias, m, n_out - 1, n_in)
        got2 = _dropin(kern, w, x, qt, bias, m, n_out - 1, n_in)
        assert_tol(got2, want2, S1[:, : n_out - 1], "other shape")
    finally:
        assert kern.edgexpu_kernels_unregister_weight(_p(w, _u8p)) == 1
    assert kern.edgexpu_kernels_lookup_weight(_p(w, _u8p)) is None
    assert kern.edgexpu_kernels_unregister_weight(_p(w, _u8p)) == 0
    # unregistered: the current bytes
    assert_tol(_dropin(kern, w, x, qt, bias, m, n_out, n_in), want1, S1, "after unregister")


@pytest.mark.parametrize("qt,n_in,n_out,m", [(Q4_K, 4096, 300, 1), (Q4_K, 2560, 129, 5), (Q6_K, 2560, 64, 2),
                                             (Q8_0, 576, 100, 4), (F32, 4096, 40, 1), (F32, 300, 17, 3)])
@pytest.mark.parametrize("wrap", [False, True])
def test_weight_handles_linear(hipdev, ora, qt, n_in, n_out, m, wrap):
    """edgexpu_hip_weight_upload (host bytes copied once) and
    edgexpu_hip_weight_wrap (device bytes not owned) behind
    edgexpu_hip_linear_quant_batch with host x and out; the handle's bias is
    applied and its accessors report what was given."""
    L = hipdev
    rng = np.random.default_rng(7300 + qt + n_out + m)
    w = np.ascontiguousarray(synth.np_weights(qt, n_out, n_in, rng))
    x = np.ascontiguousarray(synth.np_activations(m, n_in, rng))
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    if wrap:
        dw, db = dev(w), dev(bias)
        h = L.weight_wrap(dw.data_ptr(), qt, n_out, n_in, db.data_ptr())
    else:
        h = L.weight_upload(w.ctypes.data, qt, n_out, n_in, bias.ctypes.data)
    assert h, L.last_error()
    lib = L.lib
    for name, rt in (("edgexpu_hip_weight_type", C.c_uint32), ("edgexpu_hip_weight_n_out", C.c_int),
                     ("edgexpu_hip_weight_n_in", C.c_int), ("edgexpu_hip_weight_data", C.c_void_p)):
        getattr(lib, name).restype = rt
        getattr(lib, name).argtypes = [C.c_void_p]
    try:
        assert lib.edgexpu_hip_weight_type(h) == qt
        assert lib.edgexpu_hip_weight_n_out(h) == n_out and lib.edgexpu_hip_weight_n_in(h) == n_in
        data = lib.edgexpu_hip_weight_data(h)
        assert data == dw.data_ptr() if wrap else data not in (None, w.ctypes.data)
        out = np.full((m, n_out), np.nan, np.float32)
        L.check(L.linear_host_w(out.ctypes.data, x.ctypes.data, h, m), "linear_quant_batch")
    finally:
        L.weight_free(h)
    want = ora.linear_quant_batch(x, w, qt, bias, m, n_out, n_in)
    assert_tol(out, want, scales(qt, w, x) + np.abs(bias)[None, :], f"handle {qt} wrap={wrap}")


def test_weight_handles_reject_bad_arguments(hipdev):
    L = hipdev
    w = np.zeros(2304, np.uint8)
    assert not L.weight_upload(None, Q4_K, 1, 4096, None)
    assert not L.weight_upload(w.ctypes.data, Q4_K, 1, 4000, None)      # not whole super-blocks
    assert not L.weight_upload(w.ctypes.data, 5, 1, 4096, None)         # no such type
    assert not L.weight_wrap(None, Q4_K, 1, 4096, None)
    assert not L.weight_wrap(w.ctypes.data, Q4_K, 0, 4096, None)
    L.clear_error()
    out = np.zeros(4, np.float32)
    assert L.linear_host_w(out.ctypes.data, out.ctypes.data, None, 1) == 0
    L.clear_error()


@pytest.mark.parametrize("qt,n,vocab,bias_on", [(Q4_K, 4096, 20000, True), (Q6_K, 2560, 15001, False),
                                                (Q8_0, 576, 9001, True), (F32, 1000, 3001, True)])
def test_host_logits_entry(hipdev, ora, qt, n, vocab, bias_on):
    """edgexpu_hip_logits: a device-resident output weight handle, host hidden
    vector in, host scores and the greedy argmax out (src/native.c:2292-2401);
    scores may be NULL (the argmax alone)."""
    L = hipdev
    rng = np.random.default_rng(7500 + qt + vocab)
    w = np.ascontiguousarray(synth.np_weights(qt, vocab, n, rng))
    h = rng.normal(0, 1, n).astype(np.float32)
    bias = rng.normal(0, 0.01, vocab).astype(np.float32) if bias_on else None
    want, want_best = ora.logits(h, w, qt, bias, vocab, n, 0)
    hd = L.weight_upload(w.ctypes.data, qt, vocab, n, None if bias is None else bias.ctypes.data)
    assert hd, L.last_error()
    try:
        scores = np.full(vocab, np.nan, np.float32)
        best = C.c_uint32(0xFFFFFFFF)
        L.check(L.logits_host(scores.ctypes.data, C.byref(best), h.ctypes.data, hd, 0), "logits")
        best_only = C.c_uint32(0xFFFFFFFF)
        L.check(L.logits_host(None, C.byref(best_only), h.ctypes.data, hd, 8192), "logits (argmax only)")
    finally:
        L.weight_free(hd)
    sample = rng.choice(vocab, 300, replace=False)
    xs = h[None, :]
    S = scales(qt, w[sample], xs, f32_act=qt != Q8_0)[0] + (np.abs(bias[sample]) if bias is not None else 0.0)
    assert_tol(scores[sample], want[sample], S, "host logits")
    assert best.value == int(np.argmax(scores))
    assert best_only.value == best.value
    top2 = np.sort(want)[-2:]
    if top2[1] - top2[0] > 8 * TOL * S.max():
        assert best.value == want_best
