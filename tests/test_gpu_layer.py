"""GPU parity of the elementwise layer ops (device-resident activations).

The oracle's rmsnorm / silu / mul / add are bit-identical to the reference
build (tests/test_oracle.py).  Here the HIP versions, called through the
C-ABI, are held to:

* rmsnorm, mul, add: bit-exact against the oracle;
* silu, silu*mul: within four ulp of the oracle per element (the device
  expf is within about one ulp, the host libm's within 0.502, and the
  quotient x / (1 + e) can double a difference in e), and equal to the
  oracle on the special values.
"""
import numpy as np
import pytest
import torch

import edgexpu_amd as E

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def rows(rng, m, n):
    x = rng.normal(0, 1, (m, n)).astype(np.float32)
    if m > 1:
        x[1] *= 300.0
    if m > 2:
        x[2] *= 1e-3
    return x


@pytest.mark.parametrize("n", [576, 2560, 4096, 9728, 14336, 100])
@pytest.mark.parametrize("m", [1, 3])
@pytest.mark.parametrize("eps", [1e-5, 1e-6])
def test_rmsnorm_bit_exact(hipdev, ora, n, m, eps):
    rng = np.random.default_rng(n * 10 + m)
    x = rows(rng, m, n)
    w = rng.normal(1, 0.2, n).astype(np.float32)
    got = E.rmsnorm(dev(x), dev(w), eps).cpu().numpy()
    want = ora.rmsnorm(x, w, eps)
    assert np.array_equal(bits(got), bits(want))


def test_rmsnorm_edge_rows(hipdev, ora):
    """All-zero row (scale 1/sqrt(eps)), a single nonzero, in-place call."""
    n = 4096
    x = np.zeros((3, n), dtype=np.float32)
    x[1, 17] = -3.5
    x[2] = np.linspace(-1e4, 1e4, n, dtype=np.float32)
    w = np.linspace(0.5, 1.5, n, dtype=np.float32)
    want = ora.rmsnorm(x, w, 1e-5)
    t = dev(x)
    E.rmsnorm(t, dev(w), 1e-5, out=t)  # out == x
    assert np.array_equal(bits(t.cpu().numpy()), bits(want))


def _ulp_diff(a, b):
    """|a - b| in units of the last place of b (float32)."""
    a = a.astype(np.float64)
    bb = b.astype(np.float64)
    return np.abs(a - bb) / np.spacing(np.abs(b)).astype(np.float64)


def test_silu_within_four_ulp(hipdev, ora):
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 4, 1 << 20), rng.uniform(-90, 90, 1 << 16)]).astype(np.float32)
    got = E.silu(dev(x)).cpu().numpy()
    want = ora.silu(x)
    ok = np.isfinite(want)
    d = _ulp_diff(got[ok], want[ok])
    frac = float(np.mean(bits(got) != bits(want)))
    print(f"silu: {frac:.2e} of {x.size} elements differ from the reference, at most {d.max():.0f} ulp")
    assert np.all(d <= 4.0)


def test_silu_special_values(hipdev, ora):
    x = np.array([0.0, -0.0, 100.0, 1e30, -200.0, -1e30, 1e-30, -1e-30, np.inf, -np.inf], dtype=np.float32)
    got = E.silu(dev(x)).cpu().numpy()
    want = ora.silu(x)
    fin = np.isfinite(want)
    assert np.array_equal(bits(got[fin]), bits(want[fin]))
    nan = E.silu(dev(np.array([np.nan], dtype=np.float32))).cpu().numpy()
    assert np.isnan(nan[0])


def test_mul_add_bit_exact(hipdev, ora):
    rng = np.random.default_rng(5)
    a = rng.normal(0, 10, 1 << 18).astype(np.float32)
    b = rng.normal(0, 10, 1 << 18).astype(np.float32)
    assert np.array_equal(bits(E.mul(dev(a), dev(b)).cpu().numpy()), bits(ora.mul(a, b)))
    assert np.array_equal(bits(E.add(dev(a), dev(b)).cpu().numpy()), bits(ora.add(a, b)))


@pytest.mark.parametrize("n", [14336, 9728, 1536, 1000])
def test_silu_mul_matches_silu_then_mul(hipdev, ora, n):
    """silu(gate) * up in one pass equals the device silu followed by the
    device mul bit for bit, and the reference's two calls within five ulp."""
    rng = np.random.default_rng(n)
    g = rng.normal(0, 3, (4, n)).astype(np.float32)
    u = rng.normal(0, 3, (4, n)).astype(np.float32)
    fused = E.silu_mul(dev(g), dev(u)).cpu().numpy()
    two = E.mul(E.silu(dev(g)), dev(u)).cpu().numpy()
    assert np.array_equal(bits(fused), bits(two))
    want = ora.mul(ora.silu(g), u)
    assert np.all(_ulp_diff(fused, want) <= 5.0)


# ------------------------------------------------------------ layer_linear

from edgexpu_amd import synth  # noqa: E402

TOL = 1e-5


def _cond(ora, qt, w, x, n_out, n_in):
    """Per-output conditioning scale sum |w x| (float64) of the f32 product."""
    deq = ora.dequantize(w.reshape(-1), qt, n_out * n_in).reshape(n_out, n_in).astype(np.float64)
    return np.abs(x.astype(np.float64)) @ np.abs(deq).T


def _separate(ws, qt, x, n_outs, n_in, x2=None, nw=None, eps=1e-5, biases=None, residuals=None):
    """The same layer step as separate device calls: layer op, grouped
    projection, residual add."""
    act = x
    if nw is not None:
        act = E.rmsnorm(x, nw, eps)
    elif x2 is not None:
        act = E.silu_mul(x, x2)
    outs = E.linear_quant_group(ws, qt, act, n_outs, n_in, biases=biases)
    if residuals is not None:
        outs = [o if r is None else E.add(r, o) for o, r in zip(outs, residuals)]
    return outs


@pytest.mark.parametrize("qt,n_in,n_outs", [(12, 4096, (4096, 1024, 1024)), (12, 4096, (14336, 14336)),
                                            (8, 576, (576, 192, 192)), (14, 2560, (1000,)),
                                            (12, 14336, (4096,)), (12, 8192, (515, 33)),
                                            (12, 12288, (700, 33)), (14, 9728, (300,))])
def test_layer_linear_rmsnorm(hipdev, ora, qt, n_in, n_outs):
    """act = rmsnorm(x) in the GEMV's staging (one token): equal to the
    separate device rmsnorm + projection bit for bit, and within the bound of
    the oracle's rmsnorm + linear_quant_batch."""
    rng = np.random.default_rng(qt + n_in + len(n_outs))
    wts = [synth.np_weights(qt, n, n_in, rng) for n in n_outs]
    x = (rng.normal(0, 1, (1, n_in)) * 3).astype(np.float32)
    nw = rng.normal(1, 0.2, n_in).astype(np.float32)
    biases = [rng.normal(0, 0.5, n).astype(np.float32) for n in n_outs]
    ws = [dev(w) for w in wts]
    got = E.layer_linear(ws, qt, dev(x), n_outs, n_in, norm_weight=dev(nw), eps=1e-5,
                         biases=[dev(b) for b in biases])
    sep = _separate(ws, qt, dev(x), n_outs, n_in, nw=dev(nw), biases=[dev(b) for b in biases])
    act = ora.rmsnorm(x, nw, 1e-5)
    for z, n in enumerate(n_outs):
        g = got[z].cpu().numpy()
        assert np.array_equal(bits(g), bits(sep[z].cpu().numpy())), f"matrix {z}"
        want = ora.linear_quant_batch(act, wts[z], qt, biases[z], 1, n, n_in)
        S = _cond(ora, qt, wts[z], act, n, n_in) + np.abs(biases[z])[None, :]
        assert np.all(np.abs(g - want) <= TOL * S), f"matrix {z}"


@pytest.mark.parametrize("qt,n_in,n_out", [(12, 14336, 4096), (14, 9728, 2560), (8, 1536, 576), (12, 4096, 300),
                                           (12, 9728, 1000)])
def test_layer_linear_silu_mul_residual(hipdev, ora, qt, n_in, n_out):
    """down: act = silu(gate) * up in the staging, out = residual + proj in
    the store, written over the residual (in place)."""
    rng = np.random.default_rng(qt * 7 + n_in)
    w = synth.np_weights(qt, n_out, n_in, rng)
    g = rng.normal(0, 2, (1, n_in)).astype(np.float32)
    u = rng.normal(0, 2, (1, n_in)).astype(np.float32)
    res = rng.normal(0, 4, (1, n_out)).astype(np.float32)
    wd = dev(w)
    sep = _separate([wd], qt, dev(g), (n_out,), n_in, x2=dev(u), residuals=[dev(res)])[0].cpu().numpy()
    rt = dev(res)
    E.layer_linear([wd], qt, dev(g), (n_out,), n_in, x2=dev(u), residuals=[rt], outs=[rt])
    got = rt.cpu().numpy()
    assert np.array_equal(bits(got), bits(sep))
    act = ora.mul(ora.silu(g), u)
    want = ora.add(res, ora.linear_quant_batch(act, w, qt, None, 1, n_out, n_in))
    S = _cond(ora, qt, w, act, n_out, n_in) + np.abs(res)
    # the device silu is within two ulp of the reference's (test above): a
    # rare Q8 code one step apart moves an output by at most ~1e-5 of S
    assert np.all(np.abs(got - want) <= 2 * TOL * S)


def test_layer_linear_residual_only(hipdev, ora):
    """o: out = residual + (bias + W x), no prologue; grouped with a matrix
    that has no residual."""
    qt, n_in, n_outs = 12, 4096, (4096, 1024)
    rng = np.random.default_rng(99)
    wts = [synth.np_weights(qt, n, n_in, rng) for n in n_outs]
    x = rng.normal(0, 1, (1, n_in)).astype(np.float32)
    res = rng.normal(0, 4, (1, n_outs[0])).astype(np.float32)
    bias = [rng.normal(0, 0.5, n).astype(np.float32) for n in n_outs]
    ws = [dev(w) for w in wts]
    got = E.layer_linear(ws, qt, dev(x), n_outs, n_in, biases=[dev(b) for b in bias], residuals=[dev(res), None])
    sep = _separate(ws, qt, dev(x), n_outs, n_in, biases=[dev(b) for b in bias], residuals=[dev(res), None])
    for z in range(2):
        assert np.array_equal(bits(got[z].cpu().numpy()), bits(sep[z].cpu().numpy()))


@pytest.mark.parametrize("m", [2, 3, 70])
def test_layer_linear_steps_beyond_one_token(hipdev, ora, m):
    """More than one token: the separate-launch path (rmsnorm kernel,
    projection, add), equal to the separate device calls bit for bit."""
    qt, n_in, n_out = 12, 4096, 515
    rng = np.random.default_rng(m)
    w = synth.np_weights(qt, n_out, n_in, rng)
    x = rng.normal(0, 1, (m, n_in)).astype(np.float32)
    nw = rng.normal(1, 0.2, n_in).astype(np.float32)
    res = rng.normal(0, 4, (m, n_out)).astype(np.float32)
    wd = dev(w)
    got = E.layer_linear([wd], qt, dev(x), (n_out,), n_in, norm_weight=dev(nw), residuals=[dev(res)])[0]
    sep = _separate([wd], qt, dev(x), (n_out,), n_in, nw=dev(nw), residuals=[dev(res)])[0]
    assert np.array_equal(bits(got.cpu().numpy()), bits(sep.cpu().numpy()))
    act = ora.rmsnorm(x, nw, 1e-5)
    want = ora.add(res, ora.linear_quant_batch(act, w, qt, None, m, n_out, n_in))
    S = _cond(ora, qt, w, act, n_out, n_in) + np.abs(res)
    assert np.all(np.abs(got.cpu().numpy() - want) <= TOL * S)


def test_layer_linear_rejects_both_prologues(hipdev):
    L = E.hip()
    w = torch.zeros(2304 * 8, dtype=torch.uint8, device="cuda:0")
    x = torch.zeros((1, 4096), device="cuda:0")
    out = torch.empty((1, 8), device="cuda:0")
    import ctypes as C
    arr = C.c_void_p * 4
    ok = L.layer_linear_dev(1, arr(out.data_ptr()), x.data_ptr(), x.data_ptr(), x.data_ptr(), 1e-5,
                            arr(w.data_ptr()), 12, None, None, (C.c_int * 4)(8), 1, 4096, None)
    assert ok == 0
    code, msg = L.last_error()
    L.clear_error()
    assert "not both" in msg


@pytest.mark.parametrize("qt,n_in,n_ff", [(12, 4096, 14336), (14, 2560, 1000), (8, 576, 1536), (12, 14336, 4096),
                                          (12, 8192, 515), (12, 4096, 300), (12, 9728, 700), (14, 12288, 301)])
@pytest.mark.parametrize("norm", [True, False])
def test_gate_up_silu(hipdev, ora, qt, n_in, n_ff, norm):
    """act = silu(gate) * up from one launch (gate row j and up row j in the
    same wave): equal to the separate device steps (gate/up projection, then
    silu_mul) bit for bit, and within the bound of the oracle's composition."""
    rng = np.random.default_rng(qt * 31 + n_in + n_ff + norm)
    wg = synth.np_weights(qt, n_ff, n_in, rng)
    wu = synth.np_weights(qt, n_ff, n_in, rng)
    x = (rng.normal(0, 1, (1, n_in)) * 2).astype(np.float32)
    nw = rng.normal(1, 0.2, n_in).astype(np.float32) if norm else None
    bg = rng.normal(0, 0.5, n_ff).astype(np.float32)
    bu = rng.normal(0, 0.5, n_ff).astype(np.float32)
    dg, du = dev(wg), dev(wu)
    got = E.gate_up_silu(dg, du, qt, dev(x), n_ff, n_in, norm_weight=None if nw is None else dev(nw),
                         b_gate=dev(bg), b_up=dev(bu)).cpu().numpy()
    sep = _separate([dg, du], qt, dev(x), (n_ff, n_ff), n_in, nw=None if nw is None else dev(nw),
                    biases=[dev(bg), dev(bu)])
    two = E.silu_mul(sep[0], sep[1]).cpu().numpy()
    assert np.array_equal(bits(got), bits(two))
    a = ora.rmsnorm(x, nw, 1e-5) if norm else x
    g = ora.linear_quant_batch(a, wg, qt, bg, 1, n_ff, n_in)
    u = ora.linear_quant_batch(a, wu, qt, bu, 1, n_ff, n_in)
    want = ora.mul(ora.silu(g), u)
    # |d(silu(g) u)| <= (|silu'(g)| |u| + 1.1 |silu(g)|) * error of the products
    Sg = _cond(ora, qt, wg, a, n_ff, n_in) + np.abs(bg)[None, :]
    Su = _cond(ora, qt, wu, a, n_ff, n_in) + np.abs(bu)[None, :]
    bound = TOL * (1.2 * np.abs(u) * Sg + 1.2 * np.abs(ora.silu(g)) * Su) + 6 * np.spacing(np.abs(want))
    assert np.all(np.abs(got - want) <= bound)


def test_gate_up_silu_steps_beyond_one_token(hipdev, ora):
    qt, n_in, n_ff, m = 12, 4096, 1000, 3
    rng = np.random.default_rng(5)
    wg = synth.np_weights(qt, n_ff, n_in, rng)
    wu = synth.np_weights(qt, n_ff, n_in, rng)
    x = rng.normal(0, 1, (m, n_in)).astype(np.float32)
    nw = rng.normal(1, 0.2, n_in).astype(np.float32)
    dg, du = dev(wg), dev(wu)
    got = E.gate_up_silu(dg, du, qt, dev(x), n_ff, n_in, norm_weight=dev(nw)).cpu().numpy()
    sep = _separate([dg, du], qt, dev(x), (n_ff, n_ff), n_in, nw=dev(nw))
    assert np.array_equal(bits(got), bits(E.silu_mul(sep[0], sep[1]).cpu().numpy()))
