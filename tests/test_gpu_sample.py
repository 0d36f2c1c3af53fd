"""GPU parity of temperature sampling (edgexpu_hip_sample_softmax_dev and the
edgexpu_cpu_sample_softmax / edgexpu_cpu_softmax drop-ins, the reference's
src/cpu_kernel.c:328-353 and 762-849) against the oracle.

The bar: the generator state equal; every probability within 4 float ulp
of the oracle's (the device expf and the host libm expf differ by an ulp or
two; sums are double); the token equal to the definition's draw over the
device's own probabilities, and equal to the oracle's token where the
probabilities are well separated (a few-ulp difference cannot move the pick
across a running sum or reorder the top-p part there).
"""
import ctypes as C

import numpy as np
import pytest
import torch

import npref
import edgexpu_amd as E

pytestmark = pytest.mark.gpu

_f32p = C.POINTER(C.c_float)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_ulp(got, want, k=4):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    tol = k * np.spacing(np.abs(want).astype(np.float32)).astype(np.float64) + 1e-37
    bad = np.abs(got - want) > tol
    assert not bad.any(), f"{int(bad.sum())} probabilities off; first {np.nonzero(bad)[0][:5]}"


def dev_sample(logits, top_p, seed):
    x = torch.from_numpy(logits.copy()).to("cuda:0")
    tok, s = E.sample_softmax(x, top_p, seed)
    torch.cuda.synchronize()
    return int(tok.item()), x.cpu().numpy(), s


@pytest.mark.parametrize("n", [1, 2, 5, 257, 1000, 32000, 128256, 151936])
@pytest.mark.parametrize("top_p", [1.0, 0.9, 0.5, 0.0])
def test_sample_vs_oracle(hipdev, ora, n, top_p):
    rng = np.random.default_rng(n + int(top_p * 1000))
    for seed, scale in ((0, 1.0), (12345, 4.0), (0xDEADBEEFCAFE, 15.0)):
        logits = (rng.standard_normal(n) * scale).astype(np.float32)
        print(f"sample n={n} top_p={top_p} seed={seed}", flush=True)
        tok, p, s = dev_sample(logits, top_p, seed)
        t_o, p_o, s_o = ora.sample_softmax(logits, top_p, seed)
        assert s == s_o
        assert_ulp(p, p_o)
        assert tok == npref.draw(p, top_p, s)


@pytest.mark.parametrize("n", [2, 10, 300, 2000])
@pytest.mark.parametrize("top_p", [1.0, 0.8, 0.3])
def test_sample_token_equals_oracle(hipdev, ora, n, top_p):
    """Well-separated logits (distinct steps of 0.05): tokens equal the
    oracle's over a run of generator states."""
    rng = np.random.default_rng(n)
    logits = rng.permutation(np.arange(n, dtype=np.float32) * np.float32(0.05)).astype(np.float32)
    seed = 7
    for _ in range(25):
        tok, p, s = dev_sample(logits, top_p, seed)
        t_o, p_o, s_o = ora.sample_softmax(logits, top_p, seed)
        assert (tok, s) == (t_o, s_o)
        seed = s


def test_sample_reference_known_answers(hipdev):
    """src/cpu_kernel.c:951-968: {0, 20, 0, 0} with state 1 draws 1 (top_p
    1.0, then 0.9 with the advanced state); softmax {0, 0} = {0.5, 0.5}."""
    tok, _, s = dev_sample(np.float32([0, 20, 0, 0]), 1.0, 1)
    assert tok == 1 and s == npref.xorshift(1)
    tok, _, _ = dev_sample(np.float32([0, 20, 0, 0]), 0.9, s)
    assert tok == 1
    x = torch.zeros(2, device="cuda:0")
    E.softmax(x)
    assert np.array_equal(x.cpu().numpy(), np.float32([0.5, 0.5]))


@pytest.mark.parametrize("n", [5, 1000])
@pytest.mark.parametrize("top_p", [1.0, 0.9])
def test_sample_degenerate_scores(hipdev, ora, n, top_p):
    """All scores -inf: the reference's max is -inf, every exp is NaN, and the
    draw falls through to the last index; a single finite score wins."""
    logits = np.full(n, -np.inf, np.float32)
    tok, _, _ = dev_sample(logits, top_p, 3)
    assert tok == ora.sample_softmax(logits, top_p, 3)[0] == n - 1
    logits[n // 2] = 1.0
    tok, p, _ = dev_sample(logits, top_p, 3)
    assert tok == n // 2 and p[n // 2] == 1.0 and np.count_nonzero(p) == 1


@pytest.mark.parametrize("n", [128256, 151936])
@pytest.mark.parametrize("top_p", [0.9, 0.5, 0.05])
@pytest.mark.parametrize("kind", ["equal", "few_values", "near_uniform", "one_tail"])
def test_sample_top_p_ties_and_flat(hipdev, ora, n, top_p, kind):
    """Top-p over large vocabularies whose probabilities tie or crowd: all
    equal (the draw is the j-th index among n equal items), a few distinct
    values (tie groups of tens of thousands), nearly equal (the softmax of
    probabilities: every item in one first digit), and one large value over
    equal small ones.  The token equals the definition's draw over the
    device probabilities, over a run of generator states."""
    rng = np.random.default_rng(n + int(top_p * 100) + len(kind))
    if kind == "equal":
        logits = np.zeros(n, np.float32)
    elif kind == "few_values":
        logits = rng.integers(0, 3, n).astype(np.float32)
    elif kind == "near_uniform":
        logits = ora.softmax((rng.standard_normal(n) * 3.0).astype(np.float32))
    else:
        logits = np.zeros(n, np.float32)
        logits[n // 3] = 12.0
    seed = 11
    for _ in range(6):
        tok, p, s = dev_sample(logits, top_p, seed)
        assert tok == npref.draw(p, top_p, s), (kind, n, top_p, seed)
        seed = s


@pytest.mark.parametrize("n", [1000003, 4194305])
@pytest.mark.parametrize("kind", ["normal", "near_uniform"])
def test_sample_top_p_large_vocabulary(hipdev, ora, n, kind):
    """Top-p over vocabularies far beyond the LDS-resident case, of odd size
    (gathered keys read from memory, the tied indices gathered into LDS,
    indices of 20+ bits): the token equals the definition's draw."""
    rng = np.random.default_rng(n + len(kind))
    logits = (rng.standard_normal(n) * 3.0).astype(np.float32)
    if kind == "near_uniform":
        logits = ora.softmax(logits)
    seed = 5
    for top_p in (0.9, 0.3):
        tok, p, s = dev_sample(logits, top_p, seed)
        assert tok == npref.draw(p, top_p, s), (kind, n, top_p)
        seed = s


@pytest.mark.parametrize("n", [1, 3, 4096, 151936])
def test_softmax_vs_oracle(hipdev, ora, n):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 6.0).astype(np.float32)
    d = torch.from_numpy(x).to("cuda:0")
    E.softmax(d)
    assert_ulp(d.cpu().numpy(), ora.softmax(x))


@pytest.fixture(scope="module")
def kern(hipdev):
    k = C.CDLL(E.KERNELS_SO)
    k.edgexpu_cpu_softmax.restype = None
    k.edgexpu_cpu_softmax.argtypes = [_f32p, C.c_int]
    k.edgexpu_cpu_sample_softmax.restype = C.c_int
    k.edgexpu_cpu_sample_softmax.argtypes = [_f32p, C.c_int, C.c_float, C.POINTER(C.c_uint64),
                                             C.POINTER(C.c_uint32)]
    return k


@pytest.mark.parametrize("n,top_p", [(4, 1.0), (32000, 0.9), (128256, 1.0)])
def test_dropin_sample_softmax(kern, ora, n, top_p):
    rng = np.random.default_rng(n)
    logits = (rng.standard_normal(n) * 3.0).astype(np.float32)
    io = logits.copy()
    st = C.c_uint64(99)
    out = C.c_uint32(0)
    assert kern.edgexpu_cpu_sample_softmax(io.ctypes.data_as(_f32p), n, top_p, C.byref(st), C.byref(out)) == 1
    t_o, p_o, s_o = ora.sample_softmax(logits, top_p, 99)
    assert st.value == s_o
    assert_ulp(io, p_o)
    assert out.value == npref.draw(io, top_p, st.value)
    io = logits.copy()
    kern.edgexpu_cpu_softmax(io.ctypes.data_as(_f32p), n)
    assert_ulp(io, ora.softmax(logits))


def test_dropin_sample_bad_arguments(kern):
    io = np.zeros(4, np.float32)
    st = C.c_uint64(1)
    out = C.c_uint32(77)
    assert kern.edgexpu_cpu_sample_softmax(io.ctypes.data_as(_f32p), 0, 1.0, C.byref(st), C.byref(out)) == 0
    assert kern.edgexpu_cpu_sample_softmax(None, 4, 1.0, C.byref(st), C.byref(out)) == 0
    assert kern.edgexpu_cpu_sample_softmax(io.ctypes.data_as(_f32p), 4, 1.0, None, C.byref(out)) == 0
    assert st.value == 1 and out.value == 77
    kern.edgexpu_cpu_softmax(None, 4)
    kern.edgexpu_cpu_softmax(io.ctypes.data_as(_f32p), 0)
    assert np.array_equal(io, np.zeros(4, np.float32))


@pytest.mark.parametrize("n", [1, 1000, 128256, 3000001])
@pytest.mark.parametrize("temp", [0.7, 1.3, 3.0])
def test_temperature_division_bit_exact(hipdev, n, temp):
    """logits[i] = score / temperature (src/native.c:2339): float division,
    bit-identical to numpy's."""
    rng = np.random.default_rng(n)
    x = (rng.standard_normal(n) * 10.0).astype(np.float32)
    d = torch.from_numpy(x).to("cuda:0")
    E.div_scalar(d, temp)
    assert np.array_equal(bits(d.cpu().numpy()), bits(x / np.float32(temp)))


def test_sample_vs_golden(hipdev, golden):
    """The reference build's fixtures: state equal, probabilities within 4
    ulp, token = the definition's draw over the device probabilities, and
    the reference's token in all but a pick that lands within a few ulp of a
    running sum (at most 3 of the 60 cases)."""
    from test_oracle import _sample_cases

    g = golden("sample")
    same = total = 0
    for n, seed, top_p, x, p, tok, st in _sample_cases(g):
        t_d, p_d, s_d = dev_sample(x, top_p, seed)
        assert s_d == st
        assert_ulp(p_d, p)
        assert t_d == npref.draw(p_d, top_p, s_d), (n, seed, top_p)
        same += t_d == tok
        total += 1
    assert total == 60 and same >= total - 3
