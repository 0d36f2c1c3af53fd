"""GPU parity of the HIP kernels against the oracle, through the C-ABI.

Bars (the numerics contract of the path):
  * dequant and activation quantizers: bit-exact;
  * integer block sums: exact (checked end to end with inputs whose fp32
    combination is exact, so any integer error shows as a wrong output);
  * fp32 outputs: |y - y_ref| <= TOL * S_i with S_i the row's conditioning
    scale (sum of |block terms| for the Q8 paths, sum |w_k x_k| for the f32
    logits paths), TOL = 1e-5.
"""
import numpy as np
import pytest
import torch

import npref
import oracle as O
import edgexpu_amd as E
from edgexpu_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
DEV = "cuda:0"
TN = E.TYPE_NAMES


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def q8_scales(ora, qt, w, x):
    """S_i for every (token, row): the element-level conditioning scale of
    each row's own dot (npref.q8_dot_f64), vectorized over rows."""
    m, n = x.shape
    S = np.zeros((m, w.shape[0]))
    for t in range(m):
        xq = ora.quantize_q8_0(x[t]) if qt in (2, 6, 8) else ora.quantize_q8_k(x[t])
        S[t] = npref.q8_rows_f64(qt, w, xq)[1]
    return S


def f32_scales(qt, w, h):
    """S_i = sum_k |w_ik h_k| of each row (float64), one hidden vector."""
    return npref.f32_rows_f64(qt, w, h)[1]


def assert_tol(got, want, S, what=""):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = err > TOL * S + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} outside tolerance, worst ratio {(err / np.maximum(S, 1e-30)).max():.3e}"


# ------------------------------------------------------------------ dequant


@pytest.mark.parametrize("qt", [8, 12, 14])
def test_dequant_golden_bit_exact(hipdev, golden, qt):
    g = golden(f"dequant_{TN[qt]}")
    out = E.dequantize(dev(g["src"]), qt, g["out"].size)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(g["out"]))


@pytest.mark.parametrize("qt,nblocks", [(8, 300001), (12, 40001), (14, 40003)])
def test_dequant_random_bit_exact(hipdev, ora, qt, nblocks):
    rng = np.random.default_rng(900 + qt)
    bs = {8: 32, 12: 256, 14: 256}[qt]
    src = synth.np_weights(qt, 1, nblocks * bs, rng).reshape(-1)
    out = E.dequantize(dev(src), qt, nblocks * bs)
    torch.cuda.synchronize()
    assert np.array_equal(bits(out.cpu().numpy()), bits(ora.dequantize(src, qt, nblocks * bs)))


# ------------------------------------------------------------------ quantizers


# 1 GiB of blocks per format as whole rows: floor(2^30 / block bytes) blocks
FULL_GIB = {8: (87481, 11552), 12: (372827, 5120), 14: (319566, 4096)}


@pytest.mark.parametrize("qt", [8, 12, 14])
def test_dequant_full_gib_bit_exact(hipdev, ora, qt):
    """The bulk-dequant workload at full size: 1 GiB of distinct seeded
    blocks per format dequantized on the GPU, every output word compared with
    the oracle (in chunks of ~32 MB of output)."""
    L = hipdev
    rows, n_in = FULL_GIB[qt]
    be = 32 if qt == 8 else 256
    gen = torch.Generator(device=DEV)
    gen.manual_seed(4000 + qt)
    src = synth.torch_weights_bulk(qt, rows, n_in, gen, DEV)
    assert rows * n_in // be == (1 << 30) // (src.shape[1] // (n_in // be))
    n = rows * n_in
    dst = torch.empty(n, dtype=torch.float32, device=DEV)
    L.check(L.dequant_dev(src.data_ptr(), qt, n, dst.data_ptr(), torch.cuda.current_stream().cuda_stream), "dequant")
    torch.cuda.synchronize()
    src_h = src.cpu().numpy()
    del src
    rows_per = max(1, (1 << 25) // (n_in * 4))
    for r0 in range(0, rows, rows_per):
        r1 = min(rows, r0 + rows_per)
        want = ora.dequantize(src_h[r0:r1].reshape(-1), qt, (r1 - r0) * n_in).view(np.uint32)
        got = dst[r0 * n_in:r1 * n_in].cpu().numpy().view(np.uint32)
        if not np.array_equal(got, want):
            bad = np.nonzero(got != want)[0][:5]
            raise AssertionError(f"type {qt}: rows {r0}..{r1} differ first at elements {bad.tolist()}")
    del dst
    torch.cuda.empty_cache()


def test_quantizers_golden_bit_exact(hipdev, golden):
    g = golden("quantize")
    for name, x, q80, q8k in zip(g["names"], g["x"], g["q8_0"], g["q8_k"]):
        xd = dev(x)
        assert np.array_equal(E.quantize_q8_0(xd).cpu().numpy(), q80), f"q8_0 {name}"
        assert np.array_equal(E.quantize_q8_k(xd).cpu().numpy(), q8k), f"q8_k {name}"
    xr = dev(g["x_rand"])
    assert np.array_equal(E.quantize_q8_0(xr).cpu().numpy(), g["q8_0_rand"].reshape(-1))
    assert np.array_equal(E.quantize_q8_k(xr).cpu().numpy(), g["q8_k_rand"].reshape(-1))


@pytest.mark.parametrize("n", [576, 1536, 4096, 14336])
def test_quantizers_random_bit_exact(hipdev, ora, n):
    rng = np.random.default_rng(n)
    x = (rng.normal(0, 1, (7, n)) * rng.uniform(1e-3, 1e3, (7, 1))).astype(np.float32)
    q80 = E.quantize_q8_0(dev(x)).cpu().numpy()
    assert np.array_equal(q80, np.concatenate([ora.quantize_q8_0(r) for r in x]))
    if n % 256 == 0:
        q8k = E.quantize_q8_k(dev(x)).cpu().numpy()
        assert np.array_equal(q8k, np.concatenate([ora.quantize_q8_k(r) for r in x]))


# ------------------------------------------------------------------ GEMV


LINEAR = ["linear_q8_0_576", "linear_q8_0_1536", "linear_q4_k_4096", "linear_q4_k_2560", "linear_q4_k_14336",
          "linear_q6_k_2560", "linear_q6_k_9728"]


@pytest.mark.parametrize("name", LINEAR)
def test_linear_golden(hipdev, ora, golden, name):
    g = golden(name)
    qt, w, x, bias = int(g["type"]), g["w"], g["x"], g["bias"]
    n_out, (m, n_in) = w.shape[0], x.shape
    S = q8_scales(ora, qt, w, x)
    y = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in).cpu().numpy()
    assert_tol(y, g["out"], S, name)
    yb = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    assert_tol(yb, g["out_bias"], S + np.abs(bias)[None, :], name + "+bias")


@pytest.mark.parametrize("qt,n_in,n_out", [(8, 576, 577), (8, 1536, 300), (12, 4096, 1001), (12, 2560, 515),
                                           (12, 14336, 130), (14, 2560, 260), (14, 9728, 129), (12, 256, 70),
                                           (14, 256, 33), (8, 32, 65), (12, 16384, 67), (14, 16384, 35),
                                           (12, 4352, 21), (14, 8192, 513), (12, 12288, 77), (12, 9728, 300),
                                           (14, 8448, 65)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 11])
def test_linear_random_vs_oracle(hipdev, ora, qt, n_in, n_out, m):
    rng = np.random.default_rng(qt * 1000 + n_in + n_out + m)
    w = synth.np_weights(qt, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    want = ora.linear_quant_batch(x, w, qt, bias, m, n_out, n_in)
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    S = q8_scales(ora, qt, w, x)  # each (token, row) against its own scale
    # out = bias + dot: the final addition is conditioned by |bias| too
    assert_tol(got, want, S + np.abs(bias)[None, :], f"{TN[qt]} {n_out}x{n_in} m={m}")


@pytest.mark.parametrize("qt,n_in,n_outs", [(12, 2560, (4096, 1024, 1024)), (12, 2560, (9728, 9728)),
                                            (14, 9728, (2560,)), (12, 4096, (4096, 1024, 1024))])
@pytest.mark.parametrize("m", [2, 4])
def test_multi_token_decode_shapes(hipdev, ora, qt, n_in, n_outs, m):
    """The 2- and 4-token decode launches at the shapes the hybrid ~4B step
    times them on (grouped q/k/v and gate/up over K = 2560, the Q6_K down
    [2560 x 9728]; the grouped q/k/v of the Llama-3-8B step too): every row of
    every token within 1e-5 of its own conditioning scale against the oracle
    (src/cpu_kernel.c:545-644 with its token loop at :616-627)."""
    rng = np.random.default_rng(qt * 100 + n_in + m + sum(n_outs))
    ws = [synth.np_weights(qt, n, n_in, rng) for n in n_outs]
    x = synth.np_activations(m, n_in, rng)
    outs = E.linear_quant_group([dev(w) for w in ws], qt, dev(x), list(n_outs), n_in)
    for z, (w, n) in enumerate(zip(ws, n_outs)):
        got = outs[z].cpu().numpy()
        want = ora.linear_quant_batch(x, w, qt, None, m, n, n_in)
        assert_tol(got, want, q8_scales(ora, qt, w, x), f"{TN[qt]} [{n} x {n_in}] m={m} matrix {z}")


@pytest.mark.parametrize("qt,n_in,n_out", [(12, 4096, 14336), (12, 14336, 4096), (8, 576, 49152), (14, 9728, 2560)])
def test_linear_full_shape(hipdev, ora, qt, n_in, n_out):
    """Workload shapes at full size: every row within 1e-5 of its own
    conditioning scale, against the oracle and against the float64
    restatement (exact block integers)."""
    rng = np.random.default_rng(5 + qt + n_in)
    w = synth.np_weights(qt, n_out, n_in, rng)
    x = synth.np_activations(1, n_in, rng)
    want = ora.linear_quant_batch(x, w, qt, None, 1, n_out, n_in)
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in).cpu().numpy()
    xq = ora.quantize_q8_0(x[0]) if qt == 8 else ora.quantize_q8_k(x[0])
    exact, S = npref.q8_rows_f64(qt, w, xq)
    assert_tol(want[0], exact.astype(np.float32), S, "oracle vs float64")
    assert_tol(got[0], want[0], S, f"{TN[qt]} {n_out}x{n_in} every row")


@pytest.mark.parametrize("qt", [8, 12, 14])
def test_integer_sums_exact_end_to_end(hipdev, qt):
    """Unit scales and integer activations make every fp32 step exact, so the
    output must equal the int64 closed form exactly (N2 through the kernel)."""
    rng = np.random.default_rng(60 + qt)
    n_in, n_out = (1536, 64) if qt == 8 else (2048, 64)
    w = synth.np_weights(qt, n_out, n_in, rng)
    one = np.array([1.0], np.float16).view(np.uint8)
    if qt == 8:
        wb = w.reshape(n_out, -1, 34)
        wb[:, :, 0:2] = one
        x = rng.integers(-127, 128, (1, n_in)).astype(np.float32)
        x.reshape(-1, 32)[:, 0] = 127.0  # amax 127 -> d = 1, id = 1: q = x
    elif qt == 12:
        wb = w.reshape(n_out, -1, 144)
        wb[:, :, 0:2] = one
        wb[:, :, 2:4] = one
        x = rng.integers(-127, 128, (1, n_in)).astype(np.float32)
        x.reshape(-1, 256)[:, 0] = -127.0  # first max -127 -> iscale = 1: q = x, d = 1
    else:
        wb = w.reshape(n_out, -1, 210)
        wb[:, :, 208:210] = one
        x = rng.integers(-127, 128, (1, n_in)).astype(np.float32)
        x.reshape(-1, 256)[:, 0] = -127.0
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in).cpu().numpy()[0]
    xq = npref.quantize_q8_0(x[0]) if qt == 8 else npref.quantize_q8_k(x[0])
    want = np.array([npref.q8_dot_f64(qt, w[i], xq)[0] for i in range(n_out)])
    assert np.all(np.abs(want) < 2**24)
    assert np.array_equal(got.astype(np.float64), want)


# ------------------------------------------------------------------ prefill GEMM (m >= 64)


def _q8k_rows(ora, x):
    return np.stack([ora.quantize_q8_k(x[t]) for t in range(x.shape[0])])


@pytest.mark.parametrize("n_in,n_out,m", [(4096, 300, 64), (2560, 515, 100), (256, 70, 129), (14336, 130, 64),
                                          (4096, 257, 200), (1024, 128, 128), (1280, 200, 64), (2048, 16385, 70),
                                          (4096, 300, 16), (2560, 515, 23), (14336, 260, 40), (1280, 1100, 63)])
def test_prefill_gemm_vs_oracle(hipdev, ora, n_in, n_out, m):
    """m >= 16 Q4_K products run on the matrix cores with exact block integers;
    every output within the fp32 bound of the reference (oracle) on its
    conditioning scale.  Shapes cover ragged token and row counts, one
    super-block, the K range split in two (odd super-block count 5 included)
    and unsplit (129 row blocks)."""
    rng = np.random.default_rng(900 + n_in + n_out + m)
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    want = ora.linear_quant_batch(x, w, 12, bias, m, n_out, n_in)
    got = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    exact, S = npref.q4k_q8k_gemm_f64(w, _q8k_rows(ora, x))
    # the float64 restatement agrees with the oracle to its own fp32 bound
    assert_tol(want - bias[None, :], exact.astype(np.float32), S, "oracle vs float64")
    assert_tol(got, want, S + np.abs(bias)[None, :], f"gemm {n_out}x{n_in} m={m}")


def _at_offset(w, off):
    """w's bytes on the device starting `off` bytes past a 256-byte boundary."""
    buf = torch.zeros(w.nbytes + 256, dtype=torch.uint8, device=DEV)
    view = buf[off:off + w.nbytes].view(w.shape)
    view.copy_(torch.from_numpy(np.ascontiguousarray(w)).to(DEV))
    assert view.data_ptr() % 256 == off
    return view


@pytest.mark.parametrize("qt,off", [(12, 8), (12, 4), (12, 1), (13, 3), (13, 8), (14, 2), (14, 6), (8, 2), (2, 6),
                                    (6, 2), (1, 1), (0, 2)])
@pytest.mark.parametrize("m", [1, 4, 16, 64])
def test_unaligned_weights_take_the_gemv(hipdev, ora, qt, off, m):
    """Blocks at an address the streaming and matrix-core kernels cannot read
    (Q4_K rows off 16 bytes, the repacked formats off 4) still give the
    oracle's results, decode and prefill token counts: the product takes
    the fused or plain GEMV instead.  Alone and grouped with an aligned
    matrix (K = 2560 / 4096 Q4_K rows at m = 1 would stream)."""
    n_in, n_out = (576, 300) if qt in (2, 6, 8) else (4096, 1100) if qt == 12 else (2560, 300)
    rng = np.random.default_rng(77 + qt * 10 + off + m)
    w = synth.np_weights(qt, n_out, n_in, rng)
    w2 = synth.np_weights(qt, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    want = ora.linear_quant_batch(x, w, qt, None, m, n_out, n_in)
    want2 = ora.linear_quant_batch(x, w2, qt, None, m, n_out, n_in)
    if qt in (0, 1):  # F32 / F16 rows: the f32-activation dot
        S, S2 = (np.stack([f32_scales(qt, v, x[t]) for t in range(m)]) for v in (w, w2))
    else:
        S, S2 = q8_scales(ora, qt, w, x), q8_scales(ora, qt, w2, x)
    wd = _at_offset(w, off)
    got = E.linear_quant_batch(wd, qt, dev(x), n_out, n_in).cpu().numpy()
    assert_tol(got, want, S, f"{TN[qt]} at +{off} m={m}")
    outs = E.linear_quant_group([dev(w2), wd], qt, dev(x), [n_out, n_out], n_in)
    assert_tol(outs[0].cpu().numpy(), want2, S2, f"{TN[qt]} grouped aligned m={m}")
    assert_tol(outs[1].cpu().numpy(), want, S, f"{TN[qt]} grouped at +{off} m={m}")


@pytest.mark.parametrize("qt", [8, 2, 6, 14])
def test_odd_weight_addresses_are_refused(hipdev, qt):
    """Q8_0 / Q4_0 / Q5_0 / Q6_K blocks are 2-byte-aligned formats: a device
    pointer at an odd address is refused with error -2 by every device entry
    point that reads blocks, before any launch."""
    L = hipdev
    n_in = 576 if qt in (2, 6, 8) else 2560
    rng = np.random.default_rng(qt)
    w = synth.np_weights(qt, 8, n_in, rng)
    wd = _at_offset(w, 1)
    x = dev(synth.np_activations(1, n_in, rng))
    out = torch.empty((1, 8), device=DEV)
    calls = {
        "linear_quant_batch": lambda: L.linear_dev(out.data_ptr(), x.data_ptr(), wd.data_ptr(), qt, None, 1, 8, n_in,
                                                   None),
        "logits": lambda: L.logits_dev(out.data_ptr(), None, x.data_ptr(), wd.data_ptr(), qt, None, 1, 8, n_in, 0,
                                       None),
        "dequantize": lambda: L.dequant_dev(wd.data_ptr(), qt, 8 * n_in,
                                               torch.empty(8 * n_in, device=DEV).data_ptr(), None),
    }
    for who, call in calls.items():
        assert call() == 0, who
        code, msg = L.last_error()
        assert code == -2 and "even device address" in msg, (who, msg)
        L.clear_error()
    torch.cuda.synchronize()


@pytest.mark.parametrize("n_in,n_out", [(4096, 4096), (4096, 14336), (14336, 4096)])
def test_prefill_gemm_full_shape(hipdev, ora, n_in, n_out):
    """The three prefill shapes at m = 512 against the float64 restatement
    (exact integers, float64 combine); a row sample also against the oracle."""
    m = 512
    rng = np.random.default_rng(77 + n_in + n_out)
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    got = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in).cpu().numpy()
    xq = _q8k_rows(ora, x)
    rows = np.sort(rng.choice(n_out, 256, replace=False))
    exact, S = npref.q4k_q8k_gemm_f64(w[rows], xq)
    assert_tol(got[:, rows], exact.astype(np.float32), S, f"gemm {n_out}x{n_in} m=512 (sampled rows)")
    tok = rng.choice(m, 4, replace=False)
    want = ora.linear_quant_batch(x[tok], w[rows], 12, None, 4, rows.size, n_in)
    assert_tol(got[tok][:, rows], want, S[tok], "vs oracle")


@pytest.mark.parametrize("qt", [13, 14])
@pytest.mark.parametrize("n_in,n_out,m", [(2560, 300, 16), (4096, 257, 64), (256, 70, 129), (9728, 130, 100),
                                          (1280, 515, 200), (2048, 384, 512), (1024, 16385, 33), (512, 129, 47)])
def test_prefill_gemm_kq_vs_oracle(hipdev, ora, qt, n_in, n_out, m):
    """Q6_K products from 16 tokens and Q5_K from 32 run on the matrix cores
    over a per-call repack, two exact chains per K-step (scale split
    16 s1 + s0; Q5_K at 16 tokens takes the GEMV); every
    output within the fp32 bound of the oracle on its conditioning scale.
    Shapes cover one super-block, ragged tokens and rows, the K split (odd
    super-block counts), 129 row blocks and a full 512-token block."""
    rng = np.random.default_rng(4100 + 7 * qt + n_in + n_out + m)
    w = synth.np_weights(qt, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    want = ora.linear_quant_batch(x, w, qt, bias, m, n_out, n_in)
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    exact, S = npref.kq_q8k_gemm_f64(qt, w, _q8k_rows(ora, x))
    assert_tol(want - bias[None, :], exact.astype(np.float32), S, "oracle vs float64")
    assert_tol(got, want, S + np.abs(bias)[None, :], f"{TN[qt]} gemm {n_out}x{n_in} m={m}")


@pytest.mark.parametrize("qt", [13, 14])
def test_prefill_gemm_kq_from_q8k(hipdev, ora, qt):
    """The same GEMM fed with Q8_K blocks already in memory (the activation
    pack built from the blocks, not from f32 rows): identical to the f32 entry."""
    n_in, n_out, m = 2304, 200, 40
    rng = np.random.default_rng(4400 + qt)
    w = synth.np_weights(qt, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    xq = _q8k_rows(ora, x)
    got = E.gemv_q8(dev(w), qt, dev(xq), m, n_out, n_in).cpu().numpy()
    ref = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in).cpu().numpy()
    assert np.array_equal(got, ref)
    exact, S = npref.kq_q8k_gemm_f64(qt, w, xq)
    assert_tol(got, exact.astype(np.float32), S, f"{TN[qt]} from Q8_K")


@pytest.mark.parametrize("qt", [13, 14])
def test_prefill_gemm_kq_integers_exact(hipdev, qt):
    """Unit d, zero dmin and integer activations with a first element of
    -127 (so the Q8_K codes equal x and dx = 1): every super-block integer,
    including the largest scale / quant combinations, must come out exactly."""
    n_in, n_out, m = 512, 96, 32
    rng = np.random.default_rng(4500 + qt)
    w = synth.np_weights(qt, n_out, n_in, rng)
    one = np.array([1.0], np.float16).view(np.uint8)
    if qt == 14:
        wb = w.reshape(n_out, -1, 210)
        wb[:, :, 208:210] = one
        sc = wb[:, :, 192:208].view(np.int8)
        sc[:, :, 0] = -128  # s1 = -8, s0 = 0
        sc[:, :, 1] = 127   # s1 = 7, s0 = 15
    else:
        wb = w.reshape(n_out, -1, 176)
        wb[:, :, 0:2] = one
        wb[:, :, 2:4] = 0
        wb[:, :, 4:8] = 63  # scales 0..3 at their maximum
    x = rng.integers(-127, 128, (m, n_in)).astype(np.float32)
    x.reshape(m, -1, 256)[:, :, 0] = -127.0
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in).cpu().numpy()
    xq = np.stack([npref.quantize_q8_k(x[t]) for t in range(m)])
    want, _ = npref.kq_q8k_gemm_f64(qt, w, xq)
    assert np.all(np.abs(want) < 2**24)
    assert np.array_equal(got.astype(np.float64), want)


def test_prefill_gemm_q6k_full_shape(hipdev, ora):
    """Q6_K at the [2560 x 9728] down-projection shape, m = 512: a row sample
    against the float64 restatement, a token sample also against the oracle."""
    n_in, n_out, m = 9728, 2560, 512
    rng = np.random.default_rng(4600)
    w = synth.np_weights(14, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    got = E.linear_quant_batch(dev(w), 14, dev(x), n_out, n_in).cpu().numpy()
    xq = _q8k_rows(ora, x)
    rows = np.sort(rng.choice(n_out, 192, replace=False))
    exact, S = npref.kq_q8k_gemm_f64(14, w[rows], xq)
    assert_tol(got[:, rows], exact.astype(np.float32), S, "q6_k gemm 2560x9728 m=512 (sampled rows)")
    tok = rng.choice(m, 4, replace=False)
    want = ora.linear_quant_batch(x[tok], w[rows], 14, None, 4, rows.size, n_in)
    assert_tol(got[tok][:, rows], want, S[tok], "vs oracle")


def _q80_rows(ora, x):
    return np.stack([ora.quantize_q8_0(x[t]) for t in range(x.shape[0])])


@pytest.mark.parametrize("qt", [8, 2, 6])
@pytest.mark.parametrize("n_in,n_out,m", [(576, 1536, 16), (1536, 576, 64), (4096, 257, 100), (96, 70, 129),
                                          (2048, 300, 512), (1024, 16385, 33), (160, 129, 47), (14336, 130, 20)])
def test_prefill_gemm_g32_vs_oracle(hipdev, ora, qt, n_in, n_out, m):
    """m >= 16 Q8_0 / Q4_0 / Q5_0 products run on the matrix cores over a
    per-call repack into 128-element records, one exact chain per block and
    a per-block combine; every output within the fp32 bound of the oracle on
    its conditioning scale.  Shapes: the 576 / 1536 hidden sizes, rows that
    end inside a record (96, 160, 576), the K split, 129 row blocks, a full
    512-token block."""
    rng = np.random.default_rng(4700 + 11 * qt + n_in + n_out + m)
    w = synth.np_weights(qt, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    want = ora.linear_quant_batch(x, w, qt, bias, m, n_out, n_in)
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    exact, S = npref.g32_q80_gemm_f64(qt, w, _q80_rows(ora, x))
    assert_tol(want - bias[None, :], exact.astype(np.float32), S, "oracle vs float64")
    assert_tol(got, want, S + np.abs(bias)[None, :], f"{TN[qt]} gemm {n_out}x{n_in} m={m}")


@pytest.mark.parametrize("qt", [8, 2, 6])
def test_prefill_gemm_g32_from_q80(hipdev, ora, qt):
    """The same GEMM fed with Q8_0 blocks already in memory: identical to the
    f32 entry (the packer's quantization is the Q8_0 quantizer's)."""
    n_in, n_out, m = 1248, 200, 40
    rng = np.random.default_rng(4800 + qt)
    w = synth.np_weights(qt, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    xq = _q80_rows(ora, x)
    got = E.gemv_q8(dev(w), qt, dev(xq), m, n_out, n_in).cpu().numpy()
    ref = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in).cpu().numpy()
    assert np.array_equal(got, ref)
    exact, S = npref.g32_q80_gemm_f64(qt, w, xq)
    assert_tol(got, exact.astype(np.float32), S, f"{TN[qt]} from Q8_0")


@pytest.mark.parametrize("qt", [8, 2, 6])
def test_prefill_gemm_g32_integers_exact(hipdev, qt):
    """Unit block scales and integer activations with one +-127 per block (so
    the Q8_0 codes equal x and dx = 1), the largest codes included: every
    output is an exact integer and must come out exactly."""
    n_in, n_out, m = 640, 96, 24
    rng = np.random.default_rng(4900 + qt)
    w = synth.np_weights(qt, n_out, n_in, rng)
    bb = {2: 18, 6: 22, 8: 34}[qt]
    wb = w.reshape(n_out, -1, bb)
    wb[:, :, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    if qt == 8:
        wb[:, :, 2] = 0x80  # q = -128 in the first slot of every block
    x = rng.integers(-127, 128, (m, n_in)).astype(np.float32)
    x.reshape(m, -1, 32)[:, :, 5] = 127.0
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in).cpu().numpy()
    xq = np.stack([npref.quantize_q8_0(x[t]) for t in range(m)])
    want, _ = npref.g32_q80_gemm_f64(qt, w, xq)
    assert np.all(np.abs(want) < 2**24)
    assert np.array_equal(got.astype(np.float64), want)


@pytest.mark.parametrize("n_in,n_out", [(576, 1536), (4096, 4096)])
def test_prefill_gemm_q80_full_shape(hipdev, ora, n_in, n_out):
    """Q8_0 at m = 512: a row sample against the float64 restatement, a token
    sample also against the oracle."""
    m = 512
    rng = np.random.default_rng(5000 + n_in)
    w = synth.np_weights(8, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    got = E.linear_quant_batch(dev(w), 8, dev(x), n_out, n_in).cpu().numpy()
    xq = _q80_rows(ora, x)
    rows = np.sort(rng.choice(n_out, 192, replace=False))
    exact, S = npref.g32_q80_gemm_f64(8, w[rows], xq)
    assert_tol(got[:, rows], exact.astype(np.float32), S, f"q8_0 gemm {n_out}x{n_in} m=512 (sampled rows)")
    tok = rng.choice(m, 4, replace=False)
    want = ora.linear_quant_batch(x[tok], w[rows], 8, None, 4, rows.size, n_in)
    assert_tol(got[tok][:, rows], want, S[tok], "vs oracle")


F16_TOL = 1e-3  # prefill bound for the fp16 matrix-core path (each factor rounded once to fp16)


@pytest.mark.parametrize("n_in,n_out,m", [(4096, 300, 64), (2560, 515, 100), (256, 70, 129), (14336, 130, 64),
                                          (4096, 257, 200), (2048, 260, 300), (1024, 384, 512), (1024, 136, 520)])
def test_prefill_gemm_f16_vs_oracle(hipdev, ora, n_in, n_out, m):
    """EDGEXPU_HIP_PREFILL_F16: fp16 operands, fp32 sums; every output within
    1e-3 of its conditioning scale, and typically ~2^-11 of it."""
    L = hipdev
    rng = np.random.default_rng(1900 + n_in + n_out + m)
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    want = ora.linear_quant_batch(x, w, 12, bias, m, n_out, n_in)
    assert L.set_prefill_mode(1) == 1
    try:
        got = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    finally:
        assert L.set_prefill_mode(0) == 1
    _, S = npref.q4k_q8k_gemm_f64(w, _q8k_rows(ora, x))
    err = np.abs(got.astype(np.float64) - want) / (S + np.abs(bias)[None, :])
    assert err.max() <= F16_TOL, f"worst {err.max():.3e}"
    assert np.median(err) < 1e-4


def test_prefill_gemm_f16_full_shape(hipdev, ora):
    """EDGEXPU_HIP_PREFILL_F16 at the [14336 x 4096] prefill shape, m = 512:
    a row sample within 1e-3 of its conditioning scale (float64 restatement)."""
    L = hipdev
    n_in, n_out, m = 4096, 14336, 512
    rng = np.random.default_rng(8811)
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    assert L.set_prefill_mode(1) == 1
    try:
        got = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in).cpu().numpy()
    finally:
        assert L.set_prefill_mode(0) == 1
    rows = np.sort(rng.choice(n_out, 256, replace=False))
    exact, S = npref.q4k_q8k_gemm_f64(w[rows], _q8k_rows(ora, x))
    err = np.abs(got[:, rows].astype(np.float64) - exact) / S
    assert err.max() <= F16_TOL, f"worst {err.max():.3e}"


@pytest.mark.parametrize("n_in,n_out,m", [(4096, 300, 200), (2560, 130, 64), (2048, 140, 300), (2048, 11008, 300)])
def test_prefill_gemm_f16_range(hipdev, ora, n_in, n_out, m):
    """Activations and dequantized weights far beyond fp16's 65504 (token rows
    of |x| ~ 1e7, weight rows with d = 300, dmin = 200 throughout or from the
    middle of the row on): the exact per-row power-of-two prescales keep the
    fp16 path within its bound, with the K range split over workgroups (the
    first three shapes: at most 6 output tiles) and unsplit (the last: 258
    tiles, enough workgroups without a split)."""
    L = hipdev
    rng = np.random.default_rng(2300 + n_in + m)
    w = synth.np_weights(12, n_out, n_in, rng).copy()
    rb = w.shape[1]
    big = np.frombuffer(np.array([300.0, 200.0], dtype=np.float16).tobytes(), dtype=np.uint8)
    nb = n_in // 256
    for o, first in ((5, 0), (n_out - 1, nb // 2)):  # the second from mid-row on
        for sb in range(first, nb):
            w[o, sb * 144:sb * 144 + 4] = big
    x = synth.np_activations(m, n_in, rng)
    x[3] *= 5e6
    x[m - 1] *= 2e6
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    want = ora.linear_quant_batch(x, w, 12, bias, m, n_out, n_in)
    assert np.isfinite(want).all()
    assert L.set_prefill_mode(1) == 1
    try:
        got = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    finally:
        assert L.set_prefill_mode(0) == 1
    assert np.isfinite(got).all()
    _, S = npref.q4k_q8k_gemm_f64(w, _q8k_rows(ora, x))
    err = np.abs(got.astype(np.float64) - want) / (S + np.abs(bias)[None, :])
    assert err.max() <= F16_TOL, f"worst {err.max():.3e} at {np.unravel_index(err.argmax(), err.shape)}"


def test_prefill_mode_switch(hipdev):
    L = hipdev
    assert L.prefill_mode() == 0
    assert L.set_prefill_mode(7) == 0
    L.clear_error()
    assert L.prefill_mode() == 0


def test_prefill_equals_decode_rows(hipdev, ora):
    """Prefill (matrix cores) and decode (GEMV) agree per token to the bound."""
    rng = np.random.default_rng(4242)
    n_in, n_out, m = 4096, 512, 96
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    big = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in).cpu().numpy()
    _, S = npref.q4k_q8k_gemm_f64(w, _q8k_rows(ora, x))
    for t in (0, 37, 95):
        one = E.linear_quant_batch(dev(w), 12, dev(x[t:t + 1]), n_out, n_in).cpu().numpy()[0]
        assert_tol(big[t], one, 2 * S[t], f"token {t}")


def _q4k_headers(w, d, dmin):
    hb = np.frombuffer(np.array([d, dmin], dtype=np.float16).tobytes(), dtype=np.uint8)
    wb = w.reshape(w.shape[0], -1, 144)
    wb[:, :, 0:4] = hb
    return w


@pytest.mark.parametrize("n_in,n_out,m", [(2048, 256, 64), (2048, 4224, 512)])
def test_prefill_gemm_integers_exact(hipdev, n_in, n_out, m):
    """Unit scales (d = dmin = 1) and integer activations that are their own
    Q8_K codes (each block's first element -127: d = 1): every fp32 step of the
    GEMM is then exact, so the output equals the int64 closed form exactly --
    the block integers are exact through the matrix cores, with the K range
    split in two (2 tiles) and unsplit (132 tiles)."""
    rng = np.random.default_rng(5150 + n_out)
    w = _q4k_headers(synth.np_weights(12, n_out, n_in, rng), 1.0, 1.0)
    x = rng.integers(-127, 128, (m, n_in)).astype(np.float32)
    x.reshape(m, -1, 256)[:, :, 0] = -127.0
    got = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in).cpu().numpy()
    xq = np.stack([npref.quantize_q8_k(x[t]) for t in range(m)])
    want, _ = npref.q4k_q8k_gemm_f64(w, xq)
    assert np.abs(want).max() < 2**24
    assert np.array_equal(got.astype(np.float64), want)


def test_prefill_gemm_two_chains(hipdev, ora):
    """Tokens whose Q8_K codes are all +-127 (sum |q8| = 32512 per super-block,
    beyond the 17753 one exact chain allows) run every super-block as two
    chains; rows with every scale and min 63 and every code 15 push sumi to
    30.7 M.  Mixed with ordinary tokens in other workgroups' token blocks.
    Outputs within the bound of the float64 restatement and of the oracle."""
    rng = np.random.default_rng(6161)
    n_in, n_out, m = 2048, 300, 200
    w = synth.np_weights(12, n_out, n_in, rng)
    for o in (0, 1, 150, n_out - 1):
        wb = w[o].reshape(-1, 144)
        wb[:, 4:144] = 0xFF
    x = synth.np_activations(m, n_in, rng)
    x[:128] = np.where(rng.random((128, n_in)) < 0.5, -1.0, 1.0).astype(np.float32)
    x[:128] *= rng.uniform(0.5, 2.0, (128, 1)).astype(np.float32)
    got = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in).cpu().numpy()
    xq = _q8k_rows(ora, x)
    exact, S = npref.q4k_q8k_gemm_f64(w, xq)
    assert_tol(got, exact.astype(np.float32), S, "two chains vs float64")
    want = ora.linear_quant_batch(x[:4], w, 12, None, 4, n_out, n_in)
    assert_tol(got[:4], want, S[:4], "two chains vs oracle")


@pytest.mark.parametrize("qt", [12, 13, 14])
def test_prefill_pack_special_blocks(hipdev, ora, qt):
    """The f32 activation pack of the K-quant prefill GEMMs (four tokens per
    wavefront) quantizes as the reference's quantize_row_q8_K does
    (src/gguf_dot_q8.c:360-412) up to the sign of a block's codes and scale,
    which cancels in the GEMM: the GEMM over it equals, bit for bit, the GEMM
    over the oracle's Q8_K bytes of the same activations.  Blocks: all
    zero, the largest magnitude twice with opposite signs (negative first,
    positive first, in one lane and in lanes far apart), NaN elements, -0.0
    and subnormals, codes at exact .5 ties, a block whose maximum is its last
    element, and a token count that leaves a wavefront's last tokens past m."""
    rng = np.random.default_rng(4242 + qt)
    n_in, n_out, m = 1024, 96, 37
    x = synth.np_activations(m, n_in, rng)
    x[0, 0:256] = 0.0                                   # all-zero block
    x[1, 256:512] = -0.0
    x[1, 256 + 77] = np.float32(1e-40)                  # only a subnormal
    x[2, 0:256] = rng.uniform(-1, 1, 256)
    x[2, 10], x[2, 200] = -3.0, 3.0                      # tie, negative first (lanes apart)
    x[3, 0:256] = rng.uniform(-1, 1, 256)
    x[3, 40], x[3, 41] = 2.5, -2.5                       # tie, positive first (one lane)
    x[4, 0:256] = rng.uniform(-1, 1, 256)
    x[4, 3] = np.nan
    x[4, 250] = np.nan                                  # NaN never the maximum
    x[5, 0:256] = rng.uniform(-1, 1, 256)
    x[5, 255] = -5.0                                    # the maximum is the last element
    x[6, 0] = -127.0                                    # iscale = 1: the codes are x itself,
    x[6, 1:256] = (np.arange(255) - 127) * 0.5          # .5 ties round to even
    x[6, 256:512] = rng.uniform(-1, 1, 256) * 1e-38      # subnormal-range block
    x[7, 512:768] = 0.0
    x[7, 512 + 100] = -7.0                              # one element, negative
    x[8, 768:1024] = x[8, 768:1024] * 1e6
    x = x.astype(np.float32)
    w = synth.np_weights(qt, n_out, n_in, rng)
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    got = E.linear_quant_batch(dev(w), qt, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    xq = _q8k_rows(ora, x)
    want = E.gemv_q8(dev(w), qt, dev(xq), m, n_out, n_in, bias=dev(bias)).cpu().numpy()
    assert np.array_equal(bits(got), bits(want))
    finite = np.isfinite(x).all(axis=1)
    ref = ora.linear_quant_batch(x[finite], w, qt, bias, int(finite.sum()), n_out, n_in)
    S = q8_scales(ora, qt, w, x[finite]) + np.abs(bias)[None, :]
    assert_tol(got[finite], ref, S, "pack special blocks vs oracle")


def test_prefill_gemm_q8k_input_and_repeat(hipdev, ora):
    """The GEMM over Q8_K block bytes already in memory (edgexpu_hip_gemv_q8_dev)
    equals the GEMM over the f32 activations bit for bit (same codes, same
    operand pack), and a second call gives the same bits (the split-K flags
    the first call used are back at zero)."""
    rng = np.random.default_rng(7272)
    n_in, n_out, m = 4096, 300, 100
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    bias = rng.normal(0, 0.5, n_out).astype(np.float32)
    a = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    b = E.linear_quant_batch(dev(w), 12, dev(x), n_out, n_in, bias=dev(bias)).cpu().numpy()
    xq = _q8k_rows(ora, x)
    c = E.gemv_q8(dev(w), 12, dev(xq), m, n_out, n_in, bias=dev(bias)).cpu().numpy()
    assert np.array_equal(bits(a), bits(b))
    assert np.array_equal(bits(a), bits(c))


# ------------------------------------------------------------------ logits


@pytest.mark.parametrize("name", ["dotf32_q4_k_4096", "dotf32_q4_k_2560", "dotf32_q6_k_2560", "dotf32_q8_0_576"])
def test_f32_dots_golden(hipdev, golden, name):
    g = golden(name)
    qt, w, h = int(g["type"]), g["w"], g["h"]
    rows, n = w.shape[0], h.size
    scores, best = E.logits(dev(w), qt, dev(h[None, :]), rows, n)
    got = scores.cpu().numpy()[0]
    if qt == 8:  # Q8_0 logits go through the Q8_0-activation dot (src/native.c:2317-2319)
        ora = O.load_oracle()
        xq = ora.quantize_q8_0(h)
        want = np.array([ora.dot_q8(8, w[i], xq, n) for i in range(rows)], np.float32)
        S = np.array([npref.q8_dot_f64(8, w[i], xq)[1] for i in range(rows)])
    else:
        want = g["scores"]
        S = np.array([npref.f32_dot_f64(qt, w[i], h)[1] for i in range(rows)])
    assert_tol(got, want, S, name)


@pytest.mark.parametrize("qt,n,vocab,chunk", [(12, 4096, 20000, 8192), (14, 2560, 15001, 0), (8, 576, 49152, 0),
                                              (12, 2560, 3000, 1000)])
def test_logits_and_argmax(hipdev, ora, qt, n, vocab, chunk):
    rng = np.random.default_rng(qt + vocab)
    w = synth.np_weights(qt, vocab, n, rng)
    h = rng.normal(0, 1, n).astype(np.float32)
    bias = rng.normal(0, 0.01, vocab).astype(np.float32)
    want, want_best = ora.logits(h, w, qt, bias, vocab, n, chunk)
    scores, best = E.logits(dev(w), qt, dev(h[None, :]), vocab, n, bias=dev(bias), chunk_rows=chunk)
    got = scores.cpu().numpy()[0]
    # each score against its own row's scale (+ |bias|): Q8_0 rows take the
    # Q8_0-activation dot (src/native.c:2317-2319), the K-quants the f32 dot
    S = (q8_scales(ora, qt, w, h[None, :])[0] if qt == 8 else f32_scales(qt, w, h)) + np.abs(bias)
    assert_tol(got, want, S, f"logits {TN[qt]} [{vocab} x {n}]")
    b = int(best.cpu().numpy()[0])
    assert b == int(np.argmax(got))           # GPU argmax is exact over GPU scores
    top = np.argsort(want)[-2:]
    if want[top[1]] - want[top[0]] > 2 * TOL * S[top].max():  # unambiguous winner: must agree with the oracle
        assert b == want_best


@pytest.mark.parametrize("qt,n,vocab,chunk", [(12, 4096, 128256, 8192), (14, 2560, 151936, 0)])
def test_logits_full_vocabulary(hipdev, ora, qt, n, vocab, chunk):
    """The full output matrices the decode step times: [128256 x 4096] Q4_K in
    8192-row chunks and [151936 x 2560] Q6_K, f32 hidden vector.  Every score
    within 1e-5 of its row's conditioning scale sum |w x| (float64
    restatement), against the oracle; the greedy index is the lowest one of
    the largest device score, and the oracle's when its winner is clear."""
    rng = np.random.default_rng(31 + qt + vocab)
    w = synth.np_weights(qt, vocab, n, rng)
    h = rng.normal(0, 1, n).astype(np.float32)
    want, want_best = ora.logits(h, w, qt, None, vocab, n, chunk)
    scores, best = E.logits(dev(w), qt, dev(h[None, :]), vocab, n, chunk_rows=chunk)
    got = scores.cpu().numpy()[0]
    exact, S = npref.f32_rows_f64(qt, w, h)
    assert_tol(want, exact.astype(np.float32), S, "oracle vs float64")
    assert_tol(got, want, S, f"logits {TN[qt]} [{vocab} x {n}]")
    b = int(best.cpu().numpy()[0])
    assert b == int(np.argmax(got))
    top2 = np.sort(want)[-2:]
    if top2[1] - top2[0] > 2 * TOL * S[np.argsort(want)[-2:]].max():
        assert b == want_best


@pytest.mark.parametrize("qt,n,vocab", [(12, 4096, 3001), (14, 2560, 2050), (8, 576, 4000)])
@pytest.mark.parametrize("m", [2, 3, 4, 8])
def test_logits_multi_token(hipdev, ora, qt, n, vocab, m):
    """m hidden vectors in one call: each row equals the one-token call bit
    for bit (a score does not depend on how many vectors share the call, as
    in the reference's per-token loop), within the bound of the oracle, and
    the argmax is per row."""
    rng = np.random.default_rng(7 * qt + vocab + m)
    w = synth.np_weights(qt, vocab, n, rng)
    h = rng.normal(0, 1, (m, n)).astype(np.float32)
    scores, best = E.logits(dev(w), qt, dev(h), vocab, n)
    got = scores.cpu().numpy()
    for t in range(m):
        one, _ = E.logits(dev(w), qt, dev(h[t:t + 1]), vocab, n)
        assert np.array_equal(bits(got[t]), bits(one.cpu().numpy()[0])), f"token {t}"
        want, _ = ora.logits(h[t], w, qt, None, vocab, n, 0)
        S = q8_scales(ora, qt, w, h[t:t + 1])[0] if qt == 8 else f32_scales(qt, w, h[t])
        assert_tol(got[t], want, S, f"token {t}")
    assert np.array_equal(best.cpu().numpy(), np.argmax(got, axis=1))


@pytest.mark.parametrize("qt,n,vocab", [(12, 4096, 20000), (14, 2560, 15001), (12, 2560, 3001), (8, 576, 49152),
                                        (8, 2048, 7001)])
def test_logits_fused_argmax(hipdev, qt, n, vocab):
    """K-quant and Q8_0 logits with the argmax in the GEMV's store: the scores equal the
    scores-only launch bit for bit, the index is the lowest one of the largest
    score (two rows made equal and largest), and a NaN score never wins."""
    rng = np.random.default_rng(qt * 31 + vocab)
    w = synth.np_weights(qt, vocab, n, rng)
    w[vocab - 7] = w[13]                       # identical rows: equal scores
    h = rng.normal(0, 1, n).astype(np.float32)
    bias = np.zeros(vocab, np.float32)
    bias[[13, vocab - 7]] = 1e4                # ... and the largest
    s1, best = E.logits(dev(w), qt, dev(h[None, :]), vocab, n, bias=dev(bias))
    s0, _ = E.logits(dev(w), qt, dev(h[None, :]), vocab, n, bias=dev(bias), want_best=False)
    got = s1.cpu().numpy()[0]
    assert np.array_equal(bits(got), bits(s0.cpu().numpy()[0]))
    assert got[13] == got[vocab - 7]
    assert int(best.cpu().numpy()[0]) == 13
    bias[5] = np.nan                           # NaN never wins
    bias[vocab - 1] = 2e4
    s2, best2 = E.logits(dev(w), qt, dev(h[None, :]), vocab, n, bias=dev(bias))
    assert np.isnan(s2.cpu().numpy()[0][5]) and int(best2.cpu().numpy()[0]) == vocab - 1


def test_argmax_rules(hipdev):
    # A Q8_0 matrix whose rows are all zero except rows 10 and 4000: equal best
    # scores, so the lowest index must win (src/native.c:2380).
    n = 32
    rows = 5000
    wq = np.zeros((rows, 34), np.uint8)
    one = np.array([1.0], np.float16).view(np.uint8)
    for r in (10, 4000):
        wq[r, 0:2] = one
        wq[r, 2:] = 1
    h = np.ones(n, np.float32)
    scores, best = E.logits(dev(wq), 8, dev(h[None, :]), rows, n)
    assert int(best.cpu().numpy()[0]) == 10
    # NaN never wins: a NaN bias on the lowest winner hands the win to row 4000
    bias = np.zeros(rows, np.float32)
    bias[10] = np.nan
    scores, best = E.logits(dev(wq), 8, dev(h[None, :]), rows, n, bias=dev(bias))
    assert int(best.cpu().numpy()[0]) == 4000
    # all -inf -> index 0
    bias = np.full(rows, -np.inf, np.float32)
    scores, best = E.logits(dev(wq), 8, dev(h[None, :]), rows, n, bias=dev(bias))
    assert int(best.cpu().numpy()[0]) == 0


def test_argmax_signed_zero_tie(hipdev):
    """A largest score of zero held as -0.0 at one row and +0.0 at a later
    one: the reference's `score > best` sees them equal and keeps the lower
    index (src/native.c:2370-2380), whichever sign it carries.  F32 rows make
    the signed zeros: a product of -1e-30 and 1e-30 is -1e-60 in double,
    which rounds to -0.0 in float; every other row scores -inf."""
    vocab, n = 300, 8
    h = np.zeros(n, np.float32)
    h[0] = 1e-30
    for lo_sign, hi_sign in ((-1.0, 1.0), (1.0, -1.0)):
        w = np.zeros((vocab, n), np.float32)
        w[3, 0] = lo_sign * 1e-30
        w[7, 0] = hi_sign * 1e-30
        bias = np.full(vocab, -np.inf, np.float32)
        bias[[3, 7]] = -0.0
        scores, best = E.logits(dev(w.view(np.uint8)), 0, dev(h[None, :]), vocab, n, bias=dev(bias))
        got = scores.cpu().numpy()[0]
        assert got[3] == 0.0 and got[7] == 0.0
        assert np.signbit(got[3]) == (lo_sign < 0) and np.signbit(got[7]) == (hi_sign < 0)
        assert int(best.cpu().numpy()[0]) == 3


# ------------------------------------------------------------------ errors


def test_bad_arguments_are_rejected(hipdev):
    L = hipdev
    x = torch.zeros((1, 100), device=DEV)
    w = torch.zeros(1000, dtype=torch.uint8, device=DEV)
    out = torch.zeros((1, 4), device=DEV)
    assert L.linear_dev(out.data_ptr(), x.data_ptr(), w.data_ptr(), 12, None, 1, 4, 100, None) == 0
    code, msg = L.last_error()
    assert code != 0 and "multiple" in msg
    L.clear_error()
    assert L.linear_dev(out.data_ptr(), x.data_ptr(), w.data_ptr(), 5, None, 1, 4, 96, None) == 0  # no such type
    code, msg = L.last_error()
    assert "not supported" in msg
    L.clear_error()
    assert L.gemv_q8_dev(out.data_ptr(), x.data_ptr(), w.data_ptr(), 1, None, 1, 4, 96, None) == 0  # F16: f32 x only
    code, msg = L.last_error()
    assert code != 0 and "F16" in msg
    L.clear_error()
    sc = torch.zeros((1, 4), device=DEV)
    assert L.logits_dev(sc.data_ptr(), None, x.data_ptr(), w.data_ptr(), 12, None, 1, 4, 256, -1, None) == 0
    code, msg = L.last_error()
    assert code != 0 and "chunk_rows" in msg
    L.clear_error()
    xq = torch.zeros(2 * 292 + 8, dtype=torch.uint8, device=DEV)  # Q8_K codes, misaligned by one byte
    assert L.gemv_q8_dev(out.data_ptr(), xq.data_ptr() + 1, w.data_ptr(), 12, None, 1, 4, 256, None) == 0
    code, msg = L.last_error()
    assert code != 0 and "aligned" in msg
    L.clear_error()
    assert L.last_error()[0] == 0


# ------------------------------------------------------------------ grouped launches


@pytest.mark.parametrize("qt,n_in,n_outs", [(12, 4096, (4096, 1024, 1024)), (12, 4096, (14336, 14336)),
                                            (8, 576, (576, 192, 192)), (14, 2560, (300, 7)),
                                            (12, 14336, (4096,)), (12, 2560, (4096, 1024, 1024, 33))])
@pytest.mark.parametrize("m", [1, 3])
def test_linear_group_matches_single(hipdev, ora, qt, n_in, n_outs, m):
    """One grouped launch == the per-projection calls (and the oracle)."""
    rng = np.random.default_rng(sum(n_outs) + n_in + m)
    ws = [synth.np_weights(qt, n, n_in, rng) for n in n_outs]
    x = synth.np_activations(m, n_in, rng)
    biases = [rng.normal(0, 0.1, n).astype(np.float32) if z % 2 == 0 else None for z, n in enumerate(n_outs)]
    outs = E.linear_quant_group([dev(w) for w in ws], qt, dev(x), list(n_outs), n_in,
                                biases=[None if b is None else dev(b) for b in biases])
    for z, (w, n) in enumerate(zip(ws, n_outs)):
        got = outs[z].cpu().numpy()
        single = E.linear_quant_batch(dev(w), qt, dev(x), n, n_in,
                                      bias=None if biases[z] is None else dev(biases[z])).cpu().numpy()
        assert np.array_equal(got.view(np.uint32), single.view(np.uint32)), f"matrix {z}"
        want = ora.linear_quant_batch(x, w, qt, biases[z], m, n, n_in)
        sample = np.arange(min(n, 48))
        S = q8_scales(ora, qt, w[sample], x) + (0 if biases[z] is None else np.abs(biases[z][sample]))
        assert_tol(got[:, sample], want[:, sample], S, f"group matrix {z}")


def _staging_edge_blocks(golden, rng):
    """256-element activation blocks that steer the Q8_K quantizer through
    every branch: the golden edge cases (zeros, ties of +-amax in either
    order, halfway rounding, huge, tiny and subnormal maxima whose -127/max
    overflows), plus +-amax held by different 16-element groups (the earlier
    group decides), both signs inside the first group holding amax (its
    first element decides), NaN and infinite elements."""
    g = golden("quantize")
    blocks = [np.asarray(x, np.float32) for x in g["x"]]

    def base():
        return rng.normal(0, 1, 256).astype(np.float32)

    b = base(); b[3 * 16 + 5] = 9.0; b[1 * 16 + 7] = -9.0; blocks.append(b)     # -9 in an earlier group
    b = base(); b[2 * 16 + 9] = -9.0; b[2 * 16 + 3] = 9.0; blocks.append(b)     # same group, + first
    b = base(); b[2 * 16 + 3] = -9.0; b[2 * 16 + 9] = 9.0; b[5 * 16] = 9.0; blocks.append(b)  # same group, - first
    b = base(); b[0] = 9.0; b[15] = -9.0; b[16] = -9.0; blocks.append(b)         # group 0 both, + first
    b = base(); b[40] = np.nan; b[41] = 5.0; blocks.append(b)                    # NaN never enters amax
    b = base(); b[77] = np.inf; blocks.append(b)                                 # amax = inf: iscale = -0
    b = base(); b[100] = -np.inf; b[7] = np.inf; blocks.append(b)                # first infinity decides
    b = np.zeros(256, np.float32); b[200] = 1e-39; b[201] = -1e-39; blocks.append(b)  # subnormal tie
    return blocks


@pytest.mark.parametrize("gemv_mode", [1, 2])
@pytest.mark.parametrize("qt,n_in", [(12, 4096), (12, 14336), (14, 9728), (14, 2560)])
def test_fused_staging_quantizer_edge_cases(hipdev, ora, golden, qt, n_in, gemv_mode):
    """The GEMV's in-kernel Q8_K quantizer (one token: the activation is
    quantized in LDS inside the launch) on every branch of the reference's
    quantize_row_q8_K: equal bit for bit to quantizing with the standalone
    kernel (itself bit-exact against the reference's golden vectors) and
    running the GEMV over those bytes; the standalone codes equal the
    oracle's.  Shapes: 8-wave, 16-wave (rows split over 4 waves) and 12-wave
    (3 waves per row) workgroups; the fused kernel's staging and the
    streaming kernel's (gemv_mode 2, where it covers the shape)."""
    rng = np.random.default_rng(n_in + qt)
    blocks = _staging_edge_blocks(golden, rng)
    nb = n_in // 256
    x = np.concatenate([blocks[i % len(blocks)] for i in range(nb)]).astype(np.float32)[None, :]
    n_out = 300
    w = synth.np_weights(qt, n_out, n_in, rng)
    wd = dev(w)
    xq = E.quantize_q8_k(dev(x))
    assert np.array_equal(xq.cpu().numpy(), ora.quantize_q8_k(x[0]))
    L = hipdev
    try:
        assert L.set_gemv_mode(gemv_mode) == 1
        sep = E.gemv_q8(wd, qt, xq, 1, n_out, n_in).cpu().numpy()
        fused = E.linear_quant_batch(wd, qt, dev(x), n_out, n_in).cpu().numpy()
    finally:
        L.set_gemv_mode(0)
    fin = np.isfinite(sep)
    assert np.array_equal(fin, np.isfinite(fused))
    assert np.array_equal(bits(fused[fin]), bits(sep[fin]))
