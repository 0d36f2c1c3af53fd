"""The two decode GEMV kernels for one token of Q4_K rows agree bit for bit.

One to four tokens of Q4_K rows of 2560, 4096 or 14336 elements, or of
Q6_K rows of 9728 (several tokens: plain projections), runs on either the
fused kernel (csrc/gemv_fused_kernel.h) or the streaming kernel
(csrc/gemv_stream.hip: rows through LDS by DMA), chosen by launch size
(edgexpu_hip_set_gemv_mode).  Both compute each lane's unit partial with the
same roundings and sum the lanes with the same xor tree, so every output is
the same word whichever kernel runs -- the plain projection, grouped
launches, the RMSNorm and SiLU-mul staging prologues, the residual store,
gate/up pairs with silu(gate) * up, activations given as Q8_K block bytes,
and (rows of 2560, or of 4096 at two to four tokens, in long launches,
every matrix of an even row count) two adjacent rows per step.  Each variant is also held to the oracle (the reference's
edgexpu_cpu_linear_quant_batch, src/cpu_kernel.c:545-644) within the usual
1e-5 of the conditioning scale, so the agreement is between two correct
results, not two copies of one mistake.
"""
import numpy as np
import pytest
import torch

import edgexpu_amd as E
import npref
from edgexpu_amd import synth

pytestmark = pytest.mark.gpu

AUTO, FUSED, STREAM = 0, 1, 2
TOL = 1e-5


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def both(L, fn):
    """fn() under the fused kernel and under the streaming kernel."""
    out = {}
    try:
        for mode in (FUSED, STREAM):
            assert L.set_gemv_mode(mode) == 1
            out[mode] = [t.cpu().numpy() for t in fn()]
    finally:
        L.set_gemv_mode(AUTO)
    return out[FUSED], out[STREAM]


def cond(ora, w, x):
    """S_i of each output row: the sum over blocks of |block terms| (float64)."""
    xq = ora.quantize_q8_k(x[0])
    return np.array([npref.q8_dot_f64(12, w[i], xq)[1] for i in range(w.shape[0])])[None, :]


SHAPES = [(4096, (14336, 14336)), (4096, (4096, 1024, 1024)), (4096, (4096,)), (4096, (33,)),
          (14336, (4096,)), (14336, (2048,)), (14336, (300,)), (2560, (9728, 9728)), (2560, (4096, 1024, 1024)),
          (2560, (7,)), (2560, (2, 18430, 6)), (4096, (2, 18430, 6)), (2560, (4, 1031))]


@pytest.mark.parametrize("n_in,n_outs", SHAPES)
def test_plain_group_fused_equals_stream(hipdev, ora, n_in, n_outs):
    rng = np.random.default_rng(n_in + sum(n_outs))
    ws = [synth.np_weights(12, n, n_in, rng) for n in n_outs]
    x = synth.np_activations(1, n_in, rng)
    biases = [rng.normal(0, 0.3, n).astype(np.float32) if z % 2 == 0 else None for z, n in enumerate(n_outs)]
    wd = [dev(w) for w in ws]
    bd = [None if b is None else dev(b) for b in biases]
    f, s = both(hipdev, lambda: E.linear_quant_group(wd, 12, dev(x), list(n_outs), n_in, biases=bd))
    for z, n in enumerate(n_outs):
        assert np.array_equal(bits(f[z]), bits(s[z])), f"matrix {z}"
        sample = np.arange(min(n, 64))
        want = ora.linear_quant_batch(x, ws[z][sample], 12, None if biases[z] is None else biases[z][sample], 1,
                                      len(sample), n_in)
        S = cond(ora, ws[z][sample], x) + (0 if biases[z] is None else np.abs(biases[z][sample]))
        assert np.all(np.abs(s[z][:, sample] - want) <= TOL * S), f"matrix {z}"


@pytest.mark.parametrize("n_in,n_out", [(4096, 1000), (14336, 2100), (2560, 515)])
def test_q8k_input_fused_equals_stream(hipdev, ora, n_in, n_out):
    """Activations already in Q8_K block bytes (edgexpu_hip_gemv_q8_dev): the
    streaming kernel reads the blocks instead of quantizing, same words."""
    rng = np.random.default_rng(n_in * 3 + n_out)
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(1, n_in, rng)
    xq = dev(ora.quantize_q8_k(x[0]))
    wd = dev(w)
    f, s = both(hipdev, lambda: [E.gemv_q8(wd, 12, xq, 1, n_out, n_in)])
    assert np.array_equal(bits(f[0]), bits(s[0]))
    # and equal to quantizing inside the launch
    staged = E.linear_quant_batch(wd, 12, dev(x), n_out, n_in).cpu().numpy()
    assert np.array_equal(bits(staged), bits(s[0]))


@pytest.mark.parametrize("n_in,n_outs", [(4096, (4096, 1024, 1024)), (4096, (14336, 14336)), (14336, (4096,)),
                                         (2560, (4096, 1024, 1024))])
def test_rmsnorm_prologue_fused_equals_stream(hipdev, ora, n_in, n_outs):
    rng = np.random.default_rng(n_in + 7 * len(n_outs))
    ws = [dev(synth.np_weights(12, n, n_in, rng)) for n in n_outs]
    x = (rng.normal(0, 1, (1, n_in)) * 3).astype(np.float32)
    nw = dev(rng.normal(1, 0.2, n_in).astype(np.float32))
    biases = [dev(rng.normal(0, 0.5, n).astype(np.float32)) for n in n_outs]
    f, s = both(hipdev, lambda: E.layer_linear(ws, 12, dev(x), n_outs, n_in, norm_weight=nw, eps=1e-5, biases=biases))
    for z in range(len(n_outs)):
        assert np.array_equal(bits(f[z]), bits(s[z])), f"matrix {z}"


@pytest.mark.parametrize("n_in,n_out", [(14336, 4096), (4096, 2560), (2560, 2560)])
def test_silu_mul_residual_fused_equals_stream(hipdev, ora, n_in, n_out):
    rng = np.random.default_rng(n_in + n_out)
    w = dev(synth.np_weights(12, n_out, n_in, rng))
    g = dev(rng.normal(0, 2, (1, n_in)).astype(np.float32))
    u = dev(rng.normal(0, 2, (1, n_in)).astype(np.float32))
    res = rng.normal(0, 4, (1, n_out)).astype(np.float32)
    f, s = both(hipdev, lambda: E.layer_linear([w], 12, g, (n_out,), n_in, x2=u, residuals=[dev(res)]))
    assert np.array_equal(bits(f[0]), bits(s[0]))


def test_residual_only_fused_equals_stream(hipdev):
    n_in, n_outs = 4096, (4096, 1024)
    rng = np.random.default_rng(11)
    ws = [dev(synth.np_weights(12, n, n_in, rng)) for n in n_outs]
    x = dev(synth.np_activations(1, n_in, rng))
    res = dev(rng.normal(0, 4, (1, n_outs[0])).astype(np.float32))
    bias = [dev(rng.normal(0, 0.5, n).astype(np.float32)) for n in n_outs]
    f, s = both(hipdev, lambda: E.layer_linear(ws, 12, x, n_outs, n_in, biases=bias, residuals=[res, None]))
    for z in range(2):
        assert np.array_equal(bits(f[z]), bits(s[z]))


@pytest.mark.parametrize("n_in,n_ff", [(4096, 14336), (2560, 9728), (14336, 4096), (4096, 300)])
@pytest.mark.parametrize("norm", [True, False])
def test_gate_up_pairs_fused_equals_stream(hipdev, ora, n_in, n_ff, norm):
    rng = np.random.default_rng(n_in + n_ff + norm)
    wg, wu = dev(synth.np_weights(12, n_ff, n_in, rng)), dev(synth.np_weights(12, n_ff, n_in, rng))
    x = dev((rng.normal(0, 1, (1, n_in)) * 2).astype(np.float32))
    nw = dev(rng.normal(1, 0.2, n_in).astype(np.float32)) if norm else None
    bg, bu = dev(rng.normal(0, 0.5, n_ff).astype(np.float32)), dev(rng.normal(0, 0.5, n_ff).astype(np.float32))
    f, s = both(hipdev, lambda: [E.gate_up_silu(wg, wu, 12, x, n_ff, n_in, norm_weight=nw, b_gate=bg, b_up=bu)])
    assert np.array_equal(bits(f[0]), bits(s[0]))


TOKEN_SHAPES = [(4096, (4096, 1024, 1024)), (4096, (14336, 14336)), (4096, (4096,)), (4096, (301,)),
                (2560, (4096, 1024, 1024)), (2560, (9728, 9728)), (2560, (2560,)), (2560, (77,)),
                (14336, (4096,)), (14336, (2048, 300)), (4096, (2, 18430, 6))]


def fused_stages(m, n_in):
    """True when the fused kernel holds m tokens' Q8_K codes, scales and sums
    (and its 256-byte reduction buffers) in its 64 KB of LDS; otherwise the
    library's other path for those tokens is the generic GEMV, whose lane
    order differs (four tokens of 14336)."""
    return m * n_in + m * n_in // 64 + m * n_in // 8 + 256 <= 64 * 1024


@pytest.mark.parametrize("n_in,n_outs", TOKEN_SHAPES)
@pytest.mark.parametrize("m", [2, 3, 4])
def test_tokens_fused_equals_stream(hipdev, ora, n_in, n_outs, m):
    """Two to four tokens in one launch (plain projections, as the batched
    decode issues them): each token's rows equal the fused kernel's bit for
    bit where the fused kernel stages them, and the oracle's (its token loop,
    src/cpu_kernel.c:616-627) within 1e-5 of each row's conditioning scale."""
    rng = np.random.default_rng(n_in * m + sum(n_outs))
    ws = [synth.np_weights(12, n, n_in, rng) for n in n_outs]
    x = synth.np_activations(m, n_in, rng)
    biases = [rng.normal(0, 0.3, n).astype(np.float32) if z % 2 == 0 else None for z, n in enumerate(n_outs)]
    wd = [dev(w) for w in ws]
    bd = [None if b is None else dev(b) for b in biases]
    f, s = both(hipdev, lambda: E.linear_quant_group(wd, 12, dev(x), list(n_outs), n_in, biases=bd))
    for z, n in enumerate(n_outs):
        assert f[z].shape == (m, n)
        if fused_stages(m, n_in):
            assert np.array_equal(bits(f[z]), bits(s[z])), f"matrix {z}"
        sample = np.arange(min(n, 48))
        want = ora.linear_quant_batch(x, ws[z][sample], 12, None if biases[z] is None else biases[z][sample], m,
                                      len(sample), n_in)
        S = np.stack([cond(ora, ws[z][sample], x[t:t + 1])[0] for t in range(m)])
        if biases[z] is not None:
            S = S + np.abs(biases[z][sample])[None, :]
        assert np.all(np.abs(s[z][:, sample] - want) <= TOL * S), f"matrix {z}"


@pytest.mark.parametrize("m,pairs", [(1, False), (2, False), (1, True), (3, True)])
def test_more_than_64_steps_per_wave(hipdev, ora, m, pairs):
    """A launch long enough that every wave takes more than 64 steps: the
    totals kept in lanes are flushed every 64 steps and the bias prefetched
    again, then a partial flush at the end (131 849 rows of 2560: 64 full
    steps of the 2048 waves of 256 CUs, and 777 rows more; an even count of
    rows: 131 849 steps of two adjacent rows)."""
    n_in, n_out = 2560, (2048 * 64 + 777) * (2 if pairs else 1)
    rng = np.random.default_rng(64 + m + 10 * pairs)
    w = synth.np_weights(12, n_out, n_in, rng)
    x = synth.np_activations(m, n_in, rng)
    bias = rng.normal(0, 0.3, n_out).astype(np.float32)
    wd, bd = dev(w), dev(bias)
    f, s = both(hipdev, lambda: [E.linear_quant_batch(wd, 12, dev(x), n_out, n_in, bias=bd)])
    assert np.array_equal(bits(f[0]), bits(s[0]))
    r = 2 if pairs else 1
    sample = np.unique(np.concatenate([np.arange(0, n_out, 997), np.arange(n_out - 40, n_out),
                                       np.arange(r * 2048 * 63, r * 2048 * 63 + 40),
                                       np.arange(r * 2048 * 64 - 20, r * 2048 * 64 + 20)]))
    want = ora.linear_quant_batch(x, w[sample], 12, bias[sample], m, len(sample), n_in)
    S = np.stack([cond(ora, w[sample], x[t:t + 1])[0] for t in range(m)]) + np.abs(bias[sample])[None, :]
    assert np.all(np.abs(s[0][:, sample] - want) <= TOL * S)


def cond6(ora, w, x):
    """S_i of Q6_K rows against one token's Q8_K codes (float64)."""
    xq = ora.quantize_q8_k(x[0])
    return np.array([npref.q8_dot_f64(14, w[i], xq)[1] for i in range(w.shape[0])])[None, :]


@pytest.mark.parametrize("n_outs", [(2560,), (2560, 2560), (77,), (1, 3000), (4097,)])
def test_q6k_fused_equals_stream(hipdev, ora, n_outs):
    """One token of Q6_K rows of 9728 (the hybrid ~4B down projection): rows
    of 210-byte super-blocks start 4-byte aligned in the stream's slots and
    are read with byte shifts; every output equals the fused kernel's bit for
    bit and the oracle's within 1e-5 of its conditioning scale."""
    n_in = 9728
    rng = np.random.default_rng(6000 + sum(n_outs))
    ws = [synth.np_weights(14, n, n_in, rng) for n in n_outs]
    x = synth.np_activations(1, n_in, rng)
    biases = [rng.normal(0, 0.3, n).astype(np.float32) if z % 2 == 0 else None for z, n in enumerate(n_outs)]
    wd = [dev(w) for w in ws]
    bd = [None if b is None else dev(b) for b in biases]
    f, s = both(hipdev, lambda: E.linear_quant_group(wd, 14, dev(x), list(n_outs), n_in, biases=bd))
    for z, n in enumerate(n_outs):
        assert np.array_equal(bits(f[z]), bits(s[z])), f"matrix {z}"
        sample = np.unique(np.concatenate([np.arange(min(n, 40)), np.arange(max(0, n - 8), n)]))
        want = ora.linear_quant_batch(x, ws[z][sample], 14, None if biases[z] is None else biases[z][sample], 1,
                                      len(sample), n_in)
        S = cond6(ora, ws[z][sample], x) + (0 if biases[z] is None else np.abs(biases[z][sample]))
        assert np.all(np.abs(s[z][:, sample] - want) <= TOL * S), f"matrix {z}"


@pytest.mark.parametrize("n_outs", [(2560,), (77, 3000)])
@pytest.mark.parametrize("m", [2, 3, 4])
def test_q6k_tokens_fused_equals_stream(hipdev, ora, n_outs, m):
    """Two to four tokens of Q6_K rows of 9728 in one launch (the hybrid ~4B
    down projection of a batched decode): each token's rows equal the fused
    kernel's bit for bit, and the oracle's token loop (src/cpu_kernel.c:616-627)
    within 1e-5 of each row's conditioning scale."""
    n_in = 9728
    rng = np.random.default_rng(6200 + 10 * m + len(n_outs))
    ws = [synth.np_weights(14, n, n_in, rng) for n in n_outs]
    x = synth.np_activations(m, n_in, rng)
    biases = [rng.normal(0, 0.3, n).astype(np.float32) if z % 2 == 0 else None for z, n in enumerate(n_outs)]
    wd = [dev(w) for w in ws]
    bd = [None if b is None else dev(b) for b in biases]
    f, s = both(hipdev, lambda: E.linear_quant_group(wd, 14, dev(x), list(n_outs), n_in, biases=bd))
    for z, n in enumerate(n_outs):
        assert f[z].shape == (m, n)
        assert np.array_equal(bits(f[z]), bits(s[z])), f"matrix {z}"
        sample = np.unique(np.concatenate([np.arange(min(n, 32)), np.arange(max(0, n - 8), n)]))
        want = ora.linear_quant_batch(x, ws[z][sample], 14, None if biases[z] is None else biases[z][sample], m,
                                      len(sample), n_in)
        S = np.stack([cond6(ora, ws[z][sample], x[t:t + 1])[0] for t in range(m)])
        if biases[z] is not None:
            S = S + np.abs(biases[z][sample])[None, :]
        assert np.all(np.abs(s[z][:, sample] - want) <= TOL * S), f"matrix {z}"


def f32_scales(qt, w, h):
    """S_i of the f32-activation dot of the rows of w with h (float64)."""
    return np.array([npref.f32_dot_f64(qt, w[i], h)[1] for i in range(w.shape[0])])


@pytest.mark.parametrize("qt,n", [(12, 4096), (14, 2560)])
@pytest.mark.parametrize("vocab,m,with_bias", [(20000, 1, True), (3001, 1, False), (2048 * 64 + 5, 1, False),
                                               (20000, 2, True), (3001, 3, False), (1, 1, True), (7, 2, False)])
def test_logits_f32_fused_equals_stream(hipdev, ora, qt, n, vocab, m, with_bias):
    """The f32-activation logits of Q4_K rows of 4096 and Q6_K rows of 2560
    (one hidden vector with the greedy-argmax keys, or several in launches
    of two): scores and greedy indices equal the fused kernel's bit for bit,
    every score within 1e-5 of its row's scale of the oracle's
    (src/native.c:445-462, 2355-2396).  Sizes: a few rows per wave, fewer
    than three, and more than 64 (the kept totals flushed, the argmax keys
    carried across flushes)."""
    rng = np.random.default_rng(7000 + vocab + m + qt)
    w = synth.np_weights(qt, vocab, n, rng)
    h = rng.normal(0, 1, (m, n)).astype(np.float32)
    bias = rng.normal(0, 0.01, vocab).astype(np.float32) if with_bias else None
    wd, hd, bd = dev(w), dev(h), None if bias is None else dev(bias)
    f, s = both(hipdev, lambda: E.logits(wd, qt, hd, vocab, n, bias=bd))
    assert np.array_equal(bits(f[0]), bits(s[0]))
    assert np.array_equal(f[1], s[1])
    for t in range(m):
        assert int(s[1][t]) == int(np.argmax(s[0][t]))
    rows = np.unique(np.concatenate([np.arange(min(vocab, 40)), np.arange(max(0, vocab - 40), vocab),
                                     rng.integers(0, vocab, 200)]))
    for t in range(m):
        want, _ = ora.logits(h[t], w[rows], qt, None if bias is None else bias[rows], len(rows), n, 0)
        S = f32_scales(qt, w[rows], h[t]) + (0 if bias is None else np.abs(bias[rows]))
        assert np.all(np.abs(s[0][t][rows] - want) <= TOL * S), f"token {t}"


def test_q6k_logits_row_triples_more_than_64_steps(hipdev, ora):
    """One token of Q6_K logits rows of 2560 runs three rows per step over
    two passes of 64 lanes: a vocabulary long enough that every wave takes
    more than 64 steps (the kept totals flushed and the argmax keys carried
    across flushes) and ends in a triple of one row (the rows past the matrix
    read as zeros and are never stored): scores and the greedy index equal
    the fused kernel's bit for bit, and sampled rows (every flush boundary,
    the last triple) the oracle's within 1e-5 of their scale."""
    n = 2560
    vocab = 2048 * 3 * 65 + 1          # 65 steps for every wave, then one row
    gen = torch.Generator(device="cuda:0")
    gen.manual_seed(7321)
    wd = synth.torch_weights_bulk(14, vocab, n, gen, "cuda:0")
    hd = torch.randn((1, n), generator=gen, device="cuda:0")
    bd = torch.randn((vocab,), generator=gen, device="cuda:0") * 0.01
    f, s = both(hipdev, lambda: E.logits(wd, 14, hd, vocab, n, bias=bd))
    assert np.array_equal(bits(f[0]), bits(s[0]))
    assert np.array_equal(f[1], s[1])
    assert int(s[1][0]) == int(np.argmax(s[0][0]))
    edge = 2048 * 3 * 64
    rows = np.unique(np.concatenate([np.arange(12), np.arange(edge - 6, edge + 6), np.arange(vocab - 8, vocab),
                                     np.random.default_rng(5).integers(0, vocab, 64)]))
    w = wd[torch.from_numpy(rows).to("cuda:0")].cpu().numpy()
    h = hd.cpu().numpy()[0]
    b = bd.cpu().numpy()[rows]
    want, _ = ora.logits(h, w, 14, b, len(rows), n, 0)
    S = f32_scales(14, w, h) + np.abs(b)
    assert np.all(np.abs(s[0][0][rows] - want) <= TOL * S)


@pytest.mark.parametrize("qt,n,off", [(12, 4096, 8), (12, 4096, 4), (14, 2560, 2), (14, 2560, 6)])
@pytest.mark.parametrize("m", [1, 2])
def test_logits_at_unaligned_weights_take_the_fused_kernel(hipdev, qt, n, off, m):
    """The streaming logits read 16-byte transfers from 16-byte-aligned rows;
    a matrix at another address takes the fused kernel, whose words are the
    same: scores and greedy indices equal those of the aligned copy."""
    vocab = 9001
    rng = np.random.default_rng(7100 + qt + off + m)
    w = synth.np_weights(qt, vocab, n, rng)
    h = dev(rng.normal(0, 1, (m, n)).astype(np.float32))
    buf = torch.zeros(w.nbytes + 256, dtype=torch.uint8, device="cuda:0")
    wu = buf[off:off + w.nbytes].view(w.shape)
    wu.copy_(dev(w))
    assert wu.data_ptr() % 16 == off % 16
    s_al, b_al = E.logits(dev(w), qt, h, vocab, n)
    s_un, b_un = E.logits(wu, qt, h, vocab, n)
    assert np.array_equal(bits(s_al.cpu().numpy()), bits(s_un.cpu().numpy()))
    assert np.array_equal(b_al.cpu().numpy(), b_un.cpu().numpy())


@pytest.mark.parametrize("pro", ["rmsnorm", "silu_mul", "silu_mul_residual", "residual"])
def test_q6k_layer_variants_fused_equals_stream(hipdev, ora, pro):
    """The Q6_K down projection as a layer issues it (SiLU-mul prologue and
    residual) and the other staging variants: the two kernels agree."""
    n_in, n_out = 9728, 2560
    rng = np.random.default_rng(6100 + len(pro))
    w = dev(synth.np_weights(14, n_out, n_in, rng))
    x = dev((rng.normal(0, 1, (1, n_in)) * 2).astype(np.float32))
    x2 = dev(rng.normal(0, 2, (1, n_in)).astype(np.float32))
    nw = dev(rng.normal(1, 0.2, n_in).astype(np.float32))
    res = dev(rng.normal(0, 4, (1, n_out)).astype(np.float32))
    bias = [dev(rng.normal(0, 0.5, n_out).astype(np.float32))]
    kw = {"rmsnorm": dict(norm_weight=nw, eps=1e-5), "silu_mul": dict(x2=x2),
          "silu_mul_residual": dict(x2=x2, residuals=[res]), "residual": dict(residuals=[res])}[pro]
    f, s = both(hipdev, lambda: E.layer_linear([w], 14, x, (n_out,), n_in, biases=bias, **kw))
    assert np.array_equal(bits(f[0]), bits(s[0]))


def test_gemv_mode_switch(hipdev):
    L = hipdev
    assert L.gemv_mode() == AUTO
    assert L.set_gemv_mode(3) == 0
    code, msg = L.last_error()
    assert code != 0 and "unknown mode" in msg
    L.clear_error()
    assert L.gemv_mode() == AUTO
