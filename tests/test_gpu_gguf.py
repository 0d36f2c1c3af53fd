"""GPU tests of the one-time model upload (include/edgexpu_gguf_upload.h):
a synthetic GGUF v3 file written from the format's definition
(tests/gguf_writer.py) is uploaded once; every tensor's device bytes equal the
file's bytes, projections and logits through the device tensors equal the
oracle on the same blocks (within 1e-5 of the row's conditioning scale), an
embedding row dequantized on the device is bit-identical, and the weight
handles refuse what load_qweight refuses (src/native.c:611-640)."""
import ctypes as C

import numpy as np
import pytest
import torch

import gguf_writer as G
import npref
import edgexpu_amd as E
from edgexpu_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _assert_tol(got, want, S, what):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = err > TOL * S + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} outside tolerance"


@pytest.fixture(scope="module")
def model(tmp_path_factory, hipdev):
    rng = np.random.default_rng(2027)
    t = [("token_embd.weight", E.Q8_0, 320, 576), ("blk.0.attn_q.weight", E.Q4_K, 300, 4096),
         ("blk.0.ffn_down.weight", E.Q6_K, 260, 2560), ("output.weight", E.Q6_K, 3000, 2560),
         ("blk.0.ffn_gate.weight", E.Q8_0, 513, 576)]
    arrays = {name: synth.np_weights(qt, rows, n, rng) for name, qt, rows, n in t}
    norm = rng.normal(0, 1, 576).astype(np.float32)
    path = str(tmp_path_factory.mktemp("gguf") / "model.gguf")
    tensors = [(name, [n, rows], qt, G.as_bytes(arrays[name])) for name, qt, rows, n in t]
    tensors.append(("output_norm.weight", [576], E.F32, G.as_bytes(norm)))
    G.write_gguf(path, [("general.architecture", G.STRING, "llama")], tensors)
    gg = E.Gguf()
    h = gg.upload(path)
    yield gg, h, path, t, arrays, norm
    gg.free(h)


def test_device_bytes_equal_file_bytes(model):
    gg, h, path, t, arrays, norm = model
    L = E.hip()
    raw = open(path, "rb").read()
    tab = gg.device_table(h)
    assert len(tab["tensors"]) == len(t) + 1
    for e in tab["tensors"]:
        dp = gg.device_tensor(h, e["name"])
        assert dp is not None
        got = np.empty(e["nbytes"], np.uint8)
        L.check(L.download_bytes(got.ctypes.data_as(C.c_void_p), dp, e["nbytes"]), "download")
        lo = tab["data_offset"] + e["offset"]
        assert got.tobytes() == raw[lo:lo + e["nbytes"]], e["name"]
    assert gg.device_tensor(h, "no.such.tensor") is None


@pytest.mark.parametrize("name", ["blk.0.attn_q.weight", "blk.0.ffn_down.weight", "blk.0.ffn_gate.weight"])
@pytest.mark.parametrize("m", [1, 3])
def test_linear_through_the_device_tensor(model, ora, name, m):
    gg, h, _, t, arrays, _ = model
    L = E.hip()
    _, qt, rows, n = next(e for e in t if e[0] == name)
    w_host = arrays[name]
    rng = np.random.default_rng(m + rows)
    x = synth.np_activations(m, n, rng)
    wh = gg.device_weight(h, name, rows, n)
    try:
        out = np.zeros((m, rows), np.float32)
        L.check(L.linear_host_w(out.ctypes.data_as(C.c_void_p), x.ctypes.data_as(C.c_void_p), wh, m), "linear")
    finally:
        L.weight_free(wh)
    want = ora.linear_quant_batch(x, w_host, qt, None, m, rows, n)
    for tok in range(m):
        xq = ora.quantize_q8_0(x[tok]) if qt == E.Q8_0 else ora.quantize_q8_k(x[tok])
        _, S = npref.q8_rows_f64(qt, w_host, xq)
        _assert_tol(out[tok], want[tok], S, f"{name} token {tok}")


def test_logits_through_the_device_tensor(model, ora):
    gg, h, _, t, arrays, _ = model
    _, qt, vocab, n = next(e for e in t if e[0] == "output.weight")
    rng = np.random.default_rng(77)
    hid = rng.normal(0, 1, n).astype(np.float32)
    dp = gg.device_tensor(h, "output.weight")
    wt = torch.empty(0)  # the device tensor is addressed by pointer
    scores = torch.empty((1, vocab), dtype=torch.float32, device="cuda:0")
    best = torch.empty(1, dtype=torch.int32, device="cuda:0")
    hd = torch.from_numpy(hid[None, :]).to("cuda:0")
    L = E.hip()
    L.check(L.logits_dev(scores.data_ptr(), best.data_ptr(), hd.data_ptr(), dp, qt, None, 1, vocab, n, 0,
                         torch.cuda.current_stream().cuda_stream), "logits")
    got = scores.cpu().numpy()[0]
    want, want_best = ora.logits(hid, arrays["output.weight"], qt, None, vocab, n, 0)
    _, S = npref.f32_rows_f64(qt, arrays["output.weight"], hid)
    _assert_tol(got, want, S, "logits")
    assert int(best.cpu().numpy()[0]) == int(np.argmax(got))
    del wt


def test_embedding_rows_from_the_device_tensor(model):
    gg, h, _, t, arrays, _ = model
    _, qt, rows, n = next(e for e in t if e[0] == "token_embd.weight")
    ids = torch.tensor([0, 7, 319, 7], dtype=torch.int32, device="cuda:0")
    out = torch.empty((4, n), dtype=torch.float32, device="cuda:0")
    L = E.hip()
    dp = gg.device_tensor(h, "token_embd.weight")
    L.check(L.embed_rows_dev(out.data_ptr(), dp, qt, rows, n, ids.data_ptr(), 4, None,
                             torch.cuda.current_stream().cuda_stream), "embed rows")
    want = npref.dequant(qt, arrays["token_embd.weight"][[0, 7, 319, 7]]).reshape(4, n)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.astype(np.float32).view(np.uint32))


def test_weight_handle_refusals(model):
    gg, h, _, _, _, _ = model
    with pytest.raises(ValueError, match="shape mismatch"):
        gg.device_weight(h, "blk.0.attn_q.weight", 301, 4096)
    with pytest.raises(ValueError, match="missing tensor"):
        gg.device_weight(h, "blk.9.attn_q.weight", 300, 4096)
    with pytest.raises(ValueError, match="unsupported type"):
        gg.device_weight(h, "blk.0.attn_q.weight", 4096 * 300 // 100, 100)  # rows of 100 have no Q4_K layout
