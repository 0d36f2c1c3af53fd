"""The no-allocation logits entry (edgexpu_hip_logits_noalloc_dev) against the
allocating one (edgexpu_hip_logits_dev) through the C-ABI: the same kernels
over a fixed device array instead of the library workspace, so scores and
greedy argmax agree bit for bit, on two calls in a row (the second with fewer
vectors, a shorter vocabulary and a shorter hidden vector) and for every
weight family (Q4_K / Q6_K fused argmax, Q8_0 two-pass argmax).  The first
call of each pair goes to the no-allocation entry, and it is also captured
into a HIP graph in global capture mode, where any device allocation would
end the capture with an error; every replay of that graph, with other device
work between replays, equals the eager allocating call bit for bit.  Sizes
past the fixed array are refused with a message, before any launch."""
import numpy as np
import pytest
import torch

import edgexpu_amd as E
from edgexpu_amd import synth

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def _both(L, w, qt, h, vocab, n, bias):
    """(allocating, no-allocation) results; the no-allocation call runs first."""
    m = h.shape[0]
    out = []
    for fn in (L.logits_noalloc_dev, L.logits_dev):
        scores = torch.full((m, vocab), float("nan"), device=DEV)
        best = torch.full((m,), -1, dtype=torch.int32, device=DEV)
        ok = fn(scores.data_ptr(), best.data_ptr(), h.data_ptr(), w.data_ptr(), qt,
                None if bias is None else bias.data_ptr(), m, vocab, n, 0,
                torch.cuda.current_stream().cuda_stream)
        L.check(ok, "logits")
        torch.cuda.synchronize()
        out.append((scores.cpu().numpy(), best.cpu().numpy()))
    return out[1], out[0]


@pytest.mark.parametrize("qt,calls", [
    (12, [(4096, 20000, 3), (2560, 3001, 1)]),
    (14, [(2560, 15001, 2), (2560, 2050, 1)]),
    (8, [(576, 49152, 4), (576, 4000, 2)]),
])
def test_logits_noalloc_equals_logits(hipdev, qt, calls):
    L = hipdev
    L.check(L.init(0), "init")
    rng = np.random.default_rng(99 + qt)
    for n, vocab, m in calls:
        w = _dev(synth.np_weights(qt, vocab, n, rng))
        h = _dev(rng.normal(0, 1, (m, n)).astype(np.float32))
        bias = _dev(rng.normal(0, 0.01, vocab).astype(np.float32))
        (s0, b0), (s1, b1) = _both(L, w, qt, h, vocab, n, bias)
        assert np.isfinite(s0).all()
        assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32)), f"scores n={n} vocab={vocab} m={m}"
        assert np.array_equal(b0, b1), f"argmax n={n} vocab={vocab} m={m}"
        assert np.array_equal(b1, np.argmax(s1, axis=1))


def test_logits_noalloc_refuses_oversize(hipdev):
    L = hipdev
    L.check(L.init(0), "init")
    x = torch.zeros((9, 16640), device=DEV)
    w = torch.zeros(1 << 20, dtype=torch.uint8, device=DEV)
    sc = torch.zeros((9, 4), device=DEV)
    s = torch.cuda.current_stream().cuda_stream
    assert L.logits_noalloc_dev(sc.data_ptr(), None, x.data_ptr(), w.data_ptr(), 12, None, 1, 4, 16640, 0, s) == 0
    code, msg = L.last_error()
    assert code != 0 and "fixed scratch" in msg
    L.clear_error()
    assert L.logits_noalloc_dev(sc.data_ptr(), None, x.data_ptr(), w.data_ptr(), 12, None, 9, 4, 256, 0, s) == 0
    code, msg = L.last_error()
    assert code != 0 and "at most 8" in msg
    L.clear_error()


@pytest.mark.parametrize("qt,n,vocab,m", [(12, 4096, 20000, 2), (14, 2560, 15001, 1), (8, 576, 49152, 3)])
def test_logits_noalloc_under_graph_capture(hipdev, qt, n, vocab, m):
    L = hipdev
    L.check(L.init(0), "init")
    rng = np.random.default_rng(7 + qt)
    w = _dev(synth.np_weights(qt, vocab, n, rng))
    h = _dev(rng.normal(0, 1, (m, n)).astype(np.float32))
    bias = _dev(rng.normal(0, 0.01, vocab).astype(np.float32))
    ref_s = torch.empty((m, vocab), device=DEV)
    ref_b = torch.empty((m,), dtype=torch.int32, device=DEV)
    L.check(L.logits_dev(ref_s.data_ptr(), ref_b.data_ptr(), h.data_ptr(), w.data_ptr(), qt, bias.data_ptr(), m,
                         vocab, n, 0, torch.cuda.current_stream().cuda_stream), "logits")
    torch.cuda.synchronize()
    want_s, want_b = ref_s.cpu().numpy().view(np.uint32), ref_b.cpu().numpy()
    scores = torch.empty((m, vocab), device=DEV)
    best = torch.empty((m,), dtype=torch.int32, device=DEV)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):  # global capture mode
        ok = L.logits_noalloc_dev(scores.data_ptr(), best.data_ptr(), h.data_ptr(), w.data_ptr(), qt,
                                  bias.data_ptr(), m, vocab, n, 0, torch.cuda.current_stream().cuda_stream)
    L.check(ok, "logits_noalloc under capture")
    other = _dev(rng.normal(0, 1, (m, n)).astype(np.float32))
    junk_s = torch.empty((m, vocab), device=DEV)
    for rep in range(3):
        scores.fill_(float("nan"))
        best.fill_(-1)
        # eager work on the same scratch between replays
        L.check(L.logits_noalloc_dev(junk_s.data_ptr(), None, other.data_ptr(), w.data_ptr(), qt, None, m, vocab, n,
                                     0, torch.cuda.current_stream().cuda_stream), "eager noalloc")
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(scores.cpu().numpy().view(np.uint32), want_s), f"replay {rep} scores"
        assert np.array_equal(best.cpu().numpy(), want_b), f"replay {rep} argmax"
    del graph
