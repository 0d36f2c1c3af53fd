"""Writes the golden fixtures of the quantized-weight path from the reference.

Runs only where oracle/_ref/libedgexpu_ref.so exists (built by ``make -C oracle``
from the reference's src/gguf_quant.c, src/gguf_dot_q8.c and src/cpu_kernel.c).
Every fixture stores its inputs and the reference's outputs, so tests never need
the reference itself: the seeded inputs are kept as data, not regenerated.

    python tests/golden/make_golden.py        # rewrites tests/golden/*.npz
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "edgexpu-llm_amd"))

import oracle as O  # noqa: E402
from edgexpu_amd import synth  # noqa: E402

SEED = 20261201
TNAME = {1: "f16", 2: "q4_0", 6: "q5_0", 8: "q8_0", 12: "q4_k", 13: "q5_k", 14: "q6_k"}


def edge_activations() -> dict[str, np.ndarray]:
    """256-element activation vectors covering the quantizers' special cases."""
    rng = np.random.default_rng(SEED + 99)
    cases = {}
    cases["zeros"] = np.zeros(256, np.float32)
    t = np.zeros(256, np.float32)
    t[5], t[9] = 2.0, -2.0
    cases["tie_pos_first"] = t
    t = np.zeros(256, np.float32)
    t[5], t[9] = -2.0, 2.0
    cases["tie_neg_first"] = t
    t = np.zeros(256, np.float32)
    t[3], t[7] = 1e-40, -5e-41
    cases["subnormal"] = t
    cases["tiny_normal"] = np.full(256, 1e-38, np.float32)
    cases["tiny_ramp"] = (np.linspace(-1, 1, 256) * 3e-37).astype(np.float32)
    cases["halfway"] = ((np.arange(256) - 128) * 0.5).astype(np.float32)
    cases["huge"] = rng.normal(0, 1e30, 256).astype(np.float32)
    cases["one_hot_neg"] = np.where(np.arange(256) == 200, -3.0, 0.001).astype(np.float32)
    cases["normal"] = rng.normal(0, 1, 256).astype(np.float32)
    cases["block_zero_then_normal"] = np.concatenate([np.zeros(32), rng.normal(0, 1, 224)]).astype(np.float32)
    return cases


def main() -> int:
    ref = O.load_reference()
    if ref is None:
        print("oracle/_ref/libedgexpu_ref.so not built: run `make -C oracle` where the reference exists")
        return 1
    ok, msg = ref.selftest()
    assert ok, msg
    rng = np.random.default_rng(SEED)
    manifest = {}

    def save(name, **arrays):
        path = os.path.join(HERE, name + ".npz")
        # a fixture whose arrays are unchanged keeps its file (and checksum)
        same = False
        if os.path.exists(path):
            with np.load(path) as old:
                same = sorted(old.files) == sorted(arrays) and all(
                    old[k].dtype == v.dtype and np.array_equal(old[k], v) for k, v in arrays.items())
        if not same:
            np.savez_compressed(path, **arrays)
        with open(path, "rb") as f:
            manifest[name] = {"sha256": hashlib.sha256(f.read()).hexdigest(),
                              "arrays": {k: [str(v.dtype), list(v.shape)] for k, v in arrays.items()}}

    # 1. bulk dequant: 64 blocks per format (src/gguf_quant.c:139-155,223-302)
    for qt, name in ((O.Q8_0, "q8_0"), (O.Q4_K, "q4_k"), (O.Q6_K, "q6_k")):
        bs, _ = O.BLOCK[qt]
        n = 64 * bs
        w = synth.np_weights(qt, 1, n, rng).reshape(-1)
        save(f"dequant_{name}", src=w, out=ref.dequantize(w, qt, n))

    # 2. activation quantizers on edge cases and random rows (src/gguf_dot_q8.c:269-412)
    cases = edge_activations()
    names = sorted(cases)
    xs = np.stack([cases[k] for k in names])
    q80 = np.stack([ref.quantize_q8_0(x) for x in xs])
    q8k = np.stack([ref.quantize_q8_k(x) for x in xs])
    xr = synth.np_activations(8, 4096, rng)
    save("quantize", names=np.array(names), x=xs, q8_0=q80, q8_k=q8k, x_rand=xr,
         q8_0_rand=np.stack([ref.quantize_q8_0(x) for x in xr]),
         q8_k_rand=np.stack([ref.quantize_q8_k(x) for x in xr]))

    # 3. linear_quant_batch at the workloads' row widths (src/cpu_kernel.c:545-644)
    shapes = [(O.Q8_0, 576, 32, 3), (O.Q8_0, 1536, 32, 1), (O.Q4_K, 4096, 16, 3), (O.Q4_K, 2560, 16, 4),
              (O.Q6_K, 2560, 16, 2), (O.Q6_K, 9728, 8, 1), (O.Q4_K, 14336, 4, 1)]
    for qt, n_in, n_out, m in shapes:
        w = synth.np_weights(qt, n_out, n_in, rng)
        x = synth.np_activations(m, n_in, rng)
        bias = rng.normal(0, 0.1, n_out).astype(np.float32)
        out = ref.linear_quant_batch(x, w, qt, None, m, n_out, n_in)
        outb = ref.linear_quant_batch(x, w, qt, bias, m, n_out, n_in)
        save(f"linear_{TNAME[qt]}_{n_in}",
             type=np.array(qt), w=w, x=x, bias=bias, out=out, out_bias=outb)

    # 4. f32-activation row dots of the logits path (src/gguf_quant.c:539-794)
    for qt, n in ((O.Q4_K, 4096), (O.Q6_K, 2560), (O.Q8_0, 576), (O.Q4_K, 2560)):
        rows = 16
        w = synth.np_weights(qt, rows, n, rng)
        h = synth.np_activations(1, n, rng)[0]
        scores = np.array([ref.dot_f32(qt, w[i], h, n) for i in range(rows)], np.float32)
        save(f"dotf32_{TNAME[qt]}_{n}", type=np.array(qt), w=w, h=h, scores=scores)

    # 5. the dispatcher's other formats (src/gguf_quant.c:157-353, 672-892;
    #    src/gguf_dot_q8.c:482-601, 764-895): dequant, the batch driver and
    #    the f32-activation dots.  The driver's f32-activation fallback (F16
    #    rows) shares its token index across OpenMP threads
    #    (src/cpu_kernel.c:560,632-641), so its F16 fixture is bias + the
    #    reference's own row dot per token, the value that loop computes
    #    with one thread.
    for qt in (O.Q4_0, O.Q5_0, O.Q5_K, O.F16):
        bs = {O.Q4_0: 32, O.Q5_0: 32, O.Q5_K: 256, O.F16: 32}[qt]
        n = 64 * bs
        w = synth.np_weights(qt, 1, n, rng).reshape(-1)
        save(f"dequant_{TNAME[qt]}", src=w, out=ref.dequantize(w, qt, n))
    for qt, n_in, n_out, m in ((O.Q4_0, 576, 32, 3), (O.Q5_0, 1536, 24, 2), (O.Q5_K, 2560, 16, 3),
                               (O.Q5_K, 4096, 12, 1), (O.F16, 576, 24, 2)):
        w = synth.np_weights(qt, n_out, n_in, rng)
        x = synth.np_activations(m, n_in, rng)
        bias = rng.normal(0, 0.1, n_out).astype(np.float32)
        if qt == O.F16:
            dots = np.array([[ref.dot_f32(qt, w[o], x[t], n_in) for o in range(n_out)] for t in range(m)],
                            np.float32)
            out, outb = dots, (bias[None, :] + dots).astype(np.float32)
        else:
            out = ref.linear_quant_batch(x, w, qt, None, m, n_out, n_in)
            outb = ref.linear_quant_batch(x, w, qt, bias, m, n_out, n_in)
        save(f"linear_{TNAME[qt]}_{n_in}", type=np.array(qt), w=w, x=x, bias=bias, out=out, out_bias=outb)
    for qt, n in ((O.Q4_0, 576), (O.Q5_0, 1536), (O.Q5_K, 2560), (O.F16, 576)):
        rows = 16
        w = synth.np_weights(qt, rows, n, rng)
        h = synth.np_activations(1, n, rng)[0]
        scores = np.array([ref.dot_f32(qt, w[i], h, n) for i in range(rows)], np.float32)
        save(f"dotf32_{TNAME[qt]}_{n}", type=np.array(qt), w=w, h=h, scores=scores)

    # 6. softmax and sampling (src/cpu_kernel.c:328-353,762-849): per (n, seed)
    # one score vector and its probabilities; per top_p the token and state
    srng = np.random.default_rng(SEED + 6)
    sizes, seeds, tops = [1, 4, 7, 300, 2000], [0, 1, 0xDEADBEEF], [1.0, 0.9, 0.5, 0.0]
    logits, probs, toks, states = [], [], [], []
    for n in sizes:
        for seed in seeds:
            x = (srng.standard_normal(n) * srng.choice([1.0, 4.0, 12.0])).astype(np.float32)
            logits.append(x)
            probs.append(ref.softmax(x))
            for top_p in tops:
                t, _, st = ref.sample_softmax(x, top_p, seed)
                toks.append(t)
                states.append(st)
    save("sample", sizes=np.array(sizes, np.int32), seeds=np.array(seeds, np.uint64),
         top_p=np.array(tops, np.float32), logits=np.concatenate(logits), probs=np.concatenate(probs),
         tokens=np.array(toks, np.uint32), states=np.array(states, np.uint64))

    with open(os.path.join(HERE, "MANIFEST.json"), "w") as f:
        json.dump({"seed": SEED, "generator": "tests/golden/make_golden.py",
                   "reference_build": "oracle/Makefile target ref", "fixtures": manifest}, f, indent=1,
                  sort_keys=True)
    total = sum(os.path.getsize(os.path.join(HERE, k + ".npz")) for k in manifest)
    print(f"wrote {len(manifest)} fixtures, {total / 1024:.0f} KiB")
    return 0


if __name__ == "__main__":
    sys.exit(main())
