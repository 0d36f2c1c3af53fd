#!/usr/bin/env python3
"""Quantized-weight matrix path on one MI355X: decode-step GEMV throughput.

A step is one decode token through the matrix path of a model: every layer's
projections (edgexpu_cpu_linear_quant for q, k, v, o, gate, up, down;
src/native.c:2530-2580) followed by the chunked output.weight logits product
with greedy argmax (src/native.c:2292-2401).  Weights are distinct per layer,
seeded synthetic GGUF blocks resident in HBM before the timed region (so no
two launches share cached weights), activations are synthetic f32 N(0,1).

Prints one JSON line: value = algorithmic bytes of the step (weights + x + y)
per second, a `roofline` object for the dominant kernel (the grouped
gate+up launch, [2 x 14336 x 4096] Q4_K x Q8_K for the default workload,
timed with HIP events on the stream it is launched on) and a `cpu_baseline`
object (the reference's own CPU kernels built from source, oracle/_ref, timed
on this host's cores on a bounded sample).

`roofline.traffic` is the HBM bytes per launch of that kernel as measured by
rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, calibrated against a plain copy of
known size (--calibrate-copy runs that copy before the timed region); the
figures are read from profiles/traffic_<workload>.json when present.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "edgexpu-llm_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, 8 TB/s

WORKLOADS = {
    # Llama-3-8B-shaped decode, all Q4_K, logits [128256 x 4096] in 8192-row chunks
    "llama3-8b-q4k-decode": dict(layers=32, hidden=4096, qdim=4096, kv=1024, ffn=14336, vocab=128256,
                                 wtype=12, down_type=12, logits_type=12, logits_chunk=8192),
    # SmolLM2-135M-shaped decode, all Q8_0, logits [49152 x 576]
    "smollm2-135m-q8_0-decode": dict(layers=30, hidden=576, qdim=576, kv=192, ffn=1536, vocab=49152,
                                     wtype=8, down_type=8, logits_type=8, logits_chunk=0),
    # Q4_K_M hybrid ~4B (Qwen3-4B-like projections assumed), Q6_K down + logits
    "hybrid-4b-q4km-decode": dict(layers=36, hidden=2560, qdim=4096, kv=1024, ffn=9728, vocab=151936,
                                  wtype=12, down_type=14, logits_type=14, logits_chunk=0),
}


def parse():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--workload", default="llama3-8b-q4k-decode", choices=sorted(WORKLOADS))
    p.add_argument("--batch", type=int, default=1, help="tokens per step (decode batch m)")
    p.add_argument("--kernel-reps", type=int, default=4, help="passes over the layers for the per-kernel timing")
    p.add_argument("--cpu-seconds", type=float, default=12.0, help="bound on the CPU-baseline sample")
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--seed", type=int, default=20261203)
    p.add_argument("--no-extra", action="store_true", help="skip the prefill-GEMM and bulk-dequant legs")
    p.add_argument("--prefill-only", action="store_true", help="run only the prefill-GEMM leg (one JSON line)")
    p.add_argument("--dequant-only", action="store_true",
                   help="run only the bulk-dequant leg with its write ceilings (one JSON line)")
    p.add_argument("--launch-sweep", action="store_true",
                   help="time one Q4_K [rows x 4096] m=1 launch over row counts; fit fixed + marginal cost")
    p.add_argument("--layer-step", action="store_true",
                   help="time the decode step with the layer ops on device: fused layer entry vs separate launches")
    p.add_argument("--sync-costs", action="store_true",
                   help="time an empty dependent launch against a grid barrier inside one launch (one JSON line)")
    p.add_argument("--read-ceiling", action="store_true",
                   help="time a plain streaming read of each decode launch's weight bytes (one JSON line)")
    p.add_argument("--formats", action="store_true",
                   help="decode GEMV [14336 x 4096] m=1 and 1 GiB dequant for every GPU format (one JSON line)")
    p.add_argument("--sample", action="store_true",
                   help="softmax + temperature / top-p draw over a 128256-entry vocabulary on device (one JSON line)")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="first copy a 256 MiB buffer 4 times (device to device) for counter calibration")
    return p.parse_args()


COPY_BYTES = 256 << 20
MIN_ROTATION_BYTES = 600e6  # weights in rotation per timed step sequence (MI355X MALL: 256 MB)


def traffic_from_profile(workload):
    """HBM bytes per launch of the dominant kernel, from a committed counter summary."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.json")
    try:
        with open(path) as fh:
            d = json.load(fh)
        return d.get("bytes_per_launch"), d
    except (OSError, ValueError):
        return None, None


def projections(cfg):
    h, q, kv, f = cfg["hidden"], cfg["qdim"], cfg["kv"], cfg["ffn"]
    t, td = cfg["wtype"], cfg["down_type"]
    # (name, type, n_out, n_in, input vector)
    return [("q", t, q, h, "h"), ("k", t, kv, h, "h"), ("v", t, kv, h, "h"), ("o", t, h, q, "q"),
            ("gate", t, f, h, "h"), ("up", t, f, h, "h"), ("down", td, h, f, "f")]


def cpu_info():
    model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return model


def capture(fn):
    """HIP graph of fn(stream); the library's device entry points allocate
    nothing once a warm-up call has sized the workspace."""
    import torch

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn(side.cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return graph


def timed(run, n):
    """ms per run over n runs, HIP events on the stream the work is issued to."""
    import torch

    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    a.record(stream)
    for _ in range(n):
        run()
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported (across GPUs the path would "
              "split each matrix by rows, with the activation broadcast and the outputs gathered)", file=sys.stderr)
        sys.exit(2)

    # the host's CPU share, before an OpenMP runtime binds this thread; then
    # the placement for the CPU baselines (read once, when the reference's
    # libgomp loads): one thread per core, packed from the master's core
    host_cpus()
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")

    import torch

    import edgexpu_amd as E
    from edgexpu_amd import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    L = E.hip()
    L.check(L.init(0), "init")
    cfg = WORKLOADS[args.workload]
    m = args.batch
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)
    if args.launch_sweep:
        print(json.dumps(launch_sweep(L, E, synth, gen, dev)), flush=True)
        return
    if args.layer_step:
        print(json.dumps(layer_step(L, E, synth, gen, dev, cfg, args.workload, m, args.steps, args.warmup)),
              flush=True)
        return
    if args.read_ceiling:
        print(json.dumps(read_ceiling(E, cfg, args.workload, dev)), flush=True)
        return
    if args.sync_costs:
        print(json.dumps(sync_costs(dev)), flush=True)
        return
    if args.formats:
        print(json.dumps(formats_leg(L, E, synth, gen, dev, no_cpu=args.no_cpu)), flush=True)
        return
    if args.sample:
        print(json.dumps(sample_leg(L, gen, dev, no_cpu=args.no_cpu)), flush=True)
        return
    if args.prefill_only:
        # the prefill GEMM leg alone (for counter runs): one JSON line
        res = prefill_leg(L, E, synth, gen, dev, capture, timed)
        print(json.dumps({"metric": "prefill quant-GEMM TOPS, 1 GPU", "n_gpus": 1, "prefill": res}), flush=True)
        return
    if args.dequant_only:
        # the bulk dequant leg alone (for counter runs), with the calibration
        # copy first: one JSON line
        src_buf = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst_buf = torch.empty_like(src_buf)
        for _ in range(4):
            dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        del src_buf, dst_buf
        res = dequant_leg(L, E, synth, gen, dev, no_cpu=args.no_cpu)
        print(json.dumps({"metric": "bulk dequant GB/s, 1 GPU", "n_gpus": 1, "dequant": res}), flush=True)
        return

    if args.calibrate_copy:
        # a plain device copy of known size before the timed region: the
        # counter passes scale FETCH_SIZE / WRITE_SIZE by what it reads
        src_buf = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device=dev).fill_(1.0)
        dst_buf = torch.empty_like(src_buf)
        for _ in range(4):
            dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        del src_buf, dst_buf

    res = decode_leg(L, E, synth, gen, dev, args.workload, m, args.steps, args.warmup, args.kernel_reps,
                     per_kernel=True, keep_model=not args.no_cpu)
    extra = {}
    if not args.no_extra:
        extra["prefill"] = prefill_leg(L, E, synth, gen, dev, capture, timed)
        extra["dequant"] = dequant_leg(L, E, synth, gen, dev, args.no_cpu)

    # ---------------------------------------------------------------- CPU baseline
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(args, res.pop("_model"), m)
        torch.cuda.empty_cache()

    # the other decode workloads, one token per step: ms / step, GB/s, HBM
    # fraction, the grouped launches by weight format, and their CPU baselines
    if not args.no_extra:
        others = {}
        for wl in WORKLOADS:
            if wl == args.workload:
                continue
            r = decode_leg(L, E, synth, gen, dev, wl, 1, args.steps, args.warmup, args.kernel_reps, per_kernel=True,
                           keep_model=not args.no_cpu)
            model = r.pop("_model", None)
            others[wl] = {k: r[k] for k in ("ms_per_step", "value", "unit", "step_bytes", "hbm_frac_step", "kernels",
                                            "per_format", "weight_copies_rotated")}
            if model is not None:
                others[wl]["cpu_baseline"] = cpu_baseline(args, model, 1)
                del model
            torch.cuda.empty_cache()
            if wl == "hybrid-4b-q4km-decode":
                # its configuration spans batch 1-4: the step at 2 and 4 tokens
                others[wl]["batches"] = {}
                for mb in (2, 4):
                    rb = decode_leg(L, E, synth, gen, dev, wl, mb, args.steps, args.warmup, args.kernel_reps,
                                    per_kernel=False)
                    others[wl]["batches"][str(mb)] = {k: rb[k] for k in ("ms_per_step", "value", "unit",
                                                                         "hbm_frac_step")}
                    torch.cuda.empty_cache()
        extra["workloads"] = others
        # the decode step with the layer ops on device and every dependency
        # respected (rmsnorm -> q/k/v, o + residual, rmsnorm -> gate/up ->
        # silu * up, down + residual, logits), one token, each workload
        extra["layer_step"] = {}
        for wl in WORKLOADS:
            r = layer_step(L, E, synth, gen, dev, WORKLOADS[wl], wl, 1, args.steps, args.warmup, full=False)
            extra["layer_step"][wl] = {"ms_per_step": r["ms_per_step"]["fused"],
                                       "weight_GBps": r["weight_GBps"]["fused"], "launches_per_layer": 4}
            torch.cuda.empty_cache()

    cfg = WORKLOADS[args.workload]
    line = {
        "metric": "quant GEMV weight GB/s (% of HBM peak) + prefill quant-GEMM TOPS, 1 GPU",
        "value": res["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": res["ms_per_step"],
        "eager_ms_per_step": res["eager_ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8" if cfg["wtype"] != 0 else "f32",
        "data": "synthetic",
        "config": {"workload": args.workload, "batch": m, "layers": cfg["layers"], "hidden": cfg["hidden"],
                   "ffn": cfg["ffn"], "vocab": cfg["vocab"], "weights": E.TYPE_NAMES[cfg["wtype"]],
                   "down": E.TYPE_NAMES[cfg["down_type"]], "logits": E.TYPE_NAMES[cfg["logits_type"]],
                   "logits_chunk_rows": cfg["logits_chunk"], "step_bytes": res["step_bytes"],
                   "weight_bytes": res["weight_bytes"], "weight_copies_rotated": res["weight_copies_rotated"],
                   "hbm_frac_step": res["hbm_frac_step"]},
        "roofline": res["roofline"],
        "cpu_baseline": cpu,
        "kernels": res["kernels"],
        "per_format": res["per_format"],
    }
    line.update(extra)
    print(json.dumps(line), flush=True)


def decode_leg(L, E, synth, gen, dev, workload, m, steps, warmup, kernel_reps, per_kernel=True, keep_model=False):
    """One decode workload: its model resident in HBM (replicated to >= 600 MB
    when smaller than the MALL), a step = every layer's grouped projection
    launches + the chunked logits with greedy argmax, captured in a HIP graph
    and timed with HIP events; per-launch timings of each group over distinct
    layers; GB/s by weight format.  keep_model: the result also carries the
    device tensors (key "_model") for the CPU baseline."""
    import torch

    cfg = WORKLOADS[workload]
    projs = projections(cfg)
    one_copy = sum(cfg["layers"] * n_out * E.row_bytes(t, n_in) for _, t, n_out, n_in, _ in projs) \
        + cfg["vocab"] * E.row_bytes(cfg["logits_type"], cfg["hidden"])
    # a model smaller than the 256 MB MALL is replicated so that consecutive
    # steps read distinct weights (>= 600 MB in rotation): HBM, not cache
    copies = max(1, -(-int(MIN_ROTATION_BYTES) // one_copy))
    model = []
    for _ in range(copies):
        layers = [{name: synth.torch_weights_bulk(t, n_out, n_in, gen, dev) for name, t, n_out, n_in, _ in projs}
                  for _ in range(cfg["layers"])]
        wout = synth.torch_weights_bulk(cfg["logits_type"], cfg["vocab"], cfg["hidden"], gen, dev)
        model.append((layers, wout))
    layers, wout = model[0]
    xin = {"h": torch.randn((m, cfg["hidden"]), generator=gen, device=dev),
           "q": torch.randn((m, cfg["qdim"]), generator=gen, device=dev),
           "f": torch.randn((m, cfg["ffn"]), generator=gen, device=dev)}
    yout = {name: torch.empty((m, n_out), device=dev) for name, _, n_out, _, _ in projs}
    scores = torch.empty((m, cfg["vocab"]), device=dev)
    best = torch.empty(m, dtype=torch.int32, device=dev)
    torch.cuda.synchronize()

    step_bytes = 0
    for name, t, n_out, n_in, _ in projs:
        step_bytes += cfg["layers"] * (n_out * E.row_bytes(t, n_in) + m * n_in * 4 + m * n_out * 4)
    step_bytes += cfg["vocab"] * E.row_bytes(cfg["logits_type"], cfg["hidden"]) + m * cfg["hidden"] * 4 \
        + m * cfg["vocab"] * 4
    weight_bytes = one_copy

    # launches of one decode step: projections sharing an input are one
    # grouped launch (q/k/v, gate/up), as src/native.c:2530-2532,2576-2577
    # issue them back to back on the same normed hidden state
    groups = [(["q", "k", "v"], "h"), (["o"], "q"), (["gate", "up"], "h"), (["down"], "f")]
    pinfo = {name: (t, n_out, n_in) for name, t, n_out, n_in, _ in projs}
    arr = C.c_void_p * 4
    copy_args = []
    for c_layers, c_wout in model:
        launch_args = []
        for lw in c_layers:
            for names, src in groups:
                t, _, n_in = pinfo[names[0]]
                assert all(pinfo[nm][0] == t and pinfo[nm][2] == n_in for nm in names)
                launch_args.append((len(names), arr(*[yout[nm].data_ptr() for nm in names]), xin[src].data_ptr(),
                                    arr(*[lw[nm].data_ptr() for nm in names]), t,
                                    (C.c_int * 4)(*[pinfo[nm][1] for nm in names]), n_in))
        copy_args.append((launch_args, c_wout))

    def one_step(sp, c):
        launch_args, c_wout = copy_args[c]
        for nmat, outs, x, ws, t, nouts, n_in in launch_args:
            if not L.linear_group_dev(nmat, outs, x, ws, t, None, nouts, m, n_in, sp):
                L.check(0, "linear group")
        if not L.logits_dev(scores.data_ptr(), best.data_ptr(), xin["h"].data_ptr(), c_wout.data_ptr(),
                            cfg["logits_type"], None, m, cfg["vocab"], cfg["hidden"], cfg["logits_chunk"], sp):
            L.check(0, "logits")

    def step(sp):
        """`copies` consecutive decode steps, one per weight copy."""
        for c in range(copies):
            one_step(sp, c)

    cur = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    for _ in range(warmup):
        step(cur())
    eager_ms = timed(lambda: step(cur()), max(1, min(steps, 5)))
    graph = capture(step)
    for _ in range(warmup):
        graph.replay()
    ms_per_step = timed(graph.replay, steps) / copies
    eager_ms /= copies
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    del graph

    # ------------------------------------------------ per-kernel timing (GEMV only)
    def time_gemv(names, reps):
        """One product launch (fused quantize + GEMV) per layer, distinct
        matrices each time so nothing is re-read from cache."""
        t, _, n_in = pinfo[names[0]]
        src = next(p[4] for p in projs if p[0] == names[0])
        nmat = len(names)
        per_layer = [(arr(*[yout[nm].data_ptr() for nm in names]), arr(*[lw[nm].data_ptr() for nm in names]))
                     for c_layers, _ in model for lw in c_layers]
        nouts = (C.c_int * 4)(*[pinfo[nm][1] for nm in names])

        def launches(sp):
            for _ in range(reps):
                for outs, ws in per_layer:
                    L.linear_group_dev(nmat, outs, xin[src].data_ptr(), ws, t, None, nouts, m, n_in, sp)

        g = capture(launches)
        g.replay()
        # the median of five timed runs of three replays: one slow run (a
        # clock or power-state change on the box) does not set the figure
        us = sorted(timed(g.replay, 3) for _ in range(5))[2] * 1e3 / (reps * len(per_layer))
        algo = sum(pinfo[nm][1] * E.row_bytes(t, n_in) + m * pinfo[nm][1] * 4 for nm in names) + m * n_in * 4
        return {"shape": [sum(pinfo[nm][1] for nm in names), n_in], "type": E.TYPE_NAMES[t], "us": round(us, 3),
                "bytes": algo, "GBps": round(algo / (us * 1e-6) / 1e9, 1)}

    kernels = {}
    if per_kernel:
        kernels = {name: time_gemv([name], kernel_reps) for name, *_ in projs}
        kernels["qkv"] = time_gemv(["q", "k", "v"], kernel_reps)
        kernels["gate_up"] = time_gemv(["gate", "up"], kernel_reps)

        def logits_only(sp):
            for _ in range(5):
                for _, c_wout in model:
                    L.logits_dev(scores.data_ptr(), None, xin["h"].data_ptr(), c_wout.data_ptr(), cfg["logits_type"],
                                 None, m, cfg["vocab"], cfg["hidden"], cfg["vocab"], sp)

        lg = capture(logits_only)
        lg.replay()
        lus = sorted(timed(lg.replay, 2) for _ in range(5))[2] * 1e3 / (5 * len(model))
        lbytes = cfg["vocab"] * E.row_bytes(cfg["logits_type"], cfg["hidden"]) + m * cfg["hidden"] * 4 \
            + m * cfg["vocab"] * 4
        kernels["logits"] = {"shape": [cfg["vocab"], cfg["hidden"]], "type": E.TYPE_NAMES[cfg["logits_type"]],
                             "us": round(lus, 3), "bytes": lbytes, "GBps": round(lbytes / (lus * 1e-6) / 1e9, 1)}
        del lg

    # GB/s by weight format over one step's launches (grouped launches as the
    # step issues them: q+k+v, o, gate+up, down; the logits)
    per_format = {}
    if per_kernel:
        for key, mult in (("qkv", cfg["layers"]), ("o", cfg["layers"]), ("gate_up", cfg["layers"]),
                          ("down", cfg["layers"]), ("logits", 1)):
            k = kernels[key]
            f = per_format.setdefault(k["type"], {"bytes": 0, "us": 0.0})
            f["bytes"] += mult * k["bytes"]
            f["us"] += mult * k["us"]
        for f in per_format.values():
            f["GBps"] = round(f["bytes"] / (f["us"] * 1e-6) / 1e9, 1)
            f["us"] = round(f["us"], 1)

    roofline = None
    if per_kernel:
        dom = kernels["gate_up"]
        traffic, tinfo = traffic_from_profile(workload)
        roofline = {"bound": "hbm", "achieved": dom["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                    "kernel": f"{decode_kernel_name(cfg['wtype'], dom['shape'][1], m, dom['shape'][0])} "
                              f"({E.TYPE_NAMES[cfg['wtype']]}, gate+up grouped) "
                              f"{dom['shape'][0]}x{dom['shape'][1]} m={m}",
                    "us_per_launch": dom["us"], "bytes_per_launch": dom["bytes"]}
        if tinfo is not None:
            roofline["traffic_source"] = tinfo.get("source")

    out = {"workload": workload, "batch": m, "ms_per_step": round(ms_per_step, 4),
           "eager_ms_per_step": round(eager_ms, 4), "value": round(value, 1), "unit": "GB/s",
           "step_bytes": step_bytes, "weight_bytes": weight_bytes, "weight_copies_rotated": copies,
           "hbm_frac_step": round(value / HBM_PEAK_GBS, 4), "kernels": kernels, "per_format": per_format,
           "roofline": roofline}
    if keep_model:
        out["_model"] = {"cfg": cfg, "workload": workload, "projs": projs, "layers": layers, "wout": wout,
                         "xin": xin, "step_bytes": step_bytes}
    del model, copy_args
    return out


def decode_kernel_name(t, n_in, m, rows):
    """The kernel the library picks for a decode launch in its default mode
    (csrc/gemv_stream.hip gemv_stream_take): the streaming kernel for one to
    four tokens of Q4_K rows of 2560 or 4096, of 14336 from 2048 rows on (four
    tokens at any size), and of Q6_K rows of 9728 from 2048 rows on; the
    fused kernel otherwise."""
    if t == 12 and 1 <= m <= 4 and (n_in in (2560, 4096) or (n_in == 14336 and (rows >= 2048 or m == 4))):
        return "gemv_stream_q4k"
    if t == 14 and 1 <= m <= 4 and n_in == 9728 and rows >= 2048:
        return "gemv_stream_q4k"
    return "gemv_fused_kernel"


INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA
F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA


def prefill_leg(L, E, synth, gen, dev, capture, timed):
    """Prefill GEMM at m = 512 tokens on the 8B Q4_K shapes (f32 activations,
    weights distinct per launch), both prefill modes; each call quantizes the
    activations into the GEMM's operand layout and runs the GEMM.  TOPS =
    2*M*N*K per call-second.  Exact mode: fp16 matrix cores on exact integer
    operands, one MFMA per product plus one per 16 for the min term, so the
    MFMA pipes run at (17/16) x TOPS / fp16 peak of their capacity; reported
    also against the int8 peak.  fp16 mode: fp16-rounded operands, 1e-3."""
    import torch

    M = 512
    out = {}
    out_f16 = {}
    for n_out, n_in in ((4096, 4096), (14336, 4096), (4096, 14336)):
        ws = [synth.torch_weights_bulk(12, n_out, n_in, gen, dev) for _ in range(2)]
        x = torch.randn((M, n_in), generator=gen, device=dev)
        y = torch.empty((M, n_out), device=dev)

        def launches(sp, ws=ws, x=x, y=y, n_out=n_out, n_in=n_in):
            for _ in range(2):
                for w in ws:
                    if not L.linear_dev(y.data_ptr(), x.data_ptr(), w.data_ptr(), 12, None, M, n_out, n_in, sp):
                        L.check(0, "prefill gemm")

        for mode, res in ((0, out), (1, out_f16)):
            L.check(L.set_prefill_mode(mode), "prefill mode")
            g = capture(launches)
            g.replay()
            us = timed(g.replay, 3) * 1e3 / 4
            tops = 2.0 * M * n_out * n_in / (us * 1e-6) / 1e12
            if mode == 0:
                res[f"{n_out}x{n_in}"] = {"us": round(us, 2), "TOPS": round(tops, 1),
                                          "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4),
                                          "frac_f16_peak": round(tops / F16_PEAK_TFLOPS, 4),
                                          "mfma_pipe_frac": round(17.0 / 16.0 * tops / F16_PEAK_TFLOPS, 4)}
            else:
                res[f"{n_out}x{n_in}"] = {"us": round(us, 2), "TOPS": round(tops, 1),
                                          "frac_f16_peak": round(tops / F16_PEAK_TFLOPS, 4)}
            del g
        L.check(L.set_prefill_mode(0), "prefill mode")
        del ws, x, y
    # the other formats (exact mode only): the hybrid model's Q6_K down
    # projection, the SmolLM2 Q8_0 gate/up, and [4096 x 4096] per format; each
    # call packs the activations, repacks the weights and runs the GEMM
    others = {}
    for qt, n_out, n_in in ((14, 2560, 9728), (8, 1536, 576), (13, 4096, 4096), (14, 4096, 4096),
                            (8, 4096, 4096), (2, 4096, 4096), (6, 4096, 4096)):
        ws = [synth.torch_weights_bulk(qt, n_out, n_in, gen, dev) for _ in range(2)]
        x = torch.randn((M, n_in), generator=gen, device=dev)
        y = torch.empty((M, n_out), device=dev)

        def launches(sp, ws=ws, x=x, y=y, n_out=n_out, n_in=n_in, qt=qt):
            for _ in range(2):
                for w in ws:
                    if not L.linear_dev(y.data_ptr(), x.data_ptr(), w.data_ptr(), qt, None, M, n_out, n_in, sp):
                        L.check(0, "prefill gemm")

        g = capture(launches)
        g.replay()
        us = timed(g.replay, 3) * 1e3 / 4
        tops = 2.0 * M * n_out * n_in / (us * 1e-6) / 1e12
        others[f"{E.TYPE_NAMES[qt]} {n_out}x{n_in}"] = {"us": round(us, 2), "TOPS": round(tops, 1),
                                                        "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        del g, ws, x, y
    return {"m": M, "weights": "q4_k", "input": "f32 activations (quantize + GEMM per call)",
            "exact": {"peak_int8_TOPS": INT8_PEAK_TOPS, "peak_f16_TFLOPS": F16_PEAK_TFLOPS, "tolerance": 1e-5,
                      "shapes": out},
            "f16": {"peak_TFLOPS": F16_PEAK_TFLOPS, "tolerance": 1e-3, "shapes": out_f16},
            "exact_other_formats": {"note": "pack + per-call weight repack + GEMM per call", "shapes": others}}


def launch_sweep(L, E, synth, gen, dev):
    """Per-launch time of the decode GEMV ([rows x 4096] Q4_K, m = 1, 32
    distinct matrices per size so nothing is re-read from cache) against the
    row count, and a least-squares fit time = fixed + bytes / rate over the
    sizes of at least 4096 rows.  The empty-kernel time is a one-element torch
    add in the same kind of graph."""
    import numpy as np
    import torch

    K, NL = 4096, 32
    x = torch.randn((1, K), generator=gen, device=dev)
    arr = C.c_void_p * 4
    rows_list = (64, 1024, 4096, 8192, 14336, 28672, 57344)
    res = {}
    for rows in rows_list:
        ws = [synth.torch_weights_bulk(12, rows, K, gen, dev) for _ in range(NL)]
        y = torch.empty((1, rows), device=dev)
        nouts = (C.c_int * 4)(rows)

        def launches(sp, ws=ws, y=y, nouts=nouts):
            for _ in range(2):
                for w in ws:
                    if not L.linear_group_dev(1, arr(y.data_ptr()), x.data_ptr(), arr(w.data_ptr()), 12, None, nouts,
                                              1, K, sp):
                        L.check(0, "linear group")

        g = capture(launches)
        g.replay()
        us = timed(g.replay, 3) * 1e3 / (2 * NL)
        byts = rows * E.row_bytes(12, K)
        res[rows] = {"us": round(us, 3), "bytes": byts, "GBps": round(byts / (us * 1e-6) / 1e9, 1)}
        del ws, y, g
    t = torch.zeros(1, device=dev)

    def tiny(sp):
        for _ in range(256):
            t.add_(1.0)

    g = capture(tiny)
    g.replay()
    empty_us = timed(g.replay, 3) * 1e3 / 256
    big = [r for r in rows_list if r >= 4096]
    A = np.array([[1.0, res[r]["bytes"]] for r in big])
    b = np.array([res[r]["us"] for r in big])
    (fixed, per_byte), *_ = np.linalg.lstsq(A, b, rcond=None)
    return {"metric": "decode GEMV per-launch time vs rows, 1 GPU", "k": K, "type": "q4_k", "m": 1,
            "launches": {str(r): v for r, v in res.items()}, "empty_kernel_us": round(empty_us, 3),
            "fit": {"fixed_us": round(float(fixed), 3), "marginal_GBps": round(1e-3 / float(per_byte), 1),
                    "rows_fitted": list(big)}}


def layer_step(L, E, synth, gen, dev, cfg, workload, m, steps, warmup, full=True):
    """The decode step's matrix path with the ops between the projections on
    device (src/native.c:2529-2580; attention itself is not on this path, so
    o reads q):  rmsnorm -> q/k/v, o + residual, rmsnorm -> gate/up,
    silu(gate) * up -> down + residual, then the logits.  Timed two ways,
    HIP graphs of whole steps, HIP events: through
    edgexpu_hip_layer_linear_dev and edgexpu_hip_gate_up_silu_dev (the layer
    ops inside the projection launches: 4 launches per layer) and as separate
    launches (rmsnorm, the grouped projection, add, silu_mul: 9 per layer)."""
    import torch

    projs = projections(cfg)
    pinfo = {name: (t, n_out, n_in) for name, t, n_out, n_in, _ in projs}
    one_copy = sum(cfg["layers"] * n_out * E.row_bytes(t, n_in) for _, t, n_out, n_in, _ in projs)
    copies = max(1, -(-int(MIN_ROTATION_BYTES) // one_copy))
    h = cfg["hidden"]
    model = []
    for _ in range(copies):
        model.append([{name: synth.torch_weights_bulk(t, n_out, n_in, gen, dev) for name, t, n_out, n_in, _ in projs}
                      for _ in range(cfg["layers"])])
    wout = synth.torch_weights_bulk(cfg["logits_type"], cfg["vocab"], h, gen, dev)
    norms = [(1 + 0.1 * torch.randn(h, generator=gen, device=dev), 1 + 0.1 * torch.randn(h, generator=gen, device=dev))
             for _ in range(cfg["layers"])]
    hidden = torch.randn((m, h), generator=gen, device=dev)
    buf = {name: torch.empty((m, n_out), device=dev) for name, _, n_out, _, _ in projs}
    normed = torch.empty((m, h), device=dev)
    tmp = torch.empty((m, h), device=dev)
    act = torch.empty((m, cfg["ffn"]), device=dev)
    scores = torch.empty((m, cfg["vocab"]), device=dev)
    best = torch.empty(m, dtype=torch.int32, device=dev)
    arr = C.c_void_p * 4
    eps = 1e-5

    def ptrs(ts):
        return arr(*[t.data_ptr() for t in ts])

    def nouts(names):
        return (C.c_int * 4)(*[pinfo[n][1] for n in names])

    def lin(sp, names, x, outs, lw, x2=None, nw=None, resid=None):
        t, _, n_in = pinfo[names[0]]
        ok = L.layer_linear_dev(len(names), ptrs(outs), x.data_ptr(), None if x2 is None else x2.data_ptr(),
                                None if nw is None else nw.data_ptr(), eps, ptrs([lw[n] for n in names]), t, None,
                                None if resid is None else arr(*[resid.data_ptr()]), nouts(names), m, n_in, sp)
        L.check(ok, "layer_linear")

    def group(sp, names, x, outs, lw):
        t, _, n_in = pinfo[names[0]]
        L.check(L.linear_group_dev(len(names), ptrs(outs), x.data_ptr(), ptrs([lw[n] for n in names]), t, None,
                                   nouts(names), m, n_in, sp), "linear group")

    def logits(sp):
        L.check(L.logits_dev(scores.data_ptr(), best.data_ptr(), hidden.data_ptr(), wout.data_ptr(),
                             cfg["logits_type"], None, m, cfg["vocab"], h, cfg["logits_chunk"], sp), "logits")

    def gate_up_silu(sp, lw, fn):
        t, _, n_in = pinfo["gate"]
        L.check(L.gate_up_silu_dev(act.data_ptr(), hidden.data_ptr(), fn.data_ptr(), eps, lw["gate"].data_ptr(),
                                   lw["up"].data_ptr(), t, None, None, m, cfg["ffn"], n_in, sp), "gate_up_silu")

    def fused(sp):
        for layers in model:
            for lw, (an, fn) in zip(layers, norms):
                lin(sp, ["q", "k", "v"], hidden, [buf["q"], buf["k"], buf["v"]], lw, nw=an)
                lin(sp, ["o"], buf["q"], [hidden], lw, resid=hidden)
                gate_up_silu(sp, lw, fn)
                lin(sp, ["down"], act, [hidden], lw, resid=hidden)
            logits(sp)

    def separate(sp):
        for layers in model:
            for lw, (an, fn) in zip(layers, norms):
                L.check(L.rmsnorm_dev(normed.data_ptr(), hidden.data_ptr(), an.data_ptr(), m, h, eps, sp), "rmsnorm")
                group(sp, ["q", "k", "v"], normed, [buf["q"], buf["k"], buf["v"]], lw)
                group(sp, ["o"], buf["q"], [tmp], lw)
                L.check(L.add_dev(hidden.data_ptr(), hidden.data_ptr(), tmp.data_ptr(), m * h, sp), "add")
                L.check(L.rmsnorm_dev(normed.data_ptr(), hidden.data_ptr(), fn.data_ptr(), m, h, eps, sp), "rmsnorm")
                group(sp, ["gate", "up"], normed, [buf["gate"], buf["up"]], lw)
                L.check(L.silu_mul_dev(act.data_ptr(), buf["gate"].data_ptr(), buf["up"].data_ptr(),
                                       m * cfg["ffn"], sp), "silu_mul")
                group(sp, ["down"], act, [tmp], lw)
                L.check(L.add_dev(hidden.data_ptr(), hidden.data_ptr(), tmp.data_ptr(), m * h, sp), "add")
            logits(sp)

    res = {}
    for name, fn in (("fused", fused), ("separate", separate)) if full else (("fused", fused),):
        g = capture(fn)
        for _ in range(max(1, warmup)):
            g.replay()
        res[name] = round(timed(g.replay, steps) / copies, 4)
        del g
    # each fused launch kind alone over the layers (us per launch)
    layers0 = model[0]
    kinds = {
        "qkv_rmsnorm": lambda sp, lw, an, fn: lin(sp, ["q", "k", "v"], hidden, [buf["q"], buf["k"], buf["v"]], lw,
                                                  nw=an),
        "o_residual": lambda sp, lw, an, fn: lin(sp, ["o"], buf["q"], [hidden], lw, resid=hidden),
        "gate_up_rmsnorm": lambda sp, lw, an, fn: lin(sp, ["gate", "up"], hidden, [buf["gate"], buf["up"]], lw,
                                                      nw=fn),
        "gate_up_rmsnorm_silu_mul": lambda sp, lw, an, fn: gate_up_silu(sp, lw, fn),
        "down_residual": lambda sp, lw, an, fn: lin(sp, ["down"], act, [hidden], lw, resid=hidden),
        "down_silu_mul_residual": lambda sp, lw, an, fn: lin(sp, ["down"], buf["gate"], [hidden], lw, x2=buf["up"],
                                                             resid=hidden),
    }
    per = {}
    for kname, kfn in kinds.items() if full else ():
        def body(sp, kfn=kfn):
            for _ in range(4):
                for lw, (an, fn) in zip(layers0, norms):
                    kfn(sp, lw, an, fn)
        g = capture(body)
        g.replay()
        per[kname] = round(timed(g.replay, 3) * 1e3 / (4 * len(layers0)), 3)
        del g
    weight_bytes = sum(cfg["layers"] * n_out * E.row_bytes(t, n_in) for _, t, n_out, n_in, _ in projs) \
        + cfg["vocab"] * E.row_bytes(cfg["logits_type"], h)
    return {"metric": "decode step with the layer ops on device, ms per step, 1 GPU", "workload": workload,
            "batch": m, "layers": cfg["layers"], "ms_per_step": res, "fused_us_per_launch": per,
            "launches_per_layer": {"fused": 4, "separate": 9},
            "weight_GBps": {k: round(weight_bytes / (v * 1e-3) / 1e9, 1) for k, v in res.items()}}


def read_ceiling(E, cfg, workload, dev):
    """A plain streaming read (lib/libexq_bench_read.so: one 16-byte load per
    lane, grid-stride, no arithmetic) of each decode launch's weight bytes,
    timed like the GEMV launches: a HIP graph of launches over distinct
    buffers (>= 600 MB in rotation), HIP events around it.  The best of three
    grid sizes per launch."""
    import torch

    lib = C.CDLL(os.path.join(ROOT, "edgexpu-llm_amd", "lib", "libexq_bench_read.so"))
    lib.exq_bench_read.argtypes = [C.c_void_p, C.c_longlong, C.c_void_p, C.c_int, C.c_void_p]
    lib.exq_bench_read.restype = C.c_int
    h, t, td = cfg["hidden"], cfg["wtype"], cfg["down_type"]
    launches = {
        "qkv": (cfg["qdim"] + 2 * cfg["kv"]) * E.row_bytes(t, h),
        "o": h * E.row_bytes(t, cfg["qdim"]),
        "gate_up": 2 * cfg["ffn"] * E.row_bytes(t, h),
        "down": h * E.row_bytes(td, cfg["ffn"]),
        "logits": cfg["vocab"] * E.row_bytes(cfg["logits_type"], h),
    }
    grids = (1024, 2048, 4096)
    out = torch.empty(max(grids) * 256, dtype=torch.int32, device=dev)
    res = {}
    for name, nbytes in launches.items():
        nbytes -= nbytes % 256
        n = max(4, -(-int(MIN_ROTATION_BYTES) // nbytes))
        buf = torch.ones(n * nbytes, dtype=torch.uint8, device=dev)
        best = None
        for grid in grids:
            def launches_fn(sp, grid=grid):
                for i in range(n):
                    if lib.exq_bench_read(buf.data_ptr() + i * nbytes, nbytes, out.data_ptr(), grid, sp) != 0:
                        raise RuntimeError("exq_bench_read failed")

            g = capture(launches_fn)
            g.replay()
            us = min(timed(g.replay, 3) for _ in range(2)) * 1e3 / n
            if best is None or us < best[0]:
                best = (us, grid)
            del g
        res[name] = {"bytes": nbytes, "us": round(best[0], 3), "GBps": round(nbytes / (best[0] * 1e-6) / 1e9, 1),
                     "grid": best[1]}
        del buf
    return {"metric": "plain read of each decode launch's weight bytes, us per launch, 1 GPU",
            "workload": workload, "launches": res}


def sync_costs(dev):
    """What a persistent multi-phase decode kernel would pay per phase
    instead of a dependent launch (lib/libexq_bench_read.so): an empty
    launch in a HIP graph, against a grid barrier of one workgroup per CU
    (all 256, or the 32 of XCD 0) with agent-scope release/acquire (every
    store visible to every later load on any XCD) or with relaxed atomics
    only (no data visibility); and a hierarchical barrier (per-XCD arrival
    counters and release words, relaxed atomics), alone and with a phase's
    data exchanged through write-through atomic stores and loads (no L2
    writeback or invalidate).  Barrier cost = (launch of 101 barriers -
    launch of 1) / 100."""
    import torch

    lib = C.CDLL(os.path.join(ROOT, "edgexpu-llm_amd", "lib", "libexq_bench_read.so"))
    lib.exq_bench_empty.argtypes = [C.c_int, C.c_int, C.c_void_p]
    lib.exq_bench_barrier.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p]
    lib.exq_bench_barrier_words.restype = C.c_longlong
    words = torch.zeros(int(lib.exq_bench_barrier_words()) // 4, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    res = {"cus": cus, "empty_launch_us": {}, "barrier_us": {}}
    for grid, threads in ((1, 64), (cus, 1024)):
        def empties(sp, grid=grid, threads=threads):
            for _ in range(200):
                if lib.exq_bench_empty(grid, threads, sp) != 0:
                    raise RuntimeError("exq_bench_empty failed")

        g = capture(empties)
        res["empty_launch_us"][f"{grid}x{threads}"] = round(min(timed(g.replay, 3) for _ in range(2)) * 1e3 / 200, 3)
        del g
    for xcd0, mode in ((0, 0), (0, 1), (1, 0), (1, 1), (0, 2), (0, 3)):
        per = {}
        for rounds in (1, 101):
            def barriers(sp, rounds=rounds, mode=mode, xcd0=xcd0):
                for _ in range(20):
                    if lib.exq_bench_barrier(words.data_ptr(), cus, 1024, rounds, mode, xcd0, sp) != 0:
                        raise RuntimeError("exq_bench_barrier failed")

            g = capture(barriers)
            per[rounds] = min(timed(g.replay, 2) for _ in range(2)) * 1e3 / 20
            del g
        key = ("xcd0_32wg" if xcd0 else f"all_{cus}wg") + {0: "_release_acquire", 1: "_relaxed",
                                                           2: "_per_xcd_relaxed",
                                                           3: "_per_xcd_relaxed_write_through_data"}[mode]
        res["barrier_us"][key] = {"launch_1_barrier": round(per[1], 3),
                                  "per_barrier": round((per[101] - per[1]) / 100, 3)}
    torch.cuda.synchronize()
    err = int(words.view(-1)[64].item())
    if err != 0:
        raise RuntimeError("a barrier wait ran out of polls (grid not co-resident)")
    return {"metric": "dependent launch vs grid barrier, us, 1 GPU", **res}


def formats_leg(L, E, synth, gen, dev, no_cpu=False):
    """One decode GEMV launch (m = 1, [14336 x 4096], f32 x quantized inside
    the launch where the format takes quantized activations) per GPU format,
    through the grouped entry point, in a HIP graph over distinct matrices
    (>= 600 MB in rotation); GB/s = (weights + x + y bytes) / launch time.
    Then 1 GiB bulk dequant of the formats beyond Q8_0 / Q4_K / Q6_K."""
    import torch

    K, N = 4096, 14336
    x = torch.randn((1, K), generator=gen, device=dev)
    y = torch.empty((1, N), device=dev)
    arr = C.c_void_p * 4
    nouts = (C.c_int * 4)(N)
    gemv = {}
    for qt in (8, 2, 6, 12, 13, 14, 1):
        rb = E.row_bytes(qt, K)
        nmat = max(2, -(-int(MIN_ROTATION_BYTES) // (N * rb)))
        ws = [synth.torch_weights_bulk(qt, N, K, gen, dev) for _ in range(nmat)]

        def launches(sp, ws=ws, qt=qt):
            for _ in range(2):
                for w in ws:
                    if not L.linear_group_dev(1, arr(y.data_ptr()), x.data_ptr(), arr(w.data_ptr()), qt, None, nouts,
                                              1, K, sp):
                        L.check(0, "linear group")

        g = capture(launches)
        g.replay()
        us = timed(g.replay, 5) * 1e3 / (2 * nmat)
        byts = N * rb + K * 4 + N * 4
        gemv[E_name(qt)] = {"us": round(us, 3), "bytes": byts, "GBps": round(byts / (us * 1e-6) / 1e9, 1),
                            "frac": round(byts / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "matrices": nmat}
        del ws, g
        torch.cuda.empty_cache()
    deq = dequant_leg(L, E, synth, gen, dev, no_cpu=no_cpu, types=((2, "q4_0"), (6, "q5_0"), (13, "q5_k"), (1, "f16")))
    return {"metric": "decode GEMV and bulk dequant per GGUF format, 1 GPU", "gemv_shape": [N, K], "m": 1,
            "gemv": gemv, "dequant_1GiB": deq}


def sample_leg(L, gen, dev, no_cpu=False, vocab=128256, reps=50):
    """Softmax of a [vocab] f32 score vector in place and one draw
    (edgexpu_hip_sample_softmax_dev), eager launches on one stream (the
    generator's uniform is a kernel argument, so a draw is not replayed from
    a graph); top_p 1.0 (index-order draw) and 0.9 (radix selection of the
    kept prefix's end and of the drawn item).  Each call starts from fresh
    scores (seeded normal x 3.0, copied in before the call; the copy's own
    time, measured alone, is subtracted).  The top-p draw's work depends on
    the distribution, so it is also timed on a flat one: calls that run on
    the previous call's probabilities ("top_p_0.9_flat").  Beside it, unless
    no_cpu, the reference's edgexpu_cpu_sample_softmax on one host core over
    the same scores."""
    import torch

    base = torch.randn(vocab, generator=gen, device=dev) * 3.0
    x = torch.empty_like(base)
    out = torch.empty(1, dtype=torch.int32, device=dev)
    st = C.c_uint64(1)
    sp = torch.cuda.current_stream().cuda_stream
    res = {}

    def copy_in():
        x.copy_(base)

    copy_in()
    copy_us = timed(copy_in, reps) * 1e3
    for top_p in (1.0, 0.9):

        def run(top_p=top_p):
            if not L.sample_dev(x.data_ptr(), vocab, top_p, C.byref(st), out.data_ptr(), sp):
                L.check(0, "sample_softmax")

        def fresh(run=run):
            copy_in()
            run()

        fresh()
        us = timed(fresh, reps) * 1e3 - copy_us
        res[f"top_p_{top_p}"] = {"us": round(us, 2)}
        if top_p < 1.0:
            copy_in()
            run()
            res[f"top_p_{top_p}_flat"] = {"us": round(timed(run, reps) * 1e3, 2)}
    res["copy_us"] = round(copy_us, 2)
    if not no_cpu:
        import oracle as O

        ref, kind = O.load_reference(), "reference"
        if ref is None:
            ref, kind = O.load_oracle(), "port"
        scores = base.cpu().numpy()
        for top_p in (1.0, 0.9):
            t0 = time.perf_counter()
            for _ in range(5):
                ref.sample_softmax(scores, top_p, 1)
            res[f"top_p_{top_p}"]["cpu_us"] = round((time.perf_counter() - t0) / 5 * 1e6, 1)
        res["cpu_kind"] = kind
    return {"metric": "softmax + draw per decode step, 1 GPU", "vocab": vocab, "unit": "us", "sample": res}


def _write_ceilings(dst, dst_bytes, src, src_bytes, sp):
    """ms of a plain write of dst_bytes, and of a read of src_bytes feeding a
    write of dst_bytes (lib/libexq_bench_read.so), best over grid sizes."""
    import torch

    lib = C.CDLL(os.path.join(ROOT, "edgexpu-llm_amd", "lib", "libexq_bench_read.so"))
    lib.exq_bench_write.argtypes = [C.c_void_p, C.c_longlong, C.c_int, C.c_void_p]
    lib.exq_bench_write.restype = C.c_int
    lib.exq_bench_read_write.argtypes = [C.c_void_p, C.c_longlong, C.c_void_p, C.c_longlong, C.c_int, C.c_void_p]
    lib.exq_bench_read_write.restype = C.c_int
    db = dst_bytes // 16 * 16

    def best(fn):
        res = []
        for grid in (2048, 4096, 8192, 16384):
            if fn(grid) != 0:
                raise RuntimeError("ceiling kernel refused its arguments")
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(3):
                fn(grid)
            b.record()
            torch.cuda.synchronize()
            res.append(a.elapsed_time(b) / 3)
        return min(res)

    w = best(lambda g: lib.exq_bench_write(dst.data_ptr(), db, g, sp))
    rw = best(lambda g: lib.exq_bench_read_write(src.data_ptr(), src_bytes, dst.data_ptr(), db, g, sp))
    return w, rw


def dequant_leg(L, E, synth, gen, dev, no_cpu=False, types=((8, "q8_0"), (12, "q4_k"), (14, "q6_k"))):
    """Bulk dequantization of 1 GiB of blocks per format to f32 (the block
    contents are a 16 MiB seeded tile repeated); GB/s = (src + dst bytes) / s.
    Beside it the same bytes without the arithmetic (a plain write of the
    output; a read of the source feeding the write), and, unless no_cpu, the
    reference's own dequant on one host core."""
    import torch

    out = {}
    tile_bytes = 16 << 20
    ref, kind = None, None
    if not no_cpu:
        import oracle as O

        ref, kind = O.load_reference(), "reference"
        if ref is None:
            ref, kind = O.load_oracle(), "port"
    for qt, name in types:
        be = {1: 32, 2: 32, 6: 32, 8: 32}.get(qt, 256)
        bb = E.row_bytes(qt, be)
        nblk = (1 << 30) // bb
        tile_rows = tile_bytes // (bb * 64)
        tile = synth.torch_weights_bulk(qt, tile_rows, 64 * be, gen, dev).reshape(-1)
        src = tile.repeat((nblk * bb + tile.numel() - 1) // tile.numel())[: nblk * bb].contiguous()
        n = nblk * be
        dst = torch.empty(n, dtype=torch.float32, device=dev)
        sp = torch.cuda.current_stream().cuda_stream
        L.check(L.dequant_dev(src.data_ptr(), qt, n, dst.data_ptr(), sp), "dequant")
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(3):
            L.dequant_dev(src.data_ptr(), qt, n, dst.data_ptr(), sp)
        b.record()
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / 3
        byts = nblk * bb + n * 4
        out[name] = {"blocks": nblk, "src_bytes": nblk * bb, "dst_bytes": n * 4, "ms": round(ms, 3),
                     "GBps": round(byts / (ms * 1e-3) / 1e9, 1)}
        # ceilings of the same bytes without the arithmetic (best grid):
        # writing the output alone, and reading the source while writing it
        cw, crw = _write_ceilings(dst, n * 4, src, (nblk * bb) // 16 * 16, sp)
        out[name]["ceiling"] = {"write_only_ms": round(cw, 3), "read_write_ms": round(crw, 3),
                                "read_write_GBps": round(byts / (crw * 1e-3) / 1e9, 1),
                                "frac_of_read_write": round(crw / ms, 3)}
        if ref is not None:
            # the reference's dequant is single-threaded (no OpenMP): the same
            # 1 GiB of blocks in host memory, 64 MiB pieces in turn (source and
            # output beyond the last-level cache) on one host core
            import numpy as np

            host_src = src.cpu().numpy()
            piece = (64 << 20) // bb * bb
            ns = piece // bb * be
            dst_host = np.empty(ns, np.float32)
            f32p, u8p = C.POINTER(C.c_float), C.POINTER(C.c_uint8)
            ebuf = C.create_string_buffer(256)
            tail = (ebuf, 256) if kind == "reference" else ()
            args_at = [(host_src[o:o + piece].ctypes.data_as(u8p), qt, ns, dst_host.ctypes.data_as(f32p)) + tail
                       for o in range(0, host_src.size - piece + 1, piece)]
            ref._deq(*args_at[0])
            reps, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < 1.0 or reps < len(args_at):
                ref._deq(*args_at[reps % len(args_at)])
                reps += 1
            dt = (time.perf_counter() - t0) / reps
            out[name]["cpu_baseline"] = {"value": round((piece + ns * 4) / dt / 1e9, 2), "unit": "GB/s",
                                         "cores": 1, "kind": kind,
                                         "sample": f"{reps} pieces of 64 MiB of blocks in turn over the 1 GiB "
                                                   f"source ({len(args_at)} distinct), one thread"}
            del host_src, dst_host
        del tile, src, dst
        torch.cuda.empty_cache()
    return out


_HOST = {}


def host_cpus():
    """CPUs this process may run on (its affinity set, taken once before any
    OpenMP runtime binds the calling thread) and the share used for the CPU
    baselines: OMP_NUM_THREADS when set, else that set, at most 16."""
    if not _HOST:
        try:
            n = len(os.sched_getaffinity(0))
        except OSError:
            n = os.cpu_count() or 1
        _HOST["nproc"] = n
        share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
        _HOST["share"] = share if share > 0 else min(16, n)
    return _HOST


def lscpu_info():
    """CPU model, sockets, physical cores, threads per core, L3 and the
    process's CPU set / quota (the host's share of cores)."""
    info = {"model": cpu_info()}
    try:
        import subprocess

        txt = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "Socket(s)":
                info["sockets"] = int(v)
            elif k == "Core(s) per socket":
                info["cores_per_socket"] = int(v)
            elif k == "Thread(s) per core":
                info["threads_per_core"] = int(v)
            elif k in ("L3 cache", "L3"):
                info["l3"] = v
    except (OSError, ValueError):
        pass
    info["nproc"] = host_cpus()["nproc"]
    try:
        with open("/sys/fs/cgroup/cpu.max") as fh:
            q, per = fh.read().split()
            if q != "max":
                info["cgroup_cpus"] = round(int(q) / int(per), 2)
    except (OSError, ValueError):
        pass
    return info


_PROBE = {}


def _capture_fd2(fn):
    """Runs fn() with file descriptor 2 (C stderr) captured; returns (result, text)."""
    import tempfile

    sys.stderr.flush()
    saved = os.dup(2)
    with tempfile.TemporaryFile(mode="w+b") as tmp:
        os.dup2(tmp.fileno(), 2)
        try:
            r = fn()
        finally:
            os.dup2(saved, 2)
            os.close(saved)
        tmp.seek(0)
        text = tmp.read().decode(errors="replace")
    return r, text


def cpu_baseline(args, model, m):
    """The reference's CPU path on the same decode step:
    every layer's projections through edgexpu_cpu_linear_quant_batch of the
    reference built from its own sources (oracle/_ref), the logits through
    src/native.c's greedy chunked loop (2292-2401: Q8_0 hidden state for the
    Q8_0 family, OpenMP rows, per-thread argmax) over the same build's row
    dots (oracle/ref_logits.c), on this host's cores; where the reference was
    never built, both through the oracle's restatements.  The
    weights are copied to host memory (the whole step: beyond the LLC), the
    step is timed over a bounded number of repetitions, twice:
      (a) OpenMP threads = the host's share of cores (OMP_NUM_THREADS, else
          the CPU set, at most 16), bound one per core (OMP_PROC_BIND=close,
          OMP_PLACES=cores);
      (b) the reference's own thread probe (src/cpu_kernel.c:28-177), which
          runs only while OMP_NUM_THREADS is unset, over 1, 2, 4 .. that share.
    value = run (a)."""
    import numpy as np

    import oracle as O

    cfg, projs = model["cfg"], model["projs"]
    ref = O.load_reference()
    ora = O.load_oracle()
    kind = "reference" if ref is not None else "port"
    lin = ref if ref is not None else ora
    share = host_cpus()["share"]
    host = [{name: lw[name].cpu().numpy() for name, *_ in projs} for lw in model["layers"]]
    wout = model["wout"].cpu().numpy()
    x = {k: np.ascontiguousarray(v.cpu().numpy().astype(np.float32)) for k, v in model["xin"].items()}
    # a step whose weights fit in the host's last-level cache is replicated
    # (distinct copies, >= 600 MB in rotation, as on the GPU side)
    one = sum(a.nbytes for lw in host for a in lw.values()) + wout.nbytes
    rot = [(host, wout)] + [([{k: a.copy() for k, a in lw.items()} for lw in host], wout.copy())
                            for _ in range(max(1, -(-int(MIN_ROTATION_BYTES) // one)) - 1)]
    # the calls with their arguments bound once (no per-call wrapping in the
    # timed loop); outputs reused
    ys = {name: np.zeros((m, n_out), np.float32) for name, _, n_out, _, _ in projs}
    scores = np.zeros(cfg["vocab"], np.float32)
    f32p, u8p = C.POINTER(C.c_float), C.POINTER(C.c_uint8)
    calls = []
    for c_host, c_wout in rot:
        cl = [(lin._lin, (ys[name].ctypes.data_as(f32p), x[src].ctypes.data_as(f32p), lw[name].ctypes.data_as(u8p), t,
                          None, m, n_out, n_in)) for lw in c_host for name, t, n_out, n_in, src in projs]
        cl += [(lin._logits, (scores.ctypes.data_as(f32p), x["h"][tok].ctypes.data_as(f32p),
                              c_wout.ctypes.data_as(u8p), cfg["logits_type"], None, cfg["vocab"], cfg["hidden"],
                              cfg["logits_chunk"])) for tok in range(m)]
        calls.append(cl)
    turn = [0]

    def step():
        cl = calls[turn[0] % len(calls)]
        turn[0] += 1
        for fn, a in cl:
            fn(*a)

    gomp = None
    try:
        gomp = C.CDLL("libgomp.so.1")
    except OSError:
        pass

    def run(budget):
        step()
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < budget or reps < 2:
            step()
            reps += 1
        return (time.perf_counter() - t0) / reps, reps

    budget = max(0.5, args.cpu_seconds / 4)
    # (b) the reference's own choice: its probe runs at the first call while
    # OMP_NUM_THREADS is unset (once per process; later workloads reuse it)
    auto = None
    if ref is not None and gomp is not None:
        if "threads" not in _PROBE:
            saved = os.environ.pop("OMP_NUM_THREADS", None)
            os.environ["EDGEXPU_DEBUG_THREADS"] = "1"
            gomp.omp_set_num_threads(share)
            try:
                _, text = _capture_fd2(lambda: ref.linear_quant_batch(x["h"], host[0][projs[0][0]], projs[0][1], None,
                                                                      m, projs[0][2], projs[0][3]))
            finally:
                os.environ.pop("EDGEXPU_DEBUG_THREADS", None)
                if saved is not None:
                    os.environ["OMP_NUM_THREADS"] = saved
            sel = [ln for ln in text.splitlines() if "selected" in ln]
            _PROBE["threads"] = int(sel[-1].split()[-1]) if sel else None
            _PROBE["log"] = [ln.strip() for ln in text.splitlines() if "thread probe" in ln]
        if _PROBE.get("threads"):
            gomp.omp_set_num_threads(_PROBE["threads"])
            dt, reps = run(budget)
            auto = {"value": round(model["step_bytes"] / dt / 1e9, 2), "unit": "GB/s",
                    "ms_per_step": round(dt * 1e3, 3), "threads": _PROBE["threads"], "steps_timed": reps,
                    "probe": _PROBE.get("log")}
    if gomp is not None:
        gomp.omp_set_num_threads(share)
    dt, reps = run(budget)
    res = {"value": round(model["step_bytes"] / dt / 1e9, 2), "unit": "GB/s", "cores": share, "kind": kind,
           "ms_per_step": round(dt * 1e3, 3),
           "sample": f"the whole {model['workload']} step m={m} ({len(host)} layers x "
                     f"{len(projs)} projections through "
                     f"{'the reference build' if kind == 'reference' else 'the oracle'}'s "
                     f"edgexpu_cpu_linear_quant_batch + [{cfg['vocab']} x {cfg['hidden']}] logits through "
                     f"src/native.c's chunked greedy loop on "
                     f"{'that build' if kind == 'reference' else 'the oracle'}'s row dots), {reps} steps over "
                     f"{len(rot)} distinct host cop"
                     f"{'y' if len(rot) == 1 else 'ies'} of {one >> 20} MiB",
           "omp": {"OMP_NUM_THREADS": share, "OMP_PROC_BIND": os.environ.get("OMP_PROC_BIND"),
                   "OMP_PLACES": os.environ.get("OMP_PLACES")},
           "cpu": lscpu_info(), "auto_probe": auto}
    del host, wout, rot, calls
    return res


def E_name(t):
    return {1: "f16", 2: "q4_0", 6: "q5_0", 8: "q8_0", 12: "q4_k", 13: "q5_k", 14: "q6_k"}[t]


if __name__ == "__main__":
    main()
