"""Seeded synthetic GGUF blocks and activations for the quantized-weight path.

Distributions (the workloads' definitions):
  Q8_0  d = fp16(|N(0, 0.02)| / 127), q ~ U{-127..127}
  Q4_K  d, dmin = fp16(|N(0, 0.01)|); 12 scale bytes uniform (6-bit sc/m in
        [0, 63]); 128 qs bytes uniform (4-bit codes 0..15)
  Q6_K  d = fp16(|N(0, 0.01)|) (sigma chosen here; not given by the workload);
        ql/qh bytes uniform; 16 int8 sub-scales uniform in [-128, 127]
  Q4_0, Q5_0  d = fp16(|N(0, 0.02)| / 16); qs (and Q5_0's qh) bytes uniform
  Q5_K  as Q4_K, with the 32 qh bytes uniform
  F16   N(0, 0.02) rounded to fp16
  F32   N(0, 0.02)
  activations f32 N(0, 1)

``np_*`` functions build host arrays with numpy's PCG64 (tests); ``torch_*``
build device tensors on the GPU with torch's generator (benchmarks, where the
weights are gigabytes).  Scales come from distributions, never raw random
bits, so no block holds NaN/Inf scales.
"""
from __future__ import annotations

import numpy as np

F32, F16, Q4_0, Q5_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 6, 8, 12, 13, 14


def _f16_bytes(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a.astype(np.float16)).view(np.uint8)


def np_weights(qtype: int, rows: int, n: int, rng: np.random.Generator) -> np.ndarray:
    """[rows, row_bytes] uint8 GGUF rows."""
    if qtype == Q8_0:
        nb = n // 32
        d = _f16_bytes(np.abs(rng.normal(0.0, 0.02, (rows, nb))) / 127.0).reshape(rows, nb, 2)
        q = rng.integers(-127, 128, (rows, nb, 32), dtype=np.int16).astype(np.int8).view(np.uint8)
        return np.concatenate([d, q], axis=2).reshape(rows, nb * 34)
    if qtype == Q4_K:
        nb = n // 256
        dd = _f16_bytes(np.abs(rng.normal(0.0, 0.01, (rows, nb, 2)))).reshape(rows, nb, 4)
        rest = rng.integers(0, 256, (rows, nb, 140), dtype=np.int16).astype(np.uint8)
        return np.concatenate([dd, rest], axis=2).reshape(rows, nb * 144)
    if qtype == Q5_K:
        nb = n // 256
        dd = _f16_bytes(np.abs(rng.normal(0.0, 0.01, (rows, nb, 2)))).reshape(rows, nb, 4)
        rest = rng.integers(0, 256, (rows, nb, 172), dtype=np.int16).astype(np.uint8)
        return np.concatenate([dd, rest], axis=2).reshape(rows, nb * 176)
    if qtype in (Q4_0, Q5_0):
        nb = n // 32
        nq = 16 if qtype == Q4_0 else 20
        d = _f16_bytes(np.abs(rng.normal(0.0, 0.02, (rows, nb))) / 16.0).reshape(rows, nb, 2)
        q = rng.integers(0, 256, (rows, nb, nq), dtype=np.int16).astype(np.uint8)
        return np.concatenate([d, q], axis=2).reshape(rows, nb * (2 + nq))
    if qtype == F16:
        return _f16_bytes(rng.normal(0.0, 0.02, (rows, n))).reshape(rows, 2 * n)
    if qtype == F32:
        return np.ascontiguousarray(rng.normal(0.0, 0.02, (rows, n)).astype(np.float32)).view(np.uint8)
    if qtype == Q6_K:
        nb = n // 256
        qlh = rng.integers(0, 256, (rows, nb, 192), dtype=np.int16).astype(np.uint8)
        sc = rng.integers(-128, 128, (rows, nb, 16), dtype=np.int16).astype(np.int8).view(np.uint8)
        d = _f16_bytes(np.abs(rng.normal(0.0, 0.01, (rows, nb)))).reshape(rows, nb, 2)
        return np.concatenate([qlh, sc, d], axis=2).reshape(rows, nb * 210)
    raise ValueError(qtype)


def np_activations(m: int, n: int, rng: np.random.Generator) -> np.ndarray:
    return rng.normal(0.0, 1.0, (m, n)).astype(np.float32)


def torch_weights(qtype: int, rows: int, n: int, generator, device="cuda"):
    """[rows, row_bytes] uint8 device tensor, generated on the GPU."""
    import torch

    def f16b(t):
        return t.to(torch.float16).view(torch.uint8)

    if qtype == Q8_0:
        nb = n // 32
        d = f16b(torch.randn((rows, nb, 1), generator=generator, device=device).abs_() * (0.02 / 127.0))
        q = torch.randint(-127, 128, (rows, nb, 32), generator=generator, device=device, dtype=torch.int8)
        return torch.cat([d.view(rows, nb, 2), q.view(torch.uint8)], dim=2).reshape(rows, nb * 34)
    if qtype == Q4_K:
        nb = n // 256
        dd = f16b(torch.randn((rows, nb, 2), generator=generator, device=device).abs_() * 0.01)
        rest = torch.randint(0, 256, (rows, nb, 140), generator=generator, device=device, dtype=torch.uint8)
        return torch.cat([dd.view(rows, nb, 4), rest], dim=2).reshape(rows, nb * 144)
    if qtype == Q5_K:
        nb = n // 256
        dd = f16b(torch.randn((rows, nb, 2), generator=generator, device=device).abs_() * 0.01)
        rest = torch.randint(0, 256, (rows, nb, 172), generator=generator, device=device, dtype=torch.uint8)
        return torch.cat([dd.view(rows, nb, 4), rest], dim=2).reshape(rows, nb * 176)
    if qtype in (Q4_0, Q5_0):
        nb = n // 32
        nq = 16 if qtype == Q4_0 else 20
        d = f16b(torch.randn((rows, nb, 1), generator=generator, device=device).abs_() * (0.02 / 16.0))
        q = torch.randint(0, 256, (rows, nb, nq), generator=generator, device=device, dtype=torch.uint8)
        return torch.cat([d.view(rows, nb, 2), q], dim=2).reshape(rows, nb * (2 + nq))
    if qtype == F16:
        return f16b(torch.randn((rows, n), generator=generator, device=device) * 0.02).reshape(rows, 2 * n)
    if qtype == F32:
        return (torch.randn((rows, n), generator=generator, device=device) * 0.02).view(torch.uint8)
    if qtype == Q6_K:
        nb = n // 256
        qlh = torch.randint(0, 256, (rows, nb, 192), generator=generator, device=device, dtype=torch.uint8)
        sc = torch.randint(-128, 128, (rows, nb, 16), generator=generator, device=device, dtype=torch.int8)
        d = f16b(torch.randn((rows, nb, 1), generator=generator, device=device).abs_() * 0.01)
        return torch.cat([qlh, sc.view(torch.uint8), d.view(rows, nb, 2)], dim=2).reshape(rows, nb * 210)
    raise ValueError(qtype)


def torch_weights_bulk(qtype: int, rows: int, n: int, generator, device="cuda", rows_per_piece: int = 16384):
    """Like torch_weights, built piecewise to bound the temporary memory."""
    import torch

    from . import row_bytes

    out = torch.empty((rows, row_bytes(qtype, n)), dtype=torch.uint8, device=device)
    for r0 in range(0, rows, rows_per_piece):
        r1 = min(rows, r0 + rows_per_piece)
        out[r0:r1] = torch_weights(qtype, r1 - r0, n, generator, device)
    return out
