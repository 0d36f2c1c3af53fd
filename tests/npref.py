"""Independent numpy restatement of the quantized-weight path (test helper).

Written from the block formats and formulas, not from the C oracle, so that the
two pin each other: dequant and quantizers are bit-exact closed forms in
float32 (numpy never fuses a multiply-add), the integer block sums are int64
brute force, and the fp32 row results get a float64 value plus the
conditioning scale S = sum |w_k x_k| of the tolerance rule |y - y^| <= tol * S.
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def f16(b: np.ndarray) -> np.ndarray:
    """little-endian fp16 bytes [..., 2] -> float32 (exact)."""
    return np.ascontiguousarray(b).view(np.float16).astype(np.float32)[..., 0]


# ------------------------------------------------------------ unpack codes


def q8_0_parts(blocks: np.ndarray):
    """[nb, 34] -> d [nb] f32, q [nb, 32] int."""
    b = blocks.reshape(-1, 34)
    return f16(b[:, 0:2]), b[:, 2:].view(np.int8).astype(np.int64)


def q4_k_parts(sb: np.ndarray):
    """[nb, 144] -> d, dmin [nb]; sc, m [nb, 8]; codes [nb, 256] (element order)."""
    s = sb.reshape(-1, 144)
    d, dmin = f16(s[:, 0:2]), f16(s[:, 2:4])
    sc12 = s[:, 4:16].astype(np.int64)
    sc = np.zeros((s.shape[0], 8), np.int64)
    m = np.zeros((s.shape[0], 8), np.int64)
    sc[:, :4] = sc12[:, 0:4] & 63
    m[:, :4] = sc12[:, 4:8] & 63
    sc[:, 4:] = (sc12[:, 8:12] & 15) | ((sc12[:, 0:4] >> 6) << 4)
    m[:, 4:] = (sc12[:, 8:12] >> 4) | ((sc12[:, 4:8] >> 6) << 4)
    qs = s[:, 16:].reshape(-1, 4, 32).astype(np.int64)       # [nb, chunk j, l]
    codes = np.stack([qs & 15, qs >> 4], axis=2)              # [nb, j, half, l]
    return d, dmin, sc, m, codes.reshape(-1, 256)


def q6_k_parts(sb: np.ndarray):
    """[nb, 210] -> d [nb]; sc [nb, 16] (int8); codes [nb, 256] unsigned 0..63."""
    s = sb.reshape(-1, 210)
    ql = s[:, 0:128].reshape(-1, 2, 2, 32).astype(np.int64)   # [nb, half, ql-half, l]
    qh = s[:, 128:192].reshape(-1, 2, 32).astype(np.int64)    # [nb, half, l]
    sc = s[:, 192:208].view(np.int8).astype(np.int64)
    d = f16(s[:, 208:210])
    codes = np.empty((s.shape[0], 2, 4, 32), np.int64)        # [nb, half, quarter k, l]
    for k in range(4):
        lo = ql[:, :, k & 1, :]
        lo = (lo >> 4) if k >= 2 else (lo & 15)
        codes[:, :, k, :] = lo | (((qh >> (2 * k)) & 3) << 4)
    return d, sc, codes.reshape(-1, 256)


def q4_0_parts(blocks: np.ndarray):
    """[nb, 18] -> d [nb]; signed values c - 8 [nb, 32] (low nibbles first)."""
    b = blocks.reshape(-1, 18)
    qs = b[:, 2:].astype(np.int64)
    return f16(b[:, 0:2]), np.concatenate([qs & 15, qs >> 4], axis=1) - 8


def q5_0_parts(blocks: np.ndarray):
    """[nb, 22] -> d [nb]; signed values c - 16 [nb, 32]; bit e of qh is the
    fifth bit of element e."""
    b = blocks.reshape(-1, 22)
    qh = b[:, 2:6].copy().view(np.uint32).astype(np.int64)       # [nb, 1]
    qs = b[:, 6:].astype(np.int64)
    nib = np.concatenate([qs & 15, qs >> 4], axis=1)
    hb = (qh >> np.arange(32)[None, :]) & 1
    return f16(b[:, 0:2]), (nib | (hb << 4)) - 16


def q5_k_parts(sb: np.ndarray):
    """[nb, 176] -> d, dmin; sc, m [nb, 8]; codes [nb, 256] (0..31).  Chunk j
    takes bit 2j (first 32 elements) and 2j+1 (next 32) of qh[l]."""
    s = sb.reshape(-1, 176)
    as_q4 = np.concatenate([s[:, 0:16], s[:, 48:176]], axis=1)   # same header + qs layout as Q4_K
    d, dmin, sc, m, codes = q4_k_parts(as_q4)
    qh = s[:, 16:48].astype(np.int64)                              # [nb, l]
    hb = np.stack([(qh >> (2 * j + h)) & 1 for j in range(4) for h in range(2)], axis=1)   # [nb, 8, l]
    return d, dmin, sc, m, codes + 16 * hb.reshape(-1, 256)


# ------------------------------------------------------------ dequant


def dequant(qtype: int, src: np.ndarray) -> np.ndarray:
    if qtype == 8:
        d, q = q8_0_parts(src)
        return (d[:, None] * q.astype(f32)).astype(f32).reshape(-1)
    if qtype == 12:
        d, dmin, sc, m, codes = q4_k_parts(src)
        ds = (d[:, None] * sc.astype(f32)).astype(f32)        # [nb, 8]
        ms = (dmin[:, None] * m.astype(f32)).astype(f32)
        sub = np.repeat(np.arange(8), 32)
        prod = (ds[:, sub] * codes.astype(f32)).astype(f32)
        return (prod - ms[:, sub]).astype(f32).reshape(-1)
    if qtype == 14:
        d, sc, codes = q6_k_parts(src)
        ds = (d[:, None] * sc.astype(f32)).astype(f32)        # [nb, 16]
        sub = np.repeat(np.arange(16), 16)
        return (ds[:, sub] * (codes - 32).astype(f32)).astype(f32).reshape(-1)
    if qtype == 2:   # ((float)c - 8) * d
        d, v = q4_0_parts(src)
        return (v.astype(f32) * d[:, None]).astype(f32).reshape(-1)
    if qtype == 6:   # (float)(c - 16) * d
        d, v = q5_0_parts(src)
        return (v.astype(f32) * d[:, None]).astype(f32).reshape(-1)
    if qtype == 13:  # (d*sc) * c - (dmin*m)
        d, dmin, sc, m, codes = q5_k_parts(src)
        ds = (d[:, None] * sc.astype(f32)).astype(f32)
        ms = (dmin[:, None] * m.astype(f32)).astype(f32)
        sub = np.repeat(np.arange(8), 32)
        prod = (ds[:, sub] * codes.astype(f32)).astype(f32)
        return (prod - ms[:, sub]).astype(f32).reshape(-1)
    if qtype == 1:
        return np.ascontiguousarray(src).view(np.float16).astype(f32).reshape(-1)
    if qtype == 0:
        return np.ascontiguousarray(src).view(f32).reshape(-1)
    raise ValueError(qtype)


# ------------------------------------------------------------ quantizers


def _cvt_avx(r: np.ndarray) -> np.ndarray:
    """rounded float -> int32 as _mm256_cvtps_epi32: NaN / out of range -> INT32_MIN."""
    ok = np.isfinite(r) & (r >= -2147483648.0) & (r < 2147483648.0)
    out = np.full(r.shape, -2147483648, np.int64)
    out[ok] = r[ok].astype(np.int64)
    return out


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    xb = x.astype(f32).reshape(-1, 32)
    with np.errstate(all="ignore"):
        amax = np.abs(xb).max(axis=1)
        d = (amax / f32(127.0)).astype(f32)
        idv = np.where(amax != 0, f32(127.0) / np.where(amax != 0, amax, f32(1)), f32(0)).astype(f32)
        q = _cvt_avx(np.rint((xb * idv[:, None]).astype(f32)))
    q = np.clip(q, -128, 127).astype(np.int8)
    with np.errstate(over="ignore"):
        dh = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return np.concatenate([dh, q.view(np.uint8)], axis=1).reshape(-1)


def quantize_q8_k(x: np.ndarray) -> np.ndarray:
    xb = x.astype(f32).reshape(-1, 256)
    out = np.zeros((xb.shape[0], 292), np.uint8)
    for b in range(xb.shape[0]):
        a = np.abs(xb[b])
        i = int(np.argmax(a))                 # first index of the largest |x|
        if a[i] == 0:
            continue
        with np.errstate(all="ignore"):
            iscale = f32(f32(-127.0) / xb[b, i])
            p = (iscale * xb[b]).astype(f32)
            q = np.where(np.isfinite(p), np.rint(p), 0).astype(np.int64)   # lrintf: non-finite -> 0
            d = f32(f32(1.0) / iscale)
        q = np.clip(q, -127, 127)
        out[b, 0:4] = np.array([d], f32).view(np.uint8)
        out[b, 4:260] = q.astype(np.int8).view(np.uint8)
        out[b, 260:292] = q.reshape(16, 16).sum(axis=1).astype(np.int16).view(np.uint8)
    return out.reshape(-1)


# ------------------------------------------------------------ integer block sums


def q8_0_lanes(wblk, xblk):
    _, qw = q8_0_parts(wblk)
    _, qx = q8_0_parts(xblk)
    return (qw[0] * qx[0]).reshape(8, 4).sum(axis=1)


def q4_k_lanes(wsb, xsb):
    _, _, sc, m, codes = q4_k_parts(wsb)
    q8 = xsb[4:260].view(np.int8).astype(np.int64)
    bs = xsb[260:292].view(np.int16).astype(np.int64)
    e = np.arange(256)
    lanes = np.array([np.sum((sc[0][e // 32] * codes[0] * q8)[((e % 32) // 4) == u]) for u in range(8)])
    s32 = bs.reshape(8, 2).sum(axis=1)
    mins = (m[0] * s32).reshape(4, 2).sum(axis=1)
    return lanes, mins


def q6_k_lanes(wsb, xsb):
    _, sc, codes = q6_k_parts(wsb)
    q8 = xsb[4:260].view(np.int8).astype(np.int64)
    bs = xsb[260:292].view(np.int16).astype(np.int64)
    e = np.arange(256)
    lanes = []
    for u in range(8):
        sel = ((e % 32) // 4) == u
        v = np.sum((sc[0][e // 16] * codes[0] * q8)[sel])
        v -= 32 * (bs[2 * u] * sc[0][2 * u] + bs[2 * u + 1] * sc[0][2 * u + 1])
        lanes.append(v)
    return np.array(lanes)


def q4_0_lanes(wblk, xblk):
    _, v = q4_0_parts(wblk)
    _, qx = q8_0_parts(xblk)
    return (v[0] * qx[0]).reshape(8, 4).sum(axis=1)


def q5_0_lanes(wblk, xblk):
    _, v = q5_0_parts(wblk)
    _, qx = q8_0_parts(xblk)
    return (v[0] * qx[0]).reshape(8, 4).sum(axis=1)


def q5_k_lanes(wsb, xsb):
    """(lanes[8], min total) of one Q5_K super-block against Q8_K."""
    _, _, sc, m, codes = q5_k_parts(wsb)
    q8 = xsb[4:260].view(np.int8).astype(np.int64)
    bs = xsb[260:292].view(np.int16).astype(np.int64)
    e = np.arange(256)
    lanes = np.array([np.sum((sc[0][e // 32] * codes[0] * q8)[((e % 32) // 4) == u]) for u in range(8)])
    return lanes, int((m[0] * bs.reshape(8, 2).sum(axis=1)).sum())


# ------------------------------------------------------------ f64 results + scale


def q8_dot_f64(qtype: int, wrow: np.ndarray, xq: np.ndarray):
    """Exact-integer, float64-combined row dot against quantized activations.

    Returns (value, S) with S the element-level conditioning scale
    sum_k |dx*dw*sc*q_k*q8_k| (+ sum_k |dx*dmin*m*q8_k| for Q4_K): any fp32
    summation order of the row, the reference's AVX2 lanes included, stays
    within a few ulp of S."""
    if qtype in (2, 6, 8):
        dw, qw = {2: q4_0_parts, 6: q5_0_parts, 8: q8_0_parts}[qtype](wrow)
        dx, qx = q8_0_parts(xq)
        isum = (qw * qx).sum(axis=1)
        scale = dw.astype(np.float64) * dx.astype(np.float64)
        return (scale * isum).sum(), (np.abs(scale)[:, None] * np.abs(qw * qx)).sum()
    xb = xq.reshape(-1, 292)
    dx = xb[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
    q8 = xb[:, 4:260].view(np.int8).astype(np.int64)
    bs = xb[:, 260:292].copy().view(np.int16).astype(np.int64)
    if qtype in (12, 13):
        d, dmin, sc, m, codes = (q4_k_parts if qtype == 12 else q5_k_parts)(wrow)
        sub = np.repeat(np.arange(8), 32)
        isum = (sc[:, sub] * codes * q8).sum(axis=1)
        imin = (m * bs.reshape(-1, 8, 2).sum(axis=2)).sum(axis=1)
        a = dx * d.astype(np.float64) * isum
        b = dx * dmin.astype(np.float64) * imin
        mag = (np.abs(dx * d.astype(np.float64))[:, None] * np.abs(sc[:, sub] * codes * q8)).sum() + \
            (np.abs(dx * dmin.astype(np.float64))[:, None] * np.abs(m[:, sub] * q8)).sum()
        return (a - b).sum(), mag
    if qtype == 14:
        d, sc, codes = q6_k_parts(wrow)
        sub = np.repeat(np.arange(16), 16)
        terms = sc[:, sub] * (codes - 32) * q8
        a = dx * d.astype(np.float64) * terms.sum(axis=1)
        return a.sum(), (np.abs(dx * d.astype(np.float64))[:, None] * np.abs(terms)).sum()
    raise ValueError(qtype)


def f32_dot_f64(qtype: int, wrow: np.ndarray, x: np.ndarray):
    """float64 row dot against f32 activations: (value, S = sum |w_k x_k|)."""
    w = dequant(qtype, wrow).astype(np.float64)
    p = w * x.astype(np.float64)
    return p.sum(), np.abs(p).sum()


def kq_q8k_gemm_f64(qtype: int, w: np.ndarray, xq: np.ndarray):
    """Many-token K-quant (Q4_K 12, Q5_K 13, Q6_K 14) x Q8_K product in
    float64 with exact integer block sums.

    w: [n_out, row_bytes] rows; xq: [m, nb*292] Q8_K rows.  Returns
    (value [m, n_out], S [m, n_out]) with S the element-level conditioning
    scale of q8_dot_f64, computed with matrix products (every partial sum is
    an integer below 2**53, so float64 products are exact)."""
    n_out = w.shape[0]
    m = xq.shape[0]
    bb = {12: 144, 13: 176, 14: 210}[qtype]
    nb = w.shape[1] // bb
    if qtype == 14:
        d, sc, codes = q6_k_parts(w.reshape(-1, bb))
        dmin = np.zeros_like(d)
        mn = np.zeros((d.shape[0], 8), np.int64)
        sub = np.repeat(np.arange(16), 16)
        sc = sc.reshape(n_out, nb, 16)
        codes = codes.astype(np.int64) - 32
    else:
        d, dmin, sc, mn, codes = (q4_k_parts if qtype == 12 else q5_k_parts)(w.reshape(-1, bb))
        sub = np.repeat(np.arange(8), 32)
        sc = sc.reshape(n_out, nb, 8)
    d = d.astype(np.float64).reshape(n_out, nb)
    dmin = dmin.astype(np.float64).reshape(n_out, nb)
    mn = mn.reshape(n_out, nb, 8)
    codes = codes.reshape(n_out, nb, 256)
    xb = xq.reshape(m, nb, 292)
    dx = xb[:, :, 0:4].copy().view(np.float32)[:, :, 0].astype(np.float64)
    q8 = xb[:, :, 4:260].copy().view(np.int8).astype(np.float64)
    msub = np.repeat(np.arange(8), 32)
    val = np.zeros((m, n_out))
    mag = np.zeros((m, n_out))
    for b in range(nb):
        ws = (sc[:, b, sub] * codes[:, b, :]).astype(np.float64)     # [n_out, 256]
        wm = mn[:, b, msub].astype(np.float64)                         # [n_out, 256]
        isum = q8[:, b, :] @ ws.T                                      # [m, n_out]
        imin = q8[:, b, :] @ wm.T
        aq = np.abs(q8[:, b, :])
        val += dx[:, b:b + 1] * (d[None, :, b] * isum - dmin[None, :, b] * imin)
        mag += np.abs(dx[:, b:b + 1]) * (np.abs(d[None, :, b]) * (aq @ np.abs(ws).T) +
                                         np.abs(dmin[None, :, b]) * (aq @ wm.T))
    return val, mag


def g32_q80_gemm_f64(qtype: int, w: np.ndarray, xq: np.ndarray):
    """Many-token Q8_0 (8) / Q4_0 (2) / Q5_0 (6) x Q8_0 product in float64
    with exact integer block sums: w [n_out, row_bytes], xq [m, nb*34].
    Returns (value [m, n_out], S [m, n_out]) like q8_rows_f64."""
    bb = {2: 18, 6: 22, 8: 34}[qtype]
    parts = {2: q4_0_parts, 6: q5_0_parts, 8: q8_0_parts}[qtype]
    n_out, m = w.shape[0], xq.shape[0]
    nb = w.shape[1] // bb
    dw, qw = parts(w.reshape(-1, bb))
    dw = dw.astype(np.float64).reshape(n_out, nb)
    qw = qw.reshape(n_out, nb, 32).astype(np.float64)
    dx, qx = q8_0_parts(xq.reshape(-1, 34))
    dx = dx.astype(np.float64).reshape(m, nb)
    qx = qx.reshape(m, nb, 32).astype(np.float64)
    val = np.zeros((m, n_out))
    mag = np.zeros((m, n_out))
    for b in range(nb):
        sc = dx[:, b:b + 1] * dw[None, :, b]
        val += sc * (qx[:, b, :] @ qw[:, b, :].T)
        mag += np.abs(sc) * (np.abs(qx[:, b, :]) @ np.abs(qw[:, b, :]).T)
    return val, mag


def q4k_q8k_gemm_f64(w: np.ndarray, xq: np.ndarray):
    """kq_q8k_gemm_f64 for Q4_K rows."""
    return kq_q8k_gemm_f64(12, w, xq)


def q8_rows_f64(qtype: int, w: np.ndarray, xq: np.ndarray, chunk: int = 2048):
    """q8_dot_f64 for every row of w against one token's quantized activation
    xq, vectorized over rows (chunks of `chunk` rows): (value [n_out],
    S [n_out]) with the same exact integers and conditioning scale."""
    n_out = w.shape[0]
    val = np.zeros(n_out)
    mag = np.zeros(n_out)
    if qtype in (2, 6, 8):
        bb = {2: 18, 6: 22, 8: 34}[qtype]
        parts = {2: q4_0_parts, 6: q5_0_parts, 8: q8_0_parts}[qtype]
        nb = w.shape[1] // bb
        dx, qx = q8_0_parts(xq)
        for r0 in range(0, n_out, chunk):
            r1 = min(n_out, r0 + chunk)
            dw, qw = parts(w[r0:r1].reshape(-1, bb))
            prod = qw.reshape(r1 - r0, nb, 32) * qx[None]
            scale = dw.astype(np.float64).reshape(r1 - r0, nb) * dx.astype(np.float64)[None]
            val[r0:r1] = (scale * prod.sum(axis=2)).sum(axis=1)
            mag[r0:r1] = (np.abs(scale) * np.abs(prod).sum(axis=2)).sum(axis=1)
        return val, mag
    xb = xq.reshape(-1, 292)
    nb = xb.shape[0]
    dx = xb[:, 0:4].copy().view(np.float32)[:, 0].astype(np.float64)
    q8 = xb[:, 4:260].view(np.int8).astype(np.int64)
    bs = xb[:, 260:292].copy().view(np.int16).astype(np.int64)
    for r0 in range(0, n_out, chunk):
        r1 = min(n_out, r0 + chunk)
        n = r1 - r0
        if qtype in (12, 13):
            bb = 144 if qtype == 12 else 176
            d, dmin, sc, m, codes = (q4_k_parts if qtype == 12 else q5_k_parts)(w[r0:r1].reshape(-1, bb))
            sub = np.repeat(np.arange(8), 32)
            t = (sc[:, sub] * codes).reshape(n, nb, 256) * q8[None]
            isum = t.sum(axis=2)
            mm = m.reshape(n, nb, 8)
            imin = (mm * bs.reshape(nb, 8, 2).sum(axis=2)[None]).sum(axis=2)
            dd = d.astype(np.float64).reshape(n, nb) * dx[None]
            dm = dmin.astype(np.float64).reshape(n, nb) * dx[None]
            val[r0:r1] = (dd * isum - dm * imin).sum(axis=1)
            tm = np.abs(mm[:, :, sub] * q8[None]).sum(axis=2)
            mag[r0:r1] = (np.abs(dd) * np.abs(t).sum(axis=2) + np.abs(dm) * tm).sum(axis=1)
        elif qtype == 14:
            d, sc, codes = q6_k_parts(w[r0:r1].reshape(-1, 210))
            sub = np.repeat(np.arange(16), 16)
            t = (sc[:, sub] * (codes - 32)).reshape(n, nb, 256) * q8[None]
            dd = d.astype(np.float64).reshape(n, nb) * dx[None]
            val[r0:r1] = (dd * t.sum(axis=2)).sum(axis=1)
            mag[r0:r1] = (np.abs(dd) * np.abs(t).sum(axis=2)).sum(axis=1)
        else:
            raise ValueError(qtype)
    return val, mag


def f32_rows_f64(qtype: int, w: np.ndarray, x: np.ndarray, chunk: int = 4096):
    """f32_dot_f64 for every row of w (chunks of `chunk` rows): (value, S)."""
    n_out, n = w.shape[0], x.size
    xv = x.astype(np.float64)
    val = np.zeros(n_out)
    mag = np.zeros(n_out)
    for r0 in range(0, n_out, chunk):
        r1 = min(n_out, r0 + chunk)
        wd = dequant(qtype, w[r0:r1]).reshape(r1 - r0, n).astype(np.float64)
        val[r0:r1] = wd @ xv
        mag[r0:r1] = np.abs(wd) @ np.abs(xv)
    return val, mag


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """src/cpu_kernel.c:220-242 in numpy: the squares summed in float64 in
    index order (np.add.accumulate is sequential), the mean rounded to
    float32, scale = 1 / sqrt(mean + eps) in float32 (correctly rounded
    sqrt and division), then x * scale and * w, each rounded to float32."""
    x = np.asarray(x, dtype=np.float32)
    x64 = x.astype(np.float64)
    ss = np.add.accumulate(x64 * x64)[-1]
    mean = np.float32(ss / np.float64(x.size))
    scale = np.float32(1.0) / np.sqrt(np.float32(mean + np.float32(eps)))
    return (x * scale) * np.asarray(w, dtype=np.float32)


# ------------------------------------------------------------ sampling


def draw(p, top_p, rng_after):
    """The draw written from its definition with numpy: the uniform u =
    (state & 0xFFFFFFF) / 2^28; with 0 < top_p < 1 the (p desc, id asc) order
    and its smallest prefix whose running double sum reaches top_p, else the
    index order; then the first position whose running sum reaches u * (sum
    of that prefix)."""
    u = float(rng_after & 0xFFFFFFF) / float(1 << 28)
    ids = np.arange(p.size)
    if 0.0 < np.float32(top_p) < 1.0:
        order = np.lexsort((ids, -p.astype(np.float64)))
        c = np.cumsum(p[order].astype(np.float64))
        hit = np.nonzero(c >= np.float64(np.float32(top_p)))[0]
        kept = int(hit[0]) + 1 if hit.size else p.size
        order = order[:kept]
    else:
        order = ids
    c = np.cumsum(p[order].astype(np.float64))
    if c[-1] <= 0.0:  # a NaN sum falls through: no position reaches it, the last is drawn
        return int(order[0])
    hit = np.nonzero(c >= u * c[-1])[0]
    return int(order[hit[0]]) if hit.size else int(order[-1])


def xorshift(s):
    s = s or 0x00ED6E50
    s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
    s ^= s >> 7
    s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
    return s
