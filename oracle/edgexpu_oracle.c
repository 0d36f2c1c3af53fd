/*
 * edgexpu_oracle.c -- TEST INFRASTRUCTURE ONLY (see edgexpu_oracle.h).
 *
 * Scalar C restatement of the reference quantized-weight path.  The AVX2
 * kernels of the reference are restated lane by lane: an "AVX lane" below is
 * one 32-bit element of a 256-bit register, and every fp32 operation is done
 * in the same order and with the same rounding (fmaf where the reference
 * issues _mm256_fmadd_ps, separate multiply/add where it does not).  Build
 * with -std=c11 -ffp-contract=off so the compiler adds no contraction.
 */
#include "edgexpu_oracle.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

#define QK32 32
#define QKK 256
#define B_Q8_0 34
#define B_Q4_0 18
#define B_Q5_0 22
#define B_Q4_K 144
#define B_Q5_K 176
#define B_Q6_K 210
#define B_Q8_K 292
#define LOGIT_CHUNK_BYTES ((size_t)48u * 1024u * 1024u) /* include/edgexpu/scheduler.h:34 */

/* ---------------------------------------------------------------- fp16 */

float ora_fp16_to_fp32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t bits;
    float v;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in fp32 */
        v = (float)m * 0x1p-24f;
        memcpy(&bits, &v, 4);
        bits |= sign;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13) | (m ? 0x00400000u : 0u);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&v, &bits, 4);
    return v;
}

uint16_t ora_fp32_to_fp16(float f) {
    uint32_t x;
    uint32_t sign;
    uint32_t a;
    memcpy(&x, &f, 4);
    sign = (x >> 16) & 0x8000u;
    a = x & 0x7fffffffu;
    if (a > 0x7f800000u) {
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    }
    if (a >= 0x477ff000u) { /* >= 65520 rounds to infinity */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (a >= 0x38800000u) { /* normal half: rebias, round mantissa 23 -> 10 bits RNE */
        uint32_t r = a - 0x38000000u;
        r += 0x0fffu + ((r >> 13) & 1u);
        return (uint16_t)(sign | (r >> 13));
    }
    if (a < 0x33000000u) { /* below 2^-25: rounds to zero */
        return (uint16_t)sign;
    }
    {
        /* subnormal half: value in units of 2^-24 is mant >> (126 - e) */
        uint32_t e = a >> 23;
        uint32_t mant = (a & 0x7fffffu) | 0x800000u;
        uint32_t sh = 126u - e;
        uint32_t q = mant >> sh;
        uint32_t rem = mant & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) {
            q++;
        }
        return (uint16_t)(sign | q);
    }
}

static float ld_f16(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return ora_fp16_to_fp32(h);
}

/* ------------------------------------------------------------- layouts */

size_t ora_block_size(uint32_t type) {
    switch (type) {
        case ORA_F32: case ORA_F16: return 1;
        case ORA_Q4_0: case ORA_Q5_0: case ORA_Q8_0: return QK32;
        case ORA_Q4_K: case ORA_Q5_K: case ORA_Q6_K: return QKK;
        default: return 0;
    }
}

size_t ora_block_bytes(uint32_t type) {
    switch (type) {
        case ORA_F32: return 4;
        case ORA_F16: return 2;
        case ORA_Q4_0: return 18;
        case ORA_Q5_0: return 22;
        case ORA_Q8_0: return B_Q8_0;
        case ORA_Q4_K: return B_Q4_K;
        case ORA_Q5_K: return 176;
        case ORA_Q6_K: return B_Q6_K;
        default: return 0;
    }
}

size_t ora_row_bytes(uint32_t type, int n) {
    size_t bs = ora_block_size(type);
    size_t bb = ora_block_bytes(type);
    if (n <= 0 || bs == 0 || bb == 0 || (size_t)n % bs != 0) {
        return 0;
    }
    return (size_t)n / bs * bb;
}

size_t ora_q8_0_nbytes(int n) {
    return (n <= 0 || n % QK32) ? 0 : (size_t)n / QK32 * B_Q8_0;
}

size_t ora_q8_k_nbytes(int n) {
    return (n <= 0 || n % QKK) ? 0 : (size_t)n / QKK * B_Q8_K;
}

/* Six-bit scale/min pair j of a K-quant super-block (src/gguf_quant.c:212-220). */
static void k4_scale_min(const uint8_t *s12, int j, int *sc, int *mn) {
    if (j < 4) {
        *sc = s12[j] & 63;
        *mn = s12[j + 4] & 63;
    } else {
        *sc = (s12[j + 4] & 0x0f) | ((s12[j - 4] >> 6) << 4);
        *mn = (s12[j + 4] >> 4) | ((s12[j] >> 6) << 4);
    }
}

/* Q6_K element e (0..255) of a super-block as the unsigned 6-bit code
 * (src/gguf_quant.c:283-300: half h = e/128, quarter k = (e%128)/32, l = e%32). */
static int q6_code(const uint8_t *sb, int e) {
    const uint8_t *ql = sb + 64 * (e / 128);
    const uint8_t *qh = sb + 128 + 32 * (e / 128);
    int k = (e % 128) / 32;
    int l = e % 32;
    int lo = (k & 1) ? ql[l + 32] : ql[l];
    lo = (k & 2) ? (lo >> 4) : (lo & 0x0f);
    return lo | (((qh[l] >> (2 * k)) & 3) << 4);
}

/* Q4_K element e (0..255): nibble code and the 64-chunk / half it lives in. */
static int q4_code(const uint8_t *sb, int e) {
    const uint8_t *qs = sb + 16 + 32 * (e / 64);
    int l = e % 32;
    return ((e % 64) < 32) ? (qs[l] & 0x0f) : (qs[l] >> 4);
}

/* Q4_0 element e (0..31) of an 18-byte block: nibble code 0..15, value
 * code - 8 (src/gguf_quant.c:193-210: low nibbles are elements 0..15). */
static int q4_0_code(const uint8_t *blk, int e) {
    return e < 16 ? (blk[2 + e] & 0x0f) : (blk[2 + e - 16] >> 4);
}

/* Q5_0 element e (0..31) of a 22-byte block: 5-bit code, value code - 16;
 * the fifth bit of element e is bit e of the 32-bit qh word
 * (src/gguf_quant.c:157-180). */
static int q5_0_code(const uint8_t *blk, int e) {
    uint32_t qh;
    int nib;
    memcpy(&qh, blk + 2, 4);
    nib = e < 16 ? (blk[6 + e] & 0x0f) : (blk[6 + e - 16] >> 4);
    return nib | (int)(((qh >> e) & 1u) << 4);
}

/* Q5_K element e (0..255) of a 176-byte super-block: 5-bit code.  Chunk
 * j = e/64 reads qs[32j + l] (low nibble for the first 32 elements, high for
 * the next 32) and bit 2j (resp. 2j+1) of qh[l], l = e%32
 * (src/gguf_quant.c:305-353). */
static int q5_k_code(const uint8_t *sb, int e) {
    int j = e / 64;
    int hi = (e % 64) >= 32;
    int l = e % 32;
    int q = sb[48 + 32 * j + l];
    int nib = hi ? (q >> 4) : (q & 0x0f);
    return nib + (((sb[16 + l] >> (2 * j + hi)) & 1) << 4);
}

/* ------------------------------------------------------------- dequant */

int ora_dequantize(const uint8_t *src, uint32_t type, uint64_t n, float *dst) {
    uint64_t b;
    size_t bs = ora_block_size(type);
    if (src == NULL || dst == NULL || n == 0 || bs == 0 || n % bs != 0) {
        return 0;
    }
    switch (type) {
        case ORA_F32:
            memcpy(dst, src, (size_t)n * 4);
            return 1;
        case ORA_Q8_0: /* src/gguf_quant.c:139-155: y = d * q, one rounding */
            for (b = 0; b < n / QK32; b++) {
                const uint8_t *blk = src + b * B_Q8_0;
                float d = ld_f16(blk);
                int j;
                for (j = 0; j < QK32; j++) {
                    dst[b * QK32 + j] = d * (float)(int8_t)blk[2 + j];
                }
            }
            return 1;
        case ORA_F16: /* src/gguf_quant.c:183-191 */
            for (b = 0; b < n; b++) {
                dst[b] = ld_f16(src + 2 * b);
            }
            return 1;
        case ORA_Q4_0: /* src/gguf_quant.c:193-210: y = ((float)c - 8) * d */
            for (b = 0; b < n / QK32; b++) {
                const uint8_t *blk = src + b * B_Q4_0;
                float d = ld_f16(blk);
                int e;
                for (e = 0; e < QK32; e++) {
                    dst[b * QK32 + (uint64_t)e] = ((float)q4_0_code(blk, e) - 8.0f) * d;
                }
            }
            return 1;
        case ORA_Q5_0: /* src/gguf_quant.c:157-180: y = (float)(c - 16) * d */
            for (b = 0; b < n / QK32; b++) {
                const uint8_t *blk = src + b * B_Q5_0;
                float d = ld_f16(blk);
                int e;
                for (e = 0; e < QK32; e++) {
                    dst[b * QK32 + (uint64_t)e] = (float)(q5_0_code(blk, e) - 16) * d;
                }
            }
            return 1;
        case ORA_Q5_K: /* src/gguf_quant.c:305-353: y = (d*sc)*c - (dmin*m) */
            for (b = 0; b < n / QKK; b++) {
                const uint8_t *sb = src + b * B_Q5_K;
                float d = ld_f16(sb);
                float dmin = ld_f16(sb + 2);
                int e;
                for (e = 0; e < QKK; e++) {
                    int sc;
                    int mn;
                    float ds;
                    float ms;
                    k4_scale_min(sb + 4, e / 32, &sc, &mn);
                    ds = d * (float)sc;
                    ms = dmin * (float)mn;
                    dst[b * QKK + (uint64_t)e] = ds * (float)q5_k_code(sb, e) - ms;
                }
            }
            return 1;
        case ORA_Q4_K: /* src/gguf_quant.c:223-266: y = (d*sc)*q - (dmin*m) */
            for (b = 0; b < n / QKK; b++) {
                const uint8_t *sb = src + b * B_Q4_K;
                float d = ld_f16(sb);
                float dmin = ld_f16(sb + 2);
                int e;
                for (e = 0; e < QKK; e++) {
                    int sc;
                    int mn;
                    float ds;
                    float ms;
                    k4_scale_min(sb + 4, e / 32, &sc, &mn);
                    ds = d * (float)sc;
                    ms = dmin * (float)mn;
                    dst[b * QKK + (uint64_t)e] = ds * (float)q4_code(sb, e) - ms;
                }
            }
            return 1;
        case ORA_Q6_K: /* src/gguf_quant.c:269-302: y = (d*sc)*(q-32) */
            for (b = 0; b < n / QKK; b++) {
                const uint8_t *sb = src + b * B_Q6_K;
                float d = ld_f16(sb + 208);
                int e;
                for (e = 0; e < QKK; e++) {
                    float s = d * (float)(int8_t)sb[192 + e / 16];
                    dst[b * QKK + (uint64_t)e] = s * (float)(q6_code(sb, e) - 32);
                }
            }
            return 1;
        default:
            return 0;
    }
}

/* ----------------------------------------------------------- quantizers */

/* _mm256_cvtps_epi32 on an already-rounded value: NaN and out-of-range
 * inputs give the integer-indefinite 0x80000000. */
static int32_t cvt_avx_i32(float r) {
    if (!(r >= -2147483648.0f && r < 2147483648.0f)) {
        return INT32_MIN;
    }
    return (int32_t)r;
}

int ora_quantize_q8_0(const float *x, int n, uint8_t *dst) {
    int b;
    if (x == NULL || dst == NULL || n <= 0 || n % QK32 != 0) {
        return 0;
    }
    for (b = 0; b < n / QK32; b++) {
        const float *xb = x + (size_t)b * QK32;
        uint8_t *blk = dst + (size_t)b * B_Q8_0;
        float amax = 0.0f;
        float d;
        float id;
        uint16_t dh;
        int e;
        for (e = 0; e < QK32; e++) {
            float a = fabsf(xb[e]);
            amax = a > amax ? a : amax;
        }
        d = amax / 127.0f;
        id = amax != 0.0f ? 127.0f / amax : 0.0f;
        dh = ora_fp32_to_fp16(d);
        memcpy(blk, &dh, 2);
        for (e = 0; e < QK32; e++) {
            int32_t q = cvt_avx_i32(rintf(xb[e] * id));
            /* packs_epi32 then packs_epi16: signed saturation to int8 */
            q = q < -128 ? -128 : (q > 127 ? 127 : q);
            blk[2 + e] = (uint8_t)(int8_t)q;
        }
    }
    return 1;
}

int ora_quantize_q8_k(const float *x, int n, uint8_t *dst) {
    int b;
    if (x == NULL || dst == NULL || n <= 0 || n % QKK != 0) {
        return 0;
    }
    for (b = 0; b < n / QKK; b++) {
        const float *xb = x + (size_t)b * QKK;
        uint8_t *blk = dst + (size_t)b * B_Q8_K;
        int8_t *qs = (int8_t *)(blk + 4);
        int16_t bsums[16];
        float amax = 0.0f;
        float maxv = 0.0f;
        float iscale;
        float d;
        int e;
        for (e = 0; e < QKK; e++) { /* strict '>' keeps the first index on ties */
            float a = fabsf(xb[e]);
            if (a > amax) {
                amax = a;
                maxv = xb[e];
            }
        }
        if (amax == 0.0f) {
            memset(blk, 0, B_Q8_K);
            continue;
        }
        iscale = -127.0f / maxv;
        for (e = 0; e < QKK; e++) {
            int v = (int)lrintf(iscale * xb[e]);
            v = v > 127 ? 127 : (v < -127 ? -127 : v);
            qs[e] = (int8_t)v;
        }
        for (e = 0; e < 16; e++) {
            int s = 0;
            int i;
            for (i = 0; i < 16; i++) {
                s += qs[e * 16 + i];
            }
            bsums[e] = (int16_t)s;
        }
        d = 1.0f / iscale;
        memcpy(blk, &d, 4);
        memcpy(blk + 4 + QKK, bsums, sizeof(bsums));
    }
    return 1;
}

/* ------------------------------------------------ integer block lanes */

void ora_q8_0_block_lanes(const uint8_t *wblk, const uint8_t *xblk, int32_t lanes[8]) {
    int u;
    for (u = 0; u < 8; u++) {
        int32_t s = 0;
        int e;
        for (e = 4 * u; e < 4 * u + 4; e++) {
            s += (int32_t)(int8_t)wblk[2 + e] * (int32_t)(int8_t)xblk[2 + e];
        }
        lanes[u] = s;
    }
}

void ora_q4_k_block_lanes(const uint8_t *wsb, const uint8_t *xsb, int32_t lanes[8], int32_t mins[4]) {
    const int8_t *q8 = (const int8_t *)(xsb + 4);
    int16_t bs[16];
    int sc[8];
    int mn[8];
    int u;
    int k;
    memcpy(bs, xsb + 4 + QKK, sizeof(bs));
    for (k = 0; k < 8; k++) {
        k4_scale_min(wsb + 4, k, &sc[k], &mn[k]);
    }
    for (u = 0; u < 8; u++) {
        int32_t s = 0;
        int sub;
        for (sub = 0; sub < 8; sub++) { /* sub-block of 32: chunk sub/2, half sub%2 */
            int32_t p = 0;
            int e;
            for (e = 4 * u; e < 4 * u + 4; e++) {
                int idx = 32 * sub + e;
                p += q4_code(wsb, idx) * (int32_t)q8[idx];
            }
            s += sc[sub] * p;
        }
        lanes[u] = s;
    }
    for (k = 0; k < 4; k++) {
        int32_t s0 = (int32_t)bs[4 * k] + bs[4 * k + 1];
        int32_t s1 = (int32_t)bs[4 * k + 2] + bs[4 * k + 3];
        mins[k] = mn[2 * k] * s0 + mn[2 * k + 1] * s1;
    }
}

void ora_q6_k_block_lanes(const uint8_t *wsb, const uint8_t *xsb, int32_t lanes[8]) {
    const int8_t *q8 = (const int8_t *)(xsb + 4);
    const int8_t *sc = (const int8_t *)(wsb + 192);
    int16_t bs[16];
    int u;
    memcpy(bs, xsb + 4 + QKK, sizeof(bs));
    for (u = 0; u < 8; u++) {
        int32_t s = 0;
        int c;
        for (c = 0; c < 8; c++) { /* 32-element chunk c of the super-block */
            int32_t p = 0;
            int e;
            for (e = 4 * u; e < 4 * u + 4; e++) {
                int idx = 32 * c + e;
                p += q6_code(wsb, idx) * (int32_t)q8[idx];
            }
            s += (int32_t)sc[2 * c + (u >= 4)] * p;
        }
        s -= 32 * ((int32_t)bs[2 * u] * sc[2 * u] + (int32_t)bs[2 * u + 1] * sc[2 * u + 1]);
        lanes[u] = s;
    }
}

/* Q4_0 / Q5_0 x Q8_0: the same eight 4-element lanes as Q8_0, on the signed
 * values c - 8 (src/gguf_dot_q8.c:552-568) and c - 16 (:482-502). */
void ora_q4_0_block_lanes(const uint8_t *wblk, const uint8_t *xblk, int32_t lanes[8]) {
    int u;
    for (u = 0; u < 8; u++) {
        int32_t s = 0;
        int e;
        for (e = 4 * u; e < 4 * u + 4; e++) {
            s += (q4_0_code(wblk, e) - 8) * (int32_t)(int8_t)xblk[2 + e];
        }
        lanes[u] = s;
    }
}

void ora_q5_0_block_lanes(const uint8_t *wblk, const uint8_t *xblk, int32_t lanes[8]) {
    int u;
    for (u = 0; u < 8; u++) {
        int32_t s = 0;
        int e;
        for (e = 4 * u; e < 4 * u + 4; e++) {
            s += (q5_0_code(wblk, e) - 16) * (int32_t)(int8_t)xblk[2 + e];
        }
        lanes[u] = s;
    }
}

/* Q5_K x Q8_K (src/gguf_dot_q8.c:772-838, AVX2): lane u sums sc[sub] times the
 * 4-element products 4u..4u+3 of each 32-element sub-block, as Q4_K; the
 * min term is one integer, sum_k m[k] * (bsum[2k] + bsum[2k+1]). */
void ora_q5_k_block_lanes(const uint8_t *wsb, const uint8_t *xsb, int32_t lanes[8], int32_t *mins) {
    const int8_t *q8 = (const int8_t *)(xsb + 4);
    int16_t bs[16];
    int sc[8];
    int mn[8];
    int u;
    int k;
    int32_t total = 0;
    memcpy(bs, xsb + 4 + QKK, sizeof(bs));
    for (k = 0; k < 8; k++) {
        k4_scale_min(wsb + 4, k, &sc[k], &mn[k]);
    }
    for (u = 0; u < 8; u++) {
        int32_t s = 0;
        int sub;
        for (sub = 0; sub < 8; sub++) {
            int32_t p = 0;
            int e;
            for (e = 4 * u; e < 4 * u + 4; e++) {
                int idx = 32 * sub + e;
                p += q5_k_code(wsb, idx) * (int32_t)q8[idx];
            }
            s += sc[sub] * p;
        }
        lanes[u] = s;
    }
    for (k = 0; k < 8; k++) {
        total += mn[k] * ((int32_t)bs[2 * k] + bs[2 * k + 1]);
    }
    *mins = total;
}

/* hsum_float_8, src/gguf_dot_q8.c:129-135 */
static float hsum8_dotq8(const float v[8]) {
    float r0 = v[4] + v[0];
    float r1 = v[5] + v[1];
    float r2 = v[6] + v[2];
    float r3 = v[7] + v[3];
    return (r0 + r2) + (r1 + r3);
}

/* hsum256, src/gguf_quant.c:488-495 */
static float hsum8_quant(const float v[8]) {
    float s0 = v[0] + v[4];
    float s1 = v[1] + v[5];
    float s2 = v[2] + v[6];
    float s3 = v[3] + v[7];
    return (s0 + s1) + (s2 + s3);
}

/* ---------------------------------------------- dots vs quantized x */

static float dot_q8_0_q8_0(const uint8_t *w, const uint8_t *xq, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int b;
    for (b = 0; b < n / QK32; b++) {
        const uint8_t *wb = w + (size_t)b * B_Q8_0;
        const uint8_t *xb = xq + (size_t)b * B_Q8_0;
        float d = ld_f16(wb) * ld_f16(xb);
        int32_t l[8];
        int u;
        ora_q8_0_block_lanes(wb, xb, l);
        for (u = 0; u < 8; u++) {
            acc[u] = fmaf(d, (float)l[u], acc[u]);
        }
    }
    return hsum8_dotq8(acc);
}

static float dot_q4_k_q8_k(const uint8_t *w, const uint8_t *xq, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float accm[4] = {0, 0, 0, 0};
    int b;
    for (b = 0; b < n / QKK; b++) {
        const uint8_t *sb = w + (size_t)b * B_Q4_K;
        const uint8_t *yb = xq + (size_t)b * B_Q8_K;
        float dx;
        float d;
        float dmin;
        int32_t l[8];
        int32_t mn[4];
        int u;
        memcpy(&dx, yb, 4);
        d = dx * ld_f16(sb);
        dmin = -dx * ld_f16(sb + 2);
        ora_q4_k_block_lanes(sb, yb, l, mn);
        for (u = 0; u < 4; u++) {
            accm[u] = fmaf(dmin, (float)mn[u], accm[u]);
        }
        for (u = 0; u < 8; u++) {
            acc[u] = fmaf(d, (float)l[u], acc[u]);
        }
    }
    return hsum8_dotq8(acc) + ((accm[0] + accm[2]) + (accm[1] + accm[3]));
}

static float dot_q6_k_q8_k(const uint8_t *w, const uint8_t *xq, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int b;
    for (b = 0; b < n / QKK; b++) {
        const uint8_t *sb = w + (size_t)b * B_Q6_K;
        const uint8_t *yb = xq + (size_t)b * B_Q8_K;
        float dx;
        float d;
        int32_t l[8];
        int u;
        memcpy(&dx, yb, 4);
        d = dx * ld_f16(sb + 208);
        ora_q6_k_block_lanes(sb, yb, l);
        for (u = 0; u < 8; u++) {
            acc[u] = fmaf(d, (float)l[u], acc[u]);
        }
    }
    return hsum8_dotq8(acc);
}

/* Q4_0 / Q5_0 x Q8_0 (src/gguf_dot_q8.c:552-568, 482-502; AVX2): per block
 * d = fp16(w.d) * fp16(x.d), eight lane FMAs, hsum_float_8 at the end. */
static float dot_q4_0_q5_0_q8_0(uint32_t type, const uint8_t *w, const uint8_t *xq, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    size_t bb = type == ORA_Q4_0 ? B_Q4_0 : B_Q5_0;
    int b;
    for (b = 0; b < n / QK32; b++) {
        const uint8_t *wb = w + (size_t)b * bb;
        const uint8_t *xb = xq + (size_t)b * B_Q8_0;
        float d = ld_f16(wb) * ld_f16(xb);
        int32_t l[8];
        int u;
        if (type == ORA_Q4_0) {
            ora_q4_0_block_lanes(wb, xb, l);
        } else {
            ora_q5_0_block_lanes(wb, xb, l);
        }
        for (u = 0; u < 8; u++) {
            acc[u] = fmaf(d, (float)l[u], acc[u]);
        }
    }
    return hsum8_dotq8(acc);
}

float ora_dot_q8(uint32_t type, const uint8_t *wrow, const uint8_t *xq, int n) {
    if (wrow == NULL || xq == NULL || n <= 0 || n % QK32 != 0) {
        return 0.0f;
    }
    switch (type) {
        case ORA_Q8_0: return dot_q8_0_q8_0(wrow, xq, n);
        case ORA_Q4_0:
        case ORA_Q5_0: return dot_q4_0_q5_0_q8_0(type, wrow, xq, n);
        default: return 0.0f;
    }
}

/* Q5_K x Q8_K (src/gguf_dot_q8.c:772-838): lanes FMA'd with d = dx * w.d;
 * the min term accumulates in one float, summs += (-dx * w.dmin) * total,
 * multiply and add rounded separately; result hsum_float_8 + summs. */
static float dot_q5_k_q8_k(const uint8_t *w, const uint8_t *xq, int n) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float summs = 0.0f;
    int b;
    for (b = 0; b < n / QKK; b++) {
        const uint8_t *sb = w + (size_t)b * B_Q5_K;
        const uint8_t *yb = xq + (size_t)b * B_Q8_K;
        float dx;
        float d;
        float dmin;
        float prod;
        int32_t l[8];
        int32_t total;
        int u;
        memcpy(&dx, yb, 4);
        d = dx * ld_f16(sb);
        dmin = -dx * ld_f16(sb + 2);
        ora_q5_k_block_lanes(sb, yb, l, &total);
        prod = dmin * (float)total;
        summs = summs + prod;
        for (u = 0; u < 8; u++) {
            acc[u] = fmaf(d, (float)l[u], acc[u]);
        }
    }
    return hsum8_dotq8(acc) + summs;
}

float ora_dot_q8k(uint32_t type, const uint8_t *wrow, const uint8_t *xq, int n) {
    if (wrow == NULL || xq == NULL || n <= 0 || n % QKK != 0) {
        return 0.0f;
    }
    if (type == ORA_Q4_K) {
        return dot_q4_k_q8_k(wrow, xq, n);
    }
    if (type == ORA_Q6_K) {
        return dot_q6_k_q8_k(wrow, xq, n);
    }
    if (type == ORA_Q5_K) {
        return dot_q5_k_q8_k(wrow, xq, n);
    }
    return 0.0f;
}

/* -------------------------------------------------- dots vs f32 x */

/* dot_u4_f32_32, src/gguf_quant.c:539-565: 8 lanes, 4 FMA steps, hsum256. */
static void u4_f32_32(const uint8_t *q, const float *x, int hi, float *qx, float *sx) {
    float vq[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float vx[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    int i;
    for (i = 0; i < 32; i += 8) {
        int l;
        for (l = 0; l < 8; l++) {
            float c = (float)(hi ? (q[i + l] >> 4) : (q[i + l] & 0x0f));
            vq[l] = fmaf(c, x[i + l], vq[l]);
            vx[l] = vx[l] + x[i + l];
        }
    }
    *qx = hsum8_quant(vq);
    *sx = hsum8_quant(vx);
}

static float dot_q4_k_f32(const uint8_t *w, const float *x, int n) {
    float acc = 0.0f;
    int b;
    for (b = 0; b < n / QKK; b++) {
        const uint8_t *sb = w + (size_t)b * B_Q4_K;
        const float *xx = x + (size_t)b * QKK;
        float d = ld_f16(sb);
        float dmin = ld_f16(sb + 2);
        int j;
        for (j = 0; j < 4; j++) {
            int sc;
            int mn;
            float d1, m1, d2, m2, qx, sx;
            k4_scale_min(sb + 4, 2 * j, &sc, &mn);
            d1 = d * (float)sc;
            m1 = dmin * (float)mn;
            k4_scale_min(sb + 4, 2 * j + 1, &sc, &mn);
            d2 = d * (float)sc;
            m2 = dmin * (float)mn;
            u4_f32_32(sb + 16 + 32 * j, xx + 64 * j, 0, &qx, &sx);
            acc += d1 * qx - m1 * sx;
            u4_f32_32(sb + 16 + 32 * j, xx + 64 * j + 32, 1, &qx, &sx);
            acc += d2 * qx - m2 * sx;
        }
    }
    return acc;
}

static float dot_q6_k_f32(const uint8_t *w, const float *x, int n) {
    float acc = 0.0f;
    int b;
    for (b = 0; b < n / QKK; b++) {
        const uint8_t *sb = w + (size_t)b * B_Q6_K;
        const int8_t *sc = (const int8_t *)(sb + 192);
        const float *xx = x + (size_t)b * QKK;
        float d = ld_f16(sb + 208);
        int h;
        for (h = 0; h < 2; h++) { /* serial order of src/gguf_quant.c:774-791 */
            int l;
            for (l = 0; l < 32; l++) {
                int k;
                for (k = 0; k < 4; k++) {
                    int e = 128 * h + 32 * k + l;
                    float q = (float)(q6_code(sb, e) - 32);
                    acc += d * (float)sc[e / 16] * q * xx[e];
                }
            }
        }
    }
    return acc;
}

static float dot_q8_0_f32(const uint8_t *w, const float *x, int n) {
    float acc = 0.0f;
    int b;
    for (b = 0; b < n / QK32; b++) { /* src/gguf_quant.c:617-640 */
        const uint8_t *blk = w + (size_t)b * B_Q8_0;
        const float *xx = x + (size_t)b * QK32;
        float d = ld_f16(blk);
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int off;
        for (off = 0; off < QK32; off += 8) {
            int l;
            for (l = 0; l < 8; l++) {
                v[l] = fmaf((float)(int8_t)blk[2 + off + l], xx[off + l], v[l]);
            }
        }
        acc += d * hsum8_quant(v);
    }
    return acc;
}

/* dot_f16, src/gguf_quant.c:796-808: double products, serial double sum. */
static float dot_f16_f32(const uint8_t *w, const float *x, int n) {
    double acc = 0.0;
    int i;
    for (i = 0; i < n; i++) {
        acc += (double)ld_f16(w + 2 * (size_t)i) * (double)x[i];
    }
    return (float)acc;
}

/* dot_f32_row, src/gguf_quant.c:506-536: eight FMA lanes over the first
 * n - n%8 elements, hsum256, then the tail in double. */
static float dot_f32_f32(const float *w, const float *x, int n) {
    float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    double acc = 0.0;
    int i = 0;
    for (; i + 8 <= n; i += 8) {
        int l;
        for (l = 0; l < 8; l++) {
            v[l] = fmaf(w[i + l], x[i + l], v[l]);
        }
    }
    acc += (double)hsum8_quant(v);
    for (; i < n; i++) {
        acc += (double)w[i] * (double)x[i];
    }
    return (float)acc;
}

/* dot_q4_0, src/gguf_quant.c:810-835: serial, acc += (d*(c-8))*x per
 * element, low-nibble element before its high-nibble partner. */
static float dot_q4_0_f32(const uint8_t *w, const float *x, int n) {
    float acc = 0.0f;
    int b;
    for (b = 0; b < n / QK32; b++) {
        const uint8_t *blk = w + (size_t)b * B_Q4_0;
        const float *xx = x + (size_t)b * QK32;
        float d = ld_f16(blk);
        int j;
        for (j = 0; j < 16; j++) {
            acc += d * ((float)q4_0_code(blk, j) - 8.0f) * xx[j];
            acc += d * ((float)q4_0_code(blk, j + 16) - 8.0f) * xx[j + 16];
        }
    }
    return acc;
}

/* dot_q5_0, src/gguf_quant.c:672-702: acc += d * (c0*x0 + c1*x1) per pair. */
static float dot_q5_0_f32(const uint8_t *w, const float *x, int n) {
    float acc = 0.0f;
    int b;
    for (b = 0; b < n / QK32; b++) {
        const uint8_t *blk = w + (size_t)b * B_Q5_0;
        const float *xx = x + (size_t)b * QK32;
        float d = ld_f16(blk);
        int j;
        for (j = 0; j < 16; j++) {
            float v0 = (float)(q5_0_code(blk, j) - 16);
            float v1 = (float)(q5_0_code(blk, j + 16) - 16);
            acc += d * (v0 * xx[j] + v1 * xx[j + 16]);
        }
    }
    return acc;
}

/* dot_q5_k, src/gguf_quant.c:837-892: serial, acc += (d1*c - m1) * x, the
 * low-nibble element of each pair before the high-nibble one. */
static float dot_q5_k_f32(const uint8_t *w, const float *x, int n) {
    float acc = 0.0f;
    int b;
    for (b = 0; b < n / QKK; b++) {
        const uint8_t *sb = w + (size_t)b * B_Q5_K;
        const float *xx = x + (size_t)b * QKK;
        float d = ld_f16(sb);
        float dmin = ld_f16(sb + 2);
        int j;
        for (j = 0; j < 4; j++) {
            int sc;
            int mn;
            float d1, m1, d2, m2;
            int l;
            k4_scale_min(sb + 4, 2 * j, &sc, &mn);
            d1 = d * (float)sc;
            m1 = dmin * (float)mn;
            k4_scale_min(sb + 4, 2 * j + 1, &sc, &mn);
            d2 = d * (float)sc;
            m2 = dmin * (float)mn;
            for (l = 0; l < 32; l++) {
                float q0 = (float)q5_k_code(sb, 64 * j + l);
                float q1 = (float)q5_k_code(sb, 64 * j + 32 + l);
                acc += (d1 * q0 - m1) * xx[64 * j + l];
                acc += (d2 * q1 - m2) * xx[64 * j + 32 + l];
            }
        }
    }
    return acc;
}

float ora_dot_f32(uint32_t type, const uint8_t *wrow, const float *x, int n) {
    if (wrow == NULL || x == NULL || n <= 0) {
        return 0.0f;
    }
    switch (type) {
        case ORA_F32: return dot_f32_f32((const float *)wrow, x, n);
        case ORA_F16: return dot_f16_f32(wrow, x, n);
        case ORA_Q4_0: return (n % QK32) ? 0.0f : dot_q4_0_f32(wrow, x, n);
        case ORA_Q5_0: return (n % QK32) ? 0.0f : dot_q5_0_f32(wrow, x, n);
        case ORA_Q5_K: return (n % QKK) ? 0.0f : dot_q5_k_f32(wrow, x, n);
        case ORA_Q8_0: return (n % QK32) ? 0.0f : dot_q8_0_f32(wrow, x, n);
        case ORA_Q4_K: return (n % QKK) ? 0.0f : dot_q4_k_f32(wrow, x, n);
        case ORA_Q6_K: return (n % QKK) ? 0.0f : dot_q6_k_f32(wrow, x, n);
        default: return 0.0f;
    }
}

/* --------------------------------------------------------- drivers */

static uint8_t *g_scratch;
static size_t g_scratch_cap;

#include <stdlib.h>

static uint8_t *scratch_ensure(size_t nbytes) {
    if (nbytes > g_scratch_cap) {
        uint8_t *p = (uint8_t *)realloc(g_scratch, nbytes);
        if (p == NULL) {
            return NULL;
        }
        g_scratch = p;
        g_scratch_cap = nbytes;
    }
    return g_scratch;
}

/* edgexpu_cpu_linear, src/cpu_kernel.c:462-523 (F32 weights, one token):
 * acc = (double)bias, eight FMA lanes, hsum256 added in double, the tail in
 * double, one final rounding. */
static void linear_f32_one(float *out, const float *x, const float *w, const float *bias, int n_out, int n_in) {
    int o;
    for (o = 0; o < n_out; o++) {
        const float *row = w + (size_t)o * (size_t)n_in;
        double acc = bias != NULL ? (double)bias[o] : 0.0;
        float v[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int i = 0;
        for (; i + 8 <= n_in; i += 8) {
            int l;
            for (l = 0; l < 8; l++) {
                v[l] = fmaf(x[i + l], row[i + l], v[l]);
            }
        }
        acc += (double)hsum8_quant(v);
        for (; i < n_in; i++) {
            acc += (double)x[i] * (double)row[i];
        }
        out[o] = (float)acc;
    }
}

/* src/cpu_kernel.c:545-644: F32 at one token -> edgexpu_cpu_linear; the
 * Q8_0 family (Q4_0, Q5_0, Q8_0) with n_in % 32 == 0 -> Q8_0 activations;
 * the K-quants with n_in % 256 == 0 -> Q8_K activations; anything else ->
 * the f32-activation row dot.  out = bias + dot. */
int ora_linear_quant_batch(float *out, const float *x, const uint8_t *w, uint32_t type,
                           const float *bias, int m, int n_out, int n_in) {
    size_t rb;
    size_t qb = 0;
    uint8_t *xq = NULL;
    int o;
    int t;
    int path; /* 0: Q8_0 activations, 1: Q8_K activations, 2: f32 */
    if (out == NULL || x == NULL || w == NULL || m <= 0 || n_out <= 0 || n_in <= 0) {
        return 0;
    }
    if (m == 1 && type == ORA_F32) {
        linear_f32_one(out, x, (const float *)w, bias, n_out, n_in);
        return 1;
    }
    rb = ora_row_bytes(type, n_in);
    if (rb == 0) {
        return 0;
    }
    if ((type == ORA_Q8_0 || type == ORA_Q4_0 || type == ORA_Q5_0) && n_in % QK32 == 0) {
        path = 0;
        qb = ora_q8_0_nbytes(n_in);
    } else if ((type == ORA_Q4_K || type == ORA_Q5_K || type == ORA_Q6_K) && n_in % QKK == 0) {
        path = 1;
        qb = ora_q8_k_nbytes(n_in);
    } else {
        path = 2;
    }
    if (path != 2) {
        xq = scratch_ensure((size_t)m * qb);
        if (xq == NULL) {
            return 0;
        }
        for (t = 0; t < m; t++) { /* quantize every token once, serially */
            if (path == 1) {
                ora_quantize_q8_k(x + (size_t)t * n_in, n_in, xq + (size_t)t * qb);
            } else {
                ora_quantize_q8_0(x + (size_t)t * n_in, n_in, xq + (size_t)t * qb);
            }
        }
    }
#pragma omp parallel for schedule(static)
    for (o = 0; o < n_out; o++) {
        const uint8_t *wr = w + (size_t)o * rb;
        float b = bias != NULL ? bias[o] : 0.0f;
        int tok;
        for (tok = 0; tok < m; tok++) {
            float dot;
            if (path == 0) {
                dot = ora_dot_q8(type, wr, xq + (size_t)tok * qb, n_in);
            } else if (path == 1) {
                dot = ora_dot_q8k(type, wr, xq + (size_t)tok * qb, n_in);
            } else {
                dot = ora_dot_f32(type, wr, x + (size_t)tok * n_in, n_in);
            }
            out[(size_t)tok * n_out + o] = b + dot;
        }
    }
    return 1;
}

uint32_t ora_logits(float *scores, const float *hidden, const uint8_t *w, uint32_t type,
                    const float *bias, int vocab, int n_embd, size_t chunk_rows) {
    size_t rb = ora_row_bytes(type, n_embd);
    uint8_t *xq = NULL;
    uint32_t best = 0;
    float best_score = -INFINITY;
    uint32_t begin;
    if (rb == 0 || vocab <= 0 || hidden == NULL || w == NULL) {
        return 0;
    }
    if (type == ORA_Q8_0 || type == ORA_Q4_0 || type == ORA_Q5_0) { /* src/native.c:2317-2319 */
        xq = (uint8_t *)malloc(ora_q8_0_nbytes(n_embd));
        if (xq == NULL || !ora_quantize_q8_0(hidden, n_embd, xq)) {
            free(xq);
            xq = NULL;
        }
    }
    if (chunk_rows == 0) {
        chunk_rows = LOGIT_CHUNK_BYTES / rb;
        if (chunk_rows < 1) {
            chunk_rows = 1;
        }
    }
    for (begin = 0; begin < (uint32_t)vocab; begin += (uint32_t)chunk_rows) {
        uint32_t end = begin + (uint32_t)chunk_rows;
        if (end > (uint32_t)vocab) {
            end = (uint32_t)vocab;
        }
#pragma omp parallel
        {
            uint32_t lbest = 0;
            float lscore = -INFINITY;
            int i;
#pragma omp for nowait schedule(static)
            for (i = (int)begin; i < (int)end; i++) {
                const uint8_t *wr = w + (size_t)i * rb;
                float s = xq != NULL ? ora_dot_q8(type, wr, xq, n_embd) : ora_dot_f32(type, wr, hidden, n_embd);
                if (bias != NULL) {
                    s += bias[i];
                }
                if (scores != NULL) {
                    scores[i] = s;
                }
                if (s > lscore) {
                    lscore = s;
                    lbest = (uint32_t)i;
                }
            }
#pragma omp critical
            {
                if (lscore > best_score || (lscore == best_score && lbest < best)) {
                    best_score = lscore;
                    best = lbest;
                }
            }
        }
    }
    free(xq);
    return best;
}

/* ----------------------------------------------------------- sampling */

/* edgexpu_cpu_softmax, src/cpu_kernel.c:328-353: first-wins max by '>',
 * e = expf(x - max) in float, double sum in index order, p = (float)(e / sum). */
void ora_softmax(float *io, int n) {
    float mx;
    double sum = 0.0;
    int i;
    if (io == NULL || n <= 0) {
        return;
    }
    mx = io[0];
    for (i = 1; i < n; i++) {
        if (io[i] > mx) {
            mx = io[i];
        }
    }
    for (i = 0; i < n; i++) {
        io[i] = expf(io[i] - mx);
        sum += (double)io[i];
    }
    if (sum <= 0.0) {
        return;
    }
    for (i = 0; i < n; i++) {
        io[i] = (float)((double)io[i] / sum);
    }
}

/* xorshift64 step of src/cpu_kernel.c:781-786 (a zero state is seeded first). */
uint64_t ora_rng_step(uint64_t *rng) {
    if (*rng == 0) {
        *rng = 0x00ED6E50ULL;
    }
    *rng ^= *rng << 13;
    *rng ^= *rng >> 7;
    *rng ^= *rng << 17;
    return *rng;
}

typedef struct {
    float p;
    uint32_t id;
} ora_item;

/* probability descending, then id ascending (src/cpu_kernel.c:744-760) */
static int ora_item_cmp(const void *a, const void *b) {
    const ora_item *x = (const ora_item *)a;
    const ora_item *y = (const ora_item *)b;
    if (y->p > x->p) {
        return 1;
    }
    if (y->p < x->p) {
        return -1;
    }
    return x->id < y->id ? -1 : (x->id > y->id ? 1 : 0);
}

/* edgexpu_cpu_sample_softmax, src/cpu_kernel.c:762-849: softmax in place,
 * one xorshift step, u = (rng & 0xFFFFFFF) / 2^28; with 0 < top_p < 1 the
 * items sorted by (p desc, id asc) are kept until their double sum reaches
 * top_p, pick = u * (sum of the kept) and the first kept item whose running
 * sum reaches pick is drawn; otherwise the same walk over all items in index
 * order.  Returns 1, or 0 for bad arguments. */
int ora_sample_softmax(float *logits, int n, float top_p, uint64_t *rng, uint32_t *out) {
    double sum = 0.0;
    double cursor = 0.0;
    double pick;
    int i;
    if (logits == NULL || rng == NULL || out == NULL || n <= 0) {
        return 0;
    }
    ora_softmax(logits, n);
    ora_rng_step(rng);
    if (top_p > 0.0f && top_p < 1.0f) {
        int kept = n;
        ora_item *items = (ora_item *)malloc((size_t)n * sizeof(ora_item));
        if (items == NULL) {
            return 0;
        }
        for (i = 0; i < n; i++) {
            items[i].p = logits[i];
            items[i].id = (uint32_t)i;
        }
        qsort(items, (size_t)n, sizeof(ora_item), ora_item_cmp);
        for (i = 0; i < n; i++) {
            sum += (double)items[i].p;
            if (sum >= (double)top_p) {
                kept = i + 1;
                break;
            }
        }
        sum = 0.0;
        for (i = 0; i < kept; i++) {
            sum += (double)items[i].p;
        }
        if (sum <= 0.0) {
            *out = items[0].id;
            free(items);
            return 1;
        }
        pick = ((double)(*rng & 0xFFFFFFFu) / (double)0x10000000u) * sum;
        *out = items[kept - 1].id;
        for (i = 0; i < kept; i++) {
            cursor += (double)items[i].p;
            if (cursor >= pick) {
                *out = items[i].id;
                break;
            }
        }
        free(items);
        return 1;
    }
    for (i = 0; i < n; i++) {
        sum += (double)logits[i];
    }
    if (sum <= 0.0) {
        *out = 0;
        return 1;
    }
    pick = ((double)(*rng & 0xFFFFFFFu) / (double)0x10000000u) * sum;
    *out = (uint32_t)(n - 1);
    for (i = 0; i < n; i++) {
        cursor += (double)logits[i];
        if (cursor >= pick) {
            *out = (uint32_t)i;
            break;
        }
    }
    return 1;
}

/* -------------------------------------------------------- self-test */

/* -------------------------------------------------- layer elementwise ops */

/* src/cpu_kernel.c:220-242. */
void ora_rmsnorm(float *out, const float *x, const float *w, int n, float eps) {
    double ss = 0.0;
    float mean, scale;
    int i;
    for (i = 0; i < n; i++) ss += (double)x[i] * (double)x[i];
    mean = (float)(ss / (double)n);
    scale = 1.0f / sqrtf(mean + eps);
    for (i = 0; i < n; i++) out[i] = x[i] * scale;
    for (i = 0; i < n; i++) out[i] *= w[i];
}

/* src/cpu_kernel.c:244-252. */
void ora_silu(float *out, const float *x, int n) {
    int i;
    for (i = 0; i < n; i++) out[i] = x[i] / (1.0f + expf(-x[i]));
}

/* src/cpu_kernel.c:210-218. */
void ora_mul(float *out, const float *a, const float *b, int n) {
    int i;
    for (i = 0; i < n; i++) out[i] = a[i] * b[i];
}

/* src/cpu_kernel.c:200-208. */
void ora_add(float *out, const float *a, const float *b, int n) {
    int i;
    for (i = 0; i < n; i++) out[i] = a[i] + b[i];
}

int ora_selftest(char *error, size_t error_size) {
    uint8_t blk[B_Q4_K];
    float x[QKK];
    float y[QKK];
    float fused;
    float expanded = 0.0f;
    uint16_t one = 0x3c00;
    int i;
    memset(blk, 0, sizeof(blk));
    memset(x, 0, sizeof(x));
    memcpy(blk, &one, 2);
    blk[4] = 1;
    blk[16] = 0x02;
    x[0] = 3.0f;
    ora_dequantize(blk, ORA_Q4_K, QKK, y);
    for (i = 0; i < QKK; i++) {
        expanded += y[i] * x[i];
    }
    fused = ora_dot_f32(ORA_Q4_K, blk, x, QKK);
    if (fabsf(fused - expanded) > 1e-4f || fabsf(fused - 6.0f) > 1e-3f) {
        snprintf(error, error_size, "q4_k fused dot %.6f expanded %.6f", fused, expanded);
        return 0;
    }
    {
        uint8_t w[B_Q8_0];
        uint8_t xq[B_Q8_0];
        float xv[QK32];
        memset(w, 0, sizeof(w));
        memcpy(w, &one, 2);
        for (i = 0; i < QK32; i++) {
            w[2 + i] = 1;
            xv[i] = 1.0f;
        }
        ora_quantize_q8_0(xv, QK32, xq);
        fused = ora_dot_q8(ORA_Q8_0, w, xq, QK32);
        if (fabsf(fused - 32.0f) > 0.5f) {
            snprintf(error, error_size, "q8_0 integer dot %.6f", fused);
            return 0;
        }
        /* Q5_0 block of zero codes (value -16 each) against the same x */
        memset(w, 0, B_Q5_0);
        memcpy(w, &one, 2);
        fused = ora_dot_q8(ORA_Q5_0, w, xq, QK32);
        if (fabsf(fused + 512.0f) > 1.0f) {
            snprintf(error, error_size, "q5_0 integer dot %.6f", fused);
            return 0;
        }
    }
    { /* Q4_0: low nibble 9 of element 0 -> value 1; x[0] = 3 */
        uint8_t q40[B_Q4_0];
        float x0[QK32];
        float y0[QK32];
        memset(q40, 0, sizeof(q40));
        memset(x0, 0, sizeof(x0));
        memcpy(q40, &one, 2);
        q40[2] = 0x09;
        x0[0] = 3.0f;
        ora_dequantize(q40, ORA_Q4_0, QK32, y0);
        expanded = 0.0f;
        for (i = 0; i < QK32; i++) {
            expanded += y0[i] * x0[i];
        }
        fused = ora_dot_f32(ORA_Q4_0, q40, x0, QK32);
        if (fabsf(fused - expanded) > 1e-4f || fabsf(fused - 3.0f) > 1e-3f) {
            snprintf(error, error_size, "q4_0 fused dot %.6f expanded %.6f", fused, expanded);
            return 0;
        }
    }
    { /* F16 row {1, 2} . {2, 3} = 8 */
        uint8_t h[4];
        float xh[2] = {2.0f, 3.0f};
        uint16_t two = 0x4000;
        memcpy(h, &one, 2);
        memcpy(h + 2, &two, 2);
        fused = ora_dot_f32(ORA_F16, h, xh, 2);
        if (fabsf(fused - 8.0f) > 1e-3f) {
            snprintf(error, error_size, "f16 dot %.6f", fused);
            return 0;
        }
    }
    { /* Q5_K: sc0 = 1, code 2 at element 0, x[0] = 3 -> 6 */
        uint8_t q5[B_Q5_K];
        memset(q5, 0, sizeof(q5));
        memset(x, 0, sizeof(x));
        memcpy(q5, &one, 2);
        q5[4] = 1;
        q5[48] = 0x02;
        x[0] = 3.0f;
        ora_dequantize(q5, ORA_Q5_K, QKK, y);
        expanded = 0.0f;
        for (i = 0; i < QKK; i++) {
            expanded += y[i] * x[i];
        }
        fused = ora_dot_f32(ORA_Q5_K, q5, x, QKK);
        if (fabsf(fused - expanded) > 1e-4f || fabsf(fused - 6.0f) > 1e-3f) {
            snprintf(error, error_size, "q5_k fused dot %.6f expanded %.6f", fused, expanded);
            return 0;
        }
    }
    return 1;
}
