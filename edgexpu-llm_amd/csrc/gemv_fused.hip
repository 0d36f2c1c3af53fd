// Fused, persistent decode GEMV: edgexpu_cpu_linear_quant_batch
// (src/cpu_kernel.c:545-644) for m <= 4 tokens in ONE launch per group of
// projections that share an input.
//
//  * The activation quantizer runs inside the kernel: every workgroup turns
//    the f32 input into Q8_K (K-quant weights) or Q8_0 (Q8_0 weights) codes in
//    LDS with exactly the arithmetic of quantize.hip (bit-identical to
//    src/gguf_dot_q8.c:276-324,360-412), while the loads of its first weight
//    tile are already in flight.  No separate quantize launch.
//  * Lanes own fixed units of K (a unit is 64 elements of a super-block, or
//    one Q8_0 block), so each lane reads its activation slice from LDS once
//    and keeps it in registers for every row it visits.  Long rows are split
//    across KS waves of the workgroup; KS partial sums meet in LDS.
//  * Workgroups are persistent over row tiles (R rows per slot, S = 64/G slots
//    per wave) and prefetch the next tile's weights before computing the
//    current one, so the dot products overlap the HBM stream.
//  * Up to 4 matrices with the same K and type (q/k/v, gate/up) are one
//    launch: tiles are numbered across the matrices.
#include <stdlib.h>

#include "formats.h"

namespace exq {

constexpr int kFusedMaxMats = 4;

struct FusedArgs {
    int nmat;
    const uint8_t *w[kFusedMaxMats];
    const float *bias[kFusedMaxMats];
    float *out[kFusedMaxMats];       // [m][n_out[z]]
    int n_out[kFusedMaxMats];
    int tile_start[kFusedMaxMats + 1];
    size_t row_bytes;
    int K;
    int nblk;
    int U;       // units per row
    int G;       // lanes per row slot (16, 32 or 64)
    int KS;      // waves splitting a row's units (1, 2 or 4)
    int ntiles;  // total row tiles over all matrices (a tile is S*R rows)
    int m;
    const float *x;  // [m][K] f32 activations
};

struct WSrc {
    const uint8_t *w;
    size_t row_bytes;
};

// Q8_K quantization of x into LDS (src/gguf_dot_q8.c:360-412) with the
// arithmetic of quantize_q8_k_kernel.  16 threads per 256-element block, each
// owning one 16-element group (so its int16 sum needs no reduction); all x
// loads of up to 4 rounds of 16 blocks are issued before any is used.  The
// first-index signed maximum is one 64-bit max over keys
//   (|x| bits << 32) | (~index << 1) | sign
// (equal magnitudes -> lowest index wins; zeros and NaN never enter, matching
// the reference's strict '>' from amax = 0).
__device__ void stage_q8_k(const FusedArgs &a, int8_t *lq, float *ld, int16_t *lbs) {
    const int tid = threadIdx.x, sub = tid & 15, bl = tid >> 4;
    const int nb = a.K / kQKK, total = a.m * nb;
    const int rounds = (total + 15) / 16;
    for (int r0 = 0; r0 < rounds; r0 += 4) {
        float4 v[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // clamped: every thread issues the same loads
            const int blk = min((r0 + r) * 16 + bl, total - 1);
            const int tok = blk / nb, b = blk - tok * nb;
            const float4 *p = reinterpret_cast<const float4 *>(a.x + (size_t)tok * a.K + (size_t)b * kQKK + 16 * sub);
#pragma unroll
            for (int k = 0; k < 4; ++k) v[r][k] = p[k];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (r0 + r >= rounds) break;  // uniform over the workgroup
            const int blk = (r0 + r) * 16 + bl;
            const bool valid = blk < total;  // uniform over each 16-thread group
            const float xs[16] = {v[r][0].x, v[r][0].y, v[r][0].z, v[r][0].w, v[r][1].x, v[r][1].y, v[r][1].z,
                                  v[r][1].w, v[r][2].x, v[r][2].y, v[r][2].z, v[r][2].w, v[r][3].x, v[r][3].y,
                                  v[r][3].z, v[r][3].w};
            unsigned long long key = 0ull;
#pragma unroll
            for (int e = 0; e < 16; ++e) {  // selects, no branches
                const float av = fabsf(xs[e]);
                const uint32_t idx = (uint32_t)(16 * sub + e);
                unsigned long long k = ((unsigned long long)__float_as_uint(av) << 32) |
                                       (((~idx) & 0x7fffffffu) << 1) | (xs[e] < 0.0f ? 1u : 0u);
                k = (valid && av > 0.0f) ? k : 0ull;
                key = k > key ? k : key;
            }
#pragma unroll
            for (int off = 8; off > 0; off >>= 1) {
                const unsigned long long o = __shfl_xor(key, off, 16);
                key = o > key ? o : key;
            }
            if (!valid) continue;
            const int tok = blk / nb, b = blk - tok * nb;
            uint32_t words[4] = {0u, 0u, 0u, 0u};
            int sum = 0;
            float d = 0.0f;
            if (key != 0ull) {
                const float amax = __uint_as_float((uint32_t)(key >> 32));
                const float maxv = (key & 1ull) ? -amax : amax;
                const float iscale = -127.0f / maxv;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const float p = iscale * xs[e];
                    // lrintf: a NaN or infinite product gives LONG_MIN, whose low 32 bits are 0
                    int q = fabsf(p) < 2147483648.0f ? (int)rintf(p) : 0;
                    q = q > 127 ? 127 : (q < -127 ? -127 : q);
                    sum += q;
                    words[e >> 2] |= (uint32_t)(q & 0xff) << (8 * (e & 3));
                }
                d = 1.0f / iscale;
            }
            *reinterpret_cast<uint4 *>(lq + (size_t)tok * a.K + (size_t)b * kQKK + 16 * sub) =
                make_uint4(words[0], words[1], words[2], words[3]);
            lbs[(size_t)tok * (a.K / 16) + 16 * b + sub] = (int16_t)sum;
            if (sub == 0) ld[tok * nb + b] = d;
        }
    }
}

// Q8_0 quantization of x into LDS (AVX2 variant, src/gguf_dot_q8.c:276-324):
// 8 threads per 32-element block, loads of up to 4 rounds issued up front;
// same arithmetic as quantize_q8_0_kernel.
__device__ void stage_q8_0(const FusedArgs &a, int8_t *lq, float *ld) {
    const int tid = threadIdx.x, part = tid & 7, bl = tid >> 3;
    const int nb = a.K / kQK8_0, total = a.m * nb;
    const int rounds = (total + 31) / 32;
    for (int r0 = 0; r0 < rounds; r0 += 4) {
        float4 v[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {  // clamped: every thread issues the same loads
            const int blk = min((r0 + r) * 32 + bl, total - 1);
            const int tok = blk / nb, b = blk - tok * nb;
            v[r] = *reinterpret_cast<const float4 *>(a.x + (size_t)tok * a.K + (size_t)b * kQK8_0 + part * 4);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            if (r0 + r >= rounds) break;
            const int blk = (r0 + r) * 32 + bl;
            if (blk >= total) continue;  // uniform within each 8-thread group
            const int tok = blk / nb, b = blk - tok * nb;
            float amax = fmaxf(fmaxf(fabsf(v[r].x), fabsf(v[r].y)), fmaxf(fabsf(v[r].z), fabsf(v[r].w)));
            amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
            amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
            amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
            const float d = amax / 127.0f;
            const float id = amax != 0.0f ? 127.0f / amax : 0.0f;
            const uint32_t dh = f32_to_f16_rne(d);
            const float xs[4] = {v[r].x, v[r].y, v[r].z, v[r].w};
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float q0 = rintf(xs[e] * id);
                int q = (q0 >= -2147483648.0f && q0 < 2147483648.0f) ? (int)q0 : INT32_MIN;
                q = q < -128 ? -128 : (q > 127 ? 127 : q);
                word |= (uint32_t)(q & 0xff) << (8 * e);
            }
            reinterpret_cast<uint32_t *>(lq + (size_t)tok * a.K + (size_t)b * kQK8_0)[part] = word;
            if (part == 0) ld[tok * nb + b] = f16_bits_to_f32(dh);
        }
    }
}

__device__ __forceinline__ void locate(const FusedArgs &a, int tile, int rows_per_tile, int &z, int &row0) {
    z = 0;
#pragma unroll
    for (int k = 1; k < kFusedMaxMats; ++k)
        if (k < a.nmat && tile >= a.tile_start[k]) z = k;
    row0 = (tile - a.tile_start[z]) * rows_per_tile;
}

// Loads of one tile.  Always issued, whatever the tile or lane: the tile index
// is clamped to the last tile and the unit to the last unit, so the number of
// loads in flight is the same on every path and the compiler's wait counts
// let the next tile's loads stay outstanding while this one is computed.
template <class Fmt, int R>
__device__ __forceinline__ void load_tile(const FusedArgs &a, int tile, int rows_per_tile, int slot, int S, int unit,
                                          int &z, int &row0, typename Fmt::W (&w)[R]) {
    locate(a, min(tile, a.ntiles - 1), rows_per_tile, z, row0);
    const WSrc src{a.w[z], a.row_bytes};
    const int u = min(unit, a.U - 1);
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + slot + S * r, a.n_out[z] - 1);
        Fmt::load_w(src, row, u, w[r]);
    }
}

// Dot products of one tile, reduction over the G lanes of each slot and, for
// KS > 1, over the KS waves of the row group.  The sums go to this round's
// slot of the LDS output buffer (ob: [round][rg][slot][idx]); global stores
// happen once after the tile loop, because on this architecture stores share
// the vector-memory counter with loads and a store inside the loop would
// make every wait on the prefetched weights also wait for its completion.
template <class Fmt, int M, int R>
__device__ __forceinline__ void tile_product(const typename Fmt::W (&w)[R], const typename Fmt::Act (&x)[M],
                                             bool compute, int S, int G, int gl, int lane, int KS, int rg, int ks,
                                             float *red, float *ob) {
    constexpr int NV = R * M;
    constexpr int V = NV <= 1 ? 1 : NV <= 2 ? 2 : NV <= 4 ? 4 : NV <= 8 ? 8 : 16;
    static_assert(NV <= 16, "too many partials per lane");
    const int slot = lane / G;
    float vals[V];
#pragma unroll
    for (int k = 0; k < V; ++k) vals[k] = 0.0f;
    if (compute) {
        const int unit = gl + G * ks;
#pragma unroll
        for (int t = 0; t < M; ++t)
#pragma unroll
            for (int r = 0; r < R; ++r) Fmt::dot1(w[r], unit, x[t], vals[r * M + t]);
    }
    group_reduce<V>(vals, G, lane);
    const int live = group_reduce_live(V, G);
    const int base = group_reduce_index(V, G, gl);
    const int spread = V < G ? G / V : 1;
    const bool writer = (gl & (spread - 1)) == 0;
    if (KS == 1) {
        if (writer) {
#pragma unroll
            for (int k = 0; k < V; ++k) {
                if (k >= live) break;
                const int idx = base + k;
                if (idx < NV) ob[(rg * S + slot) * NV + idx] = vals[k];
            }
        }
        return;
    }
    if (writer) {
#pragma unroll
        for (int k = 0; k < V; ++k) {
            if (k >= live) break;
            const int idx = base + k;
            if (idx < NV) red[((rg * KS + ks) * S + slot) * V + idx] = vals[k];
        }
    }
    __syncthreads();
    if (ks == 0 && lane < S * NV) {
        const int sl = lane / NV, idx = lane - sl * NV;
        float sum = 0.0f;
        for (int k2 = 0; k2 < KS; ++k2) sum += red[((rg * KS + k2) * S + sl) * V + idx];
        ob[(rg * S + sl) * NV + idx] = sum;
    }
    __syncthreads();
}

template <class Fmt, int M, int R>
__global__ __launch_bounds__(256) void gemv_fused_kernel(FusedArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    // wave-uniform values go through readfirstlane so that the tile, matrix
    // and pointer selection below is scalar: kernel-argument arrays are then
    // read with scalar loads that never wait on the vector-memory counter
    // (which would drain the weight prefetch)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int G = a.G, S = 64 / G, KS = a.KS, RG = 4 / KS;
    const int rg = wave / KS, ks = wave - rg * KS;
    const int slot = lane / G, gl = lane & (G - 1);
    const int unit = gl + G * ks;
    const bool active = unit < a.U;
    const int rows_per_tile = S * R;

    // LDS: activation codes | scales | 16-element sums | cross-wave partials
    constexpr bool kQ8K = Fmt::kUnitsPerBlock == 4;
    int8_t *lq = reinterpret_cast<int8_t *>(smem);
    const size_t qbytes = ((size_t)a.m * a.K + 15) & ~(size_t)15;
    float *ld = reinterpret_cast<float *>(smem + qbytes);
    const size_t dbytes = (((size_t)a.m * a.nblk * 4) + 15) & ~(size_t)15;
    int16_t *lbs = reinterpret_cast<int16_t *>(smem + qbytes + dbytes);
    const size_t bbytes = kQ8K ? ((((size_t)a.m * (a.K / 16) * 2) + 15) & ~(size_t)15) : 0;
    float *red = reinterpret_cast<float *>(smem + qbytes + dbytes + bbytes);

    // 1. the first tile's weights go out before the activation is staged
    typename Fmt::W wa[R], wb[R];
    int wt = blockIdx.x;
    int za = 0, rowa = 0;
    bool hava = wt * RG + rg < a.ntiles;
    load_tile<Fmt, R>(a, wt * RG + rg, rows_per_tile, slot, S, unit, za, rowa, wa);

    // 2. quantize the activation into LDS, then take this lane's slices
    if (kQ8K) stage_q8_k(a, lq, ld, lbs);
    else stage_q8_0(a, lq, ld);
    __syncthreads();
    const ActLds act{lq, ld, lbs, a.K, a.nblk};
    typename Fmt::Act x[M];
#pragma unroll
    for (int t = 0; t < M; ++t) Fmt::load_act_lds(act, min(unit, a.U - 1), t, x[t]);

    // 3. persistent loop over tiles, two register buffers in turn: the next
    //    tile's loads are in flight while the current one is computed.  The
    //    trip count is uniform over the workgroup, so the cross-wave barriers
    //    of the KS > 1 reduction line up.
    constexpr int NV = R * M;
    float *ob = red + 4 * 4 * 16;  // [round][rg][slot][NV]
    const int ob_round = RG * S * NV;
    int round = 0;
    const int wt0 = wt;
    while (wt * RG < a.ntiles) {
        int zb = 0, rowb = 0;
        const int wt1 = wt + gridDim.x;
        const bool havb = wt1 * RG + rg < a.ntiles;
        load_tile<Fmt, R>(a, wt1 * RG + rg, rows_per_tile, slot, S, unit, zb, rowb, wb);
        tile_product<Fmt, M, R>(wa, x, hava && active, S, G, gl, lane, KS, rg, ks, red, ob + round * ob_round);
        ++round;
        wt = wt1;
        if (wt * RG >= a.ntiles) break;
        const int wt2 = wt + gridDim.x;
        hava = wt2 * RG + rg < a.ntiles;
        load_tile<Fmt, R>(a, wt2 * RG + rg, rows_per_tile, slot, S, unit, za, rowa, wa);
        tile_product<Fmt, M, R>(wb, x, havb && active, S, G, gl, lane, KS, rg, ks, red, ob + round * ob_round);
        ++round;
        wt = wt2;
    }

    // 4. all global stores of this workgroup: out = bias + sum
    __syncthreads();
    for (int i = threadIdx.x; i < round * ob_round; i += 256) {
        const int rd = i / ob_round, rem = i - rd * ob_round;
        const int g = rem / (S * NV), rem2 = rem - g * (S * NV);
        const int sl = rem2 / NV, idx = rem2 - sl * NV;
        const int tl = (wt0 + rd * (int)gridDim.x) * RG + g;
        if (tl >= a.ntiles) continue;
        int z, row0;
        locate(a, tl, rows_per_tile, z, row0);
        const int r = idx / M, t = idx - r * M;
        const int row = row0 + sl + S * r;
        if (row < a.n_out[z]) {
            const float b = a.bias[z] != nullptr ? a.bias[z][row] : 0.0f;
            a.out[z][(size_t)t * a.n_out[z] + row] = b + ob[i];
        }
    }
}

template <class Fmt, int M, int R>
static hipError_t launch_fused_fmt(FusedArgs a, hipStream_t st) {
    const int S = 64 / a.G, RG = 4 / a.KS;
    const int rows_per_tile = S * R;
    int t = 0;
    for (int z = 0; z < a.nmat; ++z) {
        a.tile_start[z] = t;
        t += (a.n_out[z] + rows_per_tile - 1) / rows_per_tile;
    }
    for (int z = a.nmat; z <= kFusedMaxMats; ++z) a.tile_start[z] = t;
    a.ntiles = t;
    const bool q8k = Fmt::kUnitsPerBlock == 4;
    const size_t qbytes = ((size_t)a.m * a.K + 15) & ~(size_t)15;
    const size_t dbytes = (((size_t)a.m * a.nblk * 4) + 15) & ~(size_t)15;
    const size_t bbytes = q8k ? ((((size_t)a.m * (a.K / 16) * 2) + 15) & ~(size_t)15) : 0;
    constexpr int kMaxRounds = 8;
    const size_t lds = qbytes + dbytes + bbytes + 4 * 4 * 16 * sizeof(float) + kMaxRounds * 4 * 64 * sizeof(float);
    // persistent grid: enough workgroups to fill the chip a few times over,
    // each taking the same number of tile rounds
    const int wg_tiles = (t + RG - 1) / RG;
    // resident workgroups from the kernel's real occupancy (registers + LDS)
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_fused_kernel<Fmt, M, R>, 256, lds) !=
            hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    const int resident = per_cu * cus;
    int rounds = (wg_tiles + resident - 1) / resident;
    if (const char *e = getenv("EXQ_FUSED_ROUNDS")) {  // tuning override: tile rounds per workgroup
        const int r = atoi(e);
        if (r > 0) rounds = r;
    }
    if (rounds > kMaxRounds) rounds = kMaxRounds;  // the LDS output buffer holds kMaxRounds rounds
    const int grid = (wg_tiles + rounds - 1) / rounds;
    hipLaunchKernelGGL((gemv_fused_kernel<Fmt, M, R>), dim3(grid), dim3(256), lds, st, a);
    return hipGetLastError();
}

template <class Fmt>
static hipError_t launch_fused_m(FusedArgs a, hipStream_t st) {
    static const int r1 = getenv("EXQ_FUSED_R") ? atoi(getenv("EXQ_FUSED_R")) : 4;  // tuning override
    switch (a.m) {
        case 1:
            if (r1 == 1) return launch_fused_fmt<Fmt, 1, 1>(a, st);
            if (r1 == 2) return launch_fused_fmt<Fmt, 1, 2>(a, st);
            if (r1 == 8) return launch_fused_fmt<Fmt, 1, 8>(a, st);
            return launch_fused_fmt<Fmt, 1, 4>(a, st);
        case 2: return launch_fused_fmt<Fmt, 2, 2>(a, st);
        case 3: return launch_fused_fmt<Fmt, 3, 2>(a, st);
        case 4: return launch_fused_fmt<Fmt, 4, 2>(a, st);
        default: return hipErrorInvalidValue;
    }
}

// Lanes per slot G and waves per row KS for U units so that every unit is
// covered in one pass (G * KS >= U) with the best lane use.
static bool pick_fused_shape(int U, int &G, int &KS) {
    double best = -1.0;
    bool found = false;
    for (int ks = 1; ks <= 4; ks *= 2) {
        for (int g = 64; g >= 16; g >>= 1) {
            if (g * ks < U) continue;
            const double util = (double)U / (double)(g * ks);
            if (util > best + 1e-9) {
                best = util;
                G = g;
                KS = ks;
                found = true;
            }
        }
    }
    return found;
}

}  // namespace exq

using namespace exq;

// True when the fused kernel covers (type, K, m): every unit in one pass and
// the quantized activation fits the LDS budget.
bool gemv_fused_supported(int type, int K, int m) {
    if (m < 1 || m > 4) return false;
    if (type != kTypeQ8_0 && type != kTypeQ4_K && type != kTypeQ6_K) return false;
    const int U = type == kTypeQ8_0 ? K / kQK8_0 : (K / kQKK) * 4;
    int G = 64, KS = 1;
    if (!pick_fused_shape(U, G, KS)) return false;
    const size_t lds = (size_t)m * K * (type == kTypeQ8_0 ? 1.2 : 1.15);
    return lds <= 64 * 1024;
}

// nmat matrices of the same type and K, all applied to the same m tokens of x.
hipError_t launch_gemv_fused(int type, int nmat, const uint8_t *const *w, const int *n_out,
                             const float *const *bias, float *const *out, size_t row_bytes, int K, int m,
                             const float *x, hipStream_t st) {
    if (nmat < 1 || nmat > kFusedMaxMats) return hipErrorInvalidValue;
    FusedArgs a{};
    a.nmat = nmat;
    for (int z = 0; z < nmat; ++z) {
        a.w[z] = w[z];
        a.n_out[z] = n_out[z];
        a.bias[z] = bias != nullptr ? bias[z] : nullptr;
        a.out[z] = out[z];
    }
    a.row_bytes = row_bytes;
    a.K = K;
    a.m = m;
    a.x = x;
    a.nblk = type == kTypeQ8_0 ? K / kQK8_0 : K / kQKK;
    a.U = type == kTypeQ8_0 ? a.nblk : a.nblk * 4;
    if (!pick_fused_shape(a.U, a.G, a.KS)) return hipErrorInvalidValue;
    switch (type) {
        case kTypeQ8_0: return launch_fused_m<FmtQ80>(a, st);
        case kTypeQ4_K: return launch_fused_m<FmtQ4K>(a, st);
        case kTypeQ6_K: return launch_fused_m<FmtQ6K>(a, st);
        default: return hipErrorInvalidValue;
    }
}
