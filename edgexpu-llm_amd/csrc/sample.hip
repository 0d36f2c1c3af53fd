// Temperature sampling on device (src/native.c:2326-2350 through
// edgexpu_cpu_sample_softmax, src/cpu_kernel.c:762-849): softmax of the
// scores in place (src/cpu_kernel.c:328-353), then one draw from the whole
// distribution or from its top-p part.
//
// Every sum is taken in a fixed order, so a draw is reproducible: the n
// entries are cut into B contiguous segments (one workgroup each); a
// segment's sum is a fixed tree in double, and prefixes are the segments'
// sums added in segment order, then the segment's own entries one by one.
// The reference adds in index order one by one; both are double sums of
// float terms, so they agree to about 1e-16 relative.  The exponentials use
// the device expf (within a few ulp of the host libm), so a probability can
// differ from the reference's by a few ulp, and a draw differs only where
// the pick falls within that distance of a running sum.
//
// Top-p: the keys (~bits(p) << 32 | index) sorted ascending put the
// probabilities in descending order and equal ones by ascending index, the
// order of the reference's qsort comparator (src/cpu_kernel.c:744-760);
// sorted with a bitonic network over the next power of two (padding keys
// sort last).
#include <hip/hip_runtime.h>

#include <climits>
#include <cmath>
#include <cstdint>

#include "common.h"

namespace exq {

constexpr int kSampleThreads = 256;

__device__ __forceinline__ double block_sum_f64(double v, double *red) {
    v = wave_sum_f64(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    const double s = (red[0] + red[1]) + (red[2] + red[3]);
    __syncthreads();
    return s;
}

// Segment b = [b*S, min(n, (b+1)*S)): the largest entry (NaN entries never
// win a '>' comparison, as in the reference's scan).  A NaN first entry is
// the reference's maximum whatever follows: segment 0 then reports NaN, which
// no later '>' replaces.
__global__ __launch_bounds__(kSampleThreads) void seg_max_kernel(const float *__restrict__ x, int n, int S,
                                                                 float *__restrict__ pmax) {
    __shared__ float red[4];
    const int b = blockIdx.x, lo = b * S, hi = min(n, lo + S);
    float m = -INFINITY;
    for (int i = lo + threadIdx.x; i < hi; i += kSampleThreads) m = x[i] > m ? x[i] : m;
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    if (threadIdx.x == 0) {
        float r = red[0];
        for (int k = 1; k < 4; ++k) r = red[k] > r ? red[k] : r;
        if (b == 0 && x[0] != x[0]) r = x[0];
        pmax[b] = r;
    }
}

// e = expf(x - max) in place, and the segment's double sum of e.  The max
// is the reference's: x[0] if it is NaN, else the largest entry.
__global__ __launch_bounds__(kSampleThreads) void seg_exp_kernel(float *__restrict__ x, int n, int S, int B,
                                                                 const float *__restrict__ pmax,
                                                                 double *__restrict__ psum) {
    __shared__ float mred[4];
    __shared__ double red[4];
    // max over segments 1..B-1 (none of them NaN), then segment 0's value
    // first, as the reference's scan from x[0]: a NaN there stays
    float m = -INFINITY;
    for (int k = 1 + threadIdx.x; k < B; k += kSampleThreads) m = pmax[k] > m ? pmax[k] : m;
    for (int off = 32; off > 0; off >>= 1) {
        const float o = __shfl_xor(m, off, 64);
        m = o > m ? o : m;
    }
    if ((threadIdx.x & 63) == 0) mred[threadIdx.x >> 6] = m;
    __syncthreads();
    float mx = pmax[0];
#pragma unroll
    for (int k = 0; k < 4; ++k) mx = mred[k] > mx ? mred[k] : mx;
    const int b = blockIdx.x, lo = b * S, hi = min(n, lo + S);
    double s = 0.0;
    for (int i = lo + threadIdx.x; i < hi; i += kSampleThreads) {
        const float e = expf(x[i] - mx);
        x[i] = e;
        s += (double)e;
    }
    s = block_sum_f64(s, red);
    if (threadIdx.x == 0) psum[b] = s;
}

// p = (float)(e / total) in place (total <= 0: left as e, as the
// reference; a NaN total normalizes, also as the reference), and the
// segment's double sum of p.
__global__ __launch_bounds__(kSampleThreads) void seg_norm_kernel(float *__restrict__ x, int n, int S, int B,
                                                                  const double *__restrict__ esum,
                                                                  double *__restrict__ psum) {
    __shared__ double red[4];
    double t = 0.0;
    for (int k = threadIdx.x; k < B; k += kSampleThreads) t += esum[k];
    const double tot = block_sum_f64(t, red);
    const int b = blockIdx.x, lo = b * S, hi = min(n, lo + S);
    double s = 0.0;
    for (int i = lo + threadIdx.x; i < hi; i += kSampleThreads) {
        float p = x[i];
        if (!(tot <= 0.0)) {
            p = (float)((double)p / tot);
            x[i] = p;
        }
        s += (double)p;
    }
    s = block_sum_f64(s, red);
    if (threadIdx.x == 0) psum[b] = s;
}

constexpr int kDrawThreads = 1024;

// Inclusive prefix sums of v over the block (a fixed order: each wave's
// shuffle scan, then the 16 wave totals scanned by wave 0); *total is the
// block's sum, the same addition as the last prefix.
__device__ double block_scan_f64(double v, double *wtot, double *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    if (lane == 63) wtot[w] = v;
    __syncthreads();
    if (w == 0) {
        double t = lane < kDrawThreads / 64 ? wtot[lane] : 0.0;
#pragma unroll
        for (int off = 1; off < kDrawThreads / 64; off <<= 1) {
            const double o = __shfl_up(t, off, 64);
            if (lane >= off) t += o;
        }
        if (lane < kDrawThreads / 64) wtot[lane] = t;
    }
    __syncthreads();
    if (w > 0) v += wtot[w - 1];
    *total = wtot[kDrawThreads / 64 - 1];
    __syncthreads();
    return v;
}

// The smallest idx over the threads whose flag is set (INT_MAX: none).
__device__ int block_first(bool flag, int idx, int *slot) {
    if (threadIdx.x == 0) *slot = INT_MAX;
    __syncthreads();
    if (flag) atomicMin(slot, idx);
    __syncthreads();
    const int r = *slot;
    __syncthreads();
    return r;
}

// The value of thread `src`'s v on every thread.
__device__ double block_bcast(double v, int src, double *sh) {
    if (threadIdx.x == src) *sh = v;
    __syncthreads();
    const double r = *sh;
    __syncthreads();
    return r;
}

struct Sh {
    double wtot[kDrawThreads / 64];
    double b;
    int slot;
};

// The first position i in [start, lim) whose running sum carry + v[start..i]
// reaches target (-1: none), in chunks of kDrawThreads entries; *run is the
// running sum at i (at lim - 1 when none).
template <class V>
__device__ int block_walk(V val, int start, int lim, double target, double carry, double *run, Sh &sh) {
    for (int c = start; c < lim; c += kDrawThreads) {
        const int i = c + threadIdx.x;
        const double v = i < lim ? val(i) : 0.0;
        double tot;
        const double pre = carry + block_scan_f64(v, sh.wtot, &tot);
        const int hit = block_first(i < lim && pre >= target, i, &sh.slot);
        if (hit != INT_MAX) {
            *run = block_bcast(pre, hit - c, &sh.b);
            return hit;
        }
        carry += tot;
    }
    *run = carry;
    return -1;
}

// One draw over entries in index order: pick = u * total, the first index
// whose running sum reaches pick (n - 1 if rounding leaves none; 0 when the
// total is not positive).  The running sums: the segments' sums scanned,
// then the crossing segment's entries scanned on from there.  B <= 1024.
__global__ __launch_bounds__(kDrawThreads) void draw_kernel(const float *__restrict__ p, int n, int S, int B,
                                                            const double *__restrict__ psum, double u,
                                                            uint32_t *__restrict__ out) {
    __shared__ Sh sh;
    const int t = threadIdx.x;
    const double v = t < B ? psum[t] : 0.0;
    double tot;
    const double pre = block_scan_f64(v, sh.wtot, &tot);
    if (tot <= 0.0) {
        if (t == 0) *out = 0u;
        return;
    }
    const double pick = u * tot;
    const int k = block_first(t < B && pre >= pick, t, &sh.slot);
    if (k == INT_MAX) {
        if (t == 0) *out = (uint32_t)(n - 1);
        return;
    }
    const double carry = k > 0 ? block_bcast(pre, k - 1, &sh.b) : 0.0;
    double run;
    const int i = block_walk([&](int j) { return (double)p[j]; }, k * S, n, pick, carry, &run, sh);
    if (t == 0) *out = (uint32_t)(i >= 0 ? i : n - 1);
}

// keys[i] = ~bits(p_i) << 32 | i for i < n, all ones for the padding.
__global__ __launch_bounds__(kSampleThreads) void keys_kernel(const float *__restrict__ p, int n, int N2,
                                                              unsigned long long *__restrict__ keys) {
    const int i = blockIdx.x * kSampleThreads + threadIdx.x;
    if (i >= N2) return;
    keys[i] = i < n ? ((unsigned long long)(~__float_as_uint(p[i])) << 32) | (unsigned)i : ~0ull;
}

// One compare-exchange step (k, j) of the bitonic network, ascending overall.
__global__ __launch_bounds__(kSampleThreads) void bitonic_kernel(unsigned long long *__restrict__ keys, int N2,
                                                                 int j, int k) {
    const int i = blockIdx.x * kSampleThreads + threadIdx.x;
    if (i >= N2) return;
    const int l = i ^ j;
    if (l <= i) return;
    const unsigned long long a = keys[i], b = keys[l];
    const bool up = (i & k) == 0;
    if ((a > b) == up) {
        keys[i] = b;
        keys[l] = a;
    }
}

// Steps of the network inside one workgroup's kTileKeys keys (every
// j < kTileKeys, so partners stay in the tile): stage k = k_lo from step j0
// down to 1, then the whole stages k_lo*2 .. k_hi.
// TK keys per workgroup: 2048 for the first stages (more workgroups), 8192
// (64 KiB of LDS) for the later ones.
constexpr int kTileThreads = 1024;
constexpr int kTileKeys = 8192;
constexpr int kTileKeysSmall = 2048;

template <int TK>
__global__ __launch_bounds__(kTileThreads) void bitonic_tile_kernel(unsigned long long *__restrict__ keys, int j0,
                                                                    int k_lo, int k_hi) {
    constexpr int kTilePer = TK / kTileThreads;
    __shared__ unsigned long long t[TK];
    const int base = blockIdx.x * TK;
#pragma unroll
    for (int h = 0; h < kTilePer; ++h) t[threadIdx.x + h * kTileThreads] = keys[base + threadIdx.x + h * kTileThreads];
    __syncthreads();
    for (int k = k_lo; k <= k_hi; k <<= 1) {
        for (int j = k == k_lo ? j0 : k >> 1; j > 0; j >>= 1) {
            // the TK / 2 pairs (li, li ^ j) with li's bit j clear
#pragma unroll
            for (int h = 0; h < kTilePer / 2; ++h) {
                const int q = threadIdx.x + h * kTileThreads;
                const int li = ((q & ~(j - 1)) << 1) | (q & (j - 1));
                const int ll = li | j;
                const unsigned long long a = t[li], b = t[ll];
                const bool up = ((base + li) & k) == 0;
                if ((a > b) == up) {
                    t[li] = b;
                    t[ll] = a;
                }
            }
            __syncthreads();
        }
    }
#pragma unroll
    for (int h = 0; h < kTilePer; ++h) keys[base + threadIdx.x + h * kTileThreads] = t[threadIdx.x + h * kTileThreads];
}

__device__ __forceinline__ float key_p(unsigned long long k) { return __uint_as_float(~(uint32_t)(k >> 32)); }

// Segment sums of the sorted probabilities (first n keys).
__global__ __launch_bounds__(kSampleThreads) void seg_sorted_sum_kernel(const unsigned long long *__restrict__ keys,
                                                                        int n, int S, double *__restrict__ psum) {
    __shared__ double red[4];
    const int b = blockIdx.x, lo = b * S, hi = min(n, lo + S);
    double s = 0.0;
    for (int i = lo + threadIdx.x; i < hi; i += kSampleThreads) s += (double)key_p(keys[i]);
    s = block_sum_f64(s, red);
    if (threadIdx.x == 0) psum[b] = s;
}

// Top-p draw over the sorted keys: kept = 1 + the first position whose
// running sum reaches top_p (n when none does); pick = u * (running sum at
// kept); the first kept position whose running sum reaches pick
// (src/cpu_kernel.c:788-832).  Running sums as in draw_kernel.
__global__ __launch_bounds__(kDrawThreads) void draw_topp_kernel(const unsigned long long *__restrict__ keys, int n,
                                                                 int S, int B, const double *__restrict__ psum,
                                                                 double top_p, double u,
                                                                 uint32_t *__restrict__ out) {
    __shared__ Sh sh;
    const int t = threadIdx.x;
    auto val = [&](int j) { return (double)key_p(keys[j]); };
    const double v = t < B ? psum[t] : 0.0;
    double tot;
    const double pre = block_scan_f64(v, sh.wtot, &tot);
    int kept = n;
    double at_kept = tot;
    const int k = block_first(t < B && pre >= top_p, t, &sh.slot);
    if (k != INT_MAX) {
        const double carry = k > 0 ? block_bcast(pre, k - 1, &sh.b) : 0.0;
        double run;
        const int i = block_walk(val, k * S, n, top_p, carry, &run, sh);
        if (i >= 0) {
            kept = i + 1;
            at_kept = run;
        }
    }
    if (at_kept <= 0.0) {
        if (t == 0) *out = (uint32_t)(keys[0] & 0xffffffffull);
        return;
    }
    const double pick = u * at_kept;
    // segments wholly below kept by their sums, then entries up to kept
    const int kfull = kept / S;
    const int k2 = block_first(t < kfull && pre >= pick, t, &sh.slot);
    const int start_seg = k2 != INT_MAX ? k2 : kfull;
    const double carry = start_seg > 0 ? block_bcast(pre, start_seg - 1, &sh.b) : 0.0;
    double run;
    const int i = block_walk(val, start_seg * S, kept, pick, carry, &run, sh);
    if (t == 0) *out = (uint32_t)(keys[i >= 0 ? i : kept - 1] & 0xffffffffull);
}

// io[i] = io[i] / d (the temperature scaling of src/native.c:2339; float
// division, correctly rounded).
__global__ __launch_bounds__(kSampleThreads) void div_scalar_kernel(float *__restrict__ io, long long n, float d) {
    const long long stride = (long long)gridDim.x * kSampleThreads;
    for (long long i = (long long)blockIdx.x * kSampleThreads + threadIdx.x; i < n; i += stride) io[i] = io[i] / d;
}

}  // namespace exq

using namespace exq;

hipError_t launch_div_scalar(float *io, long long n, float d, hipStream_t st) {
    if (n <= 0) return hipErrorInvalidValue;
    long long blocks = (n + kSampleThreads - 1) / kSampleThreads;
    if (blocks > 4096) blocks = 4096;
    hipLaunchKernelGGL(div_scalar_kernel, dim3((unsigned)blocks), dim3(kSampleThreads), 0, st, io, n, d);
    return hipGetLastError();
}

// Bytes of workspace launch_sample_softmax needs for n entries.
size_t sample_workspace_bytes(int n) {
    int N2 = 1;
    while (N2 < n) N2 <<= 1;
    if (N2 < kTileKeys) N2 = kTileKeys;
    const size_t B = 1024;
    return B * sizeof(float) + 2 * B * sizeof(double) + (size_t)N2 * sizeof(unsigned long long) + 256;
}

// Softmax of x[0..n) in place and one draw into *out (device; null: softmax
// only).  u in [0, 1) is the caller's uniform (the reference's
// (rng & 0xFFFFFFF) / 2^28); top_p in (0, 1) draws from the top-p part.
// ws: sample_workspace_bytes(n).
hipError_t launch_sample_softmax(float *x, int n, float top_p, double u, uint32_t *out, void *ws, hipStream_t st) {
    if (out == nullptr) {
        // softmax only (edgexpu_cpu_softmax)
        if (n <= 0) return hipErrorInvalidValue;
        int B0 = (n + kSampleThreads - 1) / kSampleThreads;
        if (B0 > 1024) B0 = 1024;
        const int S0 = (n + B0 - 1) / B0;
        B0 = (n + S0 - 1) / S0;
        float *pm = reinterpret_cast<float *>(ws);
        double *es = reinterpret_cast<double *>(reinterpret_cast<uint8_t *>(ws) + 1024 * sizeof(float));
        hipLaunchKernelGGL(seg_max_kernel, dim3(B0), dim3(kSampleThreads), 0, st, x, n, S0, pm);
        hipLaunchKernelGGL(seg_exp_kernel, dim3(B0), dim3(kSampleThreads), 0, st, x, n, S0, B0, pm, es);
        hipLaunchKernelGGL(seg_norm_kernel, dim3(B0), dim3(kSampleThreads), 0, st, x, n, S0, B0, es, es + 1024);
        return hipGetLastError();
    }
    if (n <= 0 || n > (1 << 30)) return hipErrorInvalidValue;
    int B = (n + kSampleThreads - 1) / kSampleThreads;
    if (B > 1024) B = 1024;
    const int S = (n + B - 1) / B;
    B = (n + S - 1) / S;
    float *pmax = reinterpret_cast<float *>(ws);
    double *esum = reinterpret_cast<double *>(reinterpret_cast<uint8_t *>(ws) + 1024 * sizeof(float));
    double *psum = esum + 1024;
    unsigned long long *keys = reinterpret_cast<unsigned long long *>(psum + 1024);
    hipLaunchKernelGGL(seg_max_kernel, dim3(B), dim3(kSampleThreads), 0, st, x, n, S, pmax);
    hipLaunchKernelGGL(seg_exp_kernel, dim3(B), dim3(kSampleThreads), 0, st, x, n, S, B, pmax, esum);
    hipLaunchKernelGGL(seg_norm_kernel, dim3(B), dim3(kSampleThreads), 0, st, x, n, S, B, esum, psum);
    if (!(top_p > 0.0f && top_p < 1.0f)) {
        hipLaunchKernelGGL(draw_kernel, dim3(1), dim3(kDrawThreads), 0, st, x, n, S, B, psum, u, out);
        return hipGetLastError();
    }
    int N2 = 1;
    while (N2 < n) N2 <<= 1;
    if (N2 < kTileKeys) N2 = kTileKeys;
    const unsigned grid = (unsigned)((N2 + kSampleThreads - 1) / kSampleThreads);
    hipLaunchKernelGGL(keys_kernel, dim3(grid), dim3(kSampleThreads), 0, st, x, n, N2, keys);
    const unsigned tiles = (unsigned)(N2 / kTileKeys);
    // stages 2 .. kTileKeys sort each tile on its own: 2048-key tiles, then
    // their merges inside 8192-key tiles
    hipLaunchKernelGGL(bitonic_tile_kernel<kTileKeysSmall>, dim3((unsigned)(N2 / kTileKeysSmall)),
                       dim3(kTileThreads), 0, st, keys, 1, 2, kTileKeysSmall);
    hipLaunchKernelGGL(bitonic_tile_kernel<kTileKeys>, dim3(tiles), dim3(kTileThreads), 0, st, keys,
                       kTileKeysSmall, 2 * kTileKeysSmall, kTileKeys);
    for (int k = 2 * kTileKeys; k <= N2; k <<= 1) {
        int j = k >> 1;
        for (; j >= kTileKeys; j >>= 1)
            hipLaunchKernelGGL(bitonic_kernel, dim3(grid), dim3(kSampleThreads), 0, st, keys, N2, j, k);
        hipLaunchKernelGGL(bitonic_tile_kernel<kTileKeys>, dim3(tiles), dim3(kTileThreads), 0, st, keys, j, k, k);
    }
    hipLaunchKernelGGL(seg_sorted_sum_kernel, dim3(B), dim3(kSampleThreads), 0, st, keys, n, S, psum);
    hipLaunchKernelGGL(draw_topp_kernel, dim3(1), dim3(kDrawThreads), 0, st, keys, n, S, B, psum, (double)top_p, u,
                       out);
    return hipGetLastError();
}
