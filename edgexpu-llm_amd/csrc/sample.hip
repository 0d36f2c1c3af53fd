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
    __shared__ float mx_s;
    __shared__ double red[4];
    if (threadIdx.x == 0) {
        float m = pmax[0];
        for (int k = 1; k < B; ++k) m = pmax[k] > m ? pmax[k] : m;
        mx_s = m;
    }
    __syncthreads();
    const float mx = mx_s;
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
    __shared__ double tot_s;
    __shared__ double red[4];
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int k = 0; k < B; ++k) t += esum[k];
        tot_s = t;
    }
    __syncthreads();
    const double tot = tot_s;
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

// One draw over entries in index order: pick = u * total, the first index
// whose running sum reaches pick (n - 1 if rounding leaves none; 0 when the
// total is not positive).  One thread; the running sum is the segments'
// sums in order, then the crossing segment's entries one by one.
__global__ void draw_kernel(const float *__restrict__ p, int n, int S, int B, const double *__restrict__ psum,
                            double u, uint32_t *__restrict__ out) {
    if (threadIdx.x != 0) return;
    double tot = 0.0;
    for (int k = 0; k < B; ++k) tot += psum[k];
    if (tot <= 0.0) {
        *out = 0u;
        return;
    }
    const double pick = u * tot;
    double cur = 0.0;
    for (int k = 0; k < B; ++k) {
        if (cur + psum[k] >= pick) {
            const int lo = k * S, hi = min(n, lo + S);
            for (int i = lo; i < hi; ++i) {
                cur += (double)p[i];
                if (cur >= pick) {
                    *out = (uint32_t)i;
                    return;
                }
            }
        } else {
            cur += psum[k];
        }
    }
    *out = (uint32_t)(n - 1);
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

// Steps of the network inside one workgroup's 2 * kSampleThreads keys (every
// j < 2 * kSampleThreads, so partners stay in the tile): stage k = k_lo from
// step j0 down to 1, then the whole stages k_lo*2 .. k_hi.
__global__ __launch_bounds__(kSampleThreads) void bitonic_tile_kernel(unsigned long long *__restrict__ keys, int j0,
                                                                      int k_lo, int k_hi) {
    __shared__ unsigned long long t[2 * kSampleThreads];
    const int base = blockIdx.x * 2 * kSampleThreads;
    t[threadIdx.x] = keys[base + threadIdx.x];
    t[threadIdx.x + kSampleThreads] = keys[base + threadIdx.x + kSampleThreads];
    __syncthreads();
    for (int k = k_lo; k <= k_hi; k <<= 1) {
        for (int j = k == k_lo ? j0 : k >> 1; j > 0; j >>= 1) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int li = threadIdx.x + h * kSampleThreads;
                const int ll = li ^ j;
                if (ll > li) {
                    const unsigned long long a = t[li], b = t[ll];
                    const bool up = ((base + li) & k) == 0;
                    if ((a > b) == up) {
                        t[li] = b;
                        t[ll] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
    keys[base + threadIdx.x] = t[threadIdx.x];
    keys[base + threadIdx.x + kSampleThreads] = t[threadIdx.x + kSampleThreads];
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
// (src/cpu_kernel.c:788-832).  One thread.
__global__ void draw_topp_kernel(const unsigned long long *__restrict__ keys, int n, int S, int B,
                                 const double *__restrict__ psum, double top_p, double u, uint32_t *__restrict__ out) {
    if (threadIdx.x != 0) return;
    // running sum up to and including position i, walking segment by segment
    int kept = n;
    double at_kept = 0.0;
    {
        double cur = 0.0;
        bool found = false;
        for (int k = 0; k < B && !found; ++k) {
            const int lo = k * S, hi = min(n, lo + S);
            if (cur + psum[k] >= top_p) {
                for (int i = lo; i < hi; ++i) {
                    cur += (double)key_p(keys[i]);
                    if (cur >= top_p) {
                        kept = i + 1;
                        found = true;
                        break;
                    }
                }
            } else {
                cur += psum[k];
            }
        }
        at_kept = cur;
        if (!found) {
            // no prefix reached top_p: every entry is kept, the sum is the total
            double t = 0.0;
            for (int k = 0; k < B; ++k) t += psum[k];
            at_kept = t;
        }
    }
    if (at_kept <= 0.0) {
        *out = (uint32_t)(keys[0] & 0xffffffffull);
        return;
    }
    const double pick = u * at_kept;
    uint32_t res = (uint32_t)(keys[kept - 1] & 0xffffffffull);
    double cur = 0.0;
    for (int k = 0; k < B; ++k) {
        const int lo = k * S, hi = min(kept, lo + S);
        if (lo >= kept) break;
        const bool whole = lo + S <= kept;
        if (whole && cur + psum[k] < pick) {
            cur += psum[k];
            continue;
        }
        bool hit = false;
        for (int i = lo; i < hi; ++i) {
            cur += (double)key_p(keys[i]);
            if (cur >= pick) {
                res = (uint32_t)(keys[i] & 0xffffffffull);
                hit = true;
                break;
            }
        }
        if (hit) break;
    }
    *out = res;
}

}  // namespace exq

using namespace exq;

// Bytes of workspace launch_sample_softmax needs for n entries.
size_t sample_workspace_bytes(int n) {
    int N2 = 1;
    while (N2 < n) N2 <<= 1;
    if (N2 < 2 * kSampleThreads) N2 = 2 * kSampleThreads;
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
        hipLaunchKernelGGL(draw_kernel, dim3(1), dim3(64), 0, st, x, n, S, B, psum, u, out);
        return hipGetLastError();
    }
    int N2 = 1;
    while (N2 < n) N2 <<= 1;
    if (N2 < 2 * kSampleThreads) N2 = 2 * kSampleThreads;
    const unsigned grid = (unsigned)((N2 + kSampleThreads - 1) / kSampleThreads);
    hipLaunchKernelGGL(keys_kernel, dim3(grid), dim3(kSampleThreads), 0, st, x, n, N2, keys);
    const unsigned tiles = (unsigned)(N2 / (2 * kSampleThreads));
    // stages 2 .. 2 * kSampleThreads sort each tile on its own: one launch
    hipLaunchKernelGGL(bitonic_tile_kernel, dim3(tiles), dim3(kSampleThreads), 0, st, keys, 1, 2,
                       2 * kSampleThreads);
    for (int k = 4 * kSampleThreads; k <= N2; k <<= 1) {
        int j = k >> 1;
        for (; j >= 2 * kSampleThreads; j >>= 1)
            hipLaunchKernelGGL(bitonic_kernel, dim3(grid), dim3(kSampleThreads), 0, st, keys, N2, j, k);
        hipLaunchKernelGGL(bitonic_tile_kernel, dim3(tiles), dim3(kSampleThreads), 0, st, keys, j, k, k);
    }
    hipLaunchKernelGGL(seg_sorted_sum_kernel, dim3(B), dim3(kSampleThreads), 0, st, keys, n, S, psum);
    hipLaunchKernelGGL(draw_topp_kernel, dim3(1), dim3(64), 0, st, keys, n, S, B, psum, (double)top_p, u, out);
    return hipGetLastError();
}
