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
// Top-p without a sort: the reference sorts the items by (p desc, id asc)
// (its qsort comparator, src/cpu_kernel.c:744-760), keeps the shortest
// prefix whose running sum reaches top_p and draws inside it
// (src/cpu_kernel.c:788-832).  Both answers are places in that order where
// a running sum first reaches a target, so each is found by a radix
// selection on the order's key: P = (~bits(p)) & 0x3fffffff ascending is p
// descending (p <= 1 leaves bit 30 of bits(p) clear), in three 10-bit
// digits, then the index among the items of one exact p.  A digit is a
// histogram of the count and mass of the items whose higher digits match,
// and the bin where the running mass reaches the target.  The first digit
// is built by seg_norm_kernel's workgroups; topp_gather_kernel picks the
// kept prefix's first-digit bin, gathers the items up to it and builds that
// bin's second digit; topp_draw_kernel (one workgroup) resolves the rest
// over the gathered items.  Masses are integers in units of 2^-62: every p
// >= 2^-39 is exact in them and integer sums do not depend on their order,
// so the running sums are exact and a draw is reproducible.  (The
// reference's running sum is a double sum that rounds; the two agree except
// where a target lies within that rounding of a running sum.)  NaN
// probabilities sort last, as in the numpy statement of the draw.
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
// The top-p draw's first digit over every probability (filled by
// seg_norm_kernel; the draw itself is further below).
constexpr int kToppBins = 1024;  // one 10-bit digit of the order's key
constexpr int kToppReps = 8;     // copies of the histogram (workgroup b adds to copy b % 8)
struct ToppHist {
    unsigned long long mass[kToppReps][kToppBins];  // in units of 2^-62
    unsigned int cnt[kToppReps][kToppBins];
    unsigned long long mass_all[kToppBins];  // the copies added (by topp_gather_kernel's first workgroup)
    unsigned int cnt_all[kToppBins];
    // the second digit over the items of the kept prefix's first-digit bin
    // (added by topp_gather_kernel; copies as above)
    unsigned long long mass1[kToppReps][kToppBins];
    unsigned int cnt1[kToppReps][kToppBins];
    int nan_max;           // largest index of a NaN probability (-1: none)
    unsigned int n_cand;   // items gathered by topp_gather_kernel
};

// P: the order's key of p (ascending = p descending); NaN after every p.
__device__ __forceinline__ uint32_t topp_key(float p) {
    return p != p ? (1u << 30) : (~__float_as_uint(p)) & 0x3fffffffu;
}

// p in units of 2^-62, truncated (exact for p >= 2^-39; p <= 1 keeps the
// sums < 2^63), from the bits of a non-negative finite p: the 24-bit
// significand shifted by the exponent.
__device__ __forceinline__ unsigned long long topp_mass_bits(uint32_t b) {
    const int e = (int)(b >> 23);
    const unsigned long long sig = (unsigned long long)((b & 0x7fffffu) | (e != 0 ? 0x800000u : 0u));
    const int sh = e - 88;  // p = sig * 2^(e - 150), so p * 2^62 = sig * 2^(e - 88)
    return sh >= 0 ? sig << sh : (sh > -24 ? sig >> -sh : 0ull);
}
__device__ __forceinline__ unsigned long long topp_mass(float p) {
    return p > 0.0f ? topp_mass_bits(__float_as_uint(p)) : 0ull;
}

// th non-null: the workgroups also clear the top-p histograms.
__global__ __launch_bounds__(kSampleThreads) void seg_max_kernel(const float *__restrict__ x, int n, int S,
                                                                 float *__restrict__ pmax, ToppHist *th) {
    __shared__ float red[4];
    const int b = blockIdx.x, lo = b * S, hi = min(n, lo + S);
    if (th != nullptr) {
        for (int k = b * kSampleThreads + threadIdx.x; k < kToppReps * kToppBins; k += gridDim.x * kSampleThreads) {
            (&th->mass[0][0])[k] = 0ull;
            (&th->cnt[0][0])[k] = 0u;
            (&th->mass1[0][0])[k] = 0ull;
            (&th->cnt1[0][0])[k] = 0u;
        }
        if (b == 0 && threadIdx.x == 0) {
            th->nan_max = -1;
            th->n_cand = 0u;
        }
    }
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
// segment's double sum of p.  th non-null: the segment's probabilities also
// enter the top-p draw's first-digit histogram (integer adds, so the sums do
// not depend on their order).
__global__ __launch_bounds__(kSampleThreads) void seg_norm_kernel(float *__restrict__ x, int n, int S, int B,
                                                                  const double *__restrict__ esum,
                                                                  double *__restrict__ psum, ToppHist *th) {
    __shared__ double red[4];
    __shared__ unsigned long long hm[kToppBins];
    __shared__ unsigned int hc[kToppBins];
    if (th != nullptr) {
        for (int k = threadIdx.x; k < kToppBins; k += kSampleThreads) {
            hm[k] = 0ull;
            hc[k] = 0u;
        }
    }
    double t = 0.0;
    for (int k = threadIdx.x; k < B; k += kSampleThreads) t += esum[k];
    const double tot = block_sum_f64(t, red);  // (its barriers also order the clears above)
    const int b = blockIdx.x, lo = b * S, hi = min(n, lo + S);
    double s = 0.0;
    int nan_max = -1;
    for (int i = lo + threadIdx.x; i < hi; i += kSampleThreads) {
        float p = x[i];
        if (!(tot <= 0.0)) {
            p = (float)((double)p / tot);
            x[i] = p;
        }
        s += (double)p;
        if (th != nullptr) {
            if (p != p) {
                nan_max = i;
            } else {
                const uint32_t d = topp_key(p) >> 20;
                atomicAdd(&hm[d], topp_mass(p));
                atomicAdd(&hc[d], 1u);
            }
        }
    }
    s = block_sum_f64(s, red);  // (and these order the adds before the flush)
    if (threadIdx.x == 0) psum[b] = s;
    if (th != nullptr) {
        if (nan_max >= 0) atomicMax(&th->nan_max, nan_max);
        const int rep = b & (kToppReps - 1);
        for (int k = threadIdx.x; k < kToppBins; k += kSampleThreads) {
            if (hc[k] != 0u) {
                atomicAdd(&th->mass[rep][k], hm[k]);
                atomicAdd(&th->cnt[rep][k], hc[k]);
            }
        }
    }
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

// ---------------------------------------------------------------- top-p
constexpr int kToppThreads = 1024;  // one workgroup; one bin per thread in the selections
constexpr int kToppCopies = 2;      // LDS histogram copies (fewer colliding adds)
constexpr int kToppLdsKeys = 8192;  // gathered keys the draw keeps in LDS

struct ToppSh {
    unsigned long long hm[kToppCopies][kToppBins];
    unsigned int hc[kToppCopies][kToppBins];
    unsigned long long wtot[kToppThreads / 64];
    unsigned long long r[2];
    unsigned int rc;
    int slot;
    int wfirst[kToppThreads / 64];
};

// Inclusive prefix sums of v over the workgroup (each wave's shuffle scan,
// then the 16 wave totals); *total the workgroup's sum.
__device__ unsigned long long block_scan_u64(unsigned long long v, ToppSh &sh, unsigned long long *total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const unsigned long long o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    if (lane == 63) sh.wtot[w] = v;
    __syncthreads();
    if (w == 0) {
        unsigned long long t = lane < kToppThreads / 64 ? sh.wtot[lane] : 0ull;
#pragma unroll
        for (int off = 1; off < kToppThreads / 64; off <<= 1) {
            const unsigned long long o = __shfl_up(t, off, 64);
            if (lane >= off) t += o;
        }
        if (lane < kToppThreads / 64) sh.wtot[lane] = t;
    }
    __syncthreads();
    if (w > 0) v += sh.wtot[w - 1];
    *total = sh.wtot[kToppThreads / 64 - 1];
    __syncthreads();
    return v;
}

// Thread t holds bin t (mass m, count c): the first bin with items whose
// running mass from base reaches target (-1: none); *below = base + the mass
// of the bins before it, *bin_m / *bin_c its mass and count; *total the mass
// of all bins.
__device__ int topp_select(unsigned long long m, unsigned int c, unsigned long long base, unsigned long long target,
                           ToppSh &sh, unsigned long long *below, unsigned long long *bin_m, unsigned int *bin_c,
                           unsigned long long *total) {
    const unsigned long long incl = block_scan_u64(m, sh, total);
    // the first qualifying bin: each wave's first lane by ballot, then the
    // first wave that has one (one LDS word per wave; no colliding adds)
    const unsigned long long hits = __ballot(c > 0u && base + incl >= target);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) sh.wfirst[w] = hits != 0ull ? w * 64 + __ffsll((long long)hits) - 1 : INT_MAX;
    __syncthreads();
    int d = INT_MAX;
#pragma unroll
    for (int k = 0; k < kToppThreads / 64; ++k) d = min(d, sh.wfirst[k]);
    if ((int)threadIdx.x == d) {
        sh.r[0] = base + incl - m;
        sh.r[1] = m;
        sh.rc = c;
    }
    __syncthreads();
    *below = sh.r[0];
    *bin_m = sh.r[1];
    *bin_c = sh.rc;
    __syncthreads();
    return d == INT_MAX ? -1 : d;
}

// The selection's position: the resolved high digits of P, the next digit
// (3: resolved), the mass before the resolved prefix and the target; once
// resolved, the selected items (P >> shift == prefix), the rank j of the
// target's item among them and their (equal) mass.
struct ToppSel {
    int lvl;
    unsigned int prefix;
    int shift;
    unsigned int j;
    unsigned int n_sel;  // at lvl 3: the number of selected items
    unsigned long long base;
    unsigned long long target;
    unsigned long long m_item;
};

// Bin d of digit L chosen (below: the mass before it, bin_m / bin_c its
// mass and count): the next digit, or, where one item or one exact p is
// left (always after the last digit), the rank of the target's item.
__device__ ToppSel topp_descend(ToppSel c, int L, int d, unsigned long long below, unsigned long long bin_m,
                                unsigned int bin_c) {
    c.prefix = L == 0 ? (unsigned)d : (c.prefix << 10) | (unsigned)d;
    c.base = below;
    if (bin_c == 1u || L == 2) {
        const unsigned long long m = bin_m / bin_c;
        c.j = c.target <= below || m == 0ull ? 1u : (unsigned)((c.target - below + m - 1ull) / m);
        c.m_item = m;
        c.shift = 20 - 10 * L;
        c.n_sel = bin_c;
        c.lvl = 3;
    } else {
        c.lvl = L + 1;
    }
    return c;
}

// A lane's run of items in one bin (d, mass m, count c), added to the LDS
// histogram only when the bin changes: with many equal probabilities most
// items of a lane fall in the bin of its previous one, and adds to one LDS
// word from many lanes would serialise.
struct ToppRun {
    uint32_t d = 0xffffffffu;
    unsigned long long m = 0ull;
    unsigned int c = 0u;
    __device__ void add(unsigned long long *hm, unsigned int *hc, uint32_t bin, unsigned long long mass) {
        if (bin == d) {
            m += mass;
            ++c;
        } else {
            if (c != 0u) {
                if (hm != nullptr) atomicAdd(&hm[d], m);
                atomicAdd(&hc[d], c);
            }
            d = bin;
            m = mass;
            c = 1u;
        }
    }
};

// The runs left at the end of a pass: while at least 8 lanes of a wave hold
// the first pending lane's bin, they add their sums from one lane (at most 4
// rounds); the rest add one per lane.  Called by whole waves.
__device__ void topp_run_flush(unsigned long long *hm, unsigned int *hc, const ToppRun &r) {
    const int lane = threadIdx.x & 63;
    bool pending = r.c != 0u;
    for (int round = 0; round < 4; ++round) {
        const unsigned long long act = __ballot(pending);
        if (act == 0ull) return;
        const int leader = __ffsll((long long)act) - 1;
        const uint32_t d0 = __shfl(r.d, leader, 64);
        const bool mine = pending && r.d == d0;
        if (__popcll(__ballot(mine)) < 8) break;  // spread bins: plain adds
        unsigned long long sm = mine ? r.m : 0ull;
        unsigned int sc = mine ? r.c : 0u;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            sm += __shfl_xor(sm, off, 64);
            sc += __shfl_xor(sc, off, 64);
        }
        if (lane == leader) {
            if (hm != nullptr) atomicAdd(&hm[d0], sm);
            atomicAdd(&hc[d0], sc);
        }
        pending = pending && !mine;
    }
    if (pending) {
        if (hm != nullptr) atomicAdd(&hm[r.d], r.m);
        atomicAdd(&hc[r.d], r.c);
    }
}

// Every gathered key ckey[0..n_c) through f(i, P): kToppLoads 16-byte loads
// (4 keys each) in flight per thread, uniform trip counts (f is called by
// whole waves, with i >= n_c for the lanes past the end).  ckey holds n_c
// rounded up to 4 entries.
constexpr int kToppLoads = 4;
template <class F>
__device__ __forceinline__ void topp_for_cand(const uint32_t *ckey, int n_c, F &&f) {
    const uint4 *k4 = reinterpret_cast<const uint4 *>(ckey);
    const int n4 = (n_c + 3) / 4;
    for (int b = 0; b < n4; b += kToppThreads * kToppLoads) {
        uint4 v[kToppLoads];
#pragma unroll
        for (int e = 0; e < kToppLoads; ++e) {
            const int q = b + e * kToppThreads + (int)threadIdx.x;
            v[e] = q < n4 ? k4[q] : make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int e = 0; e < kToppLoads; ++e) {
            const int i = 4 * (b + e * kToppThreads + (int)threadIdx.x);
            f(i, v[e].x);
            f(i + 1, v[e].y);
            f(i + 2, v[e].z);
            f(i + 3, v[e].w);
        }
    }
}



// Digits 1 and 2 of the selection over the gathered keys (n_c of them): a
// histogram of the items whose higher digits match, then the bin where the
// running mass reaches the target.
__device__ ToppSel topp_resolve(ToppSel c, const uint32_t *ckey, int n_c, ToppSh &sh) {
    const int t = threadIdx.x;
    while (c.lvl != 3) {
        const int L = c.lvl;
        const int copy = (t >> 6) & (kToppCopies - 1);
#pragma unroll
        for (int k = 0; k < kToppCopies; ++k) {
            sh.hm[k][t] = 0ull;
            sh.hc[k][t] = 0u;
        }
        __syncthreads();
        ToppRun run;
        if (L == 1) {
            topp_for_cand(ckey, n_c, [&](int i, uint32_t P) {
                if (i < n_c && (P >> 20) == c.prefix)
                    run.add(sh.hm[copy], sh.hc[copy], (P >> 10) & 1023u, topp_mass_bits(~P & 0x3fffffffu));
            });
        } else {
            // the last digit: a bin is one exact p, so its items are counted
            // and the run's mass is its count times that p's mass
            const uint32_t hi = c.prefix << 10;
            topp_for_cand(ckey, n_c, [&](int i, uint32_t P) {
                if (i < n_c && (P >> 10) == c.prefix) {
                    const uint32_t d = P & 1023u;
                    if (d == run.d) {
                        ++run.c;
                    } else {
                        run.m = (unsigned long long)run.c * topp_mass_bits(~(hi | run.d) & 0x3fffffffu);
                        run.add(sh.hm[copy], sh.hc[copy], d, 0ull);
                    }
                }
            });
            run.m = (unsigned long long)run.c * topp_mass_bits(~(hi | run.d) & 0x3fffffffu);
        }
        topp_run_flush(sh.hm[copy], sh.hc[copy], run);
        __syncthreads();
        unsigned long long m = 0ull;
        unsigned int cn = 0u;
#pragma unroll
        for (int k = 0; k < kToppCopies; ++k) {
            m += sh.hm[k][t];
            cn += sh.hc[k][t];
        }
        unsigned long long below, bm, tot;
        unsigned int bc;
        const int d = topp_select(m, cn, c.base, c.target, sh, &below, &bm, &bc, &tot);
        c = topp_descend(c, L, d < 0 ? 0 : d, below, bm, bc);  // a bin always qualifies below the first digit
    }
    return c;
}

// The draw's target from the kept prefix's running sum sumkept: pick =
// u * sumkept with u = r28 / 2^28, and an integer running sum reaches pick
// exactly when it reaches ceil(r28 * sumkept / 2^28).
__device__ unsigned long long topp_draw_target(unsigned long long sumkept, unsigned int r28) {
    const unsigned long long hi = __umul64hi(sumkept, (unsigned long long)r28);
    const unsigned long long lo = sumkept * (unsigned long long)r28;
    return ((hi << 36) | (lo >> 28)) + ((lo & 0xfffffffull) != 0ull ? 1ull : 0ull);
}

// The first digit's histogram (thread t: bin t, the copies added) and the
// bin of the kept prefix's end: d1 (-1: the finite mass never reaches
// top_p), *below / *bm / *bc / *tot as topp_select.
__device__ int topp_first_digit(const ToppHist *__restrict__ th, unsigned long long target1, ToppSh &sh,
                                unsigned long long *m0, unsigned int *c0, unsigned long long *below,
                                unsigned long long *bm, unsigned int *bc, unsigned long long *tot) {
    const int t = threadIdx.x;
    unsigned long long m = 0ull;
    unsigned int c = 0u;
#pragma unroll
    for (int r = 0; r < kToppReps; ++r) {
        m += th->mass[r][t];
        c += th->cnt[r][t];
    }
    *m0 = m;
    *c0 = c;
    return topp_select(m, c, 0ull, target1, sh, below, bm, bc, tot);
}

// Gathers (at th->n_cand: the key into ckey, the index into cidx) the items
// that can still matter: finite p whose first digit is at most that of the
// kept prefix's end (every finite item when top_p is never reached).
// Workgroups of 1024 threads, each over kToppThreads * 4 consecutive items;
// one add to the count per workgroup.
__global__ __launch_bounds__(kToppThreads) void topp_gather_kernel(const float *__restrict__ p, int n,
                                                                   ToppHist *th, unsigned long long target1,
                                                                   uint32_t *__restrict__ ckey,
                                                                   uint32_t *__restrict__ cidx) {
    __shared__ ToppSh sh;
    __shared__ unsigned int s_base;
    const int t = threadIdx.x;
    const int lo = blockIdx.x * (kToppThreads * 4);
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {  // issued before the histogram is read
        const int i = lo + e * kToppThreads + t;
        v[e] = i < n ? p[i] : __uint_as_float(0x7fc00000u);
    }
    unsigned long long m0, below, bm, tot;
    unsigned int c0, bc;
    const int d1 = topp_first_digit(th, target1, sh, &m0, &c0, &below, &bm, &bc, &tot);
    if (blockIdx.x == 0) {
        th->mass_all[t] = m0;
        th->cnt_all[t] = c0;
    }
    if (d1 < 0 && th->nan_max >= 0) return;  // the draw is the last NaN; nothing to gather
    const unsigned int bmax = d1 < 0 ? 1023u : (unsigned)d1;
    unsigned int f = 0u;
#pragma unroll
    for (int e = 0; e < 4; ++e) f += (v[e] == v[e] && (topp_key(v[e]) >> 20) <= bmax) ? 1u : 0u;
    unsigned long long ctot;
    const unsigned long long incl = block_scan_u64(f, sh, &ctot);
    if (t == 0) s_base = ctot != 0ull ? atomicAdd(&th->n_cand, (unsigned int)ctot) : 0u;
    __syncthreads();
    unsigned int pos = s_base + (unsigned int)(incl - f);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int i = lo + e * kToppThreads + t;
        if (v[e] == v[e] && (topp_key(v[e]) >> 20) <= bmax) {
            ckey[pos] = topp_key(v[e]);
            cidx[pos] = (uint32_t)i;
            ++pos;
        }
    }
    if (d1 < 0) return;
    // the second digit over this workgroup's items of bin bmax (the kept
    // prefix's end lies there; so does the drawn item when it shares the bin)
    sh.hm[0][t] = 0ull;
    sh.hc[0][t] = 0u;
    __syncthreads();
    ToppRun run;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t P = topp_key(v[e]);
        if (v[e] == v[e] && (P >> 20) == bmax) run.add(sh.hm[0], sh.hc[0], (P >> 10) & 1023u, topp_mass(v[e]));
    }
    topp_run_flush(sh.hm[0], sh.hc[0], run);
    __syncthreads();
    const int rep = blockIdx.x & (kToppReps - 1);
    if (sh.hc[0][t] != 0u) {
        atomicAdd(&th->mass1[rep][t], sh.hm[0][t]);
        atomicAdd(&th->cnt1[rep][t], sh.hc[0][t]);
    }
}

// One workgroup: the top-p draw (top_p as target1 in units of 2^-62; u =
// r28 / 2^28) from the first digit's histogram th and the gathered items.
// Among items of one exact p the order is by index: the drawn one is the
// j-th smallest index, found over two 12-bit digits.
__global__ __launch_bounds__(kToppThreads) void topp_draw_kernel(int n, const ToppHist *__restrict__ th,
                                                                 unsigned long long target1, unsigned int r28,
                                                                 const uint32_t *__restrict__ ckey,
                                                                 const uint32_t *__restrict__ cidx,
                                                                 uint32_t *__restrict__ out) {
    __shared__ ToppSh sh;
    __shared__ __align__(16) uint32_t lkeys[kToppLdsKeys];
    const int t = threadIdx.x;
    if (t == 0) *out = (uint32_t)(n - 1);  // replaced below; no index is left unwritten
    const int n_c = (int)th->n_cand;
    // up to kToppLdsKeys gathered keys are read from LDS from here on
    if (n_c <= kToppLdsKeys) {
        for (int i = t; i < n_c; i += kToppThreads) lkeys[i] = ckey[i];
        for (int i = n_c + t; i < (n_c + 3) / 4 * 4; i += kToppThreads) lkeys[i] = 0u;
    }
    const uint32_t *keys = n_c <= kToppLdsKeys ? lkeys : ckey;
    unsigned long long m0 = th->mass_all[t], below, bm, tot;
    unsigned int c0 = th->cnt_all[t], bc;
    const int d1 = topp_select(m0, c0, 0ull, target1, sh, &below, &bm, &bc, &tot);
    const int nan_last = th->nan_max;
    if (d1 < 0 && nan_last >= 0) {
        // the finite mass never reaches top_p and the running sum turns NaN:
        // the last item of the order, the NaN of the largest index, is drawn
        if (t == 0) *out = (uint32_t)nan_last;
        return;
    }
    // the second digit over bin d1, gathered with the items (thread t: bin t)
    unsigned long long m1 = 0ull;
    unsigned int c1 = 0u;
    if (d1 >= 0) {
#pragma unroll
        for (int r = 0; r < kToppReps; ++r) {
            m1 += th->mass1[r][t];
            c1 += th->cnt1[r][t];
        }
    }
    // the kept prefix's end (without a bin every finite item is kept)
    unsigned long long sumkept = tot;
    if (d1 >= 0) {
        ToppSel k1{};
        k1.target = target1;
        k1 = topp_descend(k1, 0, d1, below, bm, bc);
        if (k1.lvl == 1) {
            const int e1 = topp_select(m1, c1, k1.base, k1.target, sh, &below, &bm, &bc, &tot);
            k1 = topp_descend(k1, 1, e1 < 0 ? 0 : e1, below, bm, bc);
        }
        k1 = topp_resolve(k1, keys, n_c, sh);
        sumkept = k1.base + (unsigned long long)k1.j * k1.m_item;
    }
    // the drawn item: its first digit from the first histogram, then the rest
    ToppSel k2{};
    k2.target = topp_draw_target(sumkept, r28);
    // target <= sumkept <= the finite mass: a bin always qualifies
    const int d2 = topp_select(m0, c0, 0ull, k2.target, sh, &below, &bm, &bc, &tot);
    k2 = topp_descend(k2, 0, d2 < 0 ? 0 : d2, below, bm, bc);
    if (k2.lvl == 1 && d1 >= 0 && k2.prefix == (unsigned)d1) {
        const int e2 = topp_select(m1, c1, k2.base, k2.target, sh, &below, &bm, &bc, &tot);
        k2 = topp_descend(k2, 1, e2 < 0 ? 0 : e2, below, bm, bc);
    }
    k2 = topp_resolve(k2, keys, n_c, sh);
    // the j-th smallest index among the gathered items with P >> shift ==
    // prefix: its high 12 bits, then its low 12 bits (n <= 2^24)
    unsigned int j = k2.j, hi_digit = 0u;
    unsigned int *hcount = reinterpret_cast<unsigned int *>(&sh.hm[0][0]);  // 4096 counters over the copies' space
    // with the keys in global memory and few selected items, their indices
    // are gathered into LDS (the keys' LDS space is free) in one pass
    const bool lds_ids = n_c > kToppLdsKeys && k2.n_sel <= (unsigned)kToppLdsKeys;
    if (lds_ids) {
        if (t == 0) sh.slot = 0;
        __syncthreads();
        topp_for_cand(keys, n_c, [&](int i, uint32_t P) {
            const bool take = i < n_c && (P >> k2.shift) == k2.prefix;
            const unsigned long long ball = __ballot(take);
            if (ball != 0ull) {
                const int lane = t & 63, leader = __ffsll((long long)ball) - 1;
                int at = 0;
                if (lane == leader) at = atomicAdd(&sh.slot, __popcll(ball));
                at = __shfl(at, leader, 64);
                if (take) lkeys[at + __popcll(ball & ((1ull << lane) - 1ull))] = cidx[i];
            }
        });
        __syncthreads();
    }
    const int n_ids = (int)k2.n_sel;
    for (int lv = 0; lv < 2; ++lv) {
#pragma unroll
        for (int k = 0; k < 4; ++k) hcount[t + k * kToppThreads] = 0u;
        __syncthreads();
        ToppRun ids;
        if (lds_ids) {
            for (int i = t; i < n_ids; i += kToppThreads) {
                const uint32_t id = lkeys[i];
                if (lv == 0 || (id >> 12) == hi_digit) ids.add(nullptr, hcount, lv == 0 ? id >> 12 : id & 4095u, 0ull);
            }
        } else {
            topp_for_cand(keys, n_c, [&](int i, uint32_t P) {
                if (i < n_c && (P >> k2.shift) == k2.prefix) {
                    const uint32_t id = cidx[i];
                    if (lv == 0 || (id >> 12) == hi_digit) ids.add(nullptr, hcount, lv == 0 ? id >> 12 : id & 4095u, 0ull);
                }
            });
        }
        topp_run_flush(nullptr, hcount, ids);
        __syncthreads();
        // thread t holds 4 consecutive digit values
        unsigned int cc[4], csum = 0u;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            cc[k] = hcount[4 * t + k];
            csum += cc[k];
        }
        unsigned long long ctot;
        const unsigned long long incl = block_scan_u64(csum, sh, &ctot);
        if (t == 0) sh.slot = INT_MAX;
        __syncthreads();
        unsigned int run = (unsigned int)(incl - csum);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if (run < j && run + cc[k] >= j) {  // one digit value over the workgroup
                sh.slot = 4 * t + k;
                sh.rc = j - run;
            }
            run += cc[k];
        }
        __syncthreads();
        const int dv = sh.slot;
        const unsigned int jr = sh.rc;
        __syncthreads();
        if (dv == INT_MAX) return;  // not expected: the index stays n - 1
        if (lv == 0) {
            hi_digit = (unsigned)dv;
            j = jr;
        } else if (t == 0) {
            *out = (hi_digit << 12) | (unsigned)dv;
        }
    }
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

// Bytes of workspace launch_sample_softmax needs for n entries: the segment
// maxima and sums, the top-p histogram, then the top-p draw's gathered keys
// and indices (n each, 256-byte aligned).
constexpr size_t kSampleHistOffset = 1024 * sizeof(float) + 2 * 1024 * sizeof(double);
constexpr size_t kSampleCandOffset = (kSampleHistOffset + sizeof(ToppHist) + 255) / 256 * 256;
static size_t cand_bytes(int n) { return ((size_t)n * sizeof(uint32_t) + 255) / 256 * 256; }
size_t sample_workspace_bytes(int n) { return kSampleCandOffset + 2 * cand_bytes(n); }

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
        hipLaunchKernelGGL(seg_max_kernel, dim3(B0), dim3(kSampleThreads), 0, st, x, n, S0, pm, nullptr);
        hipLaunchKernelGGL(seg_exp_kernel, dim3(B0), dim3(kSampleThreads), 0, st, x, n, S0, B0, pm, es);
        hipLaunchKernelGGL(seg_norm_kernel, dim3(B0), dim3(kSampleThreads), 0, st, x, n, S0, B0, es, es + 1024,
                           nullptr);
        return hipGetLastError();
    }
    if (n <= 0 || n > (1 << 24)) return hipErrorInvalidValue;
    int B = (n + kSampleThreads - 1) / kSampleThreads;
    if (B > 1024) B = 1024;
    const int S = (n + B - 1) / B;
    B = (n + S - 1) / S;
    float *pmax = reinterpret_cast<float *>(ws);
    double *esum = reinterpret_cast<double *>(reinterpret_cast<uint8_t *>(ws) + 1024 * sizeof(float));
    double *psum = esum + 1024;
    const bool topp = top_p > 0.0f && top_p < 1.0f;
    ToppHist *th = topp ? reinterpret_cast<ToppHist *>(reinterpret_cast<uint8_t *>(ws) + kSampleHistOffset) : nullptr;
    hipLaunchKernelGGL(seg_max_kernel, dim3(B), dim3(kSampleThreads), 0, st, x, n, S, pmax, th);
    hipLaunchKernelGGL(seg_exp_kernel, dim3(B), dim3(kSampleThreads), 0, st, x, n, S, B, pmax, esum);
    hipLaunchKernelGGL(seg_norm_kernel, dim3(B), dim3(kSampleThreads), 0, st, x, n, S, B, esum, psum, th);
    if (!topp) {
        hipLaunchKernelGGL(draw_kernel, dim3(1), dim3(kDrawThreads), 0, st, x, n, S, B, psum, u, out);
        return hipGetLastError();
    }
    // top_p in units of 2^-62, as the masses; u = r28 / 2^28 exactly
    const unsigned long long target = (unsigned long long)((double)top_p * 4611686018427387904.0);
    const unsigned int r28 = (unsigned int)(u * 268435456.0);
    uint32_t *ckey = reinterpret_cast<uint32_t *>(reinterpret_cast<uint8_t *>(ws) + kSampleCandOffset);
    uint32_t *cidx = reinterpret_cast<uint32_t *>(reinterpret_cast<uint8_t *>(ckey) + cand_bytes(n));
    const unsigned int gg = (unsigned)((n + kToppThreads * 4 - 1) / (kToppThreads * 4));
    hipLaunchKernelGGL(topp_gather_kernel, dim3(gg), dim3(kToppThreads), 0, st, x, n, th, target, ckey, cidx);
    hipLaunchKernelGGL(topp_draw_kernel, dim3(1), dim3(kToppThreads), 0, st, n, th, target, r28, ckey, cidx, out);
    return hipGetLastError();
}
