// Shared pieces of the prefill GEMMs (m >= 16 tokens) on the matrix cores:
// the MFMA operand types, the LDS DMA written as inline assembly with
// explicit waits, the activation-pack geometry, the K split over
// workgroups with its deterministic last-arriver sum, and the grid sizing.
//
// Geometry shared by every format: a workgroup computes 128 tokens (4 MFMA
// tiles of 32) against a block of weight rows, stepping through K in steps
// of 128 (half a 256-element super-block).  The activation codes of a step
// live in LDS as [K-step 8][token tile 4][MFMA lane 64][8 fp16] (32 KiB):
// lane L of K-step s holds token L % 32 and K slots 8 (L / 32) .. + 7, the
// order each format's packer and weight operand agree on.
//
// MFMA operand layout (v_mfma_f32_32x32x16_f16): lane l supplies row l % 32
// of A (a token) and column l % 32 of B (a weight row), K slots
// 8 (l / 32) .. + 7; accumulator register r of lane l holds
// C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32], C[token][row].
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace exq {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

constexpr int kTiles = 4;                   // MFMA token tiles of 32 per workgroup
constexpr int kTokB = 32 * kTiles;          // 128 tokens per workgroup
constexpr int kWaves = 8;                   // two per SIMD
constexpr int kThreads = 64 * kWaves;
constexpr int kGemmCounters = 1024;         // arrival counters in the workspace

// The Q8_K activation pack, one block per (super-block, 128-token block):
//   codes  [half 2][K-step 8][tile 4][MFMA lane 64][8 fp16]   64 KiB
//   mn     [tile 4][MFMA lane 64][8 fp16]  16-element bsums for the min term
//   dx     [128] f32, sq [128] int32 (sum |q8| of the super-block)
// The codes are in the K order of the Q4_K nibble layout: lane L = token +
// 32 h of K-step s in half hf holds the codes of elements 64 j + 4 s + b and
// 64 j + 32 + 4 s + b (j = 2 h + hf, b = 0..3) as
//   [lo b0, lo b2, hi b0, hi b2, lo b1, lo b3, hi b1, hi b3]
// (lo: the first group of 32, hi: the second); lane half hh of mn holds
// bsums 8 hh .. 8 hh + 7.
constexpr int kPkHalf = 8 * kTiles * 1024;  // codes of one step: 32 KiB
constexpr int kPkCodes = 2 * kPkHalf;       // codes of a 256-element super-block
constexpr int kPkMn = kTiles * 1024;
constexpr int kPkDx = kTokB * 4;
constexpr int kPkSq = kTokB * 4;
constexpr int kPkExtra = kPkMn + kPkDx + kPkSq;  // 5120
constexpr int kPkBlk = kPkCodes + kPkExtra;      // 70656
constexpr int kHalfChunks = kPkHalf / 1024;      // 1 KiB DMA chunks per step
constexpr int kExtraChunks = kPkExtra / 1024;
static_assert(kHalfChunks == 4 * kWaves, "four code chunks per wave and step");
static_assert(kExtraChunks <= kWaves && kPkExtra % 1024 == 0, "one extras chunk per wave at most");

// 128-token blocks of an activation pack for m tokens.
__host__ __device__ constexpr int pack_tblocks(int m) { return (m + kTokB - 1) / kTokB; }

// K split: enough workgroups to cover the chip's 256 CUs where the tiles
// alone cannot, at most max_split and at least two K blocks per workgroup.
__host__ __device__ inline int gemm_split_for(int ntiles, int nblk, int max_split) {
    int s = 256 / ntiles;
    if (s > max_split) s = max_split;
    if (s > nblk / 2) s = nblk / 2;
    if (ntiles > kGemmCounters) s = 1;
    return s < 1 ? 1 : s;
}

// ------------------------------------------------------------ helpers

__device__ __forceinline__ uint32_t h2_bits(int lo, int hi) {
    const _Float16 l = (_Float16)(float)lo, h = (_Float16)(float)hi;
    return (uint32_t)__builtin_bit_cast(uint16_t, l) | ((uint32_t)__builtin_bit_cast(uint16_t, h) << 16);
}

__device__ __forceinline__ int sbyte(uint32_t w, int b) { return (int)(int8_t)((w >> (8 * b)) & 0xffu); }

__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Buffer descriptor words (gfx9): base, base_hi | stride 0, num_records,
// dword format.  Loads whose per-lane offset is at or past num_records read 0.
__device__ __forceinline__ v4u rsrc_words(const void *base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return v4u{(uint32_t)a, (uint32_t)(a >> 32) & 0xffffu, bytes, 0x00020000u};
}

// One LDS DMA: each lane's 16 bytes at base + soff + voff land at LDS byte
// address lds + 16 * lane.  M0 (which holds the LDS address) is a register
// the compiler reserves, so the block restores it before returning.  Every
// global load of a GEMM main loop is one of these, and every wait for one an
// explicit s_waitcnt: the compiler then has no loads of its own in the loop
// and no reason to drain the DMA queue before LDS reads it cannot tell apart
// from the slots in flight.
__device__ __forceinline__ void dma16(uint32_t lds, uint32_t voff, const v4u &rs, uint32_t soff) {
    uint32_t saved;
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %1\n\t"
        "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "s"(lds), "v"(voff), "s"(rs), "s"(soff)
        : "memory");
}

// s_waitcnt vmcnt(N): at most N of this wave's DMAs still in flight.
template <int N>
__device__ __forceinline__ void wait_dma() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

__device__ __forceinline__ v16f mfma(v8h a, v8h b, v16f c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v8h lds_v8h(const uint8_t *p) { return *reinterpret_cast<const v8h *>(p); }
__device__ __forceinline__ v4u lds_v4u(const uint8_t *p) { return *reinterpret_cast<const v4u *>(p); }

// Wavefront maximum through DPP row shifts and broadcasts (no LDS round trips).
__device__ __forceinline__ int wave_max_dpp(int v) {
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x111, 0xf, 0xf, false));  // row_shr:1
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x112, 0xf, 0xf, false));  // row_shr:2
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x114, 0xf, 0xf, false));  // row_shr:4
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x118, 0xf, 0xf, false));  // row_shr:8
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x142, 0xa, 0xf, false));  // row_bcast:15
    v = max(v, __builtin_amdgcn_update_dpp(v, v, 0x143, 0xc, 0xf, false));  // row_bcast:31
    return __builtin_amdgcn_readlane(v, 63);
}

// Four unsigned bytes of u (values 0..255) as two fp16 pairs 1024 + byte:
// p[0] = (b0, b1), p[1] = (b2, b3).  One v_perm each, with the exponent
// byte 0x64 taken from `hi` (0x64646464 held in a register).
__device__ __forceinline__ void bytes_to_h2(uint32_t u, uint32_t hi, h2 (&p)[2]) {
    p[0] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(hi, u, 0x04010400u));
    p[1] = __builtin_bit_cast(h2, __builtin_amdgcn_perm(hi, u, 0x04030402u));
}

// ------------------------------------------------------------ K split

// The last of a tile's nsplit workgroups adds the partial tiles up in split
// order (so the result does not depend on which finishes last) and returns
// true; the others store their partial and return false.  NT accumulator
// tiles per thread.  Release: every thread's stores are complete (vmcnt 0)
// before the barrier, one thread writes them back to the device level and
// counts the arrival; the last arriver invalidates its caches (acquire)
// before any thread reads the others' partials, and resets the counter.
template <int NT>
__device__ __forceinline__ bool split_reduce(v16f (&acc)[NT], float *part_base, unsigned *cnt, int nsplit, int ntiles,
                                             int tile, int z, int *s_last) {
    const int tid = threadIdx.x;
    float4 *part = reinterpret_cast<float4 *>(part_base);
    const size_t base = ((size_t)z * ntiles + tile) * (NT * 4);
#pragma unroll
    for (int k = 0; k < NT; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            part[(base + k * 4 + i) * kThreads + tid] =
                make_float4(acc[k][4 * i], acc[k][4 * i + 1], acc[k][4 * i + 2], acc[k][4 * i + 3]);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(&cnt[tile], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
        const int last = old == (unsigned)(nsplit - 1);
        if (last) {
            __hip_atomic_store(&cnt[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        *s_last = last;
    }
    __syncthreads();
    if (!*s_last) return false;
    v16f sum[NT];
    for (int zz = 0; zz < nsplit; ++zz) {
        const size_t bz = ((size_t)zz * ntiles + tile) * (NT * 4);
#pragma unroll
        for (int k = 0; k < NT; ++k)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 p = zz == z ? make_float4(acc[k][4 * i], acc[k][4 * i + 1], acc[k][4 * i + 2],
                                                       acc[k][4 * i + 3])
                                         : part[(bz + k * 4 + i) * kThreads + tid];
                const float pv[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) sum[k][4 * i + e] = zz == 0 ? pv[e] : sum[k][4 * i + e] + pv[e];
            }
    }
#pragma unroll
    for (int k = 0; k < NT; ++k) acc[k] = sum[k];
    return true;
}

}  // namespace exq
