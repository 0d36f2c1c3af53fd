// Fused decode GEMV for the dispatcher's other quantized formats: Q4_0 and
// Q5_0 rows against Q8_0 activations (src/gguf_dot_q8.c:482-601), Q5_K rows
// against Q8_K (:764-895), quantized inside the kernel as for Q8_0 / Q4_K.
// The plain projection only (no staging prologue, residual or gate/up
// pairs), with the default tile schedules of the Q8_0 / Q4_K / Q6_K launches:
// 16-wave row-split workgroups for one token of a split K-quant row, two
// register buffers of 2-row tiles at one workgroup per CU for launches with
// more than two workgroups' worth of tiles per CU, workgroup tiles at the
// resident grid otherwise.
#include "gemv_fused_kernel.h"

namespace exq {

template <class Fmt, bool STAGE>
static hipError_t launch_basic_nw8(FusedArgs a, hipStream_t st) {
    switch (a.m) {
        case 1: break;
        case 2: return launch_fused_fmt<Fmt, 2, 1, 8, STAGE, 0>(a, st);
        case 3: return launch_fused_fmt<Fmt, 3, 1, 8, STAGE, 0>(a, st);
        case 4: return launch_fused_fmt<Fmt, 4, 1, 8, STAGE, 0>(a, st);
        default: return hipErrorInvalidValue;
    }
    int rows = 0;
    for (int z = 0; z < a.nmat; ++z) rows += a.n_out[z];
    const int r1 = a.KS == 1 && rows <= 4096 ? 2 : 4;
    if (a.KS == 1) {
        const int rows_per_tile = (64 / a.G) * r1;
        int tiles = 0;
        for (int z = 0; z < a.nmat; ++z) tiles += (a.n_out[z] + rows_per_tile - 1) / rows_per_tile;
        if (tiles > 2 * device_cus() * 8) return launch_fused_fmt<Fmt, 1, 2, 8, STAGE, 1>(a, st, 1);
    }
    return r1 == 2 ? launch_fused_fmt<Fmt, 1, 2, 8, STAGE, 0>(a, st) : launch_fused_fmt<Fmt, 1, 4, 8, STAGE, 0>(a, st);
}

template <class Fmt>
static hipError_t launch_fused_basic(const FusedArgs &a, bool stage, hipStream_t st) {
    if (a.KS > 4) return hipErrorInvalidValue;
    if constexpr (Fmt::kUnitsPerBlock == 4) {
        if (stage && a.m == 1 && a.KS > 1) {
            const int r16 = pick_r16<Fmt>(a, 0);
            if (r16 == 1) return launch_fused_fmt<Fmt, 1, 1, 16, true, 0>(a, st);
            if (r16 == 2) return launch_fused_fmt<Fmt, 1, 2, 16, true, 0>(a, st);
            if constexpr (sizeof(typename Fmt::W) <= 48) return launch_fused_fmt<Fmt, 1, 4, 16, true, 0>(a, st);
            return hipErrorInvalidValue;
        }
    }
    return stage ? launch_basic_nw8<Fmt, true>(a, st) : launch_basic_nw8<Fmt, false>(a, st);
}

hipError_t launch_gemv_fused_more(int type, const FusedArgs &a, bool stage, hipStream_t st) {
    switch (type) {
        case kTypeQ4_0: return launch_fused_basic<FmtQ40>(a, stage, st);
        case kTypeQ5_0: return launch_fused_basic<FmtQ50>(a, stage, st);
        case kTypeQ5_K: return launch_fused_basic<FmtQ5K>(a, stage, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace exq
