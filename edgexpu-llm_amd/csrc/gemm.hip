// Prefill quantized GEMM (m >= 64 tokens) on MFMA -- not yet enabled: the
// shim routes every m through the GEMV kernels in groups of 8 tokens.
#include "common.h"

bool gemm_q8_supported(int, int, int, int) { return false; }

hipError_t launch_gemm_q8(int, const uint8_t *, size_t, int, int, int, const uint8_t *, size_t, const float *,
                          float *, int, hipStream_t) {
    return hipErrorNotSupported;
}
