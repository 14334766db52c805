// Host-side interface of the NVFP4 prefill GEMM (MFMA regime).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace apex_hip {

// C[M, N] (row stride ldc) = tensor_scale * A[M, K] . W[N, K]^T; A, C bf16 bits.
struct GemmArgs {
    const uint16_t *A;
    const uint32_t *codes;  // [N, K/8]
    const uint8_t *scales;  // [N, K/16]
    uint16_t *C;
    uint32_t M, N, K, ldc;
    float tensor_scale;
};

// K % 64 == 0 and operands within the 2 GiB buffer-descriptor range.
bool gemm_supported(uint32_t M, uint32_t N, uint32_t K);

hipError_t gemm_launch(const GemmArgs &a, hipStream_t stream);

} // namespace apex_hip
