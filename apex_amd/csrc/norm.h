// RMSNorm and per-head RMSNorm + RoPE (fp32 activations, bf16 weights) for gfx950:
// the two normalisation kernels the reference engine runs around the NVFP4 matmuls
// (shaders/norm.metal, shaders/head_norm_rope.metal).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace apex_hip {

struct RmsNormArgs {
    const float *x;     // [rows, n]
    const uint16_t *w;  // [n] bf16
    float *y;           // [rows, n]
    uint32_t rows, n;
    float eps;
};

struct HeadNormRopeArgs {
    const float *x;     // [tokens, heads, head_dim]
    const uint16_t *w;  // [head_dim] bf16 (read only when has_weight)
    float *y;           // token t, head h at y + t * out_token_stride + h * out_head_stride
    uint32_t tokens, heads, head_dim, has_weight, rope_pairs;
    float rope_base;
    uint32_t abs_pos, out_token_stride, out_head_stride;
    float eps;
};

constexpr uint32_t kHeadNormMaxDim = 512; // the reference's threadgroup row buffer

hipError_t rms_norm_launch(const RmsNormArgs &a, hipStream_t stream);
hipError_t head_norm_rope_launch(const HeadNormRopeArgs &a, hipStream_t stream);

} // namespace apex_hip
