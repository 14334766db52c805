// RMSNorm (shaders/norm.metal:33-81) and per-head RMSNorm + RoPE
// (shaders/head_norm_rope.metal:5-72) for gfx950.
//
// Both are bandwidth-trivial next to the matmuls (one read and one write of the fp32
// activations), so the design goal is one pass over memory with no extra launches:
//   rms_norm      one 256-thread workgroup per row; 16-byte loads when the row is
//                 16-byte aligned, the sum of squares reduced across the wave with DPP
//                 and across the 4 waves through LDS; the row is read twice (the
//                 second time from L2).
//   head_norm_rope one wave per (token, head): lane l owns the rotation pairs
//                 i = l, l + 64, ... (elements i and head_dim/2 + i), so the
//                 normalisation, the weights and the rotation all stay in registers;
//                 the token's cos / sin table is computed once per workgroup of 8
//                 heads, in LDS.
// Arithmetic follows the reference: fp32 sums of squares, inv = 1 / sqrt(ss / n + eps),
// y = x * inv * w with w widened from bf16, and the rotation angle
// (abs_pos + token) * rope_base^(-2 i / head_dim) in fp32 with fp32 cos / sin.
#include "norm.h"
#include "nvfp4_device.h"

namespace apex_hip {
namespace {

__device__ __forceinline__ float wave_sum(float v) { return group_sum<64>(v); }

__device__ __forceinline__ float bf16_weight(const uint16_t *w, uint32_t i) {
    return bf16_bits_to_f32(w[i]);
}

// Rows of up to 256 * kRegQuads * 4 elements (16-byte aligned) stay in registers
// between the sum of squares and the scaling, and the weight loads are issued with the
// row's: one pass over HBM with every load in flight before the reduction.  The
// per-thread sums run in the same order as the two-pass loop, so results are identical.
constexpr int kRegQuads = 4;

__global__ __launch_bounds__(256) void rms_norm_kernel(RmsNormArgs a) {
    __shared__ float part[4];
    const uint32_t row = blockIdx.x;
    const float *x = a.x + (size_t)row * a.n;
    float *y = a.y + (size_t)row * a.n;
    const uint32_t n = a.n, tid = threadIdx.x;
    const bool vec = n % 4 == 0 && ((uintptr_t)x | (uintptr_t)y) % 16 == 0 && (uintptr_t)a.w % 8 == 0;
    float ss = 0.0f;
    if (vec && n / 4 <= 256u * kRegQuads) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const uint2 *w4 = reinterpret_cast<const uint2 *>(a.w);
        float4 v[kRegQuads];
        uint2 wb[kRegQuads];
#pragma unroll
        for (int r = 0; r < kRegQuads; ++r) {
            const uint32_t i = tid + 256 * r;
            const bool ok = i < n / 4;
            v[r] = ok ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            wb[r] = ok ? w4[i] : make_uint2(0, 0);
        }
#pragma unroll
        for (int r = 0; r < kRegQuads; ++r)
            ss += v[r].x * v[r].x + v[r].y * v[r].y + v[r].z * v[r].z + v[r].w * v[r].w;
        ss = wave_sum(ss);
        if ((tid & 63) == 0)
            part[tid >> 6] = ss;
        __syncthreads();
        const float total = part[0] + part[1] + part[2] + part[3];
        const float inv = 1.0f / sqrtf(total / (float)n + a.eps);
        float4 *y4 = reinterpret_cast<float4 *>(y);
#pragma unroll
        for (int r = 0; r < kRegQuads; ++r) {
            const uint32_t i = tid + 256 * r;
            if (i < n / 4) {
                float4 o;
                o.x = v[r].x * inv * __uint_as_float(wb[r].x << 16);
                o.y = v[r].y * inv * __uint_as_float(wb[r].x & 0xFFFF0000u);
                o.z = v[r].z * inv * __uint_as_float(wb[r].y << 16);
                o.w = v[r].w * inv * __uint_as_float(wb[r].y & 0xFFFF0000u);
                y4[i] = o;
            }
        }
        return;
    }
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        for (uint32_t i = tid; i < n / 4; i += 256) {
            const float4 v = x4[i];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    } else {
        for (uint32_t i = tid; i < n; i += 256)
            ss += x[i] * x[i];
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0)
        part[tid >> 6] = ss;
    __syncthreads();
    const float total = part[0] + part[1] + part[2] + part[3];
    const float inv = 1.0f / sqrtf(total / (float)n + a.eps);
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const uint2 *w4 = reinterpret_cast<const uint2 *>(a.w);
        float4 *y4 = reinterpret_cast<float4 *>(y);
        for (uint32_t i = tid; i < n / 4; i += 256) {
            const float4 v = x4[i];
            const uint2 wb = w4[i];
            float4 o;
            o.x = v.x * inv * __uint_as_float(wb.x << 16);
            o.y = v.y * inv * __uint_as_float(wb.x & 0xFFFF0000u);
            o.z = v.z * inv * __uint_as_float(wb.y << 16);
            o.w = v.w * inv * __uint_as_float(wb.y & 0xFFFF0000u);
            y4[i] = o;
        }
    } else {
        for (uint32_t i = tid; i < n; i += 256)
            y[i] = x[i] * inv * bf16_weight(a.w, i);
    }
}

// One workgroup per (kTokensPerBlock tokens, group of kHeadsPerBlock heads), one wave
// per head.  The rotation angles depend on the token and the pair only, so the
// workgroup computes each token's cos / sin table once into LDS (fp32 powf and
// sincosf, as the reference forms them) and every head of the group reads it.  A wave
// issues the loads of its head in all of the block's tokens before anything else: a
// CU holds at most 32 waves, so the loads a wave keeps in flight set the rate: two
// tokens per wave measured 4.29-4.39 -> 4.73 TB/s; four (67 VGPRs, fewer waves) gained
// nothing.
// Heads per workgroup: 16 when there are that many (one table per 16 heads: 4.78-4.85
// against 4.61-4.63 TB/s with 8 at 16 heads), else 8.
constexpr int kTokensPerBlock = 2;

template <int kHeadsPerBlock>
__global__ __launch_bounds__(64 * kHeadsPerBlock) void head_norm_rope_kernel(HeadNormRopeArgs a) {
    constexpr int kMaxPerLane = kHeadNormMaxDim / 2 / 64; // pairs per lane
    constexpr int TB = kTokensPerBlock;
    __shared__ float2 rot[TB][kHeadNormMaxDim / 2];       // (cos, sin) of pair i
    const uint32_t groups = (a.heads + kHeadsPerBlock - 1) / kHeadsPerBlock;
    const uint32_t token0 = blockIdx.x / groups * TB;
    const uint32_t head = (blockIdx.x % groups) * kHeadsPerBlock + (threadIdx.x >> 6);
    const uint32_t D = a.head_dim, half = D / 2;
    const uint32_t lane = threadIdx.x & 63;
    float lo[TB][kMaxPerLane], hi[TB][kMaxPerLane];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        const bool live = head < a.heads && token0 + t < a.tokens;   // wave-uniform
        const float *x = a.x + ((size_t)(live ? token0 + t : 0) * a.heads + (live ? head : 0)) * D;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j) {
            const uint32_t i = lane + 64 * j;
            const bool ok = live && i < half;
            lo[t][j] = ok ? x[i] : 0.0f;
            hi[t][j] = ok ? x[half + i] : 0.0f;
        }
    }
    for (uint32_t q = threadIdx.x; q < TB * a.rope_pairs; q += blockDim.x) {
        const uint32_t t = q / a.rope_pairs, i = q - t * a.rope_pairs;
        const float pos = (float)(a.abs_pos + token0 + t);
        const float angle = pos * powf(a.rope_base, -2.0f * (float)i / (float)D);
        float sn, cs;
        sincosf(angle, &sn, &cs);
        rot[t][i] = make_float2(cs, sn);
    }
    __syncthreads();
    if (head >= a.heads)
        return;
#pragma unroll
    for (int t = 0; t < TB; ++t) {
        if (token0 + t >= a.tokens)
            break;
        float ss = 0.0f;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j)
            ss += lo[t][j] * lo[t][j] + hi[t][j] * hi[t][j];
        ss = wave_sum(ss);
        const float inv = 1.0f / sqrtf(ss / (float)D + a.eps);
        float *y = a.y + (size_t)(token0 + t) * a.out_token_stride + (size_t)head * a.out_head_stride;
#pragma unroll
        for (int j = 0; j < kMaxPerLane; ++j) {
            const uint32_t i = lane + 64 * j;
            if (i >= half)
                continue;
            const float wl = a.has_weight ? bf16_weight(a.w, i) : 1.0f;
            const float wh = a.has_weight ? bf16_weight(a.w, half + i) : 1.0f;
            float u = lo[t][j] * inv * wl, v = hi[t][j] * inv * wh;
            if (i < a.rope_pairs) {
                const float2 r = rot[t][i];
                const float u2 = u * r.x - v * r.y;
                const float v2 = u * r.y + v * r.x;
                u = u2;
                v = v2;
            }
            y[i] = u;
            y[half + i] = v;
        }
    }
}

} // namespace

hipError_t rms_norm_launch(const RmsNormArgs &a, hipStream_t stream) {
    if (a.rows == 0 || a.n == 0)
        return hipSuccess;
    hipLaunchKernelGGL(rms_norm_kernel, dim3(a.rows), dim3(256), 0, stream, a);
    return hipGetLastError();
}

hipError_t head_norm_rope_launch(const HeadNormRopeArgs &a, hipStream_t stream) {
    if (a.tokens == 0 || a.heads == 0)
        return hipSuccess;
    if (a.head_dim == 0 || a.head_dim % 2 || a.head_dim > kHeadNormMaxDim || a.rope_pairs > a.head_dim / 2)
        return hipErrorInvalidValue;
    const uint32_t hpb = a.heads >= 16 ? 16 : 8;
    const uint64_t groups = (a.heads + hpb - 1) / hpb;
    const dim3 grid((uint32_t)((a.tokens + kTokensPerBlock - 1) / kTokensPerBlock * groups));
    if (hpb == 16)
        hipLaunchKernelGGL(head_norm_rope_kernel<16>, grid, dim3(64 * 16), 0, stream, a);
    else
        hipLaunchKernelGGL(head_norm_rope_kernel<8>, grid, dim3(64 * 8), 0, stream, a);
    return hipGetLastError();
}

} // namespace apex_hip
