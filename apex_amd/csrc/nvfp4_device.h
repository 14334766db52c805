// Device-side NVFP4 decode helpers for gfx950 (CDNA4).
//
// Format (src/nvfp4.h:27-43, shaders/quant.h:7-23): a row of K weights is K/8 uint32
// code words -- element 8w+i is nibble i (LSB first) of word w -- and K/16 FP8 E4M3
// scale bytes, one per 16-element block.  w = e2m1(code) * e4m3(scale).
//
// Decode strategy (measured on gfx950):
//  * v_cvt_scalef32_pk_{f32,bf16}_fp4 turns one byte (two nibbles, low nibble first)
//    into two values with the OCP E2M1 table, which is the reference's table
//    including code 8 -> -0.0.  Its scale operand contributes only its exponent
//    (0.75 acts as 0.5), so it is always passed 1.0 and the E4M3 block scale is
//    applied separately, in fp32.
//  * E4M3 scales decode with an integer construction that has no NaN encoding, so
//    0x7F / 0xFF give +-480 exactly as the reference's decoder does (the hardware
//    fp8 conversion would give NaN there).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace apex_hip {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// Buffer resource over [base, base + bytes): raw buffer loads through it are range
// checked by the hardware -- a lane whose offset falls outside returns 0 and never
// faults -- so tails need no branches.  Word 3 is the gfx9 default descriptor format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// Cache-policy bits of the weight-stream loads (the buffer instruction's aux field).
#ifndef APEX_WEIGHT_CPOL
#define APEX_WEIGHT_CPOL 2 // nt: the weights are streamed once
#endif

template <int CPOL = 0>
__device__ __forceinline__ u32x4_t load_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, CPOL));
}

template <int CPOL = 0>
__device__ __forceinline__ uint32_t load_u16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, (int)off, 0, CPOL);
}

// E4M3 byte (in the low 8 bits of `b`) -> fp32, reference semantics.
// Magnitude bits 0eeeemmm placed at float bits 20..26 give 2^(e-127) * (1 + m/8) for
// e > 0 and the fp32 denormal m * 2^-129 for e == 0; multiplying by 2^120 (exact)
// yields (1 + m/8) * 2^(e-7) and m/512.  0x7F -> 1.875 * 2^8 = 480.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
    const float mag = __uint_as_float((b & 0x7Fu) << 20) * 0x1p120f;
    return __uint_as_float(__float_as_uint(mag) | ((b & 0x80u) << 24));
}

// The same construction without the final 2^120: E4M3 byte -> 2^-120 times its value
// (a normal or denormal fp32, sign included).  Paired with e2m1x8_to_f32_x2p120 -- the
// codes converted with the power-of-two 2^120 in the conversion's scale operand -- the
// product code * scale is the same exact fp32 value with one multiply fewer per scale.
__device__ __forceinline__ float e4m3_to_f32_x2m120(uint32_t b) {
    return __uint_as_float(((b & 0x7Fu) << 20) | ((b & 0x80u) << 24));
}

// Eight E2M1 codes of one word -> four bf16 pairs (elements 2j, 2j+1 in pair j).
__device__ __forceinline__ void e2m1x8_to_bf16(uint32_t w, bf16x2_t out[4]) {
    out[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 0);
    out[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 1);
    out[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 2);
    out[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, 1.0f, 3);
}

// Eight E2M1 codes of one word -> eight fp32 values.
__device__ __forceinline__ void e2m1x8_to_f32(uint32_t w, f32x2_t out[4]) {
    out[0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 0);
    out[1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 1);
    out[2] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 2);
    out[3] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 1.0f, 3);
}

// Eight E2M1 codes of one word -> eight fp32 values times 2^120 (exact: the scale
// operand is a power of two, which the conversion applies as an exponent offset).
__device__ __forceinline__ void e2m1x8_to_f32_x2p120(uint32_t w, f32x2_t out[4]) {
    out[0] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 0x1p120f, 0);
    out[1] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 0x1p120f, 1);
    out[2] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 0x1p120f, 2);
    out[3] = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, 0x1p120f, 3);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
    return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).  Branch-free: both
// results are formed and one is selected.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t rounded = (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
    const uint32_t quiet = (u >> 16) | 0x40u;
    return (uint16_t)(__builtin_isnan(f) ? quiet : rounded);
}

// GeLU, tanh approximation, fp32 constants of shaders/geglu.metal:15-16:
// 0.5 g (1 + tanh(u)), u = 0.7978845608028654 (g + 0.044715 g^3), evaluated through the
// identity 0.5 (1 + tanh(u)) = 1 / (1 + exp(-2u)) -- one exponential and one division
// instead of a tanh.  exp overflowing to +inf gives g / inf = -0 (the limit).
__device__ __forceinline__ float gelu_tanh(float g) {
    const float u = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    return g / (1.0f + __expf(-2.0f * u));
}

// The same function for GEMM epilogues, where it runs once per output element: the
// constants folded into one base-2 exponent, -2 u log2(e) = g (k1 + k2 g^2), then
// v_exp_f32 and v_rcp_f32 (each about 1 ulp) instead of a correctly rounded division;
// a few fp32 ulps from gelu_tanh, with the same limits (+inf exponent -> g * 0 = -0).
__device__ __forceinline__ float gelu_tanh_fast(float g) {
    constexpr float k1 = -2.0f * 1.4426950408889634f * 0.7978845608028654f;
    constexpr float k2 = k1 * 0.044715f;
    const float t = g * __builtin_fmaf(k2, g * g, k1);
    return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// Sum over aligned groups of G lanes (G in {8, 16, 32, 64}) of a wave64; every lane
// of a group receives the group total.  DPP within rows of 16, then cross-row swaps.
// v(l) + v(l ^ 16) and v(l) + v(l ^ 32) by VALU lane swaps (v_permlane16_swap swaps the
// odd rows of its first operand with the even rows of its second, v_permlane32_swap
// the upper half of the first with the lower half of the second; with both operands
// v, lane l of the two results holds v(l) and its partner in row order).  Both lanes
// of a pair add the same two values in the same order, so they agree bit for bit.
__device__ __forceinline__ float add_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
    static_assert(G == 8 || G == 16 || G == 32 || G == 64, "group size");
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)); // row_half_mirror
    if constexpr (G >= 16)
        v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)); // row_mirror
    if constexpr (G >= 32)
        v = add_xor16(v);
    if constexpr (G >= 64)
        v = add_xor32(v);
    return v;
}

} // namespace apex_hip
