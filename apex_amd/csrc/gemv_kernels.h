// NVFP4 GEMV kernel templates for the decode regime (few tokens), gfx950.
// Included by the per-variant instantiation units gemv_*.hip.
//
// Computes out[t, r] = sum_k W[r, k] * x[t, k] for an NVFP4 matrix W [rows, K] (the
// op of shaders/matmul.metal:4-53 and src/tests/cpu_ref.h:48-63), optionally for two
// matrices at once with the GeGLU epilogue gelu_tanh(gate.x) * (up.x)
// (shaders/geglu.metal:6-24 fused into the producer).
//
// The work is bandwidth-bound: 0.5625 byte of weights per multiply-add.  Design:
//  * A chunk is 32 consecutive K elements: one 16-byte code load (4 words) plus the
//    chunk's two scale bytes.  A group of G lanes (G = 64, 32, 16 or 8) owns one row;
//    lane g of a group owns chunks g, g+G, g+2G, ... (SLOTS of them), so every wave
//    load instruction streams contiguous 16-byte pieces of a row.
//  * All code/scale loads of a row set are issued before any arithmetic and the next
//    row set's loads are issued before the current one is computed (two register
//    buffers), keeping ~2 x 3 KiB per wave in flight.
//  * x is staged once per workgroup in LDS in a piece-major layout (piece p of every
//    chunk is contiguous) so the 16-byte LDS reads of a wave are bank-conflict free.
//  * bf16 activations: v_cvt_scalef32_pk_bf16_fp4 (2 weights/instr) + v_dot2c_f32_bf16
//    (2 MACs/instr) -> ~1 VALU op per weight.  fp32 activations (the reference's fp32
//    contract): v_cvt_scalef32_pk_f32_fp4 + fp32 FMA.
//  * Per 16-element block the unscaled partial sum is multiplied by the block's E4M3
//    scale, as the reference kernel does (shaders/matmul.metal:38-46); group sums use
//    DPP; the per-tensor fp32 scale is applied in the epilogue.
#pragma once
#include "gemv.h"
#include "nvfp4_device.h"

namespace apex_hip {
namespace gemv_detail {


constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;

template <typename XT> struct XTraits;
template <> struct XTraits<float> {
    static constexpr int kPieces = 8; // 16-byte pieces per 32-element chunk
};
template <> struct XTraits<uint16_t> {
    static constexpr int kPieces = 4;
};

// One matrix-row's loads for all slots of a lane.
template <int SLOTS> struct RowRegs {
    u32x4_t codes[SLOTS];
    uint32_t scales[SLOTS];
};

template <int SLOTS, int G>
__device__ __forceinline__ void load_row(RowRegs<SLOTS> &r, const uint32_t *codes,
                                         const uint8_t *scales, uint32_t row, bool row_ok,
                                         int gl, int nchunks, uint32_t K) {
    const u32x4_t *crow = reinterpret_cast<const u32x4_t *>(codes + (size_t)row * (K / 8));
    const uint16_t *srow = reinterpret_cast<const uint16_t *>(scales + (size_t)row * (K / 16));
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int c = gl + s * G;
        if (row_ok && c < nchunks) {
            r.codes[s] = __builtin_nontemporal_load(crow + c);
            r.scales[s] = srow[c];
        } else {
            r.codes[s] = u32x4_t{0, 0, 0, 0};
            r.scales[s] = 0;
        }
    }
}

// Accumulate one chunk (32 weights in `cw`, scale bytes in `sc`) against token tt's x.
__device__ __forceinline__ float chunk_dot(const u32x4_t &cw, uint32_t sc, const uint4 *xl,
                                           int nchunks, int c, uint16_t) {
    const uint32_t words[4] = {cw[0], cw[1], cw[2], cw[3]};
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        float partial = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int p = 2 * b + h;
            const uint4 xv = xl[p * nchunks + c];
            bf16x2_t w[4];
            e2m1x8_to_bf16(words[p], w);
            const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                partial = __builtin_amdgcn_fdot2_f32_bf16(w[j], __builtin_bit_cast(bf16x2_t, xs[j]),
                                                          partial, false);
        }
        acc = __builtin_fmaf(e4m3_to_f32(sc >> (8 * b)), partial, acc);
    }
    return acc;
}

__device__ __forceinline__ float chunk_dot(const u32x4_t &cw, uint32_t sc, const uint4 *xl,
                                           int nchunks, int c, float) {
    const uint32_t words[4] = {cw[0], cw[1], cw[2], cw[3]};
    float acc = 0.0f;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        float partial = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int wi = 2 * b + h;
            f32x2_t w[4];
            e2m1x8_to_f32(words[wi], w);
            const uint4 x0 = xl[(2 * wi) * nchunks + c];
            const uint4 x1 = xl[(2 * wi + 1) * nchunks + c];
            const float xs[8] = {__uint_as_float(x0.x), __uint_as_float(x0.y),
                                 __uint_as_float(x0.z), __uint_as_float(x0.w),
                                 __uint_as_float(x1.x), __uint_as_float(x1.y),
                                 __uint_as_float(x1.z), __uint_as_float(x1.w)};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                partial = __builtin_fmaf(w[j][0], xs[2 * j], partial);
                partial = __builtin_fmaf(w[j][1], xs[2 * j + 1], partial);
            }
        }
        acc = __builtin_fmaf(e4m3_to_f32(sc >> (8 * b)), partial, acc);
    }
    return acc;
}

// MODE: 0 plain fp32 out, 1 plain bf16 out, 2 GeGLU bf16 out, 3 GeGLU fp32 out.
template <typename XT, int MODE, int G, int SLOTS, int TT>
__global__ __launch_bounds__(kThreads) void nvfp4_gemv_kernel(GemvArgs a) {
    constexpr int NMAT = (MODE >= 2) ? 2 : 1;
    constexpr int R = 64 / G;
    constexpr int PIECES = XTraits<XT>::kPieces;
    extern __shared__ uint4 lds_x[];

    const int nchunks = (int)(a.K / 32);
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane / G;
    const int gl = lane % G;
    const uint32_t nsets = (a.rows + R - 1) / R;
    const uint32_t wave_stride = gridDim.x * kWaves;
    const uint32_t first_set = blockIdx.x * kWaves + wave;
    const int plane = PIECES * nchunks; // uint4 entries per token in LDS

    for (uint32_t t0 = 0; t0 < a.tokens; t0 += TT) {
        // Stage x[t0 .. t0+TT) piece-major: entry (tt*PIECES + p)*nchunks + c holds
        // bytes [16p, 16p+16) of chunk c of token t0+tt.
        __syncthreads();
        const int total = TT * plane;
        for (int q = threadIdx.x; q < total; q += kThreads) {
            const int tt = q / plane;
            const int rem = q - tt * plane;
            const int c = rem / PIECES;
            const int p = rem - c * PIECES;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (t0 + tt < a.tokens)
                v = reinterpret_cast<const uint4 *>(static_cast<const XT *>(a.x) +
                                                    (size_t)(t0 + tt) * a.K)[rem];
            lds_x[(tt * PIECES + p) * nchunks + c] = v;
        }
        __syncthreads();

        RowRegs<SLOTS> cur[NMAT], nxt[NMAT];
        uint32_t set = first_set;
        if (set < nsets) {
            const uint32_t row = set * R + sub;
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                load_row<SLOTS, G>(cur[m], a.codes[m], a.scales[m], row, row < a.rows, gl,
                                   nchunks, a.K);
        }
        for (; set < nsets; set += wave_stride) {
            const uint32_t row = set * R + sub;
            const uint32_t next = set + wave_stride;
            if (next < nsets) {
                const uint32_t nrow = next * R + sub;
#pragma unroll
                for (int m = 0; m < NMAT; ++m)
                    load_row<SLOTS, G>(nxt[m], a.codes[m], a.scales[m], nrow, nrow < a.rows,
                                       gl, nchunks, a.K);
            }
            float acc[NMAT][TT];
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int tt = 0; tt < TT; ++tt)
                    acc[m][tt] = 0.0f;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const int c = gl + s * G;
                if (c < nchunks) {
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt) {
                        const uint4 *xl = lds_x + tt * plane;
#pragma unroll
                        for (int m = 0; m < NMAT; ++m)
                            acc[m][tt] += chunk_dot(cur[m].codes[s], cur[m].scales[s], xl,
                                                    nchunks, c, XT());
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
#pragma unroll
                for (int tt = 0; tt < TT; ++tt)
                    acc[m][tt] = group_sum<G>(acc[m][tt]);
            if (gl == 0 && row < a.rows) {
#pragma unroll
                for (int tt = 0; tt < TT; ++tt) {
                    const uint32_t t = t0 + tt;
                    if (t >= a.tokens)
                        break;
                    const size_t o = (size_t)t * a.out_stride + row;
                    if constexpr (MODE == 0) {
                        static_cast<float *>(a.out)[o] = acc[0][tt] * a.tensor_scale[0];
                    } else if constexpr (MODE == 1) {
                        static_cast<uint16_t *>(a.out)[o] =
                            f32_to_bf16_bits(acc[0][tt] * a.tensor_scale[0]);
                    } else {
                        const float g = acc[0][tt] * a.tensor_scale[0];
                        const float u = acc[1][tt] * a.tensor_scale[1];
                        const float h = gelu_tanh(g) * u;
                        if constexpr (MODE == 2)
                            static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_bits(h);
                        else
                            static_cast<float *>(a.out)[o] = h;
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                cur[m] = nxt[m];
        }
    }
}

// Generic path for any K % 16 == 0 and any 4-byte-aligned codes: one wave per row,
// lanes stride over 16-element blocks (the reference kernel's mapping with 64 lanes).
template <typename XT, int MODE>
__global__ __launch_bounds__(kThreads) void nvfp4_gemv_generic_kernel(GemvArgs a) {
    constexpr int NMAT = (MODE >= 2) ? 2 : 1;
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * kWaves + (threadIdx.x >> 6);
    const uint32_t t = blockIdx.y;
    if (row >= a.rows || t >= a.tokens)
        return;
    const uint32_t nblk = a.K / 16;
    const XT *x = static_cast<const XT *>(a.x) + (size_t)t * a.K;
    float acc[NMAT];
#pragma unroll
    for (int m = 0; m < NMAT; ++m) {
        const uint32_t *crow = a.codes[m] + (size_t)row * (a.K / 8);
        const uint8_t *srow = a.scales[m] + (size_t)row * nblk;
        float dot = 0.0f;
        for (uint32_t b = lane; b < nblk; b += 64) {
            const uint32_t lo = crow[2 * b], hi = crow[2 * b + 1];
            float partial = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float xv0, xv1;
                if constexpr (sizeof(XT) == 2) {
                    xv0 = bf16_bits_to_f32(x[16 * b + j]);
                    xv1 = bf16_bits_to_f32(x[16 * b + 8 + j]);
                } else {
                    xv0 = x[16 * b + j];
                    xv1 = x[16 * b + 8 + j];
                }
                const f32x2_t wl = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(lo >> (4 * j), 1.0f, 0);
                const f32x2_t wh = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(hi >> (4 * j), 1.0f, 0);
                partial = __builtin_fmaf(wl[0], xv0, partial);
                partial = __builtin_fmaf(wh[0], xv1, partial);
            }
            dot = __builtin_fmaf(e4m3_to_f32(srow[b]), partial, dot);
        }
        acc[m] = group_sum<64>(dot);
    }
    if (lane == 0) {
        const size_t o = (size_t)t * a.out_stride + row;
        if constexpr (MODE == 0) {
            static_cast<float *>(a.out)[o] = acc[0] * a.tensor_scale[0];
        } else if constexpr (MODE == 1) {
            static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_bits(acc[0] * a.tensor_scale[0]);
        } else {
            const float h = gelu_tanh(acc[0] * a.tensor_scale[0]) * (acc[NMAT - 1] * a.tensor_scale[NMAT - 1]);
            if constexpr (MODE == 2)
                static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_bits(h);
            else
                static_cast<float *>(a.out)[o] = h;
        }
    }
}

// ----------------------------------------------------------------------------
// Launch configuration
// ----------------------------------------------------------------------------

struct Shape {
    int G, SLOTS;
};

// Lanes per row and chunks per lane for a given chunk count: the fewest wasted lane
// slots, preferring wide groups (fewer reductions) on ties; SLOTS <= 4.
inline Shape pick_shape(int nchunks) {
    Shape best{64, 4};
    int best_waste = 1 << 30;
    for (int G : {64, 32, 16, 8}) {
        const int slots = (nchunks + G - 1) / G;
        if (slots > 4)
            continue;
        const int waste = slots * G - nchunks;
        if (waste < best_waste) {
            best_waste = waste;
            best = {G, slots};
        }
    }
    return best;
}

template <typename XT, int MODE, int G, int SLOTS, int TT>
hipError_t launch_fast(const GemvArgs &a, int nchunks, hipStream_t stream) {
    constexpr int R = 64 / G;
    const uint32_t nsets = (a.rows + R - 1) / R;
    // Balanced persistent grid: about kTargetWaves waves, each with the same count of
    // row sets (the last wave may have fewer).
    const uint32_t target = (uint32_t)kTargetWavesPerCU * (uint32_t)kNumCUs;
    const uint32_t per_wave = (nsets + target - 1) / target;
    const uint32_t waves = (nsets + per_wave - 1) / per_wave;
    const uint32_t grid = (waves + kWaves - 1) / kWaves;
    const size_t lds = (size_t)TT * XTraits<XT>::kPieces * nchunks * 16;
    hipLaunchKernelGGL((nvfp4_gemv_kernel<XT, MODE, G, SLOTS, TT>), dim3(grid), dim3(kThreads),
                       lds, stream, a);
    return hipGetLastError();
}

template <typename XT, int MODE, int TT>
hipError_t dispatch_shape(const GemvArgs &a, int nchunks, hipStream_t stream) {
    const Shape s = pick_shape(nchunks);
#define APEX_SHAPE(g, sl)                                                                          \
    if (s.G == g && s.SLOTS == sl)                                                                 \
        return launch_fast<XT, MODE, g, sl, TT>(a, nchunks, stream);
    APEX_SHAPE(64, 1) APEX_SHAPE(64, 2) APEX_SHAPE(64, 3) APEX_SHAPE(64, 4)
    APEX_SHAPE(32, 1) APEX_SHAPE(32, 2) APEX_SHAPE(32, 3) APEX_SHAPE(32, 4)
    APEX_SHAPE(16, 1) APEX_SHAPE(16, 2) APEX_SHAPE(16, 3) APEX_SHAPE(16, 4)
    APEX_SHAPE(8, 1) APEX_SHAPE(8, 2) APEX_SHAPE(8, 3) APEX_SHAPE(8, 4)
#undef APEX_SHAPE
    return hipErrorInvalidValue;
}

template <typename XT, int MODE>
hipError_t gemv_dispatch(const GemvArgs &a, hipStream_t stream) {
    const int nchunks = (int)(a.K / 32);
    bool fast = (a.K % 32 == 0) && nchunks <= 4 * 64;
    for (int m = 0; m < ((MODE >= 2) ? 2 : 1); ++m)
        fast = fast && ((uintptr_t)a.codes[m] % 16 == 0) && ((uintptr_t)a.scales[m] % 2 == 0);
    fast = fast && ((uintptr_t)a.x % 16 == 0);
    if (!fast) {
        dim3 grid((a.rows + kWaves - 1) / kWaves, a.tokens);
        hipLaunchKernelGGL((nvfp4_gemv_generic_kernel<XT, MODE>), grid, dim3(kThreads), 0, stream,
                           a);
        return hipGetLastError();
    }
    // Tokens per pass: the next power of two >= tokens (at most 8) whose x block fits
    // a 32 KiB LDS budget; one token always fits (K <= 8192 here).
    const size_t per_token = (size_t)a.K * sizeof(XT);
    uint32_t tt = 1;
    while (tt < a.tokens && tt < 8)
        tt *= 2;
    while (tt > 1 && tt * per_token > 32768)
        tt /= 2;
    switch (tt) {
    case 1: return dispatch_shape<XT, MODE, 1>(a, nchunks, stream);
    case 2: return dispatch_shape<XT, MODE, 2>(a, nchunks, stream);
    case 4: return dispatch_shape<XT, MODE, 4>(a, nchunks, stream);
    default: return dispatch_shape<XT, MODE, 8>(a, nchunks, stream);
    }
}

} // namespace gemv_detail
} // namespace apex_hip
