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
#include <algorithm>
#include "gemv.h"
#include "nvfp4_device.h"

namespace apex_hip {
namespace gemv_detail {


constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
// Tokens per block with the fused RMSNorm: the per-token sums stay in registers, and the
// wider blocks of the fp32 kernel are already at the register limit.
constexpr int kMaxNormTokens = 2;


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

// Loads go through buffer descriptors spanning exactly the matrix, so they need no
// branches or clamps: a row set past the last row reads zeros.  Keeping the loads
// straight-line lets the compiler count outstanding loads exactly and keep the next
// row sets' loads in flight while the current one is computed.  Slot s sits at a
// fixed immediate offset s*G*16 (codes) and s*G*2 (scales) from the lane's base,
// except the last slot, whose offset adders `last_c`/`last_s` are out of range for
// lanes past the end of the row, so those lanes read zero codes and zero scales.
template <int SLOTS, int G>
__device__ __forceinline__ void load_row(RowRegs<SLOTS> &r, __amdgpu_buffer_rsrc_t rc,
                                         __amdgpu_buffer_rsrc_t rs, uint32_t row, int gl,
                                         uint32_t K, uint32_t last_c, uint32_t last_s) {
    const uint32_t co = row * (K / 2) + (uint32_t)gl * 16;
    const uint32_t so = row * (K / 16) + (uint32_t)gl * 2;
#pragma unroll
    for (int s = 0; s < SLOTS - 1; ++s) {
        r.codes[s] = load_b128<APEX_WEIGHT_CPOL>(rc, co + s * G * 16);
        r.scales[s] = load_u16<APEX_WEIGHT_CPOL>(rs, so + s * G * 2);
    }
    r.codes[SLOTS - 1] = load_b128<APEX_WEIGHT_CPOL>(rc, co + last_c);
    r.scales[SLOTS - 1] = load_u16<APEX_WEIGHT_CPOL>(rs, so + last_s);
}

// x pieces of one chunk for one token: 16-byte piece p holds elements [8p, 8p+8)
// (bf16) or [4p, 4p+4) (fp32) of the chunk.
template <typename XT> struct XChunk {
    u32x4_t p[XTraits<XT>::kPieces];
};

template <typename XT>
__device__ __forceinline__ XChunk<XT> lds_chunk(const uint4 *xl, int nchunks, int c) {
    XChunk<XT> x;
#pragma unroll
    for (int p = 0; p < XTraits<XT>::kPieces; ++p)
        x.p[p] = __builtin_bit_cast(u32x4_t, xl[p * nchunks + c]);
    return x;
}

// The two E4M3 scales of a chunk (bytes 0 and 1 of `sc`).  The packed hardware
// conversion is exact for every code except 0x7F/0xFF, which it maps to NaN where the
// reference decodes +-480; a row that meets one comes out NaN and is recomputed with
// the exact integer decode (see compute_row_set).
template <bool EXACT>
__device__ __forceinline__ f32x2_t chunk_scales(uint32_t sc) {
    if constexpr (EXACT)
        return f32x2_t{e4m3_to_f32(sc), e4m3_to_f32(sc >> 8)};
    else
        return __builtin_amdgcn_cvt_pk_f32_fp8((int)sc, false);
}

// One chunk (32 weights in `cw`, block scales `s`) dotted with x into acc: per
// 16-element block an unscaled fp32 partial, then acc += scale * partial
// (shaders/matmul.metal:38-46 order).
__device__ __forceinline__ void chunk_dot(const u32x4_t &cw, f32x2_t s,
                                          const XChunk<uint16_t> &x, float &acc) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        float partial = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int p = 2 * b + h;
            bf16x2_t w[4];
            e2m1x8_to_bf16(cw[p], w);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                // Copy the lane out of the vector first: __builtin_bit_cast applied
                // directly to an ext-vector element reads element 0 (clang 22).
                const uint32_t xw = x.p[p][j];
                partial = __builtin_amdgcn_fdot2_f32_bf16(w[j], __builtin_bit_cast(bf16x2_t, xw),
                                                          partial, false);
            }
        }
        acc = __builtin_fmaf(s[b], partial, acc);
    }
}

__device__ __forceinline__ void chunk_dot(const u32x4_t &cw, f32x2_t s, const XChunk<float> &x,
                                          float &acc) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        float partial = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int wi = 2 * b + h;
            f32x2_t w[4];
            e2m1x8_to_f32(cw[wi], w);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4_t &xp = x.p[2 * wi + j / 2];
                partial = __builtin_fmaf(w[j][0], __uint_as_float(xp[(2 * j) % 4]), partial);
                partial = __builtin_fmaf(w[j][1], __uint_as_float(xp[(2 * j) % 4 + 1]), partial);
            }
        }
        acc = __builtin_fmaf(s[b], partial, acc);
    }
}

// Accumulate all chunks of the row set whose loads are in `r`, then sum over the
// group.  Lanes past the end of a row hold zero codes and scales and read a zero x
// chunk, so they add exactly 0.
template <bool EXACT, typename XT, int G, int SLOTS, int TT, int NMAT, bool XREG>
__device__ __forceinline__ void row_set_sums(float (&acc)[NMAT][TT], const RowRegs<SLOTS> (&r)[NMAT],
                                             const XChunk<XT> (&xr)[SLOTS], const uint4 *lds_x,
                                             int plane, int nchunks, int gl) {
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
            acc[m][tt] = 0.0f;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int c = gl + s * G;
        const int cx = c < nchunks ? c : nchunks; // entry nchunks of each LDS plane is zero
        f32x2_t sc[NMAT];
#pragma unroll
        for (int m = 0; m < NMAT; ++m)
            sc[m] = chunk_scales<EXACT>(r[m].scales[s]);
#pragma unroll
        for (int tt = 0; tt < TT; ++tt) {
            XChunk<XT> x;
            if constexpr (XREG)
                x = xr[s];
            else
                x = lds_chunk<XT>(lds_x + tt * plane, nchunks + 1, cx);
#pragma unroll
            for (int m = 0; m < NMAT; ++m)
                chunk_dot(r[m].codes[s], sc[m], x, acc[m][tt]);
        }
    }
#pragma unroll
    for (int m = 0; m < NMAT; ++m)
#pragma unroll
        for (int tt = 0; tt < TT; ++tt)
            acc[m][tt] = group_sum<G>(acc[m][tt]);
}

// Row sums (reduced over the group, one per token) of the row set whose loads are in
// `r`, for one matrix.  A NaN sum means a 0x7F/0xFF scale (or a NaN in x) was met:
// the row set is then recomputed with the exact decode.
template <typename XT, int G, int SLOTS, int TT>
__device__ __forceinline__ void row_set_result(float (&acc)[1][TT], const RowRegs<SLOTS> (&r)[1],
                                               const uint4 *lds_x, int plane, int nchunks,
                                               int gl) {
    const XChunk<XT> no_xr[SLOTS] = {};
    row_set_sums<false, XT, G, SLOTS, TT, 1, false>(acc, r, no_xr, lds_x, plane, nchunks, gl);
    bool nan = false;
#pragma unroll
    for (int tt = 0; tt < TT; ++tt)
        nan |= __builtin_isnan(acc[0][tt]);
    if (nan)
        row_set_sums<true, XT, G, SLOTS, TT, 1, false>(acc, r, no_xr, lds_x, plane, nchunks, gl);
}

// Output element of a plain GEMV (MODE 0: fp32, MODE 1: bf16).
template <int MODE>
__device__ __forceinline__ void store_plain(const GemvArgs &a, size_t o, float v) {
    if constexpr (MODE == 0)
        static_cast<float *>(a.out)[o] = v * a.tensor_scale[0];
    else
        static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_bits(v * a.tensor_scale[0]);
}

// MODE: 0 plain fp32 out, 1 plain bf16 out, 2 GeGLU bf16 out, 3 GeGLU fp32 out.
//
// Work units are row sets (R = 64/G rows).  Wave w of workgroup b owns the sets
// b*4 + w + j*step (j < kmax, step = 4*grid).  Plain GEMVs store each row's result at
// once.  GeGLU walks gate set j, then up set j, then gate set j+1, ...: the wave holds
// both sums of its rows and applies gelu_tanh(gate) * up in registers
// (shaders/geglu.metal:15-23) -- 0.7-0.8 % faster than walking all gate sets, then all
// up sets, with the sums meeting in LDS behind a barrier.
//
// x is staged per block of TT tokens in LDS, piece-major.  The staging loads are
// issued first, then the first DEPTH-1 row sets' weight loads, and only then does the
// wave wait -- for the x loads alone -- write LDS and meet the barrier, so the weight
// latency overlaps the staging.
template <typename XT, int MODE, int G, int SLOTS, int TT, int DEPTH>
__global__ __launch_bounds__(kThreads) void nvfp4_gemv_kernel(GemvArgs a) {
    constexpr int NM = (MODE >= 2) ? 2 : 1; // matrices
    constexpr int R = 64 / G;
    constexpr int PIECES = XTraits<XT>::kPieces;
    // entries per token plane <= PIECES * (SLOTS*G + 1); staging loads per thread:
    constexpr int NX = (TT * PIECES * (SLOTS * G + 1) + kThreads - 1) / kThreads;
    extern __shared__ uint4 lds_x[];

    const int nchunks = (int)(a.K / 32);
    const int lane = threadIdx.x & 63;
    const int wave = (int)__builtin_amdgcn_readfirstlane((uint32_t)threadIdx.x >> 6);
    const int sub = lane / G;
    const int gl = lane % G;
    const uint32_t nsets = (a.rows + R - 1) / R;
    const int stride_c = nchunks + 1;    // LDS entries per piece plane
    const int plane = PIECES * stride_c; // LDS entries per token
    const uint32_t kmax = a.sets_per_wave;
    const uint32_t total_k = NM * kmax;  // iterations of every wave
    static_assert(NM == 1 || DEPTH % 2 == 0, "GeGLU pairs iterations 2j (gate) and 2j + 1 (up)");

    __amdgpu_buffer_rsrc_t rc[NM], rs[NM];
#pragma unroll
    for (int m = 0; m < NM; ++m) {
        rc[m] = make_rsrc(a.codes[m], a.rows * (a.K / 2));
        rs[m] = make_rsrc(a.scales[m], a.rows * (a.K / 16));
    }

    const uint32_t base = blockIdx.x * kWaves + wave;
    const uint32_t step = gridDim.x * kWaves;
    // A row at or past a.rows lies outside the buffer descriptors: its loads read zeros
    // without touching memory.  Prefetches past the end use it.
    const uint32_t oob_row = a.rows + sub;
    // Offsets of the last slot: out of range (>= 2^31 > any descriptor size) for
    // lanes whose last chunk lies past the end of the row.
    const bool last_ok = gl + (SLOTS - 1) * G < nchunks;
    const uint32_t last_c = last_ok ? (SLOTS - 1) * G * 16 : 0x80000000u;
    const uint32_t last_s = last_ok ? (SLOTS - 1) * G * 2 : 0x80000000u;

    // Iteration k's matrix and row set: one matrix, set base + k * step; GeGLU, gate then
    // up of each set in turn (matrix k % 2, set base + (k / 2) * step), so a wave holds
    // both sums of a row and applies the activation in registers.
    auto matrix_of = [&](uint32_t k) { return NM == 2 ? (k & 1u) : 0u; };
    auto set_of = [&](uint32_t k) { return base + (NM == 2 ? k >> 1 : k) * step; };
    // Loads of iteration k into `r`.
    auto issue = [&](RowRegs<SLOTS> &r, uint32_t k) {
        const uint32_t m = matrix_of(k);
        const uint32_t set = set_of(k);
        const uint32_t row = (k < total_k && set < nsets) ? set * R + sub : oob_row;
        load_row<SLOTS, G>(r, rc[NM == 2 ? m : 0], rs[NM == 2 ? m : 0], row, gl, a.K, last_c,
                           last_s);
    };

    RowRegs<SLOTS> buf[DEPTH][1];
    for (uint32_t t0 = 0; t0 < a.tokens; t0 += TT) {
        // 1. staging loads of x[t0 .. t0+TT): thread-linear entry q = tt*plane +
        //    c*PIECES + p (natural order); the zero chunk c = nchunks and tokens past
        //    the end fall outside the descriptor and read zeros.
        const uint32_t ntok = min((uint32_t)TT, a.tokens - t0);
        const __amdgpu_buffer_rsrc_t rx =
            make_rsrc(static_cast<const XT *>(a.x) + (size_t)t0 * a.K,
                      ntok * a.K * (uint32_t)sizeof(XT));
        u32x4_t xv[NX];
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int q = threadIdx.x + i * kThreads;
            const int tt = q / plane;
            const int rem = q - tt * plane;
            const int c = rem / PIECES;
            const int p = rem - c * PIECES;
            const uint32_t off = (c < nchunks && tt < TT)
                                     ? ((uint32_t)tt * a.K * (uint32_t)sizeof(XT) +
                                        (uint32_t)(c * PIECES + p) * 16)
                                     : 0x80000000u;
            xv[i] = load_b128(rx, off);
        }
        // 2. first iterations' weights
        __syncthreads(); // readers of the previous token block are done with LDS
#pragma unroll
        for (int i = 0; i < DEPTH - 1; ++i)
            issue(buf[i][0], i);
        // 3'. fp32 x with norm_w: RMSNorm of each token row on the staged pieces (piece p
        //     of chunk c holds elements 32c + 4p .. +3), x * inv * w -- the rmsNormCpu order
        if constexpr (sizeof(XT) == 4 && TT <= kMaxNormTokens) {
            if (a.norm_w) {
                __shared__ float red[kMaxNormTokens][kWaves];
                float ss[TT] = {};
#pragma unroll
                for (int i = 0; i < NX; ++i) {
                    const int q = threadIdx.x + i * kThreads;
                    const int tt = q / plane, c = (q - tt * plane) / PIECES;
                    if (q < TT * plane && c < nchunks)
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float v = __uint_as_float(xv[i][e]);
#pragma unroll
                            for (int u = 0; u < TT; ++u)
                                if (u == tt)
                                    ss[u] += v * v;
                        }
                }
#pragma unroll
                for (int u = 0; u < TT; ++u) {
                    const float w = group_sum<64>(ss[u]);
                    if (lane == 0)
                        red[u][wave] = w;
                }
                __syncthreads();
                float inv[TT];
#pragma unroll
                for (int u = 0; u < TT; ++u) {
                    float tot = 0.0f;
#pragma unroll
                    for (int w = 0; w < kWaves; ++w)
                        tot += red[u][w];
                    inv[u] = 1.0f / sqrtf(tot / (float)a.K + a.norm_eps);
                }
#pragma unroll
                for (int i = 0; i < NX; ++i) {
                    const int q = threadIdx.x + i * kThreads;
                    const int tt = q / plane, rem = q - tt * plane;
                    const int c = rem / PIECES, p = rem - c * PIECES;
                    if (q < TT * plane && c < nchunks) {
                        float s = 0.0f;
#pragma unroll
                        for (int u = 0; u < TT; ++u)
                            if (u == tt)
                                s = inv[u];
                        const uint16_t *w = a.norm_w + 32 * c + 4 * p;
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            xv[i][e] = __float_as_uint(__uint_as_float(xv[i][e]) * s *
                                                       bf16_bits_to_f32(w[e]));
                    }
                }
            }
        }
        // 3. x into LDS, piece-major: entry tt*plane + p*stride_c + c
#pragma unroll
        for (int i = 0; i < NX; ++i) {
            const int q = threadIdx.x + i * kThreads;
            if (q < TT * plane) {
                const int tt = q / plane;
                const int rem = q - tt * plane;
                const int c = rem / PIECES;
                const int p = rem - c * PIECES;
                lds_x[tt * plane + p * stride_c + c] = __builtin_bit_cast(uint4, xv[i]);
            }
        }
        __syncthreads();

        // DEPTH-stage pipeline over rotating register sets: while iteration k is
        // computed, the loads of k+1 .. k+DEPTH-1 are in flight.  The body is unrolled
        // DEPTH times so every buffer index is a constant and the compiler can count
        // outstanding loads exactly; it is straight-line for the same reason.
        float gate[TT]; // GeGLU: the gate sums of the current set, until its up sums
        for (uint32_t k0 = 0; k0 < total_k; k0 += DEPTH) {
#pragma unroll
            for (int i = 0; i < DEPTH; ++i) {
                const uint32_t k = k0 + i;
                if ((total_k % DEPTH) != 0 && k >= total_k)
                    break;
                issue(buf[(i + DEPTH - 1) % DEPTH][0], k + DEPTH - 1);
                // A set past the last one read zeros and is computed all the same (its
                // stores are dropped below).  With a branch around the compute, the
                // compiler's load counting could not tell whether buffer i's loads had
                // been consumed on every path and waited for them before issuing the
                // next set's: one set in flight instead of two (22.5 vs 21.6 us on the
                // 130 MB decode GeGLU).
                const uint32_t set = set_of(k);
                // x stays in LDS, read per set: hoisted into registers it costs
                // occupancy, and spills for fp32 x and several tokens.
                asm volatile("" ::: "memory");
                float acc[1][TT];
                row_set_result<XT, G, SLOTS, TT>(acc, buf[i], lds_x, plane, nchunks, gl);
                if (gl != 0)
                    continue;
                const uint32_t row = set * R + sub;
                if constexpr (NM == 1) {
                    if (row < a.rows) {
#pragma unroll
                        for (int tt = 0; tt < TT; ++tt)
                            if (t0 + tt < a.tokens)
                                store_plain<MODE>(a, (size_t)(t0 + tt) * a.out_stride + row,
                                                  acc[0][tt]);
                    }
                } else if (i % 2 == 0) {
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt)
                        gate[tt] = acc[0][tt] * a.tensor_scale[0];
                } else if (row < a.rows) {
                    // gelu(gate) * up (shaders/geglu.metal:15-23)
#pragma unroll
                    for (int tt = 0; tt < TT; ++tt) {
                        if (t0 + tt >= a.tokens)
                            continue;
                        const float h = gelu_tanh(gate[tt]) * (acc[0][tt] * a.tensor_scale[1]);
                        const size_t o = (size_t)(t0 + tt) * a.out_stride + row;
                        if constexpr (MODE == 2)
                            static_cast<uint16_t *>(a.out)[o] = f32_to_bf16_bits(h);
                        else
                            static_cast<float *>(a.out)[o] = h;
                    }
                }
            }
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
hipError_t launch_fast(const GemvArgs &args, int nchunks, hipStream_t stream) {
    constexpr int R = 64 / G;
    const uint32_t nsets = (args.rows + R - 1) / R;
    // Persistent grid of about kTargetWavesPerCU waves per CU; every wave gets the
    // same count of row sets per matrix (the last ones may get one fewer).
    const uint32_t target = (uint32_t)kTargetWavesPerCU.load(std::memory_order_relaxed) *
                          (uint32_t)num_cus();
    const uint32_t per_wave = (nsets + target - 1) / target;
    const uint32_t waves = (nsets + per_wave - 1) / per_wave;
    const uint32_t grid = (waves + kWaves - 1) / kWaves;
    const uint32_t kmax = (nsets + grid * kWaves - 1) / (grid * kWaves);
    const size_t lds = (size_t)TT * XTraits<XT>::kPieces * (nchunks + 1) * 16;
    if (lds > 65536)
        return hipErrorInvalidValue;
    GemvArgs a = args;
    a.sets_per_wave = kmax;
    // two row sets in flight per wave (depth 3 measured slower at every occupancy)
    hipLaunchKernelGGL((nvfp4_gemv_kernel<XT, MODE, G, SLOTS, TT, 2>), dim3(grid),
                       dim3(kThreads), lds, stream, a);
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
    // buffer descriptors address at most 2^31 bytes per matrix
    bool fast = (a.K % 32 == 0) && nchunks <= 4 * 64 && (uint64_t)a.rows * (a.K / 2) < (1ull << 31);
    for (int m = 0; m < ((MODE >= 2) ? 2 : 1); ++m)
        fast = fast && ((uintptr_t)a.codes[m] % 16 == 0) && ((uintptr_t)a.scales[m] % 2 == 0);
    fast = fast && ((uintptr_t)a.x % 16 == 0);
    if (!fast && a.norm_w)
        return hipErrorInvalidValue; // the fused RMSNorm lives in the staged-x kernel only
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
    if (a.norm_w)
        tt = std::min(tt, (uint32_t)kMaxNormTokens);
    switch (tt) {
    case 1: return dispatch_shape<XT, MODE, 1>(a, nchunks, stream);
    case 2: return dispatch_shape<XT, MODE, 2>(a, nchunks, stream);
    case 4: return dispatch_shape<XT, MODE, 4>(a, nchunks, stream);
    default: return dispatch_shape<XT, MODE, 8>(a, nchunks, stream);
    }
}

} // namespace gemv_detail
} // namespace apex_hip
