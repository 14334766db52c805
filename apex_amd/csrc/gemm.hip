// NVFP4 prefill GEMMs for gfx950, fp32 accumulation:
//   plain  C[M,N] = A[M,K] . W[N,K]^T (x tensor_scale)
//   GeGLU  C[M,N] = gelu(A . G^T) * (A . U^T), gate and up in one tile
// with A bf16 -- or fp32 activations split into bf16 hi + lo halves -- W NVFP4 (codes
// uint32 [N, K/8], E4M3 scales [N, K/16]) and C bf16 or fp32.
//
// The reference computes prefill as one GEMV per token (src/ops.h:44, grid.y =
// tokens, shaders/matmul.metal:18); here it is a dense MFMA contraction on 256 x 256
// tiles (gemm_core.h: W dequantised exactly to bf16 in registers from LDS-staged codes,
// v_mfma_f32_32x32x16_bf16, fp32 accumulation).  A GeGLU tile's 256 W rows are 128
// gate and 128 up rows of the same 128 output columns, interleaved by 32, so each wave
// holds both halves of its outputs and the activation is applied before the store.
//
// fp32 activations (the reference's fp32 contract, src/ops.h:34-46): x = hi + lo + r
// with hi, lo bf16 and |r| <= 2^-17 |x|; A = [hi | lo] along K (2K columns) and W's K
// position wraps at K, so one tile loop sums hi . w + lo . w.  Every W element is
// exact in bf16 and every bf16 product exact in fp32, so the result carries fp32
// accumulation error plus r (rel ~1e-6), inside the reference's 1e-5 gate; it costs
// twice the MFMA work of a bf16 GEMM and one pass over X.
//
// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so
// workgroup g works on tile (g % 8) * tiles_per_xcd + g / 8, tiles M-fastest: the tiles
// resident on one XCD share A row blocks and W column blocks in its L2.  Loads use
// buffer descriptors: rows past M or N read zeros; stores are guarded.
#include "gemm.h"
#include "gemm_core.h"
#include "gemv.h"
#include "lds_attr.h"

#include <algorithm>

namespace apex_hip {
namespace {

using namespace gemm_core;
constexpr int WC = 4;                     // 1 x 4 waves (the 2 x 2 layout measured slower)
constexpr int MT = 8;                     // 32-row MFMA tiles per wave
constexpr int BM = Layout<MT, WC>::kBM;   // 256
constexpr uint32_t kGegluCols = BN / 2;   // output columns of a GeGLU tile

template <bool GEGLU, bool F32> __device__ __forceinline__ bool uniform_wide(const GemmArgs &a) {
    // 16-byte stores: 8 bf16 or 4 fp32 columns at 16-byte aligned addresses
    constexpr uint32_t q = F32 ? 4 : 8;
    return a.N % q == 0 && a.ldc % q == 0 && ((uintptr_t)a.C & 15) == 0;
}

// One tile of C: rows [m0, m0 + 256), W tile rows n0 + w_row(r) for r < 32 NTW WCW
// (plain: output columns n0 .. n0 + 32 NTW WCW - 1; GeGLU: h columns n0 .. n0 + 16 NTW
// WCW - 1).  The
// 256 x 256 tile is the 1 x 4 layout (MT 8, NTW 8); a narrow tile is the 4 x 1 layout,
// each wave on 64 rows and all NTW W blocks (MT 2): the same 256 A rows per stage, the
// decode of each W element 4 times (once per wave) but the tile as short as its width.
template <bool GEGLU, bool F32, int MTW, int WCW, int NTW, int VPM>
__device__ __forceinline__ void gemm_one_tile(const GemmArgs &a, uint8_t *lds, uint32_t m0,
                                              uint32_t n0) {
    const uint32_t K = a.K, ak = a.a_k;
    const uint32_t M = a.M, N = a.N;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, M * ak * 2);
    const __amdgpu_buffer_rsrc_t rc[2] = {make_rsrc(a.codes[0], N * (K / 2)),
                                          make_rsrc(a.codes[GEGLU ? 1 : 0], N * (K / 2))};
    const __amdgpu_buffer_rsrc_t rs[2] = {make_rsrc(a.scales[0], N * (K / 16)),
                                          make_rsrc(a.scales[GEGLU ? 1 : 0], N * (K / 16))};
    auto a_row = [=](int r) { return m0 + r < M ? (m0 + r) * ak * 2 : kOut; };
    // W tile row r -> row of its matrix: plain n0 + r; GeGLU n0 + 32 (r / 64) + r % 32
    // (the matrix, (r / 32) % 2, is the descriptor's); rows past the tile's width read
    // nothing
    auto w_row = [=](int r) { return GEGLU ? n0 + 32 * (r / 64) + r % 32 : n0 + r; };
    auto w_ok = [=](int r) { return r < 32 * NTW * WCW && w_row(r) < N; };
    auto w_code = [=](int r) { return w_ok(r) ? w_row(r) * (K / 2) : kOut; };
    auto w_scale = [=](int r) { return w_ok(r) ? w_row(r) * (K / 16) : kOut; };

    // bf16 A: chunked W loads; fp32 [hi | lo] A meets W twice, wrapping at K, which a
    // 2-stage code chunk may straddle: per-stage W there
    Acc<MTW, WCW, NTW> acc;
    gemm_tile<MTW, WCW, NTW, VPM, F32 ? 4 : 0>(lds, ra, rc, rs, ak, a_row, w_code, w_scale, acc, K);

    const bool wide = uniform_wide<GEGLU, F32>(a);
    if constexpr (GEGLU) {
        using OutT = std::conditional_t<F32, float, uint16_t>;
        store_tile_geglu<MTW, OutT, WCW, NTW>(acc, static_cast<OutT *>(a.C) + (size_t)m0 * a.ldc,
                                              a.ldc, M - m0, n0, N, a.tensor_scale[0],
                                              a.tensor_scale[1], wide);
    } else if constexpr (F32) {
        store_tile_f32<MTW, WCW, NTW>(acc, static_cast<float *>(a.C), a.ldc, m0, n0, M, N,
                                      a.tensor_scale[0], wide);
    } else {
        store_tile_bf16<MTW, WCW, NTW>(acc, static_cast<uint16_t *>(a.C), a.ldc, m0, n0, M, N,
                                       a.tensor_scale[0], wide);
    }
}

// A whole tile's 16 MFMAs per step leave room for its 2 fragments' decode at 2 VALU ops
// after each (2: 370.6 / 370.5 us, 3: 373.1 / 372.6, 4: 376.1 / 375.8 at 2048 x 21504 x
// 5376, same box).
constexpr int kWholeVpm = 2;
// A narrow tile's 2 NT MFMAs per step share NT fragments' decode: up to 8 VALU ops after
// each (3 and 5 measured the same).
constexpr int kNarrowVpm = 8;
constexpr uint32_t kNarrowMaxBlocks = 2; // widest narrow tile (32-row W blocks)
constexpr uint32_t kShortMaxBlocks = 6;  // tallest short tile worth running (32-row blocks)

// Workgroups [0, G_full): the 256 x 256 tiles of n-tiles [0, nf), XCD-aware (workgroup g
// on tile (g % 8) * per_xcd + g / 8, tiles M-fastest: the tiles resident on one XCD
// share A row blocks and W column blocks in its L2).  Workgroups past G_full: the tail
// columns past nf n-tiles, either as narrow tiles (nt = 1 or 2 W blocks each; GeGLU 2:
// one gate and one up block) or as ns short tiles (full-width 1 x 4 tiles of at most
// kShortMaxBlocks 32-row blocks of one column, short_tile), dealt the same way; they fill the CUs of
// the last round, which whole tiles would leave partly empty.
template <bool GEGLU, bool F32>
__device__ __forceinline__ void short_gemm_tile(const GemmArgs &a, uint8_t *lds, uint32_t blocks,
                                                uint32_t m0, uint32_t n0) {
    static_assert(kShortMaxBlocks == 6, "one case per short tile height");
    switch (blocks) {
    case 6: gemm_one_tile<GEGLU, F32, 6, WC, 2, 3>(a, lds, m0, n0); break;
    case 5: gemm_one_tile<GEGLU, F32, 5, WC, 2, 3>(a, lds, m0, n0); break;
    case 4: gemm_one_tile<GEGLU, F32, 4, WC, 2, 3>(a, lds, m0, n0); break;
    case 3: gemm_one_tile<GEGLU, F32, 3, WC, 2, 3>(a, lds, m0, n0); break;
    case 2: gemm_one_tile<GEGLU, F32, 2, WC, 2, 3>(a, lds, m0, n0); break;
    default: gemm_one_tile<GEGLU, F32, 1, WC, 2, 3>(a, lds, m0, n0); break;
    }
}

template <bool GEGLU, bool F32>
__global__ __launch_bounds__(kThreads) void nvfp4_gemm_kernel(GemmArgs a, uint32_t nf, uint32_t nt,
                                                              uint32_t ns) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr uint32_t TN = GEGLU ? kGegluCols : BN;
    const uint32_t tiles_m = (a.M + BM - 1) / BM;
    const uint32_t full = tiles_m * nf;
    const uint32_t g_full = 8 * ((full + 7) / 8);
    if (blockIdx.x < g_full) {
        const uint32_t per_xcd = g_full / 8;
        const uint32_t t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
        if (t >= full)
            return;
        gemm_one_tile<GEGLU, F32, MT, WC, 8 / WC, kWholeVpm>(a, lds, (t % tiles_m) * BM, (t / tiles_m) * TN);
        return;
    }
    const uint32_t c_tail = nf * TN;
    const uint32_t u = blockIdx.x - g_full;
    if (ns) {
        // consecutive short tiles (mostly of one column) on one XCD: they share W in its L2
        const uint32_t per_xcd = (ns + 7) / 8;
        const uint32_t v = (u % 8) * per_xcd + u / 8;
        if (v >= ns)
            return;
        const uint32_t C = (a.N - c_tail + TN - 1) / TN, B = (a.M + 31) / 32;
        const ShortTile st = short_tile(v, ns, C, B);
        short_gemm_tile<GEGLU, F32>(a, lds, st.blocks, 32 * st.block0, c_tail + st.col * TN);
        return;
    }
    const uint32_t tc = GEGLU ? 16 * nt : 32 * nt; // output columns of a narrow tile
    const uint32_t tiles = tiles_m * ((a.N - c_tail + tc - 1) / tc);
    const uint32_t per_xcd = (tiles + 7) / 8;
    const uint32_t t = (u % 8) * per_xcd + u / 8;
    if (t >= tiles)
        return;
    const uint32_t m0 = (t % tiles_m) * BM, n0 = c_tail + (t / tiles_m) * tc;
    if (GEGLU || nt == 2)
        gemm_one_tile<GEGLU, F32, 2, 1, 2, kNarrowVpm>(a, lds, m0, n0);
    else
        gemm_one_tile<false, F32, 2, 1, 1, kNarrowVpm>(a, lds, m0, n0);
}

// The last round of whole tiles: with tiles = R * ncu + rem (0 < rem, R >= 1), whole
// tiles cover the first nf = R * ncu / tiles_m n-tiles and narrow tiles of nt W blocks
// the remaining columns, nt the smallest width whose tiles fit in the CUs left after
// the whole tiles' R rounds plus one more round -- if that width is at most 2 blocks
// (GeGLU: 2).  The narrow tiles are decode-bound (each wave decodes every W element of
// the tile for its 64 rows): measured at 2048 x 21504 x 5376, a round of 2-block tiles
// took 0.73 of a whole-tile round (the GeGLU GEMM 835 -> 795 us), a round of 5-block
// tiles 1.16 (404 -> 426 us), so wider narrow tiles are not used.  Where no narrow
// width fits, short tiles (full width, contiguous 32-row block ranges of one tail
// column, at most kShortMaxBlocks blocks) take the last round's CUs, one each: at
// 2048 x 21504 x 5376 (20 tail columns of 64 blocks on 256 CUs, 5-6 blocks each) 407 ->
// 403 us.  nt = ns = 0: whole tiles only.
GemmTailPlan plan_tail(uint32_t M, uint32_t N, bool geglu, uint32_t ncu) {
    const uint32_t tn = geglu ? kGegluCols : BN;
    const uint32_t tiles_m = (M + BM - 1) / BM, tiles_n = (N + tn - 1) / tn;
    const uint64_t tiles = (uint64_t)tiles_m * tiles_n;
    GemmTailPlan p{tiles_n, 0, 0};
    if (ncu == 0 || tiles <= ncu || tiles % ncu == 0)
        return p;
    const uint64_t R = tiles / ncu;
    const uint32_t nf = (uint32_t)(R * ncu / tiles_m);
    if (nf == 0 || nf >= tiles_n)
        return p;
    const uint64_t cols = N - (uint64_t)nf * tn;
    const uint64_t slots = (R + 1) * ncu - (uint64_t)tiles_m * nf;
    for (uint32_t nt = geglu ? 2 : 1; nt <= kNarrowMaxBlocks; ++nt) {
        const uint64_t tc = geglu ? 16 * nt : 32 * nt;
        if (tiles_m * ((cols + tc - 1) / tc) <= slots)
            return GemmTailPlan{nf, nt, 0};
    }
    // Short tiles: the tail columns' 32-row blocks dealt over the last round's CUs; worth
    // it when no tile needs more than kShortMaxBlocks blocks (a whole tile has 8).
    const uint64_t C = (cols + tn - 1) / tn, B = (M + 31) / 32;
    if (slots >= C && slots <= 0xFFFFFFFFull) {
        const uint64_t q = slots / C;
        if ((B + q - 1) / q <= kShortMaxBlocks) // at most C * B tiles: none empty
            return GemmTailPlan{nf, 0, (uint32_t)std::min(slots, C * B)};
    }
    return p;
}

template <bool GEGLU, bool F32> hipError_t launch_kernel(const GemmArgs &a, hipStream_t stream) {
    const GemmTailPlan p = plan_tail(a.M, a.N, GEGLU, (uint32_t)num_cus());
    const uint32_t tiles_m = (a.M + BM - 1) / BM;
    uint32_t grid = 8 * ((tiles_m * p.nf + 7) / 8);
    if (p.nt) {
        const uint32_t tc = GEGLU ? 16 * p.nt : 32 * p.nt;
        const uint32_t c_tail = p.nf * (GEGLU ? kGegluCols : BN);
        grid += 8 * ((tiles_m * ((a.N - c_tail + tc - 1) / tc) + 7) / 8);
    } else if (p.ns) {
        grid += 8 * ((p.ns + 7) / 8);
    }
    constexpr size_t lds = kMaxLds;
    static std::atomic<uint64_t> attr_set{0};
    if (hipError_t e = allow_dynamic_lds(nvfp4_gemm_kernel<GEGLU, F32>, lds, attr_set); e != hipSuccess)
        return e;
    hipLaunchKernelGGL((nvfp4_gemm_kernel<GEGLU, F32>), dim3(grid), dim3(kThreads), lds, stream, a,
                       p.nf, p.nt, p.ns);
    return hipGetLastError();
}

// ---- split-K ------------------------------------------------------------------

// GeGLU partials of a tile: acc[i][0] (gate) / acc[i][1] (up) of h columns c0 + 32 wave
// + 8 (e / 4) + 4 (lane / 32) + e % 4, token row m0 + 32 i + lane % 32, into gate / up
// [M, N] fp32.
template <int MT>
__device__ __forceinline__ void store_geglu_partials(const Acc<MT, 4> &acc, float *gate, float *up,
                                                     uint32_t M, uint32_t N, uint32_t m0,
                                                     uint32_t c0) {
    const int lane = threadIdx.x & 63;
    const uint32_t wcol = c0 + 32 * (threadIdx.x >> 6);
    const uint32_t row = lane & 31;
    const uint64_t bytes = (uint64_t)(M - m0) * N * 4;
    const uint32_t nb = bytes < 0x80000000ull ? (uint32_t)bytes : 0x7FFFFFF0u;
    const __amdgpu_buffer_rsrc_t rd[2] = {make_rsrc(gate + (size_t)m0 * N, nb),
                                          make_rsrc(up + (size_t)m0 * N, nb)};
    const bool wide = N % 4 == 0;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t c = wcol + 8 * g + 4 * (lane >> 5);
                const uint32_t ro = (row + 32 * i) * N;
                if (wide) {
                    const u32x4_t v = {__float_as_uint(acc[i][j][4 * g]),
                                       __float_as_uint(acc[i][j][4 * g + 1]),
                                       __float_as_uint(acc[i][j][4 * g + 2]),
                                       __float_as_uint(acc[i][j][4 * g + 3])};
                    __builtin_amdgcn_raw_buffer_store_b128(v, rd[j], (int)(c < N ? (ro + c) * 4 : kOut),
                                                           0, 0);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        __builtin_amdgcn_raw_buffer_store_b32(
                            __float_as_uint(acc[i][j][4 * g + e]), rd[j],
                            (int)(c + e < N ? (ro + c + e) * 4 : kOut), 0, 0);
                }
            }
}

// Workgroup b: tile b / S, split b % S.  Split s of a tile covers the stages
// [s nh / Sh, (s + 1) nh / Sh) of half s / Sh (Sh = S / halves splits per half of nh
// stages; one half for bf16 A, two -- hi, lo -- for split fp32 A), so its W columns
// are its A columns less K in the lo half.
template <bool GEGLU>
__global__ __launch_bounds__(kThreads) void nvfp4_gemm_splitk_kernel(GemmArgs a, float *part,
                                                                     uint32_t S) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    constexpr uint32_t TN = GEGLU ? kGegluCols : BN;
    const uint32_t tiles_m = (a.M + BM - 1) / BM;
    const uint32_t t = blockIdx.x / S, s = blockIdx.x % S;
    const uint32_t m0 = (t % tiles_m) * BM;
    const uint32_t n0 = (t / tiles_m) * TN;

    const uint32_t K = a.K, ak = a.a_k;
    const uint32_t M = a.M, N = a.N;
    const uint32_t halves = ak / K;
    const uint32_t sh_n = S / halves, nh = K / BK;
    const uint32_t half = s / sh_n, sh = s % sh_n;
    const uint32_t st0 = sh * nh / sh_n, st1 = (sh + 1) * nh / sh_n;
    const uint32_t kw0 = st0 * BK;              // W column of the split's first stage
    const uint32_t ka0 = half * K + kw0;        // A column
    const uint32_t len = (st1 - st0) * BK;

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, M * ak * 2);
    const __amdgpu_buffer_rsrc_t rc[2] = {make_rsrc(a.codes[0], N * (K / 2)),
                                          make_rsrc(a.codes[GEGLU ? 1 : 0], N * (K / 2))};
    const __amdgpu_buffer_rsrc_t rs[2] = {make_rsrc(a.scales[0], N * (K / 16)),
                                          make_rsrc(a.scales[GEGLU ? 1 : 0], N * (K / 16))};
    auto a_row = [=](int r) { return m0 + r < M ? ((m0 + r) * ak + ka0) * 2 : kOut; };
    auto w_row = [=](int r) { return GEGLU ? n0 + 32 * (r / 64) + r % 32 : n0 + r; };
    auto w_code = [=](int r) { return w_row(r) < N ? w_row(r) * (K / 2) + kw0 / 2 : kOut; };
    auto w_scale = [=](int r) { return w_row(r) < N ? w_row(r) * (K / 16) + kw0 / 16 : kOut; };

    Acc<MT, WC> acc;
    gemm_tile<MT, WC>(lds, ra, rc, rs, len, a_row, w_code, w_scale, acc);

    const size_t mn = (size_t)M * N;
    if constexpr (GEGLU)
        store_geglu_partials<MT>(acc, part + (2 * s) * mn, part + (2 * s + 1) * mn, M, N, m0, n0);
    else
        store_tile_f32<MT, WC>(acc, part + s * mn, N, m0, n0, M, N, 1.0f,
                               N % 4 == 0);
}

// C = epilogue(sum over s = 0 .. S-1 of the partials, in that order).
template <bool GEGLU, bool F32>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *part, uint32_t S, GemmArgs a) {
    const size_t mn = (size_t)a.M * a.N;
    for (size_t q = blockIdx.x * 256ull + threadIdx.x; q < mn; q += (size_t)gridDim.x * 256) {
        float v;
        if constexpr (GEGLU) {
            float g = 0.0f, u = 0.0f;
            for (uint32_t s = 0; s < S; ++s) {
                g += part[2 * s * mn + q];
                u += part[(2 * s + 1) * mn + q];
            }
            v = gelu_tanh_fast(g * a.tensor_scale[0]) * (u * a.tensor_scale[1]);
        } else {
            float acc = 0.0f;
            for (uint32_t s = 0; s < S; ++s)
                acc += part[s * mn + q];
            v = acc * a.tensor_scale[0];
        }
        const size_t m = q / a.N, n = q - m * a.N;
        const size_t o = m * a.ldc + n;
        if constexpr (F32)
            static_cast<float *>(a.C)[o] = v;
        else
            static_cast<uint16_t *>(a.C)[o] = f32_to_bf16_bits(v);
    }
}

template <bool GEGLU> hipError_t launch_splitk(const GemmArgs &a, uint32_t S, float *part,
                                               hipStream_t stream) {
    constexpr uint32_t TN = GEGLU ? kGegluCols : BN;
    const uint32_t tiles = ((a.M + BM - 1) / BM) * ((a.N + TN - 1) / TN);
    constexpr size_t lds = Layout<MT, WC>::kLds;
    static std::atomic<uint64_t> attr_set{0};
    if (hipError_t e = allow_dynamic_lds(nvfp4_gemm_splitk_kernel<GEGLU>, lds, attr_set); e != hipSuccess)
        return e;
    hipLaunchKernelGGL((nvfp4_gemm_splitk_kernel<GEGLU>), dim3(tiles * S), dim3(kThreads), lds,
                       stream, a, part, S);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    const size_t mn = (size_t)a.M * a.N;
    const uint32_t grid = (uint32_t)std::min<size_t>((mn + 255) / 256, 256 * 8);
    if (a.out_f32)
        hipLaunchKernelGGL((splitk_reduce_kernel<GEGLU, true>), dim3(grid), dim3(256), 0, stream,
                           part, S, a);
    else
        hipLaunchKernelGGL((splitk_reduce_kernel<GEGLU, false>), dim3(grid), dim3(256), 0, stream,
                           part, S, a);
    return hipGetLastError();
}

// One workgroup per row: optional RMS statistics, then hi / lo of every element.  Rows
// of up to 256 * kSplitQuads * 4 elements (16-byte aligned x, 8-byte aligned norm_w)
// stay in registers, read with 16-byte loads and written as 8-byte pieces of 4 bf16;
// other rows take the element loop.
constexpr int kSplitThreads = 256;
constexpr int kSplitQuads = 8;

__device__ __forceinline__ uint16_t bf16_rne(float x) { return f32_to_bf16_bits(x); }

// hi / lo of one value (lo = 0 where hi is not finite)
__device__ __forceinline__ void split_one(float v, uint16_t &h, uint16_t &l) {
    h = bf16_rne(v);
    const float hf = __uint_as_float((uint32_t)h << 16);
    l = __builtin_isfinite(hf) ? bf16_rne(v - hf) : (uint16_t)0;
}

__device__ __forceinline__ float block_sum(float v, float *red) {
    v = group_sum<64>(v);
    if ((threadIdx.x & 63) == 0)
        red[threadIdx.x >> 6] = v;
    __syncthreads();
    float total = 0.0f;
#pragma unroll
    for (int w = 0; w < kSplitThreads / 64; ++w)
        total += red[w];
    return total;
}

__global__ __launch_bounds__(kSplitThreads) void split_bf16_kernel(const float *X,
                                                                   const uint16_t *norm_w,
                                                                   float eps, uint16_t *out,
                                                                   uint32_t K) {
    __shared__ float red[kSplitThreads / 64];
    const float *x = X + (size_t)blockIdx.x * K;
    uint16_t *hi = out + (size_t)blockIdx.x * 2 * K;
    uint16_t *lo = hi + K;
    const uint32_t tid = threadIdx.x;
    const bool vec = K % 4 == 0 && K / 4 <= kSplitThreads * kSplitQuads &&
                     (uintptr_t)x % 16 == 0 && (uintptr_t)hi % 8 == 0 &&
                     (!norm_w || (uintptr_t)norm_w % 8 == 0);
    if (vec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x);
        const uint2 *w4 = reinterpret_cast<const uint2 *>(norm_w);
        float4 v[kSplitQuads];
        uint2 wb[kSplitQuads];
#pragma unroll
        for (int r = 0; r < kSplitQuads; ++r) {
            const uint32_t i = tid + kSplitThreads * r;
            const bool ok = i < K / 4;
            v[r] = ok ? x4[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            wb[r] = ok && norm_w ? w4[i] : make_uint2(0, 0);
        }
        if (norm_w) {
            float ss = 0.0f;
#pragma unroll
            for (int r = 0; r < kSplitQuads; ++r)
                ss += v[r].x * v[r].x + v[r].y * v[r].y + v[r].z * v[r].z + v[r].w * v[r].w;
            const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)K + eps);
#pragma unroll
            for (int r = 0; r < kSplitQuads; ++r) {
                v[r].x = v[r].x * inv * __uint_as_float(wb[r].x << 16);
                v[r].y = v[r].y * inv * __uint_as_float(wb[r].x & 0xFFFF0000u);
                v[r].z = v[r].z * inv * __uint_as_float(wb[r].y << 16);
                v[r].w = v[r].w * inv * __uint_as_float(wb[r].y & 0xFFFF0000u);
            }
        }
#pragma unroll
        for (int r = 0; r < kSplitQuads; ++r) {
            const uint32_t i = tid + kSplitThreads * r;
            if (i >= K / 4)
                continue;
            uint16_t h[4], l[4];
            split_one(v[r].x, h[0], l[0]);
            split_one(v[r].y, h[1], l[1]);
            split_one(v[r].z, h[2], l[2]);
            split_one(v[r].w, h[3], l[3]);
            reinterpret_cast<uint2 *>(hi)[i] =
                make_uint2(h[0] | (uint32_t)h[1] << 16, h[2] | (uint32_t)h[3] << 16);
            reinterpret_cast<uint2 *>(lo)[i] =
                make_uint2(l[0] | (uint32_t)l[1] << 16, l[2] | (uint32_t)l[3] << 16);
        }
        return;
    }
    float inv = 1.0f;
    if (norm_w) {
        float ss = 0.0f;
        for (uint32_t k = tid; k < K; k += kSplitThreads)
            ss += x[k] * x[k];
        inv = 1.0f / sqrtf(block_sum(ss, red) / (float)K + eps);
    }
    for (uint32_t k = tid; k < K; k += kSplitThreads) {
        float v = x[k];
        if (norm_w)
            v = v * inv * __uint_as_float((uint32_t)norm_w[k] << 16);
        split_one(v, hi[k], lo[k]);
    }
}

} // namespace

bool gemm_supported(uint32_t M, uint32_t N, uint32_t K, uint32_t a_k, bool out_f32) {
    const uint64_t esz = out_f32 ? 4 : 2;
    return K % BK == 0 && K > 0 && M > 0 && N > 0 && (a_k == K || a_k == 2 * K) &&
           (uint64_t)M * a_k * 2 < (1ull << 31) && (uint64_t)N * (K / 2) < (1ull << 31) &&
           (uint64_t)BM * N * esz < (1ull << 31);
}

GemmTailPlan gemm_tail_plan(uint32_t M, uint32_t N, bool geglu, uint32_t ncu) {
    return plan_tail(M, N, geglu, ncu);
}

hipError_t gemm_launch(const GemmArgs &a, hipStream_t stream) {
    if (!gemm_supported(a.M, a.N, a.K, a.a_k, a.out_f32))
        return hipErrorInvalidValue;
    if (a.geglu)
        return a.out_f32 ? launch_kernel<true, true>(a, stream) : launch_kernel<true, false>(a, stream);
    return a.out_f32 ? launch_kernel<false, true>(a, stream) : launch_kernel<false, false>(a, stream);
}

// Splits when the tiles fill under half the CUs: enough that tiles x S covers the 256
// CUs, each split at least 8 stages, a multiple of the halves of A.
uint32_t gemm_splitk_splits(const GemmArgs &a) {
    const uint32_t tn = a.geglu ? kGegluCols : BN;
    const uint32_t tiles = ((a.M + BM - 1) / BM) * ((a.N + tn - 1) / tn);
    if (tiles >= 128 || a.K == 0 || a.a_k % a.K != 0)
        return 1;
    const uint32_t halves = a.a_k / a.K;
    const uint32_t per_half = (a.K / BK) / 8;   // splits of >= 8 stages in a half
    uint32_t s = std::min((256 + tiles - 1) / tiles, per_half * halves);
    s -= s % halves;
    return s >= 2 ? s : 1;
}

size_t gemm_splitk_bytes(const GemmArgs &a, uint32_t splits) {
    return (size_t)splits * (a.geglu ? 2 : 1) * a.M * a.N * 4;
}

hipError_t gemm_splitk_launch(const GemmArgs &a, uint32_t splits, float *part,
                              hipStream_t stream) {
    if (!gemm_supported(a.M, a.N, a.K, a.a_k, a.out_f32) || splits < 1 ||
        splits % (a.a_k / a.K) != 0 || splits / (a.a_k / a.K) > a.K / BK ||
        (uint64_t)a.M * a.N * 4 >= (1ull << 31))
        return hipErrorInvalidValue;
    return a.geglu ? launch_splitk<true>(a, splits, part, stream)
                   : launch_splitk<false>(a, splits, part, stream);
}

size_t gemm_split_bytes(uint32_t M, uint32_t K) { return (size_t)M * 2 * K * 2; }

hipError_t gemm_split_launch(const float *X, const uint16_t *norm_w, float eps, uint16_t *split,
                             uint32_t M, uint32_t K, hipStream_t stream) {
    if (M == 0 || K == 0)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(split_bf16_kernel, dim3(M), dim3(kSplitThreads), 0, stream, X, norm_w, eps,
                       split, K);
    return hipGetLastError();
}

} // namespace apex_hip
