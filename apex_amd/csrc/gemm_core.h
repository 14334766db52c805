// Tile core of the NVFP4 x bf16 MFMA GEMMs (dense prefill GEMM and the grouped MoE
// expert GEMMs), gfx950.
//
// One workgroup of 4 waves computes a BM x 256 tile of C = A . W^T (BM = 32*MT*(4/WC)):
//   A   bf16 rows (activations), K contiguous, 2*K bytes per row;
//   W   NVFP4 rows (codes: K/2 bytes, E4M3 scales: K/16 bytes per row);
//   C   fp32 accumulators, handed to the caller's epilogue.
// Row addressing is the caller's: `a_row(r)` gives the byte offset of tile row r of A
// inside the A descriptor, `w_code(r)` / `w_scale(r)` the byte offsets of W tile row r
// inside the code / scale descriptors, each 0x80000000 (out of range: reads zeros)
// for rows that do not exist.  That is how the grouped GEMMs gather token rows and
// place gate and up rows side by side.  W tile rows with (r % 64) < 32 are read through
// the descriptors rc[0] / rs[0], the others through rc[1] / rs[1] (gate and up matrices
// in separate buffers; pass the same descriptor twice for one matrix).  W's K position
// is the stage's, less kw_wrap once it reaches kw_wrap: an A of [hi | lo] halves along
// K (2K columns) meets the same W twice.
//
// gfx950's scaled-FP4 MFMA uses MXFP4 (32-element blocks, E8M0 scales), which cannot
// express NVFP4's 16-element E4M3 blocks, so W is dequantised to bf16 -- exactly:
// every e2m1 x e4m3 product has at most 6 significant bits -- and fed to
// v_mfma_f32_32x32x16_bf16 (measured: sustains ~90% of the bf16 peak with one wave per
// SIMD; 16x16x32 only ~55%).
//
//  * (4/WC) x WC waves: wave w owns rows [32 MT (w / WC), +32 MT) and columns
//    [32 NT (w % WC), +32 NT) (NT = 8 / WC) as MT x NT MFMA tiles.  WC = 4 (1 x 4)
//    dequantises every W element once per tile; WC = 2 (2 x 2) halves the A-fragment
//    LDS reads per MFMA and dequantises each W element twice.
//  * A streams HBM/L2 -> LDS with buffer_load ... lds (no VGPR round trip) through a
//    ring of kStages stage buffers, kStages-1 stages ahead of the MFMAs.  A rows are
//    128 bytes per stage with 16-byte pieces XOR-swizzled by (row / 2) % 8, so the 32
//    lanes reading one piece of 32 consecutive rows spread over all banks.
//  * W's packed codes (32 bytes per row per stage) and scales (4 bytes; tile row r at
//    entry 128 ((r / 32) % 2) + 32 (r / 64) + r % 32, so every 64-entry DMA load reads
//    one matrix) stream through LDS buffers of their own, one stage ahead of A: stage
//    s+1's codes and scales are in LDS while stage s runs, so a wave reads them and
//    decodes the scales during steps 1 and 2 of stage s, and the step after the
//    barrier carries only the DMA issue, the next stage's first A fragments and its
//    first dequantisation (with the W reads and the scale decode there too, that step
//    overflowed its MFMAs' issue slots).  W's load cost follows the cache lines a DMA
//    instruction touches more than its bytes: per stage a row's codes are 32 bytes and
//    its scales 4, one line each.  Chunked (WS = 0, bf16 A): codes arrive two stages
//    per load (64 bytes of a row, 16 rows per instruction) and scales four (16 bytes
//    of a row), about 3.5x fewer line touches than one stage per load.  Per stage
//    (WS = 4 buffers): fp32 [hi | lo] A, whose W wraps at K mid-chunk when K / 64 is
//    odd.  Each wave dequantises its B fragments in registers right before its MFMAs
//    (cvt_scalef32_pk_f32_fp4 with 2^120 in the scale operand, x 2^-120 E4M3 scale,
//    keep the exact high halves as bf16).  The packed form keeps W's LDS traffic 4x
//    smaller than a bf16 copy.
//  * K order: within a 64-wide stage, MFMA step q (0..3) and lane half h = lane/32
//    take the 8 k values of piece 4h + q (a permutation of k applied to A and W alike,
//    which leaves the dot products unchanged), so a lane's four code words of a stage
//    are one 16-byte LDS read and span scale blocks 2h, 2h+1.
//  * Software pipeline: the MFMAs of step q run while step q+1's A fragments are read
//    and its B fragments dequantised; one barrier per stage.
#pragma once
#include <type_traits>

#include "nvfp4_device.h"

namespace apex_hip {
namespace gemm_core {

constexpr int kThreads = 256;
constexpr int BK = 64;
constexpr int BN = 256;
constexpr int kARow = BK * 2;              // bytes per A row per stage
constexpr int kStages = 3;                 // ring depth
constexpr int kWCode = BN * (BK / 2);      // 8 KiB of W codes per stage
constexpr int kWScale = BN * (BK / 16);    // 1 KiB of W scales per stage
constexpr uint32_t kOut = 0x80000000u;     // an offset no descriptor covers
// W loads use the default cache policy: a stage takes 32 bytes of each 128-byte code
// line and 4 bytes of each scale line, so a line serves 4 (codes) or 32 (scales)
// consecutive stages and must stay in L2 between them (the streaming policy of the
// GEMV re-fetched the lines: 3.8x the L2 misses on the MoE gate/up GEMM).
constexpr int kWCpol = 0;

// NT (32-row W blocks per wave) defaults to the full 256-row W tile; with WC = 2 and
// NT = 2 only W rows 0..127 are used (the half-width tile: 2 x 2 waves, both wave rows
// on the same 128 W rows), the stage layout staying that of 256 rows.  WS: W's LDS
// buffers -- 0: chunked (two 2-stage code buffers, two 4-stage scale buffers; no K wrap);
// 4: per-stage ring, W loads with the same two stages of latency cover as A's.
constexpr int kCodeChunk = 2 * kWCode;   // 16 KiB: codes of 2 stages, 64 bytes per row
constexpr int kScaleChunk = 4 * kWScale; // 4 KiB: scales of 4 stages, 16 bytes per row
template <int MT, int WC = 4, int NT = 8 / WC, int WS = 0> struct Layout {
    static_assert(WS == 0 || WS == 4, "W buffers");
    static constexpr int kWR = 4 / WC;
    static constexpr int kNT = NT;
    static constexpr int kBM = 32 * MT * kWR;
    static constexpr int kAStage = kBM * kARow;
    static constexpr int kWStage = kWCode + kWScale;
    static constexpr size_t kLds = (size_t)kStages * kAStage +
                                   (WS == 0 ? 2 * (size_t)(kCodeChunk + kScaleChunk) : (size_t)WS * kWStage);
};
constexpr size_t kMaxLds = Layout<8>::kLds > Layout<8, 4, 2, 4>::kLds ? Layout<8>::kLds : Layout<8, 4, 2, 4>::kLds;

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t pack_bf16_hi(float lo, float hi) {
    // e2m1 x e4m3 products are exact in bf16: the low 16 bits of the fp32 are zero,
    // so taking the high halves (bytes 2,3 of lo, then of hi) is exact.
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// The MFMAs take W as their first operand and A as their second, so each 32 x 32
// accumulator holds a block of C^T: element e of MFMA tile (i, j) of wave `wave`, lane
// `lane` sits at tile row 32 MT (wave / WC) + 32 i + lane % 32 and tile column
// 32 NT (wave % WC) + 32 j + 8 (e / 4) + 4 (lane / 32) + e % 4 -- a lane holds runs of
// 4 consecutive columns of one row, which the epilogues pack into 16-byte stores.
template <int MT, int WC = 4, int NT = 8 / WC> using Acc = f32x16_t[MT][NT];

// bf16 output of one accumulator block: `v` (the lane's 16 values, already through any
// elementwise epilogue) -> two 16-byte pieces, piece p = columns 16 p + 8 (lane / 32)
// + 0..7 of the lane's row (lane % 32).  The lane halves hold columns 8 g + 0..3 and
// 8 g + 4..7 of group g; one v_permlane32_swap per register pair hands group 2p+1's
// lower half to the upper lanes and group 2p's upper half to the lower lanes.
// Rounding: v_cvt_pk_bf16_f32, round to nearest even.
__device__ __forceinline__ void pack_bf16_cols(const f32x16_t &v, u32x4_t (&out)[2]) {
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    typedef float f32x2_v __attribute__((ext_vector_type(2)));
    uint32_t pk[4][2];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int q = 0; q < 2; ++q)
            pk[g][q] = __builtin_bit_cast(
                uint32_t, __builtin_convertvector(f32x2_v{v[4 * g + 2 * q], v[4 * g + 2 * q + 1]},
                                                  bf16x2_v));
#pragma unroll
    for (int p = 0; p < 2; ++p) {
#pragma unroll
        for (int q = 0; q < 2; ++q) {
            const auto r = __builtin_amdgcn_permlane32_swap(pk[2 * p][q], pk[2 * p + 1][q], false, false);
            pk[2 * p][q] = r[0];
            pk[2 * p + 1][q] = r[1];
        }
        out[p] = u32x4_t{pk[2 * p][0], pk[2 * p][1], pk[2 * p + 1][0], pk[2 * p + 1][1]};
    }
}

template <int MT, int WC> __device__ __forceinline__ int wave_row0() {
    return 32 * MT * ((threadIdx.x >> 6) / WC);
}
template <int WC, int NT = 8 / WC> __device__ __forceinline__ int wave_col0() {
    return 32 * NT * ((threadIdx.x >> 6) % WC);
}

// VPM: VALU slots after each MFMA in the interleaved schedule (the decode work per MFMA
// grows as MT shrinks: 2 fragments of 16 ops per 2 MT MFMAs).
template <int MT, int WC, int NT = 8 / WC, int VPM = 3, int WS = 0, typename ARow, typename WCode,
          typename WScale>
__device__ __forceinline__ void gemm_tile(uint8_t *lds, __amdgpu_buffer_rsrc_t ra,
                                          const __amdgpu_buffer_rsrc_t (&rc)[2],
                                          const __amdgpu_buffer_rsrc_t (&rs)[2], uint32_t K,
                                          ARow a_row, WCode w_code, WScale w_scale,
                                          Acc<MT, WC, NT> &acc, uint32_t kw_wrap = 0xFFFFFFFFu) {
    static_assert(WC * NT * 32 <= BN, "the waves' W blocks lie in the staged W tile");
    using L = Layout<MT, WC, NT, WS>;
    constexpr int WR = 4 / WC;
    constexpr int kAStage = L::kAStage;
    constexpr int kWStage = L::kWStage;
    constexpr int kARows = 8 * MT * WR;       // A rows each wave copies per stage
    constexpr int kALoads = MT * WR;          // DMA loads of 8 A rows per wave per stage
    constexpr int kLoadsPerStage = kALoads + 2 + 1;
    uint8_t *const wring = lds + kStages * kAStage;
    // Chunked W (WS = 0): code chunk c (stages 2c, 2c+1) in buffer c % 2, scale chunk d
    // (stages 4d .. 4d+3) in buffer d % 2, each issued four stages before its first
    // stage: 4 code loads per wave per chunk, 1 scale load per wave per chunk.
    constexpr bool kChunk = WS == 0;
    constexpr int kCodeLoads = 4;
    // The loads issued after stage s's barrier (window s: W, A(s+3)) are spread over that
    // step and steps 1 and 2 of stage s+1 -- one burst of DMA instructions behind each
    // barrier stalled the waves' issue (measured: two parts 1-2 % faster than one, three
    // parts faster again).  Window s's loads all go out before stage s+1's wait.
    constexpr int kA1 = (kALoads + 2) / 3;          // A loads right after the barrier
    constexpr int kA2 = kA1 + (kALoads - kA1 + 1) / 2; // ... up to here in step 1
    uint8_t *const cring = wring;
    uint8_t *const sring = wring + 2 * kCodeChunk;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // uniform: LDS destinations (M0) and their arithmetic stay in scalar registers
    const int wave = (int)__builtin_amdgcn_readfirstlane((uint32_t)tid >> 6);
    const int wn = wave_col0<WC, NT>();  // wave's column offset in the tile
    const int wm = wave_row0<MT, WC>();  // wave's row offset in the tile
    const int frow = lane & 31;     // fragment row (A) / column (B) within a 32-wide tile
    const int h = lane >> 5;        // lane half: k pieces 4h .. 4h+3 of each stage

    // A: wave w copies rows [kARows w, kARows (w+1)) with DMA loads of 8 rows; lane l
    // lands at row 8i + l/8, physical piece l%8, so it fetches logical piece
    // (l%8) ^ ((row/2)%8) of that row.
    uint32_t a_off[kALoads];
#pragma unroll
    for (int i = 0; i < kALoads; ++i) {
        const int trow = wave * kARows + 8 * i + (lane >> 3);
        const uint32_t ro = a_row(trow);
        a_off[i] = ro == kOut ? kOut : ro + (((lane & 7) ^ ((trow >> 1) & 7)) * 16);
    }
    // W codes: 16-byte slot q of the stage holds half (q%2) ^ ((q/16)%2) of tile row
    // q/2 -- rows 8..15 of every 16 swap halves, so the 16 lanes reading one half of 16
    // consecutive rows hit distinct bank groups; wave w copies slots [128w, 128w+128)
    // with 2 DMA loads (load i: rows 64w + 32i + 0..31, all of matrix i).  Scales: wave w
    // copies entries [64w, 64w+64), 4 bytes each: rows of matrix w / 2.
    uint32_t wc_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = wave * 128 + i * 64 + lane;
        const int trow = q / 2;
        const int half = (q & 1) ^ ((trow >> 3) & 1);
        const uint32_t ro = w_code(trow);
        wc_off[i] = ro == kOut ? kOut : ro + half * 16;
    }
    const int se = wave * 64 + lane;   // scale entry -> tile row
    const uint32_t ws_off = w_scale(64 * ((se % 128) / 32) + 32 * (se / 128) + se % 32);
    // Chunked codes: 16-byte slot q of a chunk holds piece (q%4) ^ ((q/16)%4) of tile row
    // q/4 (piece p = bytes 16p .. 16p+15 of the row's 64: stage 2c + p/2, lane half p%2),
    // so the 16 lanes reading one piece of 16 consecutive rows hit distinct bank groups;
    // wave w copies slots [256w, 256w+256) with 4 DMA loads (load k: rows 64w + 16k +
    // 0..15, all of matrix k/2).
    uint32_t cc_off[kCodeLoads];
#pragma unroll
    for (int k = 0; k < kCodeLoads; ++k) {
        const int q = wave * 256 + k * 64 + lane;
        const int trow = q / 4;
        const int piece = (q & 3) ^ ((trow >> 2) & 3);
        const uint32_t ro = w_code(trow);
        cc_off[k] = ro == kOut ? kOut : ro + piece * 16;
    }

    // The stage's K position rides in the scalar offset: the per-lane offsets are fixed
    // for the whole tile (a valid row plus k0 stays inside its row; an out-of-range
    // lane offset stays out of range).
    auto load_a = [&](int buf, uint32_t k0, int i0, int i1) {
        uint8_t *base = lds + buf * kAStage;
#pragma unroll
        for (int i = i0; i < i1; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (lds_void_t *)(base + (wave * kARows + 8 * i) * kARow), 16, a_off[i],
                (int)(k0 * 2), 0, 0);
    };
    auto load_w = [&](int wbuf, uint32_t k0) {
        uint8_t *base = wring + wbuf * kWStage;
        const uint32_t kw = k0 >= kw_wrap ? k0 - kw_wrap : k0;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rc[i], (lds_void_t *)(base + (wave * 128 + i * 64) * 16), 16, wc_off[i],
                (int)(kw / 2), 0, kWCpol);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs[wave / 2], (lds_void_t *)(base + kWCode + wave * 64 * 4), 4, ws_off,
            (int)(kw / 16), 0, kWCpol);
    };

#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.0f;

    const uint32_t nk = K / BK;
    auto kofs = [&](uint32_t st) { return st < nk ? st * BK : 0u; }; // past the end: harmless re-read
    // A chunk's bytes past the row's last stage (K / 64 not a multiple of the chunk) are
    // the next row's or, past the matrix, zeros: loaded, never read.
    auto load_codes_part = [&](uint32_t c, int k0_, int k1_) {
        uint8_t *base = cring + (c & 1) * kCodeChunk;
        const uint32_t k0 = kofs(2 * c);
#pragma unroll
        for (int k = k0_; k < k1_; ++k)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rc[k >> 1], (lds_void_t *)(base + (wave * 256 + k * 64) * 16), 16, cc_off[k],
                (int)(k0 / 2), 0, kWCpol);
    };
    auto load_scales = [&](uint32_t d) {
        uint8_t *base = sring + (d & 1) * kScaleChunk;
        const uint32_t k0 = kofs(4 * d);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs[wave / 2], (lds_void_t *)(base + wave * 64 * 16), 16,
                                                 ws_off, (int)(k0 / 16), 0, kWCpol);
    };

    // Two register sets of a stage's W: codes (4 words per fragment), raw scale bytes
    // and the decoded scales; set p holds the running stage's, set 1-p is filled with
    // the next stage's during steps 1 and 2.
    u32x4_t wcode[2][NT];
    uint32_t wsraw[2][NT];
    f32x2_t wsc[2][NT];
    bf16x8_v af[2][MT], bf[2][NT];
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    // W of stage x into register set P: rows wn + 32 j + frow, half h (code words
    // 4h .. 4h+3 = scale blocks 2h, 2h+1).
    auto read_w = [&](auto P, uint32_t x) {
        constexpr int p = decltype(P)::value;
        if constexpr (kChunk) {
            const uint8_t *lwc = cring + ((x >> 1) & 1) * kCodeChunk;
            const uint8_t *lws = sring + ((x >> 2) & 1) * kScaleChunk + (x & 3) * 4 + 2 * h;
            const int piece = 2 * (int)(x & 1) + h;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const int r = wn + 32 * j + frow;
                wcode[p][j] = *reinterpret_cast<const u32x4_t *>(lwc + r * 64 + ((piece ^ ((r >> 2) & 3)) * 16));
                const int e = 128 * ((r >> 5) & 1) + 32 * (r >> 6) + (r & 31);
                wsraw[p][j] = *reinterpret_cast<const uint16_t *>(lws + e * 16);
            }
        } else {
            const uint8_t *lwc = wring + (x % WS) * kWStage;
            const uint8_t *lws = lwc + kWCode;
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                // slot 2r + (h ^ ((r/8)%2))
                const int r = wn + 32 * j + frow;
                wcode[p][j] = *reinterpret_cast<const u32x4_t *>(lwc + (2 * r + (h ^ ((r >> 3) & 1))) * 16);
                const int e = 128 * ((r >> 5) & 1) + 32 * (r >> 6) + (r & 31);
                wsraw[p][j] = *reinterpret_cast<const uint16_t *>(lws + e * 4 + 2 * h);
            }
        }
    };
    auto decode_scales = [&](auto P) {
        constexpr int p = decltype(P)::value;
#pragma unroll
        for (int j = 0; j < NT; ++j)
            wsc[p][j] = f32x2_t{e4m3_to_f32_x2m120(wsraw[p][j]), e4m3_to_f32_x2m120(wsraw[p][j] >> 8)};
    };
    // A fragments of step q: rows 32 i + frow, logical piece 4h + q.
    auto read_a = [&](bf16x8_v (&dst)[MT], int buf, int q) {
        const uint8_t *la = lds + buf * kAStage;
        const int piece = 4 * h + q;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int r = wm + i * 32 + frow;
            dst[i] = *reinterpret_cast<const bf16x8_v *>(la + r * kARow + ((piece ^ ((r >> 1) & 7)) * 16));
        }
    };
    // B fragments of step q: word q of each tile's codes (8 weights), scale block 2h + q/2;
    // (code x 2^120) x (scale x 2^-120) is the exact product.
    auto dequant_b = [&](bf16x8_v (&dst)[NT], auto P, int q) {
        constexpr int p = decltype(P)::value;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            f32x2_t v[4];
            e2m1x8_to_f32_x2p120(wcode[p][j][q], v);
            const float sc = wsc[p][j][q >> 1];
            u32x4_t bw;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                bw[e] = pack_bf16_hi(v[e][0] * sc, v[e][1] * sc);
            dst[j] = __builtin_bit_cast(bf16x8_v, bw);
        }
    };
    auto mfmas = [&](const bf16x8_v (&A)[MT], const bf16x8_v (&B)[NT]) {
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int i = 0; i < MT; ++i)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(B[j], A[i], acc[i][j], 0, 0, 0);
    };
    // One MFMA, then up to VPM VALU ops and one LDS read, for the MT*NT MFMAs of a
    // step.  Three slots (the default) leave room for the dequantisation of the MoE's
    // smaller tiles (MT 4 and 2 dequantise 2x and 4x as much per MFMA): 1.4 % faster MoE
    // prefill than two, the same dense GEMM; four was slower.
    auto interleave = [&]() {
#pragma unroll
        for (int m = 0; m < MT * NT; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, VPM, 0); // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
        }
        // Close the region: the next step's MFMAs must not be pulled into this one's
        // slots, or their fragment reads end up right before them (exposed latency).
        __builtin_amdgcn_sched_barrier(0);
    };
    // DMA windows.  A(x) lives in A buffer x % kStages; per-stage W(x) in W buffer x % WS,
    // chunked W as above.  Window s goes out after stage s's barrier and during steps 1
    // and 2 of stage s+1: A(s+3) and the W four stages ahead (per stage: W(s+4), into the
    // buffer whose stage, s+1 or s, was read before the barrier; chunked: after a stage
    // s = 0 mod 4 the scale chunk of stages s+4 .. s+7, after an even one the code chunk
    // of stages s+4, s+5).  Stage x's wait needs A(x+1) and W(x+2), both in window x-2,
    // and leaves window x-1 in flight: two stages of latency cover for every load.
    // The prologue issues windows -4 .. -1 (W(0) alone, then W(1) A(0), W(2) A(1), W(3)
    // A(2)).
    if constexpr (kChunk) {
        load_scales(0);
        load_codes_part(0, 0, kCodeLoads);
        load_a(0, kofs(0), 0, kALoads);
        load_codes_part(1, 0, kCodeLoads);
        load_a(1, kofs(1), 0, kALoads);
        load_a(2, kofs(2), 0, kA1); // the rest in stage 0's steps 1 and 2
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kCodeLoads + kALoads + kA1) : "memory");
    } else {
        load_w(0, kofs(0));
        load_w(1, kofs(1));
        load_a(0, kofs(0), 0, kALoads);
        load_w(2, kofs(2));
        load_a(1, kofs(1), 0, kALoads);
        load_w(3, kofs(3));
        load_a(2, kofs(2), 0, kA1);
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"(6 + kALoads + kA1) : "memory");
    }
    // bare barrier: __syncthreads' fence made the compiler wait for every DMA load in
    // flight here
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    read_w(I0{}, 0u);
    decode_scales(I0{});
    read_a(af[0], 0, 0);
    dequant_b(bf[0], I0{}, 0);

    // Stage s (phase PH = s % 4, A buffer s % kStages, W in register set s % 2): steps 1
    // and 2 also read W(s+1) into the other set, decode its scales and issue window s-1's
    // later parts.  After step 3's reads the wave waits, meets the barrier (A(s+1),
    // W(s+2) visible everywhere; A buffer s and the W just read retired), issues window
    // s's first part, and step 3's MFMAs hide stage s+1's first reads and dequantisation.
    auto stage = [&](uint32_t s, auto PH) {
        constexpr int ph = decltype(PH)::value;
        constexpr int p = ph & 1;
        constexpr int pph = (ph + 3) & 3; // phase of stage s-1
        using P = std::integral_constant<int, p>;
        using N = std::integral_constant<int, 1 - p>;
        const int buf = s % kStages;
        const int nbuf = (s + 1) % kStages;
        const int abuf = (s + 2) % kStages; // window s-1's A(s+2)
        read_a(af[1], buf, 1);
        dequant_b(bf[1], P{}, 1);
        read_w(N{}, s + 1);
        if constexpr (kChunk && (pph & 1) == 0)
            load_codes_part((s + 3) / 2, 0, kCodeLoads / 2);
        load_a(abuf, kofs(s + 2), kA1, kA2);
        mfmas(af[0], bf[0]);
        interleave();
        read_a(af[0], buf, 2);
        dequant_b(bf[0], P{}, 2);
        decode_scales(N{});
        if constexpr (kChunk && (pph & 1) == 0)
            load_codes_part((s + 3) / 2, kCodeLoads / 2, kCodeLoads);
        load_a(abuf, kofs(s + 2), kA2, kALoads);
        mfmas(af[1], bf[1]);
        interleave();
        read_a(af[1], buf, 3);
        dequant_b(bf[1], P{}, 3);
        mfmas(af[0], bf[0]);
        interleave();
        // The explicit wait covers what the barrier must order (this wave's LDS reads,
        // A(s+1) and W(s+2) landed), so the barrier is the bare instruction: with
        // __syncthreads' fence the compiler added a wait for every DMA load in flight.
        constexpr int kWindow = kChunk ? kALoads + ((pph & 1) == 0 ? kCodeLoads : 0) + (pph == 0 ? 1 : 0)
                                       : kLoadsPerStage;
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kWindow) : "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if constexpr (kChunk) {
            if constexpr (ph == 0)
                load_scales(s / 4 + 1);
        } else {
            load_w((int)((s + 4) % WS), kofs(s + 4));
        }
        load_a(buf, kofs(s + kStages), 0, kA1);
        read_a(af[0], nbuf, 0);
        dequant_b(bf[0], N{}, 0);
        mfmas(af[1], bf[1]);
        interleave();
    };
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    uint32_t s = 0;
    for (; s + 4 <= nk; s += 4) {
        stage(s, I0{});
        stage(s + 1, I1{});
        stage(s + 2, I2{});
        stage(s + 3, I3{});
    }
    if (s < nk)
        stage(s, I0{});
    if (s + 1 < nk)
        stage(s + 1, I1{});
    if (s + 2 < nk)
        stage(s + 2, I2{});
    // Drain the DMA loads of the stages past the end, so the LDS is free for the
    // caller (epilogue staging or the next tile).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
}

// Store a tile's accumulators (times `scale`) as bf16 into C (row stride ldc
// elements): tile row r, column c go to C[(m0 + r) * ldc + n0 + c] for m0 + r < M and
// n0 + c < N.  Branch-free: the stores go through a buffer descriptor that ends at row
// M (the hardware drops stores past it) and columns past N get an out-of-range offset.
// `wide` (N and ldc multiples of 8, C 16-byte aligned): 16-byte stores of 8 columns;
// otherwise one 2-byte store per element.
template <int MT, int WC, int NT = 8 / WC>
__device__ __forceinline__ void store_tile_bf16(const Acc<MT, WC, NT> &acc, uint16_t *C, uint32_t ldc,
                                                uint32_t m0, uint32_t n0, uint32_t M, uint32_t N,
                                                float scale, bool wide) {
    const int lane = threadIdx.x & 63;
    const int wave = (int)__builtin_amdgcn_readfirstlane((uint32_t)threadIdx.x >> 6);
    const uint32_t cm = 32 * MT * (wave / WC) + (lane & 31);         // row within the tile
    const uint32_t cn = 32 * NT * (wave % WC) + 8 * (lane >> 5);     // column within the tile
    const uint64_t rows = M - m0;
    const uint64_t bytes = rows * ldc * 2;
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(C + (size_t)m0 * ldc + n0, bytes < 0x80000000ull ? (uint32_t)bytes : 0x7FFFFFF0u);
    if (wide) {
#pragma unroll
        for (int i = 0; i < MT; ++i)
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                u32x4_t o[2];
                pack_bf16_cols(acc[i][j] * scale, o);
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const uint32_t c = cn + 32 * j + 16 * p;
                    const uint32_t off = n0 + c < N ? ((cm + 32 * i) * ldc + c) * 2 : kOut;
                    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, o[p]), rc,
                                                           (int)off, 0, 0);
                }
            }
        return;
    }
    const uint32_t cq = 32 * NT * (wave % WC) + 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t c = cq + 32 * j + 8 * (e >> 2) + (e & 3);
                const uint32_t off = n0 + c < N ? ((cm + 32 * i) * ldc + c) * 2 : kOut;
                __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(acc[i][j][e] * scale), rc,
                                                      (int)off, 0, 0);
            }
}

// The same output as store_tile_bf16 (wide form), for 1 x 4 tiles, staged through LDS: a
// lane's 16-byte pieces land in a row-major copy of the tile (16-byte chunks XOR-swizzled
// by row % 16, so neither the accumulator-order writes nor the row-order reads conflict),
// then each store instruction writes whole rows (two 512-byte rows, 8 cache lines)
// instead of 16 bytes in each of 32 rows.  Passes of at most 128 rows (64 KB of `lds`,
// which the tile loop has drained).  Requires N and ldc multiples of 8, C 16-byte aligned.
template <int MT>
__device__ __forceinline__ void store_tile_bf16_lds(const Acc<MT, 4> &acc, uint8_t *lds, uint16_t *C,
                                                    uint32_t ldc, uint32_t m0, uint32_t n0, uint32_t M,
                                                    uint32_t N, float scale) {
    constexpr int kRows = 32 * MT;
    constexpr int kPassRows = kRows > 128 ? 128 : kRows;
    constexpr int kPasses = (kRows + kPassRows - 1) / kPassRows; // the last may be partial
    constexpr int kRowBytes = BN * 2;
    constexpr int kChunks = kRowBytes / 16; // 32
    const int lane = threadIdx.x & 63;
    const int wave = (int)__builtin_amdgcn_readfirstlane((uint32_t)threadIdx.x >> 6);
    const uint64_t bytes = (uint64_t)(M - m0) * ldc * 2;
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(C + (size_t)m0 * ldc + n0, bytes < 0x80000000ull ? (uint32_t)bytes : 0x7FFFFFF0u);
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
        if (ps > 0)
            __syncthreads(); // the previous pass's reads are done
        // block (i, j), piece p -> row 32 i + lane % 32, chunk 8 wave + 4 j + 2 p + lane / 32;
        // a partial last pass stages its blocks only (its other LDS rows hold stale data
        // that is stored to rows past the tile, which the descriptor ending at row M drops)
#pragma unroll
        for (int ii = 0; ii < kPassRows / 32; ++ii) {
            const int i = ps * (kPassRows / 32) + ii;
            if (i >= MT)
                break;
            const int r = 32 * ii + (lane & 31);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                u32x4_t o[2];
                pack_bf16_cols(acc[i][j] * scale, o);
#pragma unroll
                for (int p = 0; p < 2; ++p) {
                    const int c = 8 * wave + 4 * j + 2 * p + (lane >> 5);
                    *reinterpret_cast<u32x4_t *>(lds + r * kRowBytes + ((c ^ (r & 15)) * 16)) = o[p];
                }
            }
        }
        __syncthreads();
        // thread t: chunk t % 32 of rows t / 32 + 8 s
#pragma unroll
        for (int sr = 0; sr < kPassRows / 8; ++sr) {
            const int r = (int)(threadIdx.x / kChunks) + 8 * sr;
            const int c = (int)(threadIdx.x % kChunks);
            const u32x4_t v = *reinterpret_cast<const u32x4_t *>(lds + r * kRowBytes + ((c ^ (r & 15)) * 16));
            const uint32_t col = 8 * c;
            const uint32_t off = n0 + col < N ? ((ps * kPassRows + r) * ldc + col) * 2 : kOut;
            __builtin_amdgcn_raw_buffer_store_b128(v, rc, (int)off, 0, 0);
        }
    }
}

// fp32 output of a tile (times `scale`), placed as store_tile_bf16 places it: a lane's
// runs of 4 consecutive columns go out as 16-byte stores when `wide` (N and ldc
// multiples of 4, C 16-byte aligned), otherwise one 4-byte store per element.
template <int MT, int WC, int NT = 8 / WC>
__device__ __forceinline__ void store_tile_f32(const Acc<MT, WC, NT> &acc, float *C, uint32_t ldc,
                                               uint32_t m0, uint32_t n0, uint32_t M, uint32_t N,
                                               float scale, bool wide) {
    const int lane = threadIdx.x & 63;
    const int wave = (int)__builtin_amdgcn_readfirstlane((uint32_t)threadIdx.x >> 6);
    const uint32_t cm = 32 * MT * (wave / WC) + (lane & 31);
    const uint32_t cq = 32 * NT * (wave % WC) + 4 * (lane >> 5);
    const uint64_t bytes = (uint64_t)(M - m0) * ldc * 4;
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(C + (size_t)m0 * ldc + n0, bytes < 0x80000000ull ? (uint32_t)bytes : 0x7FFFFFF0u);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t c = cq + 32 * j + 8 * g;
                const uint32_t ro = (cm + 32 * i) * ldc;
                if (wide) {
                    u32x4_t v;
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = __float_as_uint(acc[i][j][4 * g + e] * scale);
                    const uint32_t off = n0 + c < N ? (ro + c) * 4 : kOut;
                    __builtin_amdgcn_raw_buffer_store_b128(v, rc, (int)off, 0, 0);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const uint32_t off = n0 + c + e < N ? (ro + c + e) * 4 : kOut;
                        __builtin_amdgcn_raw_buffer_store_b32(
                            __float_as_uint(acc[i][j][4 * g + e] * scale), rc, (int)off, 0, 0);
                    }
                }
            }
}

// GeGLU epilogue of a tile whose W rows interleave two matrices by 32 (tile row r:
// gate if (r / 32) % 2 == 0, else up; h column c0 + 32 (r / 64) + r % 32) and whose
// waves hold NT (even) 32-row W blocks each -- the 1 x 4 tile (WC = 4, NT = 2), the
// half-width 2 x 2 tile (WC = 2, NT = 2, W rows 0..127) or a narrow 4 x 1 tile (WC = 1,
// W rows 0 .. 32 NT - 1) -- so acc[i][2p] and acc[i][2p+1] of a wave hold gate and up of
// the same h columns c0 + 16 NT (wave % WC) + 32 p + 8 (e / 4) + 4 (lane / 32) + e % 4,
// token row 32 MT (wave / WC) + 32 i + lane % 32:
//   out[r][c] = gelu_tanh(gate_scale * gate) * (up_scale * up), r < nrows, c < ncols,
// `out` at the tile's first token row, row stride ldc (shaders/geglu.metal:15-23).
// OutT uint16_t (bf16 bits, round to nearest even) or float.  `wide`: 16-byte stores
// (bf16: ncols and ldc multiples of 8; fp32: of 4; out 16-byte aligned), else one
// store per element.
template <int MT, typename OutT, int WC = 4, int NT = 2>
__device__ __forceinline__ void store_tile_geglu(const Acc<MT, WC, NT> &acc, OutT *out, uint32_t ldc,
                                                 uint32_t nrows, uint32_t c0, uint32_t ncols,
                                                 float gate_scale, float up_scale, bool wide) {
    static_assert(NT % 2 == 0, "gate and up blocks in pairs");
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t row = 32 * MT * (wave / WC) + (lane & 31);     // the wave's first row
    const uint64_t bytes = (uint64_t)nrows * ldc * sizeof(OutT);
    const __amdgpu_buffer_rsrc_t rh =
        make_rsrc(out, bytes < 0x80000000ull ? (uint32_t)bytes : 0x7FFFFFF0u);
#pragma unroll
    for (int pr = 0; pr < NT / 2; ++pr)
#pragma unroll
    for (int i = 0; i < MT; ++i) {
        const uint32_t wcol = c0 + 16 * NT * (wave % WC) + 32 * pr; // the pair's first h column
        f32x16_t v;
#pragma unroll
        for (int q = 0; q < 16; ++q)
            v[q] = gelu_tanh_fast(acc[i][2 * pr][q] * gate_scale) * (acc[i][2 * pr + 1][q] * up_scale);
        const uint32_t ro = (row + 32 * i) * ldc;
        if (wide && sizeof(OutT) == 2) {
            u32x4_t o[2];
            pack_bf16_cols(v, o);
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint32_t c = wcol + 8 * (lane >> 5) + 16 * p;
                const uint32_t off = c < ncols ? (ro + c) * 2 : kOut;
                __builtin_amdgcn_raw_buffer_store_b128(o[p], rh, (int)off, 0, 0);
            }
        } else if (wide) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const uint32_t c = wcol + 8 * g + 4 * (lane >> 5);
                const uint32_t off = c < ncols ? (ro + c) * 4 : kOut;
                const u32x4_t w = {__float_as_uint(v[4 * g]), __float_as_uint(v[4 * g + 1]),
                                   __float_as_uint(v[4 * g + 2]), __float_as_uint(v[4 * g + 3])};
                __builtin_amdgcn_raw_buffer_store_b128(w, rh, (int)off, 0, 0);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t c = wcol + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                const uint32_t off = c < ncols ? (ro + c) * (uint32_t)sizeof(OutT) : kOut;
                if constexpr (sizeof(OutT) == 2)
                    __builtin_amdgcn_raw_buffer_store_b16(f32_to_bf16_bits(v[e]), rh, (int)off, 0, 0);
                else
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v[e]), rh, (int)off, 0, 0);
            }
        }
    }
}

} // namespace gemm_core
} // namespace apex_hip
