// NVFP4 prefill GEMM for gfx950: C[M,N] = A[M,K] . W[N,K]^T (x tensor_scale), A and C
// bf16, W NVFP4 (codes uint32 [N, K/8], E4M3 scales [N, K/16]), fp32 accumulation.
//
// The reference computes prefill as one GEMV per token (src/ops.h:44, grid.y =
// tokens, shaders/matmul.metal:18); here it is a dense MFMA contraction.  gfx950's
// scaled-FP4 MFMA uses MXFP4 (32-element blocks, E8M0 scales), which cannot express
// NVFP4's 16-element E4M3 blocks, so W is dequantised to bf16 -- exactly: every
// e2m1 x e4m3 product has at most 6 significant bits -- and fed to
// v_mfma_f32_16x16x32_bf16.
//
//  * Block tile BM x BN x 64 on 4 waves (2 x 2); a wave owns (BM/2) x (BN/2) as
//    (BM/32) x (BN/32) MFMA sub-tiles.
//  * A streams HBM/L2 -> LDS with buffer_load ... lds (no VGPR round trip) through a
//    ring of kStages stage buffers, kStages-1 stages ahead of the MFMAs.  A rows are
//    128 bytes with 16-byte pieces XOR-swizzled by (row / 2) % 8: the 16 lanes of a
//    fragment read (16 consecutive rows, one piece) then cover all 64 banks once.
//  * W's packed codes (32 bytes per row per stage) and scales (4 bytes) ride the same
//    LDS ring, copied with the same DMA loads (coalesced: rows are contiguous); each
//    wave reads the code words of its own B fragments from LDS and dequantises them
//    in registers right before its MFMAs (cvt_scalef32_pk_f32_fp4, x E4M3 scale, keep
//    the exact high halves as bf16).  The packed form keeps W's LDS traffic 4x
//    smaller than a bf16 copy.
//  * K order: within a 64-wide stage, MFMA step kk and lane group g = lane/16 take
//    the 8 k values of piece 2g + kk (a permutation of k applied to A and W alike,
//    which leaves the dot products unchanged), so a lane's two code words of a stage
//    are adjacent (one 8-byte load) and lie in one scale block (one scale byte).
//  * XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so
//    workgroup g works on tile (g % 8) * tiles_per_xcd + g / 8, tiles M-fastest: the
//    tiles resident on one XCD share A row blocks and W column blocks in its L2.
//  * Loads use buffer descriptors: rows past M or N read zeros; stores are guarded.
#include "gemm.h"
#include "nvfp4_device.h"

namespace apex_hip {
namespace {

constexpr int kThreads = 256;
constexpr int BK = 64;
constexpr int kARow = BK * 2;                 // bytes per A row in LDS
constexpr int kStages = 3;                    // ring depth
constexpr int kAStage = 256 * kARow;          // 32 KiB of A per stage
constexpr int kWCode = 256 * (BK / 2);        // 8 KiB of W codes per stage
constexpr int kWScale = 256 * (BK / 16);      // 1 KiB of W scales per stage
constexpr int kStage = kAStage + kWCode + kWScale;
constexpr size_t kLds = (size_t)kStages * kStage;

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ uint32_t pack_bf16_hi(float lo, float hi) {
    // e2m1 x e4m3 products are exact in bf16: the low 16 bits of the fp32 are zero,
    // so taking the high halves (bytes 2,3 of lo, then of hi) is exact.
    return __builtin_amdgcn_perm(__float_as_uint(hi), __float_as_uint(lo), 0x07060302u);
}

// 1 x 4 waves, each wave BM rows x BN/4 columns as (BM/32) x (BN/128) tiles of
// v_mfma_f32_32x32x16_bf16 (measured: 32x32x16 sustains ~90% of the bf16 peak with one
// wave per SIMD, 16x16x32 only ~55%).  Every W element is dequantised once per tile.
//
// K order: within a 64-wide stage, MFMA step q (0..3) and lane half h = lane/32 take
// the 8 k values of piece 4h + q, so a lane's four code words of a stage are
// contiguous (one 16-byte LDS read) and span scale blocks 2h, 2h+1.
template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void nvfp4_gemm_kernel(GemmArgs a) {
    static_assert(BM == 256 && BN == 256, "tile");
    constexpr int WM = BM, WN = BN / 4;           // wave tile 256 x 64
    constexpr int MT = WM / 32, NT = WN / 32;     // 8 x 2 MFMA tiles
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    // ---- tile of this workgroup (XCD-aware order) ----
    const uint32_t tiles_m = (a.M + BM - 1) / BM;
    const uint32_t tiles_n = (a.N + BN - 1) / BN;
    const uint32_t tiles = tiles_m * tiles_n;
    const uint32_t per_xcd = (tiles + 7) / 8;
    const uint32_t t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= tiles)
        return;
    const uint32_t m0 = (t % tiles_m) * BM;
    const uint32_t n0 = (t / tiles_m) * BN;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wn = wave * WN;       // wave's column offset in the tile
    const int frow = lane & 31;     // fragment row (A) / column (B) within a 32-wide tile
    const int h = lane >> 5;        // lane half: k pieces 4h .. 4h+3 of each stage

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, a.M * a.K * 2);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.codes, a.N * (a.K / 2));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, a.N * (a.K / 16));

    // A: wave w copies rows [64w, 64w+64) of the tile into LDS with 8 buffer_load ...
    // lds instructions of 8 rows each; lane l lands at row 8i + l/8, physical piece
    // l%8, so it fetches logical piece (l%8) ^ ((row/2)%8) of that row.  Offsets of
    // rows past M are out of range (>= 2^31), so those lanes read zeros.
    uint32_t a_off[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int trow = wave * 64 + 8 * i + (lane >> 3);
        const uint32_t row = m0 + trow;
        a_off[i] = row < a.M ? row * a.K * 2 + (((lane & 7) ^ ((trow >> 1) & 7)) * 16)
                             : 0x80000000u;
    }
    // W: rows n0 .. n0+255 of the tile (rows past N read zeros).  Codes: 16-byte slot q
    // of the stage holds half (q%2) ^ ((q/16)%2) of row q/2 -- rows 8..15 of every 16
    // swap their halves, so the 16 lanes reading one half of 16 consecutive rows hit
    // 16 distinct bank groups; wave w copies slots [128w, 128w+128) with 2 DMA loads.
    // Scales: wave w copies rows [64w, 64w+64), 4 bytes each.
    uint32_t wc_off[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int q = wave * 128 + i * 64 + lane;
        const int trow = q / 2;
        const uint32_t row = n0 + trow;
        const int half = (q & 1) ^ ((trow >> 3) & 1);
        wc_off[i] = row < a.N ? row * (a.K / 2) + half * 16 : 0x80000000u;
    }
    const uint32_t ws_row = n0 + wave * 64 + lane;
    const uint32_t ws_off = ws_row < a.N ? ws_row * (a.K / 16) : 0x80000000u;

    auto load_stage = [&](int buf, uint32_t k0) {
        uint8_t *base = lds + buf * kStage;
#pragma unroll
        for (int i = 0; i < 8; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                ra, (lds_void_t *)(base + (wave * 64 + 8 * i) * kARow), 16, a_off[i] + k0 * 2, 0,
                0, 0);
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(
                rc, (lds_void_t *)(base + kAStage + (wave * 128 + i * 64) * 16), 16,
                wc_off[i] + k0 / 2, 0, 0, APEX_WEIGHT_CPOL);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (lds_void_t *)(base + kAStage + kWCode + wave * 64 * 4), 4, ws_off + k0 / 16, 0, 0,
            APEX_WEIGHT_CPOL);
    };
    constexpr int kLoadsPerStage = 8 + 2 + 1; // DMA loads per wave per stage

    f32x16_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e)
                acc[i][j][e] = 0.0f;

    const uint32_t nk = a.K / BK;
    auto kofs = [&](uint32_t st) { return st < nk ? st * BK : 0u; }; // past the end: harmless re-read

    // Per-stage register state: this lane's W code words and block scales, A and B
    // fragments of the current MFMA step and of the next one.
    u32x4_t wcode[NT];
    f32x2_t wsc[NT];
    bf16x8_v af[2][MT], bf[2][NT];
    auto read_w = [&](int buf) {
        const uint8_t *lwc = lds + buf * kStage + kAStage;
        const uint8_t *lws = lwc + kWCode;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            // rows wn + 32 j + frow, half h (code words 4h .. 4h+3 = scale blocks 2h,
            // 2h+1), slot 2r + (h ^ ((r/8)%2))
            const int r = wn + 32 * j + frow;
            wcode[j] = *reinterpret_cast<const u32x4_t *>(lwc + (2 * r + (h ^ ((r >> 3) & 1))) * 16);
            const uint32_t sb = *reinterpret_cast<const uint16_t *>(lws + r * 4 + 2 * h);
            wsc[j] = f32x2_t{e4m3_to_f32(sb), e4m3_to_f32(sb >> 8)};
        }
    };
    // A fragments of step q: rows 32 i + frow, logical piece 4h + q.
    auto read_a = [&](bf16x8_v (&dst)[MT], int buf, int q) {
        const uint8_t *la = lds + buf * kStage;
        const int piece = 4 * h + q;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int r = i * 32 + frow;
            dst[i] = *reinterpret_cast<const bf16x8_v *>(la + r * kARow + ((piece ^ ((r >> 1) & 7)) * 16));
        }
    };
    // B fragments of step q: word q of each tile's codes (8 weights), scale block 2h + q/2.
    auto dequant_b = [&](bf16x8_v (&dst)[NT], int q) {
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            f32x2_t v[4];
            e2m1x8_to_f32(wcode[j][q], v);
            const float sc = wsc[j][q >> 1];
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
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(A[i], B[j], acc[i][j], 0, 0, 0);
    };
    // One MFMA, then up to two VALU ops and one LDS read, for the MT*NT MFMAs of a step.
    auto interleave = [&]() {
#pragma unroll
        for (int m = 0; m < MT * NT; ++m) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0); // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 2, 0); // VALU
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0); // DS read
        }
    };

    // Prologue: stages 0 .. kStages-1 in flight; stage 0 visible; step 0 prepared.
#pragma unroll
    for (int st = 0; st < kStages; ++st)
        load_stage(st, kofs(st));
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoadsPerStage * (kStages - 1)) : "memory");
    __syncthreads();
    read_w(0);
    read_a(af[0], 0, 0);
    dequant_b(bf[0], 0);

    // Stage s (buffer s % kStages): the MFMAs of step q run while step q+1's A
    // fragments are read and its B fragments dequantised.  After step 2 every read of
    // the buffer has been issued: the wave waits for them and for its part of stage
    // s+1, meets the barrier (stage s+1 visible everywhere, buffer s retired) and
    // refills buffer s with stage s + kStages; step 3 then hides stage s+1's first
    // reads and dequantisation.
    for (uint32_t s = 0; s < nk; ++s) {
        const int buf = s % kStages;
        const int nbuf = (s + 1) % kStages;
        read_a(af[1], buf, 1);
        dequant_b(bf[1], 1);
        mfmas(af[0], bf[0]);
        interleave();
        read_a(af[0], buf, 2);
        dequant_b(bf[0], 2);
        mfmas(af[1], bf[1]);
        interleave();
        read_a(af[1], buf, 3);
        dequant_b(bf[1], 3);
        mfmas(af[0], bf[0]);
        interleave();
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)" ::"n"(kLoadsPerStage * (kStages - 2))
                     : "memory");
        __syncthreads();
        load_stage(buf, kofs(s + kStages));
        read_w(nbuf);
        read_a(af[0], nbuf, 0);
        dequant_b(bf[0], 0);
        mfmas(af[1], bf[1]);
        interleave();
    }

    // epilogue: acc[i][j][4 jj + ii] = C[m0 + 32 i + 8 jj + 4 h + ii][n0 + wn + 32 j + frow]
    const uint32_t cn = n0 + wn + frow;
    const uint32_t cm = m0 + 4 * h;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const uint32_t m = cm + 32 * i + 8 * (e >> 2) + (e & 3);
                const uint32_t n = cn + 32 * j;
                if (m < a.M && n < a.N)
                    a.C[(size_t)m * a.ldc + n] = f32_to_bf16_bits(acc[i][j][e] * a.tensor_scale);
            }
}

template <int BM, int BN> hipError_t launch(const GemmArgs &a, hipStream_t stream) {
    const uint32_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const uint32_t grid = 8 * ((tiles + 7) / 8);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)nvfp4_gemm_kernel<BM, BN>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLds);
        if (e != hipSuccess)
            return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((nvfp4_gemm_kernel<BM, BN>), dim3(grid), dim3(kThreads), kLds, stream, a);
    return hipGetLastError();
}

} // namespace

bool gemm_supported(uint32_t M, uint32_t N, uint32_t K) {
    return K % BK == 0 && K > 0 && (uint64_t)M * K * 2 < (1ull << 31) &&
           (uint64_t)N * (K / 2) < (1ull << 31) && M > 0 && N > 0;
}

hipError_t gemm_launch(const GemmArgs &a, hipStream_t stream) {
    if (!gemm_supported(a.M, a.N, a.K))
        return hipErrorInvalidValue;
    return launch<256, 256>(a, stream);
}

} // namespace apex_hip
