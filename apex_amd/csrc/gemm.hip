// NVFP4 prefill GEMM for gfx950: C[M,N] = A[M,K] . W[N,K]^T (x tensor_scale), A and C
// bf16, W NVFP4 (codes uint32 [N, K/8], E4M3 scales [N, K/16]), fp32 accumulation.
//
// The reference computes prefill as one GEMV per token (src/ops.h:44, grid.y =
// tokens, shaders/matmul.metal:18); here it is a dense MFMA contraction:
//  * Block tile BM x BN x 64 on 4 waves (2 x 2); a wave owns (BM/2) x (BN/2) and runs
//    v_mfma_f32_16x16x32_bf16 on (BM/32) x (BN/32) sub-tiles.  gfx950's scaled-FP4
//    MFMA uses MXFP4 (32-element blocks, E8M0 scales), which cannot express NVFP4's
//    16-element E4M3 blocks, so W is dequantised to bf16 -- exactly: e2m1 x e4m3
//    products have at most 6 significant bits -- once per stage into LDS.
//  * Stage pipeline: global loads of stage s+1 (A bf16 rows, W codes + scales) are
//    issued before the MFMAs of stage s and written to the other LDS buffer after
//    them; one barrier per stage.  LDS rows are padded to 144 bytes so the 16-byte
//    fragment reads and writes of 8 consecutive lanes hit disjoint banks.
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
constexpr int kRowBytes = BK * 2 + 16; // padded LDS row: 64 bf16 + 16 bytes
constexpr int kRows = 256;             // LDS rows per operand per stage

typedef __bf16 bf16x8_v __attribute__((ext_vector_type(8)));

__device__ __forceinline__ uint32_t pack_bf16_hi(float lo, float hi) {
    // e2m1 x e4m3 products are exact in bf16: the low 16 bits of the fp32 are zero,
    // so taking the high halves is exact (no rounding needed).
    return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xFFFF0000u);
}

template <int BM, int BN>
__global__ __launch_bounds__(kThreads) void nvfp4_gemm_kernel(GemmArgs a) {
    static_assert(BM == 256, "A staging assumes 256 rows");
    static_assert(BN % 32 == 0 && BN <= 256, "BN");
    constexpr int WM = BM / 2, WN = BN / 2; // wave tile
    constexpr int MT = WM / 16, NT = WN / 16;
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    // stage buffer b: A rows at lds + 2b*S, W rows at lds + (2b+1)*S, S = 256 rows
    auto lds_a = [&](int b) { return lds + (2 * b) * kRows * kRowBytes; };
    auto lds_w = [&](int b) { return lds + (2 * b + 1) * kRows * kRowBytes; };

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
    const int wm = (wave & 1) * WM; // wave's row offset in the tile
    const int wn = (wave >> 1) * WN;

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, a.M * a.K * 2);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.codes, a.N * (a.K / 2));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, a.N * (a.K / 16));

    // A staging: thread loads 16-byte piece (tid % 8) of rows tid/8 + 32 i, i < 8.
    const int a_piece = tid & 7;
    const int a_row0 = tid >> 3;
    // W staging: thread owns tile row n0 + tid (32 code bytes + 4 scale bytes a stage).
    const bool w_ok = tid < BN && n0 + tid < a.N;
    const uint32_t w_code_off = w_ok ? (n0 + tid) * (a.K / 2) : 0x80000000u;
    const uint32_t w_scale_off = w_ok ? (n0 + tid) * (a.K / 16) : 0x80000000u;

    u32x4_t av[8];
    u32x4_t wc[2];
    uint32_t ws;
    auto load_stage = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t row = m0 + a_row0 + 32 * i;
            const uint32_t off = row < a.M ? (row * a.K + k0) * 2 + a_piece * 16 : 0x80000000u;
            av[i] = load_b128(ra, off);
        }
        wc[0] = load_b128(rc, w_code_off + k0 / 2);
        wc[1] = load_b128(rc, w_code_off + k0 / 2 + 16);
        ws = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(w_scale_off + k0 / 16), 0, 0);
    };
    auto store_stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            *reinterpret_cast<u32x4_t *>(lds_a(buf) + (a_row0 + 32 * i) * kRowBytes + a_piece * 16) =
                av[i];
        // dequantise the 64 weights of row tid: block b = words 2b, 2b+1, scale byte b
        uint8_t *wrow = lds_w(buf) + tid * kRowBytes;
        const uint32_t words[8] = {wc[0][0], wc[0][1], wc[0][2], wc[0][3],
                                   wc[1][0], wc[1][1], wc[1][2], wc[1][3]};
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const float s = e4m3_to_f32(ws >> (8 * b));
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                f32x2_t v[4];
                e2m1x8_to_f32(words[2 * b + h], v);
                u32x4_t o;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    o[j] = pack_bf16_hi(v[j][0] * s, v[j][1] * s);
                *reinterpret_cast<u32x4_t *>(wrow + (2 * b + h) * 16) = o;
            }
        }
    };

    f32x4_t acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
            acc[i][j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    const uint32_t nk = a.K / BK;
    load_stage(0);
    store_stage(0);
    __syncthreads();

    // fragment addressing: lane l reads row (l % 16), k bytes ((l / 16) * 8 + 32 kk) * 2
    const int frow = lane & 15;
    const int fk = (lane >> 4) * 16;

    for (uint32_t ks = 0; ks < nk; ++ks) {
        const int cur = ks & 1;
        if (ks + 1 < nk)
            load_stage((ks + 1) * BK);
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            bf16x8_v af[MT], bfr[NT];
#pragma unroll
            for (int i = 0; i < MT; ++i)
                af[i] = *reinterpret_cast<const bf16x8_v *>(
                    lds_a(cur) + (wm + i * 16 + frow) * kRowBytes + kk * 64 + fk);
#pragma unroll
            for (int j = 0; j < NT; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8_v *>(
                    lds_w(cur) + (wn + j * 16 + frow) * kRowBytes + kk * 64 + fk);
#pragma unroll
            for (int i = 0; i < MT; ++i)
#pragma unroll
                for (int j = 0; j < NT; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j],
                                                                        0, 0, 0);
        }
        if (ks + 1 < nk)
            store_stage(cur ^ 1);
        __syncthreads();
    }

    // epilogue: acc[i][j][r] = C[m0 + wm + 16 i + 4 (lane/16) + r][n0 + wn + 16 j + lane%16]
    const uint32_t cn = n0 + wn + (lane & 15);
    const uint32_t cm = m0 + wm + (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < NT; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t m = cm + 16 * i + r;
                const uint32_t n = cn + 16 * j;
                if (m < a.M && n < a.N)
                    a.C[(size_t)m * a.ldc + n] = f32_to_bf16_bits(acc[i][j][r] * a.tensor_scale);
            }
}

template <int BM, int BN> hipError_t launch(const GemmArgs &a, hipStream_t stream) {
    const uint32_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const uint32_t grid = 8 * ((tiles + 7) / 8);
    const size_t lds = 4 * (size_t)kRows * kRowBytes;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)nvfp4_gemm_kernel<BM, BN>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return e;
        attr_set = true;
    }
    hipLaunchKernelGGL((nvfp4_gemm_kernel<BM, BN>), dim3(grid), dim3(kThreads), lds, stream, a);
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
    // 224-wide tiles when N divides evenly (e.g. 21504 = 96 x 224), else 256.
    if (a.N % 224 == 0 && a.N % 256 != 0)
        return launch<256, 224>(a, stream);
    return launch<256, 256>(a, stream);
}

} // namespace apex_hip
