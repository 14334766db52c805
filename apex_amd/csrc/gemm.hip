// NVFP4 prefill GEMM for gfx950: C[M,N] = A[M,K] . W[N,K]^T (x tensor_scale), A and C
// bf16, W NVFP4 (codes uint32 [N, K/8], E4M3 scales [N, K/16]), fp32 accumulation.
//
// The reference computes prefill as one GEMV per token (src/ops.h:44, grid.y =
// tokens, shaders/matmul.metal:18); here it is a dense MFMA contraction on 256 x 256
// tiles (gemm_core.h: W dequantised exactly to bf16 in registers from LDS-staged codes,
// v_mfma_f32_32x32x16_bf16, fp32 accumulation).
//
// XCD-aware tile order: workgroups are dispatched round-robin over the 8 XCDs, so
// workgroup g works on tile (g % 8) * tiles_per_xcd + g / 8, tiles M-fastest: the tiles
// resident on one XCD share A row blocks and W column blocks in its L2.  Loads use
// buffer descriptors: rows past M or N read zeros; stores are guarded.
#include "gemm.h"
#include "gemm_core.h"

namespace apex_hip {
namespace {

using namespace gemm_core;
constexpr int WC = 4;                     // 1 x 4 waves (the 2 x 2 layout measured slower)
constexpr int MT = 8;                     // 32-row MFMA tiles per wave
constexpr int BM = Layout<MT, WC>::kBM;   // 256

// 16-byte epilogue stores need 8-column row pieces at 16-byte aligned addresses.
__device__ __forceinline__ bool uniform_wide(const GemmArgs &a) {
    return a.N % 8 == 0 && a.ldc % 8 == 0 && ((uintptr_t)a.C & 15) == 0;
}

__global__ __launch_bounds__(kThreads) void nvfp4_gemm_kernel(GemmArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

    const uint32_t tiles_m = (a.M + BM - 1) / BM;
    const uint32_t tiles_n = (a.N + BN - 1) / BN;
    const uint32_t tiles = tiles_m * tiles_n;
    const uint32_t per_xcd = (tiles + 7) / 8;
    const uint32_t t = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (t >= tiles)
        return;
    const uint32_t m0 = (t % tiles_m) * BM;
    const uint32_t n0 = (t / tiles_m) * BN;

    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.A, a.M * a.K * 2);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(a.codes, a.N * (a.K / 2));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.scales, a.N * (a.K / 16));
    const uint32_t K = a.K;
    const uint32_t M = a.M, N = a.N;
    auto a_row = [=](int r) { return m0 + r < M ? (m0 + r) * K * 2 : kOut; };
    auto w_code = [=](int r) { return n0 + r < N ? (n0 + r) * (K / 2) : kOut; };
    auto w_scale = [=](int r) { return n0 + r < N ? (n0 + r) * (K / 16) : kOut; };

    Acc<MT, WC> acc;
    gemm_tile<MT, WC>(lds, ra, rc, rs, K, a_row, w_code, w_scale, acc);

    store_tile_bf16<MT, WC>(acc, a.C, a.ldc, m0, n0, M, N, a.tensor_scale, uniform_wide(a));
}

hipError_t launch(const GemmArgs &a, hipStream_t stream) {
    const uint32_t tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
    const uint32_t grid = 8 * ((tiles + 7) / 8);
    constexpr size_t lds = Layout<MT, WC>::kLds;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void *)nvfp4_gemm_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(nvfp4_gemm_kernel, dim3(grid), dim3(kThreads), lds, stream, a);
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
    return launch(a, stream);
}

} // namespace apex_hip
