// Host-side interface of the NVFP4 prefill GEMMs (MFMA regime).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace apex_hip {

// Plain:  C[M, N] = tensor_scale[0] * A . W^T                     (W = codes/scales[0])
// GeGLU:  C[M, N] = gelu(tensor_scale[0] * A . G^T) * (tensor_scale[1] * A . U^T)
//         (G = codes/scales[0], U = [1], both [N, K]; shaders/geglu.metal:15-23)
// A is bf16 [M, a_k] (row stride a_k): a_k = K for bf16 activations, a_k = 2K for the
// [hi | lo] split of fp32 activations (gemm_split_launch), whose halves both meet W.
// C is bf16 bits or fp32 (out_f32), row stride ldc.  W: codes uint32 [N, K/8], E4M3
// scales [N, K/16].
struct GemmArgs {
    const uint16_t *A;
    const uint32_t *codes[2];
    const uint8_t *scales[2];
    float tensor_scale[2];
    void *C;
    uint32_t M, N, K, ldc, a_k;
    bool geglu, out_f32;
};

// K % 64 == 0 and operands within the 2 GiB buffer-descriptor range (A of a_k columns).
bool gemm_supported(uint32_t M, uint32_t N, uint32_t K, uint32_t a_k, bool out_f32);

hipError_t gemm_launch(const GemmArgs &a, hipStream_t stream);

// How gemm_launch covers C on ncu CUs: whole tiles (256 x 256; GeGLU 256 rows x 128 h
// columns) for the first nf n-tiles, narrow tiles of nt (1 or 2) 32-row W blocks for
// the columns past them; nt = 0: whole tiles only (nf = all n-tiles).
// Tail plan of a grid whose whole tiles leave the last round of CUs partly empty: whole
// tiles cover n-tiles [0, nf); the columns past them run either as narrow tiles of nt
// 32-row W blocks (nt > 0) or as ns short tiles (ns > 0): each a contiguous range of at
// most 8 32-row blocks of one tail n-tile column, full width, one per CU of the last
// round.  nt = ns = 0: whole tiles only.
struct GemmTailPlan {
    uint32_t nf, nt, ns;
};
GemmTailPlan gemm_tail_plan(uint32_t M, uint32_t N, bool geglu, uint32_t ncu);

// Short tile v of ns over C tail columns of B 32-row blocks: column c (r_c = ns / C
// workgroups, one more for the first ns % C columns) and its i-th of r_c contiguous block
// ranges (B / r_c blocks, one more for the first B % r_c ranges).
struct ShortTile {
    uint32_t col, block0, blocks;
};
__host__ __device__ inline ShortTile short_tile(uint32_t v, uint32_t ns, uint32_t C, uint32_t B) {
    const uint32_t q = ns / C, rem = ns % C;
    uint32_t c, i, r;
    if (v < (q + 1) * rem) {
        c = v / (q + 1), i = v % (q + 1), r = q + 1;
    } else {
        const uint32_t u = v - (q + 1) * rem;
        c = rem + u / q, i = u % q, r = q;
    }
    const uint32_t base = B / r, extra = B % r;
    return ShortTile{c, i * base + (i < extra ? i : extra), base + (i < extra ? 1u : 0u)};
}

// Split-K form for grids of few tiles: S workgroups per tile each run a contiguous
// range of K stages (for a_k = 2K none crosses from the hi half to the lo half) and
// store fp32 partials, part[S][M][N] (GeGLU: gate and up, part[S][2][M][N]); a second
// kernel sums them in split order and applies the epilogue.  gemm_splitk_splits gives
// the split count for a's shape (1: run gemm_launch).
uint32_t gemm_splitk_splits(const GemmArgs &a);
size_t gemm_splitk_bytes(const GemmArgs &a, uint32_t splits);
hipError_t gemm_splitk_launch(const GemmArgs &a, uint32_t splits, float *part, hipStream_t stream);

// fp32 activations X [M, K] (row stride K) -> split [M, 2K] bf16: hi = bf16(x) and
// lo = bf16(x - hi), both rounded to nearest even (lo = 0 where hi is not finite), so
// x = hi + lo + r with |r| <= 2^-17 |x|.  With norm_w (bf16 [K]), x is first
// RMS-normalised over its row: x * (1 / sqrt(mean(x^2) + eps)) * norm_w[k].
size_t gemm_split_bytes(uint32_t M, uint32_t K);
hipError_t gemm_split_launch(const float *X, const uint16_t *norm_w, float eps, uint16_t *split,
                             uint32_t M, uint32_t K, hipStream_t stream);

} // namespace apex_hip
