// MoE expert FFN over NVFP4 expert slots, gfx950.
//
//   y[t] = sum_j w[t,j] * down_e( gelu(gate_e x_t) (*) up_e x_t ),  e = ids[t,j]
//
// with ids / w the router's top-k (ties to the lower expert id) and softmax over the
// k selected logits.  The reference has no MoE kernel: the semantics are those of
// tools/dump_reference.py:208-219 (experts combined with the router weights), each
// expert being the dense GeGLU FFN of src/ops.h:57-69 on the slot pieces of
// tools/repack.py:180-213.
//
// Routing and grouping (both regimes):
//   route   one wave per token: top-k by k rounds of a wave-wide 64-bit max over
//           (order-preserving logit bits, ~expert id) keys, then softmax in fp32.
//   plan    one workgroup: per-expert counts (LDS atomics), offsets, the ascending list
//           of active experts, and a position for every (token, slot) pair in the
//           expert-grouped order.  Pairs of one expert get their positions in
//           arbitrary order; every pair's result is computed independently of its
//           neighbours, so outputs do not depend on that order.
//
// Decode regime (T <= 32 tokens, T*k <= 256 pairs): bandwidth-bound grouped GEMVs.
//   gate/up  persistent waves over (active expert, 2 rows) units: the unit's gate and
//            up rows stream once and serve every token routed to the expert; GeGLU in
//            registers -> h[pos] (bf16).
//   down     persistent waves over (token group, 8 rows) units: a group is up to 4
//            positions of one expert whose h rows sit in LDS; each unit's down rows are
//            decoded once for the whole group -> d[pos] (bf16).
//   combine  as in the prefill regime.
// Prefill regime: MFMA grouped GEMMs on the gemm_core tile (bf16 MFMA on exactly
// dequantised weights).
//   m-tiles  per expert, 256-row tiles plus one tail tile of 1 to 8 blocks of 32 rows,
//            big tiles first; token rows are gathered through the pair list by the
//            A-tile DMA loads (no permuted copy of x).
//   gate/up  each 256-wide W tile holds 128 gate rows and the same 128 up rows, placed
//            so that a lane's two accumulator sets are gate and up of one h column:
//            GeGLU epilogue in registers -> h[pos] (bf16).
//   down     h rows are contiguous per expert -> d[pos] (bf16), over the gate/up
//            GEMM's m-tiles, one workgroup per CU.
//   combine  y[t] = sum_j w[t,j] d[pos(t,j)] in slot order j, fp32 -> bf16: a fixed
//            summation order, no float atomics, so results are deterministic.
#include <type_traits>

#include "gemm_core.h"
#include "gemv_kernels.h"
#include "lds_attr.h"
#include "moe.h"

namespace apex_hip {

std::atomic<int> kMoePath{0};

namespace {

using gemv_detail::chunk_dot;
using gemv_detail::chunk_scales;
using gemv_detail::load_row;
using gemv_detail::RowRegs;
using gemv_detail::XChunk;

constexpr uint32_t kOutOfRange = 0x80000000u;

// A value the whole wave holds alike, moved to a scalar register.  Values read from
// memory land in vector registers, and a buffer descriptor or loop bound built from a
// vector register makes the compiler wrap every load in a per-lane (waterfall) loop.
__device__ __forceinline__ uint32_t uniform(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int uniform(int v) { return (int)__builtin_amdgcn_readfirstlane((uint32_t)v); }
__device__ __forceinline__ float uniform_f(float v) {
    return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(v)));
}


struct PlanView {
    int32_t *hdr, *cnt, *off, *act, *pos_of_pair, *pair_of_pos, *tiles, *groups;
};

__host__ __device__ inline PlanView plan_view(int32_t *plan, uint32_t E, uint32_t P) {
    PlanView v;
    v.hdr = plan;
    v.cnt = plan + kMoePlanHeader;
    v.off = v.cnt + E;
    v.act = v.off + E + 1;
    v.pos_of_pair = v.act + E;
    v.pair_of_pos = v.pos_of_pair + P;
    v.groups = v.pair_of_pos + P;
    v.tiles = v.groups + 2 * P;
    return v;
}

// ---------------------------------------------------------------------------------
// Routing
// ---------------------------------------------------------------------------------

// Maximum of a 64-bit key over the wave: DPP within rows of 16 lanes (quad swaps, then
// half-row and row mirrors pair every lane with one of the other half), then the two
// cross-row steps by VALU lane swaps (v_permlane16_swap / v_permlane32_swap).
template <int CTRL> __device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, false);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
    uint64_t o;
    o = dpp_u64<0xB1>(v);  v = o > v ? o : v;  // quad_perm [1,0,3,2]
    o = dpp_u64<0x4E>(v);  v = o > v ? o : v;  // quad_perm [2,3,0,1]
    o = dpp_u64<0x141>(v); v = o > v ? o : v;  // row_half_mirror
    o = dpp_u64<0x140>(v); v = o > v ? o : v;  // row_mirror
    {
        const auto lo = __builtin_amdgcn_permlane16_swap((uint32_t)v, (uint32_t)v, false, false);
        const auto hi = __builtin_amdgcn_permlane16_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
        const uint64_t a0 = ((uint64_t)hi[0] << 32) | lo[0], a1 = ((uint64_t)hi[1] << 32) | lo[1];
        v = a0 > a1 ? a0 : a1;
    }
    {
        const auto lo = __builtin_amdgcn_permlane32_swap((uint32_t)v, (uint32_t)v, false, false);
        const auto hi = __builtin_amdgcn_permlane32_swap((uint32_t)(v >> 32), (uint32_t)(v >> 32), false, false);
        const uint64_t a0 = ((uint64_t)hi[0] << 32) | lo[0], a1 = ((uint64_t)hi[1] << 32) | lo[1];
        v = a0 > a1 ? a0 : a1;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));  // quad_perm [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false));  // quad_perm [2,3,0,1]
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false)); // row_half_mirror
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x140, 0xF, 0xF, false)); // row_mirror
    const auto r16 = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    v = max(r16[0], r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return max(r32[0], r32[1]);
}

// route_token_by for bf16 logits, whose key fits 32 bits: the order-preserving image
// of the 16 logit bits above 0xFFFF - e (larger logit first, then lower expert id,
// as route_token_by orders), so each of the k rounds is one 32-bit wave maximum.
// bits(e, q) returns expert e's logit bits (e = lane + 64 q).
template <typename Bits>
__device__ __forceinline__ void route_token_bits(Bits bits, uint32_t E, uint32_t k, int lane,
                                                 int32_t &my_id, float &my_w) {
    uint32_t key[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t e = lane + 64 * q;
        if (e < E) {
            const uint32_t b = bits(e, q);
            const uint32_t u = b == 0x8000u ? 0u : b; // -0 ties +0
            const uint32_t ord = (u & 0x8000u) ? (~u & 0xFFFFu) : (u | 0x8000u);
            key[q] = (ord << 16) | (0xFFFFu - e);
        } else {
            key[q] = 0; // below every expert's key (their low halves are >= 0xFF00)
        }
    }
    my_id = 0;
    float my_v = 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
        uint32_t best = key[0];
#pragma unroll
        for (int q = 1; q < 4; ++q)
            if (64 * q < E)
                best = max(best, key[q]);
        best = wave_max_u32(best);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (key[q] == best)
                key[q] = 0;
        if ((uint32_t)lane == j) {
            my_id = (int32_t)(0xFFFFu - (best & 0xFFFFu));
            const uint32_t ord = best >> 16;
            my_v = __uint_as_float(((ord & 0x8000u) ? (ord & 0x7FFFu) : (~ord & 0xFFFFu)) << 16);
        }
    }
    // slot 0 holds the largest logit
    const float vmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), 0));
    const float p = (uint32_t)lane < k ? expf(my_v - vmax) : 0.0f;
    my_w = p / group_sum<64>(p);
}

__device__ __forceinline__ void route_token(const uint16_t *logits, uint32_t E, uint32_t k,
                                            int lane, int32_t &my_id, float &my_w) {
    route_token_bits([&](uint32_t e, int) { return (uint32_t)logits[e]; }, E, k, lane, my_id, my_w);
}

// Top-k of one token's E logits (E <= 256; logit(e, q) returns expert e = lane + 64 q's
// as fp32) by wave
// lanes 0..63, then softmax over the k; lane j < k returns slot j's expert id and
// weight.  Keys order by logit, then by lower expert id (the reference tie-break), and
// are unique per expert.
template <typename Logit>
__device__ __forceinline__ void route_token_by(Logit logit, uint32_t E, uint32_t k, int lane,
                                               int32_t &my_id, float &my_w) {
    uint64_t key[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t e = lane + 64 * q;
        if (e < E) {
            const uint32_t f = __float_as_uint(logit(e, q));
            const uint32_t u = f == 0x80000000u ? 0u : f; // -0 ties +0
            const uint32_t ord = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
            key[q] = ((uint64_t)ord << 32) | (0xFFFFFFFFu - e);
        } else {
            key[q] = 0;
        }
    }
    my_id = 0;
    float my_v = 0.0f;
    for (uint32_t j = 0; j < k; ++j) {
        uint64_t best = key[0];
#pragma unroll
        for (int q = 1; q < 4; ++q)
            best = key[q] > best ? key[q] : best;
        best = wave_max_u64(best);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (key[q] == best)
                key[q] = 0;
        if ((uint32_t)lane == j) {
            my_id = (int32_t)(0xFFFFFFFFu - (uint32_t)best);
            const uint32_t ord = (uint32_t)(best >> 32);
            my_v = __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
        }
    }
    // slot 0 holds the largest logit
    const float vmax = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_v), 0));
    const float p = (uint32_t)lane < k ? expf(my_v - vmax) : 0.0f;
    my_w = p / group_sum<64>(p);
}

// Token t of the FFN's logits (fp32 when given, else bf16); lane j < k's weight times
// the per-expert scale of its expert when one is given.
__device__ __forceinline__ void route_token_args(const MoeArgs &a, uint32_t t, int lane,
                                                 int32_t &id, float &wt) {
    if (a.logits_f32) {
        const float *l = a.logits_f32 + (size_t)t * a.E;
        route_token_by([&](uint32_t e, int) { return l[e]; }, a.E, a.k, lane, id, wt);
    } else {
        route_token(a.logits + (size_t)t * a.E, a.E, a.k, lane, id, wt);
    }
    if (a.pes && (uint32_t)lane < a.k)
        wt *= bf16_bits_to_f32(a.pes[id]);
}

// Token t's logits for lane `lane` (experts lane + 64 q; fp32 or bf16 bits), loaded
// ahead of the routing so their latency overlaps other work.
struct TokenLogits {
    uint32_t v[4];
};
__device__ __forceinline__ TokenLogits load_token_logits(const MoeArgs &a, uint32_t t, int lane) {
    TokenLogits r;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t e = lane + 64 * q;
        r.v[q] = e >= a.E ? 0u
                 : a.logits_f32 ? __float_as_uint(a.logits_f32[(size_t)t * a.E + e])
                                : (uint32_t)a.logits[(size_t)t * a.E + e];
    }
    return r;
}

// route_token_args on logits already loaded.
__device__ __forceinline__ void route_token_loaded(const MoeArgs &a, const TokenLogits &r, int lane,
                                                   int32_t &id, float &wt) {
    if (a.logits_f32)
        route_token_by([&](uint32_t, int q) { return __uint_as_float(r.v[q]); }, a.E, a.k, lane, id, wt);
    else
        route_token_bits([&](uint32_t, int q) { return r.v[q]; }, a.E, a.k, lane, id, wt);
    if (a.pes && (uint32_t)lane < a.k)
        wt *= bf16_bits_to_f32(a.pes[id]);
}

__global__ __launch_bounds__(256) void moe_route_f32_kernel(const float *logits,
                                                            const uint16_t *pes, uint32_t T,
                                                            uint32_t E, uint32_t k, int32_t *ids,
                                                            float *w) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T)
        return;
    int32_t id;
    float wt;
    const float *l = logits + (size_t)t * E;
    route_token_by([&](uint32_t e, int) { return l[e]; }, E, k, lane, id, wt);
    if ((uint32_t)lane < k) {
        ids[(size_t)t * k + lane] = id;
        w[(size_t)t * k + lane] = pes ? wt * bf16_bits_to_f32(pes[id]) : wt;
    }
}

// Router logits (MoeRouterArgs): one workgroup of WAVES waves per tile of TT tokens.
// The tile's normalised rows xn = h * inv * w (the rmsNormCpu order) and their
// per-group sums go to LDS once.  Lane l owns experts l, l + 64, ... (EPL of them) and
// the waves split the 64-element groups of K, so each activation read is an LDS
// broadcast feeding 4 * EPL FMAs per token; the next group's codes are loaded while
// the current one is used.  Per group g:
//   logit[t][e] += scale[e][g] * sum_k xn[t][k] q[e][k] + bias[e][g] * sum_k xn[t][k]
// in fp32 (w = scale * q + bias expanded, the bias term from the shared group sum);
// the waves' partial logits are summed in wave order.
constexpr uint32_t kQGroup = 64;
constexpr size_t kMaxDynLds = 160 * 1024 - 256; // a CU's LDS, less the static arrays

template <int TT, int EPL, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void moe_router_kernel(MoeRouterArgs a) {
    extern __shared__ __attribute__((aligned(16))) float rsm[];
    __shared__ float inv_s[TT];
    const uint32_t H = a.H, E = a.E, NG = H / kQGroup;
    float *xn = rsm;                     // [TT][H]
    float *gsum = xn + TT * H;           // [TT][NG]
    float *part = gsum + TT * NG;        // [WAVES][TT][E]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t0 = blockIdx.x * TT;
    const uint32_t nt = a.T - t0 < (uint32_t)TT ? a.T - t0 : (uint32_t)TT;
    // the first group's codes and scales do not depend on h: in flight from the start
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, E * H);
    uint32_t row[EPL]; // byte offset of each owned expert's codes (out of range if none)
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const uint32_t e = lane + 64 * j;
        row[j] = e < E ? e * H : kOutOfRange;
    }
    const uint32_t g0 = wave * NG / WAVES, g1 = (wave + 1) * NG / WAVES;
    float acc[EPL][TT];
#pragma unroll
    for (int j = 0; j < EPL; ++j)
#pragma unroll
        for (int t = 0; t < TT; ++t)
            acc[j][t] = 0.0f;
    u32x4_t q4[EPL][4], nq[EPL][4];
    uint32_t sb[EPL], nsb[EPL]; // bf16 scale (low half) and bias (high half) of the group
    auto load_group = [&](u32x4_t (&dst)[EPL][4], uint32_t (&dsb)[EPL], uint32_t g) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                dst[j][i] = load_b128(rq, row[j] == kOutOfRange ? kOutOfRange : row[j] + g * kQGroup + 16 * i);
            const uint32_t e = lane + 64 * j;
            const uint32_t er = e < E ? e : E - 1;
            dsb[j] = (uint32_t)a.qs[(size_t)er * NG + g] | ((uint32_t)a.qb[(size_t)er * NG + g] << 16);
        }
    };
    if (g0 < g1)
        load_group(nq, nsb, g0);
    // the tile's rows into LDS (16-byte loads, a batch in flight per thread), then the
    // sums of squares and the scaling from there
    {
        const __amdgpu_buffer_rsrc_t rh = make_rsrc(a.h + (size_t)t0 * H, nt * H * 4);
        constexpr int kBatch = 4;
        const uint32_t n4 = TT * H / 4;
        for (uint32_t i0 = threadIdx.x; i0 < n4; i0 += kBatch * blockDim.x) {
            u32x4_t v[kBatch];
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const uint32_t i = i0 + b * blockDim.x;
                v[b] = load_b128(rh, i < n4 ? i * 16 : kOutOfRange); // rows past nt read 0
            }
#pragma unroll
            for (int b = 0; b < kBatch; ++b) {
                const uint32_t i = i0 + b * blockDim.x;
                if (i < n4)
                    *reinterpret_cast<u32x4_t *>(xn + 4 * i) = v[b];
            }
        }
    }
    __syncthreads();
    for (uint32_t t = wave; t < (uint32_t)TT; t += WAVES) {
        float ss = 0.0f;
        for (uint32_t i = lane; i < H; i += 64)
            ss += xn[t * H + i] * xn[t * H + i];
        ss = group_sum<64>(ss);
        if (lane == 0)
            inv_s[t] = t < nt ? 1.0f / sqrtf(ss / (float)H + a.eps) : 0.0f;
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < TT * H; i += blockDim.x)
        xn[i] = xn[i] * inv_s[i / H] * bf16_bits_to_f32(a.norm_w[i % H]);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < TT * NG; i += blockDim.x) {
        const float *r = xn + (i / NG) * H + (i % NG) * kQGroup;
        float sum = 0.0f;
        for (uint32_t j = 0; j < kQGroup; ++j)
            sum += r[j];
        gsum[i] = sum;
    }
    __syncthreads();
    for (uint32_t g = g0; g < g1; ++g) {
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q4[j][i] = nq[j][i];
            sb[j] = nsb[j];
        }
        if (g + 1 < g1)
            load_group(nq, nsb, g + 1);
        float aq[EPL][TT];
#pragma unroll
        for (int j = 0; j < EPL; ++j)
#pragma unroll
            for (int t = 0; t < TT; ++t)
                aq[j][t] = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            float q[EPL][4];
#pragma unroll
            for (int j = 0; j < EPL; ++j) {
                const uint32_t wv = q4[j][w / 4][w % 4];
#pragma unroll
                for (int b = 0; b < 4; ++b)
                    q[j][b] = (float)((wv >> (8 * b)) & 0xFFu);
            }
#pragma unroll
            for (int t = 0; t < TT; ++t) {
                const float4 xv = *reinterpret_cast<const float4 *>(xn + t * H + g * kQGroup + 4 * w);
#pragma unroll
                for (int j = 0; j < EPL; ++j) {
                    aq[j][t] = __builtin_fmaf(xv.x, q[j][0], aq[j][t]);
                    aq[j][t] = __builtin_fmaf(xv.y, q[j][1], aq[j][t]);
                    aq[j][t] = __builtin_fmaf(xv.z, q[j][2], aq[j][t]);
                    aq[j][t] = __builtin_fmaf(xv.w, q[j][3], aq[j][t]);
                }
            }
        }
#pragma unroll
        for (int j = 0; j < EPL; ++j) {
            const float sc = __uint_as_float(sb[j] << 16);
            const float bi = __uint_as_float(sb[j] & 0xFFFF0000u);
#pragma unroll
            for (int t = 0; t < TT; ++t)
                acc[j][t] += sc * aq[j][t] + bi * gsum[t * NG + g];
        }
    }
#pragma unroll
    for (int j = 0; j < EPL; ++j) {
        const uint32_t e = lane + 64 * j;
        if (e < E)
#pragma unroll
            for (int t = 0; t < TT; ++t)
                part[(wave * TT + t) * E + e] = acc[j][t];
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < nt * E; i += blockDim.x) {
        const uint32_t t = i / E, e = i % E;
        float v = 0.0f;
        for (int w = 0; w < WAVES; ++w)
            v += part[(w * TT + t) * E + e];
        a.logits[(size_t)(t0 + t) * E + e] = v;
    }
}

// Router logits for few tokens (decode): one workgroup per (token, 16 experts), so the
// weight stream (E x H bytes) spreads over T * E / 16 workgroups instead of T.  Wave w
// owns experts e0 + 4w .. e0 + 4w + 3, 16 lanes each; lane j of an expert owns the
// 64-element groups j, j + 16, ... (K <= 4096: at most 4), whose codes it loads at
// entry, before the token's row is normalised into LDS (the rmsNormCpu order, as the
// tiled kernel); per group `scale * sum_k xn q + bias * sum_k xn`, then the 16 lanes'
// partial logits are summed by DPP.
constexpr uint32_t kRouterSmallExperts = 16;
constexpr uint32_t kRouterSmallTokens = 64; // the (token, expert block) form up to this
constexpr int kRouterSmallSlots = (int)(kRouterMaxHidden / kQGroup / 16);

__global__ __launch_bounds__(256) void moe_router_small_kernel(MoeRouterArgs a) {
    __shared__ __attribute__((aligned(16))) float xn[kRouterMaxHidden];
    __shared__ float gsum[kRouterMaxHidden / kQGroup];
    __shared__ float red[4];
    const uint32_t t = blockIdx.x, H = a.H, E = a.E, NG = H / kQGroup;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane % 16;
    const uint32_t e = blockIdx.y * kRouterSmallExperts + 4 * wave + lane / 16;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, E * H);
    const __amdgpu_buffer_rsrc_t rqs = make_rsrc(a.qs, E * NG * 2), rqb = make_rsrc(a.qb, E * NG * 2);
    // Every load of the kernel goes out at entry, with offsets the compiler cannot see
    // through (a select it can see becomes a branch around the load) and no load
    // waited for before the last is issued: codes, group scales and biases, the token's
    // row and the norm weights.
    u32x4_t q4[kRouterSmallSlots][4];
    uint32_t sc[kRouterSmallSlots], bi[kRouterSmallSlots];
#pragma unroll
    for (int s = 0; s < kRouterSmallSlots; ++s) {
        const uint32_t g = j + 16 * s;
        const bool ok = e < E && g < NG;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t off = ok ? e * H + g * kQGroup + 16 * i : kOutOfRange;
            asm volatile("" : "+v"(off));
            q4[s][i] = load_b128(rq, off);
        }
        uint32_t so = ok ? (e * NG + g) * 2 : kOutOfRange;
        asm volatile("" : "+v"(so));
        sc[s] = load_u16(rqs, so);
        bi[s] = load_u16(rqb, so);
    }
    // the token's row (4 floats per piece) and its norm weights, all pieces at once
    constexpr int kRowPieces = kRouterMaxHidden / 4 / 256;
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(a.h + (size_t)t * H, H * 4);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.norm_w, H * 2);
    u32x4_t hv[kRowPieces];
    uint32_t wv[kRowPieces][4];
#pragma unroll
    for (int r = 0; r < kRowPieces; ++r) {
        const uint32_t i = threadIdx.x + 256 * r;
        uint32_t off = i < H / 4 ? i * 16 : kOutOfRange;
        asm volatile("" : "+v"(off));
        hv[r] = load_b128(rh, off);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            wv[r][c] = load_u16(rw, off == kOutOfRange ? kOutOfRange : off / 2 + 2 * c);
    }
    float ss = 0.0f;
#pragma unroll
    for (int r = 0; r < kRowPieces; ++r)
#pragma unroll
        for (int c = 0; c < 4; ++c)
            ss += __uint_as_float(hv[r][c]) * __uint_as_float(hv[r][c]);
    ss = group_sum<64>(ss);
    if (lane == 0)
        red[wave] = ss;
    __syncthreads();
    const float inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)H + a.eps);
#pragma unroll
    for (int r = 0; r < kRowPieces; ++r) {
        const uint32_t i = threadIdx.x + 256 * r;
        if (i < H / 4)
#pragma unroll
            for (int c = 0; c < 4; ++c)
                xn[4 * i + c] = __uint_as_float(hv[r][c]) * inv * bf16_bits_to_f32((uint16_t)wv[r][c]);
    }
    __syncthreads();
    for (uint32_t g = wave; g < NG; g += 4) { // a group of 64 per wave, summed by DPP
        const float sum = group_sum<64>(xn[g * kQGroup + lane]);
        if (lane == 0)
            gsum[g] = sum;
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < kRouterSmallSlots; ++s) {
        const uint32_t g = j + 16 * s;
        if (g >= NG)
            break;
        float aq = 0.0f;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            const uint32_t wv = q4[s][w / 4][w % 4];
            const float4 xv = *reinterpret_cast<const float4 *>(xn + g * kQGroup + 4 * w);
            aq = __builtin_fmaf(xv.x, (float)(wv & 0xFFu), aq);
            aq = __builtin_fmaf(xv.y, (float)((wv >> 8) & 0xFFu), aq);
            aq = __builtin_fmaf(xv.z, (float)((wv >> 16) & 0xFFu), aq);
            aq = __builtin_fmaf(xv.w, (float)(wv >> 24), aq);
        }
        acc += __uint_as_float(sc[s] << 16) * aq + __uint_as_float(bi[s] << 16) * gsum[g];
    }
    acc = group_sum<16>(acc);
    if (j == 0 && e < E)
        a.logits[(size_t)t * E + e] = acc;
}

template <int TT, int WAVES> size_t router_lds(const MoeRouterArgs &a) {
    const uint32_t NG = a.H / kQGroup;
    return 4 * ((size_t)TT * a.H + (size_t)TT * NG + (size_t)WAVES * TT * a.E);
}

__global__ __launch_bounds__(256) void moe_route_kernel(const uint16_t *logits, uint32_t T,
                                                        uint32_t E, uint32_t k, int32_t *ids,
                                                        float *w) {
    const int lane = threadIdx.x & 63;
    const uint32_t t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= T)
        return;
    int32_t id;
    float wt;
    route_token(logits + (size_t)t * E, E, k, lane, id, wt);
    if ((uint32_t)lane < k) {
        ids[(size_t)t * k + lane] = id;
        w[(size_t)t * k + lane] = wt;
    }
}

// Exclusive prefix sum over the 64 lanes of a wave; `total` receives the sum of all
// lanes.  Inclusive scans within rows of 16 by DPP row shifts (lanes shifted in from
// outside the row read 0), then each row adds the totals of the rows below it.
__device__ __forceinline__ int wave_excl_scan(int x, int lane, int &total) {
    int incl = x;
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xF, 0xF, true); // row_shr:1
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xF, 0xF, true); // row_shr:2
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xF, 0xF, true); // row_shr:4
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xF, 0xF, true); // row_shr:8
    const int r0 = __builtin_amdgcn_readlane(incl, 15), r1 = __builtin_amdgcn_readlane(incl, 31),
              r2 = __builtin_amdgcn_readlane(incl, 47), r3 = __builtin_amdgcn_readlane(incl, 63);
    const int row = lane >> 4;
    incl += (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
    total = r0 + r1 + r2 + r3;
    return incl - x;
}

// Plan from per-expert pair counts `cnt` (kMoeMaxExperts entries, zero from E on; one
// workgroup of >= kMoeMaxExperts threads): header, counts, offsets, the active expert
// list and the m-tile list of the grouped GEMMs -- entries (expert, first pos, rows,
// blocks): per expert, full tiles of 256 rows (8 blocks of 32) and a tail tile of as
// many 32-row blocks as its remainder needs, ordered by blocks (8 first, then 7, ...,
// 1) so the grid deals the longest tiles first.  The tail's 32-row granularity keeps
// padding low (at the 4096-token Zipf routing 34,688 MFMA rows for 32,768 pairs,
// against 38,080 with 256/128/64-row tails).  Counts, offsets and tile slots come from
// exclusive scans over the experts (a wave scan per 64 experts, then the waves'
// totals), so every expert's entries are written in parallel.  `first` receives each
// expert's first position.
constexpr int kTileClasses = 8; // tiles of 8, 7, ..., 1 blocks of 32 rows
constexpr int kPlanScans = 2 + kTileClasses; // pair counts, active flags, tiles per class

__device__ void plan_scan(const MoeArgs &a, const int *cnt, int *first, bool publish = true) {
    __shared__ int wsum[kPlanScans][kMoeMaxExperts / 64];
    const uint32_t E = a.E, P = a.T * a.k;
    const PlanView v = plan_view(a.plan, E, P);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    constexpr int kWaves = kMoeMaxExperts / 64;
    // experts 0..255 on the first 4 waves (experts >= E count 0): per scan, an exclusive
    // wave scan plus the totals of the waves below
    const bool mine = tid < (int)kMoeMaxExperts;
    const int c = tid < (int)E ? cnt[tid] : 0;
    const int full = c / 256, blocks = (c % 256 + 31) / 32; // tail tile: 0..8 blocks
    int val[kPlanScans] = {}, excl[kPlanScans] = {};
    val[0] = c;
    val[1] = c > 0;
    val[2] = full + (blocks == 8);         // class 0: tiles of 8 blocks
#pragma unroll
    for (int i = 1; i < kTileClasses; ++i) // class i: a tail of 8 - i blocks
        val[2 + i] = blocks == kTileClasses - i;
    if (mine) {
#pragma unroll
        for (int q = 0; q < kPlanScans; ++q) {
            int tot;
            excl[q] = wave_excl_scan(val[q], lane, tot);
            if (lane == 0)
                wsum[q][wave] = tot;
        }
    }
    __syncthreads();
    int total[kPlanScans];
#pragma unroll
    for (int q = 0; q < kPlanScans; ++q) {
        total[q] = 0;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            if (w < wave)
                excl[q] += wsum[q][w];
            total[q] += wsum[q][w];
        }
    }
    // first tile slot of each class: 8 blocks first, then 7, ..., 1
    int base[kTileClasses];
    base[0] = 0;
#pragma unroll
    for (int i = 1; i < kTileClasses; ++i)
        base[i] = base[i - 1] + total[2 + i - 1];
    if (tid < (int)E) {
        const int e = tid;
        const int off = excl[0];
        first[e] = off;
    }
    if (publish && tid < (int)E) {
        const int e = tid;
        const int off = excl[0];
        v.off[e] = off;
        v.cnt[e] = c;
        if (c > 0)
            v.act[excl[1]] = e;
        const int t0 = excl[2];
        for (int f = 0; f < full; ++f) {
            int32_t *t = v.tiles + 4 * (t0 + f);
            t[0] = e, t[1] = off + 256 * f, t[2] = 256, t[3] = kTileClasses;
        }
        if (blocks > 0) {
            const int cls = kTileClasses - blocks;
            const int slot = cls == 0 ? t0 + full : base[cls] + excl[2 + cls];
            int32_t *t = v.tiles + 4 * slot;
            t[0] = e, t[1] = off + 256 * full, t[2] = c % 256, t[3] = blocks;
        }
    }
    if (publish && tid == 0) {
        v.off[E] = total[0];
        v.hdr[0] = total[1];
        int nt = 0;
#pragma unroll
        for (int i = 0; i < kTileClasses; ++i)
            nt += total[2 + i];
        v.hdr[1] = nt;
        // tiles of more than 4 blocks (classes 0..3), reported with the plan
        v.hdr[2] = total[2] + total[3] + total[4] + total[5];
    }
    __syncthreads();
}

// Prefill grouping, deterministic and free of contended atomics, in three launches whose
// work is linear in the tokens (O(T/16 * E) reads in all):
// 1. moe_route_hist_kernel: each workgroup routes kRouteBlockTokens (16) tokens and marks,
//    per expert, the bit of every one of its tokens that chose it (LDS atomicOr, whose
//    result does not depend on order).  A pair's rank inside its workgroup's group is
//    the popcount of its expert's mask below its token's bit; the mask's popcount is
//    the workgroup's count for the expert -> hist[block][expert].
// 2. moe_hist_scan_kernel: per expert, an exclusive scan of hist over the blocks of each
//    of kScanChunks chunks (in place: hist[b][e] becomes the expert's pairs in the
//    chunk's blocks before b) and the chunks' totals into hist rows nb ...
// 3. moe_place_kernel (one workgroup per routing block): the totals summed and scanned
//    over the experts (plan_scan, published by workgroup 0) and pos = off[e] + (pairs in
//    earlier chunks) + hist[b][e] + rank for the block's pairs.
// kRouteBlockTokens (moe.h) tokens per workgroup of 16 waves, one per wave: a wave's
// top-k rounds are a chain of dependent wave reductions, so more tokens per wave
// lengthen the workgroup (4 per wave: 15.2 against 7.2 us at 4096 tokens).
constexpr uint32_t kRouteWaves = 16;
constexpr uint32_t kRouteTokensPerWave = kRouteBlockTokens / kRouteWaves;
static_assert(kRouteBlockTokens <= 64, "a block's tokens are bits of one 64-bit mask");

__global__ __launch_bounds__(64 * kRouteWaves) void moe_route_hist_kernel(MoeArgs a) {
    __shared__ unsigned long long mask[kMoeMaxExperts];
    __shared__ int32_t s_id[kRouteBlockTokens * kMoeMaxTopK];
    const uint32_t E = a.E, k = a.k;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t t0 = blockIdx.x * kRouteBlockTokens;
    const uint32_t nt = a.T - t0 < kRouteBlockTokens ? a.T - t0 : kRouteBlockTokens;
    TokenLogits pre[kRouteTokensPerWave];
#pragma unroll
    for (uint32_t i = 0; i < kRouteTokensPerWave; ++i) {
        const uint32_t tl = wave + kRouteWaves * i;
        if (tl < nt)
            pre[i] = load_token_logits(a, t0 + tl, lane);
    }
    for (uint32_t e = threadIdx.x; e < kMoeMaxExperts; e += blockDim.x)
        mask[e] = 0;
    __syncthreads();
#pragma unroll
    for (uint32_t i = 0; i < kRouteTokensPerWave; ++i) {
        const uint32_t tl = wave + kRouteWaves * i;
        if (tl >= nt)
            break;
        const uint32_t t = t0 + tl;
        int32_t id;
        float wt;
        route_token_loaded(a, pre[i], lane, id, wt);
        if ((uint32_t)lane < k) {
            a.ids[(size_t)t * k + lane] = id;
            a.w[(size_t)t * k + lane] = wt;
            s_id[tl * k + lane] = id;
            atomicOr(&mask[id], 1ull << tl);
        }
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < nt * k; q += blockDim.x) {
        const uint32_t tl = q / k;
        const unsigned long long below = (1ull << tl) - 1;
        a.rank[(size_t)t0 * k + q] = __popcll(mask[s_id[q]] & below);
    }
    for (uint32_t e = threadIdx.x; e < E; e += blockDim.x)
        a.hist[(size_t)blockIdx.x * E + e] = __popcll(mask[e]);
}

// Column scan of hist in kScanChunks chunks of blocks, one workgroup per (64 experts,
// chunk): lane l owns expert 64 g + l, wave w a quarter of the chunk's blocks.  Pass 1
// sums each thread's blocks; the waves' sums are scanned through LDS; pass 2 rewrites
// each block's count with the expert's pairs in the chunk's blocks before it.  The
// chunk's totals go to hist row nb + chunk.  Each entry is read twice and written once,
// and every workgroup walks at most ceil(nb / kScanChunks / 4) blocks per thread.
constexpr uint32_t kScanWaves = 4;

__global__ __launch_bounds__(64 * kScanWaves) void moe_hist_scan_kernel(MoeArgs a) {
    __shared__ int s_sum[kScanWaves][64];
    const uint32_t E = a.E;
    const uint32_t nb = (a.T + kRouteBlockTokens - 1) / kRouteBlockTokens;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t e = blockIdx.x * 64 + lane, c = blockIdx.y;
    const uint32_t bpc = (nb + kScanChunks - 1) / kScanChunks;
    const uint32_t spw = (bpc + kScanWaves - 1) / kScanWaves;
    const uint32_t c0 = min(c * bpc, nb), c1 = min(c0 + bpc, nb);
    const uint32_t b0 = min(c0 + wave * spw, c1), b1 = min(b0 + spw, c1);
    int32_t *col = a.hist + e;
    const bool mine = e < E;
    int sum = 0;
    for (uint32_t b = b0; b < b1; b += 8) {
        int v[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i)
            v[i] = mine && b + i < b1 ? col[(size_t)(b + i) * E] : 0;
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i)
            sum += v[i];
    }
    s_sum[wave][lane] = sum;
    __syncthreads();
    int run = 0, total = 0;
#pragma unroll
    for (int w = 0; w < (int)kScanWaves; ++w) {
        const int v = s_sum[w][lane];
        run += w < wave ? v : 0;
        total += v;
    }
    if (mine && wave == 0)
        col[(size_t)(nb + c) * E] = total;
    for (uint32_t b = b0; b < b1; b += 8) {
        int v[8];
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i)
            v[i] = mine && b + i < b1 ? col[(size_t)(b + i) * E] : 0;
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            if (mine && b + i < b1)
                col[(size_t)(b + i) * E] = run;
            run += v[i];
        }
    }
}

// One workgroup per routing block b of chunk c: the per-expert totals (the sums of the
// chunk totals, hist rows nb ..) scanned over the experts (plan_scan; workgroup 0
// publishes the plan), then the block's pairs: pos = off[e] + (pairs of e in the chunks
// before c) + hist[b][e] (pairs of e in c's blocks before b) + rank.
__global__ __launch_bounds__(256) void moe_place_kernel(MoeArgs a) {
    __shared__ int cnt[kMoeMaxExperts], first[kMoeMaxExperts], before[kMoeMaxExperts];
    const uint32_t E = a.E, k = a.k, b = blockIdx.x;
    const uint32_t nb = (a.T + kRouteBlockTokens - 1) / kRouteBlockTokens;
    const uint32_t c = b / ((nb + kScanChunks - 1) / kScanChunks);
    for (uint32_t e = threadIdx.x; e < kMoeMaxExperts; e += blockDim.x) {
        int tot = 0, pre = 0;
        if (e < E) {
            int v[kScanChunks];
#pragma unroll
            for (uint32_t q = 0; q < kScanChunks; ++q)
                v[q] = a.hist[(size_t)(nb + q) * E + e];
#pragma unroll
            for (uint32_t q = 0; q < kScanChunks; ++q) {
                pre += q < c ? v[q] : 0;
                tot += v[q];
            }
        }
        cnt[e] = tot;
        before[e] = pre;
    }
    __syncthreads();
    plan_scan(a, cnt, first, b == 0);
    const uint32_t P = a.T * k;
    const PlanView v = plan_view(a.plan, E, P);
    const uint32_t p0 = b * kRouteBlockTokens * k;
    const uint32_t np = min(kRouteBlockTokens * k, P - p0);
    const int32_t *pre = a.hist + (size_t)b * E;
    for (uint32_t i = threadIdx.x; i < np; i += blockDim.x) {
        const uint32_t p = p0 + i;
        const int ex = a.ids[p];
        const int pos = first[ex] + before[ex] + pre[ex] + a.rank[p];
        v.pos_of_pair[p] = pos;
        v.pair_of_pos[pos] = (int32_t)p;
    }
}

// Decode plan from the experts' token masks (bit t of mask[e]: token t chose expert e),
// by one wave: lane l owns experts 4l..4l+3.  Counts, offsets (pairs grouped by expert,
// experts ascending, each expert's tokens ascending), the active list and the token
// groups (sizes 4, 3, 2, 1 in that order, see moe_gemv_kernel) -> plan; offsets also
// -> s_off.
__device__ void plan_from_masks(const MoeArgs &a, int32_t *plan, const uint32_t *mask, int32_t *s_off,
                                int lane) {
    static_assert(kTokenGroup == 4 && kMoeMaxExperts == 256, "4 experts per lane, group sizes 4..1");
    const uint32_t E = a.E, P = a.T * a.k;
    const PlanView v = plan_view(plan, E, P);
    int c[4];
    int sum[6] = {}; // pairs, active experts, groups of 4, of 3, of 2, of 1
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t e = 4 * lane + q;
        c[q] = e < E ? __popc(mask[e]) : 0;
        sum[0] += c[q];
        sum[1] += c[q] > 0;
        sum[2] += c[q] / 4;
        sum[3] += c[q] % 4 == 3;
        sum[4] += c[q] % 4 == 2;
        sum[5] += c[q] % 4 == 1;
    }
    int base[6], total[6];
#pragma unroll
    for (int i = 0; i < 6; ++i)
        base[i] = wave_excl_scan(sum[i], lane, total[i]);
    // first group slot of each class: sizes 4, 3, 2, 1 in that order
    const int cls0[4] = {0, total[2], total[2] + total[3], total[2] + total[3] + total[4]};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t e = 4 * lane + q;
        if (e >= E)
            break;
        const int n = c[q], off = base[0];
        s_off[e] = off;
        v.off[e] = off;
        v.cnt[e] = n;
        if (n > 0)
            v.act[base[1]++] = (int32_t)e;
        for (int f = 0; f < n / 4; ++f) {
            const int g = cls0[0] + base[2]++;
            v.groups[2 * g] = (int32_t)e;
            v.groups[2 * g + 1] = (off + 4 * f) | (4 << 16);
        }
        const int r = n % 4;
        if (r > 0) {
            const int cls = 4 - r; // 1 (3 tokens) .. 3 (1 token)
            const int g = cls0[cls] + base[2 + cls]++;
            v.groups[2 * g] = (int32_t)e;
            v.groups[2 * g + 1] = (off + 4 * (n / 4)) | (r << 16);
        }
        base[0] += n;
    }
    if (lane == 0) {
        v.off[E] = total[0];
        v.hdr[0] = total[1];
        v.hdr[1] = 0;
        v.hdr[2] = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i)
            v.hdr[3 + i] = total[2 + i];
    }
}

// Decode: route all T <= 32 tokens (one per wave) and plan, in one workgroup, with
// no atomics whose order matters: each routed pair sets its token's bit in its
// expert's mask (LDS atomicOr), one wave turns the masks into the plan, and a pair's
// position is its expert's offset plus the number of its expert's tokens below its
// own (so positions do not depend on timing).  The plan goes to `plan` (global memory
// or an LDS copy); ids and weights go to a.ids / a.w when `write_routes`.
struct RoutePlanLds {
    uint32_t mask[kMoeMaxExperts];
    int32_t off[kMoeMaxExperts];
    int32_t ids[kMoeGemvMaxPairs];
};

// `meanwhile` runs in every thread between the routing and the plan's barrier -- in
// waves 1.. while wave 0 builds the plan -- for independent setup work.
template <typename Meanwhile>
__device__ void route_plan_block(const MoeArgs &a, int32_t *plan, RoutePlanLds &s, bool write_routes,
                                 Meanwhile meanwhile) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const uint32_t k = a.k, P = a.T * k, nwaves = blockDim.x / 64;
    // the wave's first two tokens' logits load while the masks are cleared
    TokenLogits pre[2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
        if (wave + i * nwaves < a.T)
            pre[i] = load_token_logits(a, wave + i * nwaves, lane);
    for (uint32_t e = threadIdx.x; e < kMoeMaxExperts; e += blockDim.x)
        s.mask[e] = 0;
    __syncthreads();
    auto record = [&](uint32_t t, int32_t id, float wt) {
        if ((uint32_t)lane < k) {
            if (write_routes) {
                a.ids[t * k + lane] = id;
                a.w[t * k + lane] = wt;
            }
            s.ids[t * k + lane] = id;
            atomicOr(&s.mask[id], 1u << t);
        }
    };
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const uint32_t t = wave + i * nwaves;
        if (t < a.T) {
            int32_t id;
            float wt;
            route_token_loaded(a, pre[i], lane, id, wt);
            record(t, id, wt);
        }
    }
    for (uint32_t t = wave + 2 * nwaves; t < a.T; t += nwaves) {
        int32_t id;
        float wt;
        route_token_args(a, t, lane, id, wt);
        record(t, id, wt);
    }
    __syncthreads();
    if (wave == 0)
        plan_from_masks(a, plan, s.mask, s.off, lane);
    meanwhile();
    __syncthreads();
    const PlanView v = plan_view(plan, a.E, P);
    for (uint32_t p = threadIdx.x; p < P; p += blockDim.x) {
        const uint32_t t = p / k;
        const int e = s.ids[p];
        const int pos = s.off[e] + __popc(s.mask[e] & ((1u << t) - 1u));
        v.pos_of_pair[p] = pos;
        v.pair_of_pos[pos] = (int32_t)p;
    }
    __syncthreads();
}

__global__ __launch_bounds__(1024) void moe_route_plan_kernel(MoeArgs a) {
    __shared__ RoutePlanLds s;
    route_plan_block(a, a.plan, s, true, [] {});
}

// ---------------------------------------------------------------------------------
// Decode: grouped GEMVs
// ---------------------------------------------------------------------------------

// x pieces of chunk c = gl + s*G of one bf16 row at byte offset `row_off` (chunks past
// the row read zeros).
template <int G>
__device__ __forceinline__ XChunk<uint16_t> load_x_slot(__amdgpu_buffer_rsrc_t r, uint32_t row_off,
                                                       int gl, int s, int nchunks) {
    const int c = gl + s * G;
    const uint32_t off = c < nchunks ? row_off + (uint32_t)c * 64 : kOutOfRange;
    XChunk<uint16_t> xc;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        xc.p[q] = load_b128(r, off + q * 16);
    return xc;
}

// Dots of NR weight rows (row sets whose loads are in `w`) with one activation row
// whose slot-s chunk `xslot(s)` returns, reduced over the G-lane groups.  The fast
// E4M3 conversion maps 0x7F/0xFF to NaN (the reference decodes +-480): a NaN result
// is recomputed with the exact decode.
template <int G, int SLOTS, int NR, bool SERIAL_X, typename XSlot>
__device__ __forceinline__ void rows_dot(float (&out)[NR], const RowRegs<SLOTS> (&w)[NR],
                                         XSlot xslot) {
    auto pass = [&](auto exact) {
#pragma unroll
        for (int r = 0; r < NR; ++r)
            out[r] = 0.0f;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const XChunk<uint16_t> xc = xslot(s);
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                // Tie the weight words to x's arrival: the compiler would otherwise decode
                // every row and slot ahead of the x wait and exceed the register budget.
                u32x4_t cw = w[r].codes[s];
                asm volatile("" : "+v"(cw) : "v"(xc.p[3]));
                chunk_dot(cw, chunk_scales<decltype(exact)::value>(w[r].scales[s]), xc, out[r]);
            }
            // SERIAL_X (x read from LDS): the next slot's reads wait for this slot's
            // dots instead of being hoisted, keeping one slot of x in registers.
            if constexpr (SERIAL_X)
                asm volatile("" ::"v"(out[NR - 1]) : "memory");
        }
#pragma unroll
        for (int r = 0; r < NR; ++r)
            out[r] = group_sum<G>(out[r]);
    };
    pass(std::false_type{});
    bool nan = false;
#pragma unroll
    for (int r = 0; r < NR; ++r)
        nan |= __builtin_isnan(out[r]);
    if (nan)
        pass(std::true_type{});
}

// chunk_dot with the chunk's codes already decoded (wd[4 p + j] = elements 8 p + 2 j
// and 8 p + 2 j + 1).
__device__ __forceinline__ void chunk_dot_decoded(const bf16x2_t (&wd)[16], f32x2_t s,
                                                  const XChunk<uint16_t> &x, float &acc) {
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        float partial = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const int p = 2 * b + h;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t xw = x.p[p][j];
                partial = __builtin_amdgcn_fdot2_f32_bf16(wd[4 * p + j],
                                                          __builtin_bit_cast(bf16x2_t, xw),
                                                          partial, false);
            }
        }
        acc = __builtin_fmaf(s[b], partial, acc);
    }
}

// Dots of NR weight rows with the activation rows of n <= TG tokens (one group of an
// expert's positions): each slot's codes are decoded once and dotted with every
// token's chunk `xslot(t, s)`, so the half-rate conversions are shared by the group.
// Same arithmetic per (row, token) as rows_dot; NaN results are recomputed with the
// exact E4M3 decode.
template <int G, int SLOTS, int NR, int TG, typename XSlot>
__device__ __forceinline__ void rows_dot_group(float (&out)[TG][NR], const RowRegs<SLOTS> (&w)[NR],
                                               int n, XSlot xslot) {
    auto pass = [&](auto exact) {
#pragma unroll
        for (int t = 0; t < TG; ++t)
#pragma unroll
            for (int r = 0; r < NR; ++r)
                out[t][r] = 0.0f;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            bf16x2_t wd[NR][16];
            f32x2_t sc[NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                // decode after the previous slot's dots: one slot of decoded rows live
                u32x4_t cw = w[r].codes[s];
                asm volatile("" : "+v"(cw) : "v"(out[0][NR - 1]));
#pragma unroll
                for (int p = 0; p < 4; ++p)
                    e2m1x8_to_bf16(cw[p], &wd[r][4 * p]);
                sc[r] = chunk_scales<decltype(exact)::value>(w[r].scales[s]);
            }
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                if (t >= n)
                    break;
                const XChunk<uint16_t> xc = xslot(t, s);
#pragma unroll
                for (int r = 0; r < NR; ++r)
                    chunk_dot_decoded(wd[r], sc[r], xc, out[t][r]);
                // one token's x chunk in registers at a time
                asm volatile("" ::"v"(out[t][NR - 1]) : "memory");
            }
        }
#pragma unroll
        for (int t = 0; t < TG; ++t) {
            if (t >= n)
                break;
#pragma unroll
            for (int r = 0; r < NR; ++r)
                out[t][r] = group_sum<G>(out[t][r]);
        }
    };
    pass(std::false_type{});
    bool nan = false;
#pragma unroll
    for (int t = 0; t < TG; ++t)
#pragma unroll
        for (int r = 0; r < NR; ++r)
            nan |= t < n && __builtin_isnan(out[t][r]);
    if (nan)
        pass(std::true_type{});
}

// Decode gate/up GEMV over the routed (token, expert) pairs, in items of equal cost per
// class that persistent waves walk round-robin, so they get equal shares however
// unevenly the tokens spread over experts.  K = H, gate and up rows side by side, GeGLU
// in registers -> h[pos][row] (bf16).
//   TG == 1: item (rb, pos) = row block rb (NB row sets of 64/G rows) of pos's expert
//     dotted with pos's activation row; item i = (i / P, i % P), so the n positions
//     of one expert are consecutive and the n items streaming the same weight rows
//     run on adjacent waves of one workgroup (all but the first read them from L2).
//   TG > 1 (x in LDS): item (rb, g) = row block rb of group g's expert dotted with the
//     rows of the group's n <= TG tokens, decoding the weights once for all of them.
//     Items are dealt class by class (groups of 4 tokens first, then 3, 2, 1), each
//     class rb-major, round-robin over workgroups first, so every CU and SIMD gets an
//     equal share of every cost class.
// XLDS: all T activation rows are staged in LDS once per workgroup (piece-major, so
// a wave's 16-byte reads of one piece of consecutive chunks are conflict-free) and
// read from there; otherwise each item's row is loaded from global memory (L2).
// Double-buffering the weights (next item's loads during this item's arithmetic)
// measured slower at every shape: four waves per SIMD already cover the latency and
// the second register set costs occupancy or spills.  (The down GEMV is
// moe_down_group_kernel.)
constexpr int kGemvBlocksPerCU = 4; // 256-thread workgroups per CU (global x)
constexpr int kXLdsThreads = 1024;  // x in LDS: one workgroup of 16 waves per CU
constexpr uint32_t kXLdsBytes = 120 * 1024;

// Activation rows staged in LDS as [row][4 pieces][nchunks + 1] 16-byte entries: entry
// (r, q, c) = bytes [64 c + 16 q, +16) of the row at byte offset row_off(r) of `rs`, and
// chunk nchunks of every (r, q) plane is zero (its load lies past the descriptor), so
// lanes past the end of a row read zeros without a branch.  Each thread issues all its
// loads (up to kStagePerThread) before its first LDS write, so the copy costs one
// memory round trip; a load-then-write loop waits for each load in turn (~1 us each
// at kernel start, when every CU copies at once).
constexpr int kStagePerThread = 8;
static_assert(kStagePerThread * kXLdsThreads * 16 >= kXLdsBytes, "one round covers the LDS budget");

// One round of the copy: entries threadIdx.x + k * blockDim.x (k < kStagePerThread)
// loaded into registers by stage_issue, written to LDS by stage_commit, so independent
// work can run while the loads are in flight.
struct StageRegs {
    u32x4_t v[kStagePerThread];
    uint32_t dst[kStagePerThread];
};

template <typename RowOff>
__device__ __forceinline__ void stage_issue(StageRegs &st, __amdgpu_buffer_rsrc_t rs, uint32_t n_rows,
                                            int nchunks, uint32_t base, RowOff row_off) {
    const uint32_t nc = (uint32_t)nchunks + 1, per_row = 4 * nc, n = n_rows * per_row;
    // (row, piece) of element i = base + tid + k * blockDim.x, stepped without a
    // division per element (the per-element divisions cost ~1 us of issue per call)
    const uint32_t i0 = base + threadIdx.x;
    uint32_t r = i0 / per_row, rem = i0 - r * per_row;
    const uint32_t step_r = blockDim.x / per_row, step_rem = blockDim.x - step_r * per_row;
#pragma unroll
    for (int k = 0; k < kStagePerThread; ++k) {
        const uint32_t i = i0 + k * blockDim.x;
        uint32_t off = kOutOfRange;
        st.dst[k] = 0xFFFFFFFFu;
        if (i < n) {
            const uint32_t c = rem / 4, q = rem % 4;
            if ((int)c < nchunks)
                off = row_off(r) + c * 64 + q * 16;
            st.dst[k] = (r * 4 + q) * nc + c;
        }
        st.v[k] = load_b128(rs, off);
        rem += step_rem;
        r += step_r;
        if (rem >= per_row) {
            rem -= per_row;
            ++r;
        }
    }
}

// Branch-free (a slot with nothing to stage writes a dummy LDS word instead), so the
// compiler's load waits count exactly: a later load (the first item's weights) is not
// waited for.
__device__ __forceinline__ void stage_commit(const StageRegs &st, uint4 *xl) {
    __shared__ uint4 s_discard;
#pragma unroll
    for (int k = 0; k < kStagePerThread; ++k) {
        uint4 *dst = st.dst[k] != 0xFFFFFFFFu ? xl + st.dst[k] : &s_discard;
        *dst = __builtin_bit_cast(uint4, st.v[k]);
    }
}

template <typename RowOff>
__device__ __forceinline__ void stage_rows(uint4 *xl, __amdgpu_buffer_rsrc_t rs, uint32_t n_rows,
                                           int nchunks, RowOff row_off) {
    const uint32_t n = n_rows * 4 * ((uint32_t)nchunks + 1);
    for (uint32_t base = 0; base < n; base += kStagePerThread * blockDim.x) {
        StageRegs st;
        stage_issue(st, rs, n_rows, nchunks, base, row_off);
        stage_commit(st, xl);
    }
}

// Plan words of the decode regime (header, counts, offsets, active list, both position
// maps and the token groups; no m-tiles) at the largest E and T * k.
constexpr uint32_t kDecodePlanWords = kMoePlanHeader + 3 * kMoeMaxExperts + 1 + 4 * kMoeGemvMaxPairs;

template <int G, int SLOTS, int NB, bool XLDS, int TG, bool ROUTE = false>
__global__ __launch_bounds__(XLDS ? kXLdsThreads : 256, XLDS ? kXLdsThreads / 256 : 4) void moe_gemv_kernel(MoeArgs a) {
    static_assert(TG == 1 || (XLDS && TG == kTokenGroup), "token groups read x from LDS");
    static_assert(!ROUTE || XLDS, "routing runs in the workgroups that stage x in LDS");
    constexpr int R = 64 / G;          // rows per row set
    constexpr int NM = 2; // gate, up
    constexpr int NR = NM * NB;
    // TG == 1: s_exp[pos] = expert of grouped position pos.  TG > 1: s_exp[g] = expert
    // of group g, s_grp[g] = its first position | size << 16.  s_xrow[pos] = activation
    // row of pos (token or pos).  Staged in LDS so the per-item lookups never wait
    // behind the weight stream.
    __shared__ int s_exp[kMoeGemvMaxPairs];
    __shared__ uint32_t s_grp[TG > 1 ? kMoeGemvMaxPairs : 1];
    __shared__ uint32_t s_xrow[kMoeGemvMaxPairs];
    __shared__ uint32_t s_next; // TG > 1: the workgroup's next unclaimed item index
    extern __shared__ uint4 xl[];                 // XLDS: [T][4 pieces][nchunks + 1]
    const int lane = threadIdx.x & 63;
    const int sub = lane / G, gl = lane % G;
    const uint32_t P = a.T * a.k, H = a.H, I = a.I;
    const uint32_t K = H, rows = I;
    const int nchunks = (int)(K / 32);
    // ROUTE: every workgroup routes the T tokens and plans into LDS itself (the same
    // deterministic plan everywhere, no launch of its own); workgroup 0 also writes the
    // routes and the plan to global memory for the down and combine kernels.
    int32_t *plan = a.plan;
    const int32_t *ids = a.ids;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.T * H * 2);
    auto x_row = [&](uint32_t t) { return t * K * 2; };
    if constexpr (ROUTE) {
        __shared__ int32_t s_plan[kDecodePlanWords];
        __shared__ RoutePlanLds s_rp;
        // x's loads fly while the tokens are routed (the host keeps x within one round)
        StageRegs st;
        stage_issue(st, rx, a.T, nchunks, 0, x_row);
        route_plan_block(a, s_plan, s_rp, blockIdx.x == 0, [&] { stage_commit(st, xl); });
        if (blockIdx.x == 0) {
            const uint32_t words = kMoePlanHeader + 3 * a.E + 1 + 4 * P;
            for (uint32_t i = threadIdx.x; i < words; i += blockDim.x)
                a.plan[i] = s_plan[i];
        }
        plan = s_plan;
        ids = s_rp.ids;
    }
    const PlanView v = plan_view(plan, a.E, P);
    uint32_t ncls[kTokenGroup] = {}; // TG > 1: groups of size 4, 3, 2, 1
    uint32_t ng = 0;
    if constexpr (TG > 1) {
#pragma unroll
        for (int q = 0; q < kTokenGroup; ++q) {
            ncls[q] = uniform(v.hdr[3 + q]);
            ng += ncls[q];
        }
    }
    const uint32_t wave = uniform(threadIdx.x >> 6);
    const uint32_t waves_per_block = blockDim.x / 64;
    const uint32_t per_e = (rows + R * NB - 1) / (R * NB);
    const uint32_t items = per_e * (TG > 1 ? ng : P);
    const bool last_ok = gl + (SLOTS - 1) * G < nchunks;
    const uint32_t last_c = last_ok ? (SLOTS - 1) * G * 16 : kOutOfRange;
    const uint32_t last_s = last_ok ? (SLOTS - 1) * G * 2 : kOutOfRange;
    const uint64_t off_w[2] = {a.slots.gate_w, a.slots.up_w};
    const uint64_t off_s[2] = {a.slots.gate_s, a.slots.up_s};
    const uint32_t wbytes = rows * K / 2, sbytes = rows * K / 16;
    const uint32_t nw = gridDim.x * waves_per_block;
    // TG > 1: group g's expert and (first position | size << 16) -- straight from the
    // plan when it is in LDS (ROUTE), else from the LDS copies made below
    auto group_expert = [&](uint32_t g) { return ROUTE ? v.groups[2 * g] : s_exp[g]; };
    auto group_info = [&](uint32_t g) {
        return ROUTE ? (uint32_t)v.groups[2 * g + 1] : s_grp[g];
    };

    // item it -> (row block, position or group)
    auto locate = [&](uint32_t it, uint32_t &rb, uint32_t &j) {
        if constexpr (TG == 1) {
            rb = it / P;
            j = it - rb * P;
        } else {
            uint32_t g0 = 0;
#pragma unroll
            for (int q = 0; q < kTokenGroup; ++q) {
                const uint32_t nq = ncls[q];
                if (it < per_e * nq) {
                    rb = it / nq;
                    j = g0 + (it - rb * nq);
                    return;
                }
                it -= per_e * nq;
                g0 += nq;
            }
        }
    };
    // Loads of item it's weight rows into `w` (nothing for an item past the end).
    auto issue = [&](RowRegs<SLOTS> (&w)[NR], uint32_t it) {
        if (it >= items)
            return;
        uint32_t rb, j;
        locate(it, rb, j);
        const uint32_t r0 = rb * R * NB;
        const int e = TG > 1 ? group_expert(j) : s_exp[j];
        const uint8_t *slot = a.slots.base + (size_t)uniform(e) * a.slots.stride;
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                const uint32_t row = r0 + b * R + sub;
                load_row<SLOTS, G>(w[m * NB + b], make_rsrc(slot + off_w[m], wbytes),
                                   make_rsrc(slot + off_s[m], sbytes), row < rows ? row : rows, gl,
                                   K, last_c, last_s);
            }
    };
    // x chunk of slot s of activation row xr, from LDS
    auto lds_x = [&](uint32_t xr, int s) {
        const int c = min(gl + s * G, nchunks); // chunk nchunks is zero
        const uint4 *plane = xl + xr * 4 * (nchunks + 1) + c;
        XChunk<uint16_t> xc;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            xc.p[q] = __builtin_bit_cast(u32x4_t, plane[q * (nchunks + 1)]);
        return xc;
    };
    // the bf16 outputs of one (row set b, position pos) from its dots
    auto store = [&](const float *dots, uint32_t r0, uint32_t pos) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const uint32_t row = r0 + b * R + sub;
            if (row >= rows)
                continue;
            a.h[(size_t)pos * I + row] = f32_to_bf16_bits(gelu_tanh_fast(dots[b]) * dots[NB + b]);
        }
    };
    // Item it's rows (loaded into `w`) against its activation rows.
    auto compute = [&](const RowRegs<SLOTS> (&w)[NR], uint32_t it) {
        uint32_t rb, j;
        locate(it, rb, j);
        const uint32_t r0 = rb * R * NB;
        if constexpr (TG == 1) {
            const uint32_t xr = uniform(s_xrow[j]);
            float dots[NR];
            if constexpr (XLDS) {
                rows_dot<G, SLOTS, NR, true>(dots, w, [&](int s) { return lds_x(xr, s); });
            } else {
                rows_dot<G, SLOTS, NR, false>(dots, w, [&](int s) {
                    return load_x_slot<G>(rx, xr * K * 2, gl, s, nchunks);
                });
            }
            if (gl == 0)
                store(dots, r0, j);
        } else {
            const uint32_t gp = uniform(group_info(j));
            const int p0 = (int)(gp & 0xFFFFu), n = (int)(gp >> 16);
            float dots[TG][NR];
            rows_dot_group<G, SLOTS, NR, TG>(dots, w, n, [&](int t, int s) {
                return lds_x(uniform(s_xrow[p0 + t]), s);
            });
            if (gl == 0)
#pragma unroll
                for (int t = 0; t < TG; ++t) {
                    if (t >= n)
                        break;
                    store(dots[t], r0, p0 + t);
                }
        }
    };

    // TG > 1 with the plan in LDS: the wave's first item's weight loads go out now,
    // while the rest of the setup runs
    RowRegs<SLOTS> w_first[NR];
    constexpr bool kEarly = ROUTE && TG > 1;
    if constexpr (kEarly)
        issue(w_first, blockIdx.x + gridDim.x * wave);
    for (uint32_t i = threadIdx.x; i < P; i += blockDim.x) {
        const uint32_t pair = (uint32_t)v.pair_of_pos[i];
        if constexpr (TG == 1)
            s_exp[i] = ids[pair];
        s_xrow[i] = pair / a.k;
    }
    if constexpr (TG > 1 && !ROUTE) {
        for (uint32_t i = threadIdx.x; i < ng; i += blockDim.x) {
            s_exp[i] = v.groups[2 * i];
            s_grp[i] = (uint32_t)v.groups[2 * i + 1];
        }
    }
    if constexpr (XLDS && !ROUTE)
        stage_rows(xl, rx, a.T, nchunks, x_row);
    if (threadIdx.x == 0)
        s_next = blockDim.x / 64;
    if constexpr (kEarly) {
        // the LDS writes above must be visible to every wave, but the first item's
        // weight loads need not land before the barrier (__syncthreads would wait for
        // them): wait for LDS only, then the bare barrier
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    } else {
        __syncthreads();
    }

    // TG == 1: consecutive items (which share weight rows) on the waves of one
    // workgroup.  TG > 1: consecutive items on consecutive workgroups, so every CU gets
    // an even share of each cost class -- workgroup b takes items b + gridDim.x j,
    // j = 0, 1, ..., its waves claiming the next j from an LDS counter as they finish
    // (each wave starts at j = its index): with static dealing (wave w on j = w mod 16)
    // a workgroup's waves finished up to 11 us apart (items differ in group size, and
    // 7-8 items per wave leave a whole item of imbalance), the kernel waiting for the
    // last; claimed, a workgroup's waves end within about an item.
    if constexpr (TG == 1) {
        for (uint32_t it = blockIdx.x * waves_per_block + wave; it < items; it += nw) {
            RowRegs<SLOTS> w[NR];
            issue(w, it);
            compute(w, it);
        }
    } else {
        bool issued = kEarly;
        for (uint32_t j = wave;; issued = false) {
            const uint32_t it = blockIdx.x + gridDim.x * j;
            if (it >= items)
                break;
            if (!issued)
                issue(w_first, it);
            uint32_t next = 0;
            if (lane == 0)
                next = atomicAdd(&s_next, 1u);
            j = uniform(next);
            compute(w_first, it);
        }
    }
}

// Decode down GEMV over token groups, h staged in LDS by segment.  At decode sizes the
// down GEMV is bound by its weight decode and dots rather than by its bytes (one
// position per item: 28 us for 8 distinct experts, 31 us for 128, at 128 positions),
// so each item decodes its weight rows once for a whole group (up to kTokenGroup
// positions of one expert, see plan_from_masks), and 8-lane row groups keep 22 of
// every 24 chunk slots busy at I = 704 (32-lane groups: 22 of 32).  Measured against
// the per-position kernel: 18 vs 28 us (8 experts), 26 vs 30 us (83 experts of 128
// positions), 34 vs 31 us (128 experts, no group larger than 1: the 8-lane groups
// read 4x the x bytes per weight byte from LDS).
//   The groups' h rows are read from LDS, and all P rows need not fit: the groups are
// split over S segments, group g in segment g % S (so every size class splits
// evenly), workgroup b serves segment b % S and stages only its segment's rows -- per
// class at most one group more than an even share, so at most ceil(P / S) + 10 rows,
// which the host sizes `cap` and S for.
//   Items (row block rb of R * NB rows, group i of the segment) are dealt class by class
// (groups of 4, 3, 2, 1 positions), rb-major, round-robin over the segment's workgroups,
// so every CU gets an even share of each cost class; a workgroup's waves claim its
// items in that order from an LDS counter.  The first item's weight loads are issued
// before the h rows are staged.
template <int G, int SLOTS, int NB>
__global__ __launch_bounds__(kXLdsThreads, kXLdsThreads / 256) void moe_down_group_kernel(MoeArgs a, uint32_t S,
                                                                                     uint32_t cap) {
    constexpr int R = 64 / G;
    constexpr int TG = kTokenGroup;
    __shared__ int s_exp[kMoeGemvMaxPairs];      // expert of the segment's group i
    __shared__ uint32_t s_grp[kMoeGemvMaxPairs]; // its first staged row | size << 16
    __shared__ uint32_t s_pos[kMoeGemvMaxPairs]; // position of staged row j
    __shared__ uint32_t s_nrows;
    __shared__ uint32_t s_next;                  // the workgroup's next unclaimed item index
    extern __shared__ uint4 xl[];                // [staged row][4 pieces][nchunks + 1]
    const int lane = threadIdx.x & 63;
    const int sub = lane / G, gl = lane % G;
    const uint32_t P = a.T * a.k, H = a.H, I = a.I;
    const int nchunks = (int)(I / 32);
    const uint32_t nc = (uint32_t)nchunks + 1;
    const PlanView v = plan_view(a.plan, a.E, P);
    const uint32_t seg = blockIdx.x % S, wg = blockIdx.x / S;
    const uint32_t nwg = (gridDim.x - seg + S - 1) / S;
    const uint32_t wave = uniform(threadIdx.x >> 6);
    // the segment's groups per size class: g in [lo, hi) with g % S == seg
    auto below = [&](uint32_t x) { return (x + S - 1 - seg) / S; };
    uint32_t ncls[TG], ngs = 0;
    {
        uint32_t lo = 0;
#pragma unroll
        for (int q = 0; q < TG; ++q) {
            const uint32_t hi = lo + uniform(v.hdr[3 + q]);
            ncls[q] = below(hi) - below(lo);
            ngs += ncls[q];
            lo = hi;
        }
    }
    if (wave == 0) {
        uint32_t base = 0;
        for (uint32_t i0 = 0; i0 < ngs; i0 += 64) {
            const uint32_t i = i0 + lane;
            int e = 0;
            uint32_t p0 = 0, n = 0;
            if (i < ngs) {
                const uint32_t g = seg + S * i;
                e = v.groups[2 * g];
                const uint32_t gp = (uint32_t)v.groups[2 * g + 1];
                p0 = gp & 0xFFFFu;
                n = gp >> 16;
            }
            int total;
            const uint32_t off = base + (uint32_t)wave_excl_scan((int)n, lane, total);
            if (i < ngs) {
                s_exp[i] = e;
                s_grp[i] = off | (n << 16);
                for (uint32_t u = 0; u < n; ++u)
                    s_pos[off + u] = p0 + u;
            }
            base += (uint32_t)total;
        }
        if (lane == 0)
            s_nrows = base;
    }
    if (threadIdx.x == 0)
        s_next = blockDim.x / 64;
    __syncthreads();

    const uint32_t per_e = (H + R * NB - 1) / (R * NB);
    const uint32_t items = per_e * ngs;
    const bool last_ok = gl + (SLOTS - 1) * G < nchunks;
    const uint32_t last_c = last_ok ? (SLOTS - 1) * G * 16 : kOutOfRange;
    const uint32_t last_s = last_ok ? (SLOTS - 1) * G * 2 : kOutOfRange;
    const uint32_t wbytes = H * I / 2, sbytes = H * I / 16;
    auto locate = [&](uint32_t it, uint32_t &rb, uint32_t &i) {
        uint32_t g0 = 0;
#pragma unroll
        for (int q = 0; q < TG; ++q) {
            const uint32_t nq = ncls[q];
            if (it < per_e * nq) {
                rb = it / nq;
                i = g0 + (it - rb * nq);
                return;
            }
            it -= per_e * nq;
            g0 += nq;
        }
    };
    // Loads of item it's weight rows; an item past the end loads row H of expert
    // s_exp[0] -- past the descriptors' end, so nothing is read (zeros) -- so a caller
    // need not branch around it.
    auto issue = [&](RowRegs<SLOTS> (&w)[NB], uint32_t it) {
        const bool ok = it < items;
        uint32_t rb = 0, i = 0;
        locate(ok ? it : 0u, rb, i);
        const uint8_t *slot = a.slots.base + (size_t)uniform(s_exp[i]) * a.slots.stride;
        const __amdgpu_buffer_rsrc_t rc = make_rsrc(slot + a.slots.down_w, wbytes);
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(slot + a.slots.down_s, sbytes);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const uint32_t row = rb * R * NB + b * R + sub;
            load_row<SLOTS, G>(w[b], rc, rs, ok && row < H ? row : H, gl, I, last_c, last_s);
        }
    };
    // x chunk of slot s of staged row j (j < cap by the segment bound; the clamp only
    // keeps the reads inside the staged rows)
    auto lds_x = [&](uint32_t j, int s) {
        const int c = min(gl + s * G, nchunks); // chunk nchunks is zero
        const uint4 *plane = xl + min(j, cap - 1) * 4 * nc + c;
        XChunk<uint16_t> xc;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            xc.p[q] = __builtin_bit_cast(u32x4_t, plane[q * nc]);
        return xc;
    };
    auto compute = [&](const RowRegs<SLOTS> (&w)[NB], uint32_t it) {
        uint32_t rb, i;
        locate(it, rb, i);
        const uint32_t gp = uniform(s_grp[i]);
        const uint32_t j0 = gp & 0xFFFFu;
        const int n = (int)(gp >> 16);
        float dots[TG][NB];
        rows_dot_group<G, SLOTS, NB, TG>(dots, w, n, [&](int t, int s) { return lds_x(j0 + t, s); });
        if (gl == 0)
#pragma unroll
            for (int t = 0; t < TG; ++t) {
                if (t >= n)
                    break;
                const uint32_t pos = uniform(s_pos[j0 + t]);
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    const uint32_t row = rb * R * NB + b * R + sub;
                    if (row < H)
                        a.d[(size_t)pos * H + row] = f32_to_bf16_bits(dots[t][b]);
                }
            }
    };

    // workgroup wg takes items wg + nwg j, j = 0, 1, ...: each wave starts at j = its
    // index and claims the next j from an LDS counter (static dealing, wave w on
    // j = w mod 16, left a workgroup's waves finishing up to 6 us apart)
    auto item = [&](uint32_t j) { return wg + nwg * j; };
    auto claim = [&]() {
        uint32_t next = 0;
        if (lane == 0)
            next = atomicAdd(&s_next, 1u);
        return item(uniform(next));
    };
    const uint32_t first = item(wave);
    RowRegs<SLOTS> wa[NB], wb[NB];
    // the segment's h rows (staged row j = h[s_pos[j]]): the first batch's loads go out,
    // then the first item's weight loads, so writing the batch to LDS waits only for
    // the h loads (a wave's loads complete in order)
    {
        const __amdgpu_buffer_rsrc_t rh = make_rsrc(a.h, P * I * 2);
        const uint32_t nrows = min(s_nrows, cap);
        auto h_row = [&](uint32_t j) { return s_pos[j] * I * 2; };
        StageRegs st;
        stage_issue(st, rh, nrows, nchunks, 0, h_row);
        asm volatile("" ::: "memory"); // keep the load order: h first
        issue(wa, first);              // unconditional: the waits above stay exact
        asm volatile("" ::: "memory");
        stage_commit(st, xl);
        const uint32_t n = nrows * 4 * ((uint32_t)nchunks + 1);
        for (uint32_t base = kStagePerThread * blockDim.x; base < n; base += kStagePerThread * blockDim.x) {
            stage_issue(st, rh, nrows, nchunks, base, h_row);
            stage_commit(st, xl);
        }
    }
    // the staged rows must be visible to every wave, but the first item's weight loads
    // need not land before the barrier (__syncthreads would wait for them): wait for
    // LDS only, then the bare barrier
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // two register sets: the next item's weight loads are in flight during this item's
    // decode and dots
    for (uint32_t it = first; it < items;) {
        const uint32_t it2 = claim();
        if (it2 < items)
            issue(wb, it2);
        compute(wa, it);
        if (it2 >= items)
            break;
        it = claim();
        if (it < items)
            issue(wa, it);
        compute(wb, it2);
    }
}

// ---------------------------------------------------------------------------------
// Prefill: grouped GEMMs
// ---------------------------------------------------------------------------------

using namespace gemm_core;
constexpr int kGateUpCols = BN / 2; // h columns per gate/up tile

// HALF: the tile's h columns past c0 + 64 do not exist (the last n-tile when I % 128 ==
// 64), so it runs as the half-width tile -- 2 x 2 waves on W rows 0..127, each wave row
// on half the token rows -- instead of leaving two of the four waves on zero W rows.
template <int MT, bool HALF>
__device__ __forceinline__ void gateup_tile(const MoeArgs &a, uint8_t *lds, const int32_t *pair_of_pos,
                                            int e, uint32_t row0, uint32_t nrows, uint32_t c0) {
    const uint32_t H = a.H, I = a.I, k = a.k;
    const uint8_t *slot = a.slots.base + (size_t)e * a.slots.stride;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.x, a.T * H * 2);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(slot, (uint32_t)a.slots.stride);
    const uint32_t gw = (uint32_t)a.slots.gate_w, uw = (uint32_t)a.slots.up_w;
    const uint32_t gs = (uint32_t)a.slots.gate_s, us = (uint32_t)a.slots.up_s;
    auto a_row = [=](int r) {
        return (uint32_t)r < nrows ? (uint32_t)pair_of_pos[row0 + r] / k * H * 2 : kOut;
    };
    // W tile row r: matrix (r % 64) / 32 (gate, up), h column c0 + 32 (r / 64) + r % 32
    auto w_code = [=](int r) {
        const uint32_t col = c0 + 32 * (r / 64) + r % 32;
        return col < I ? ((r & 32) ? uw : gw) + col * (H / 2) : kOut;
    };
    auto w_scale = [=](int r) {
        const uint32_t col = c0 + 32 * (r / 64) + r % 32;
        return col < I ? ((r & 32) ? us : gs) + col * (H / 16) : kOut;
    };
    const __amdgpu_buffer_rsrc_t rw2[2] = {rw, rw};
    // h[row0 + r][col] = gelu(gate) * up, 16-byte stores (I is a multiple of 64, so
    // 8-column pieces never straddle it); the store descriptor ends at row nrows.
    constexpr int MTW = HALF ? MT / 2 : MT; // 32-row A blocks per wave
    constexpr int WC = HALF ? 2 : 4;
    Acc<MTW, WC, 2> acc;
    gemm_tile<MTW, WC, 2>(lds, ra, rw2, rw2, H, a_row, w_code, w_scale, acc);
    store_tile_geglu<MTW, uint16_t, WC>(acc, a.h + (size_t)row0 * I, I, nrows, c0, I, 1.0f, 1.0f, true);
}

// Workgroups are dispatched round-robin over the 8 XCDs (workgroup b on XCD b % 8).
// Workgroup b takes n-tile s % nn of m-tile 8 (s / nn) + b % 8, s = b / 8: each XCD
// walks all n-tiles of one m-tile in turn, so the m-tile's A rows (gathered token rows
// or h rows) are fetched into that XCD's L2 once, and consecutive m-tiles -- big ones
// first -- are dealt to the XCDs in turn.  The grid is a multiple of 8 * nn and covers
// the largest possible m-tile count; workgroups past the device's count exit at once.
__device__ __forceinline__ void xcd_tile(uint32_t nn, uint32_t &mt, uint32_t &nt) {
    const uint32_t s = blockIdx.x / 8;
    mt = 8 * (s / nn) + blockIdx.x % 8;
    nt = s % nn;
}

__global__ __launch_bounds__(kThreads) void moe_gateup_gemm_kernel(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t E = a.E, P = a.T * a.k;
    const PlanView v = plan_view(a.plan, E, P);
    const uint32_t nn = (a.I + kGateUpCols - 1) / kGateUpCols;
    uint32_t mt, nt;
    xcd_tile(nn, mt, nt);
    if (mt >= uniform(v.hdr[1]))
        return;
    const int32_t *t = v.tiles + 4 * mt;
    const int e = uniform(t[0]), blocks = uniform(t[3]); // 32-row blocks, 1..8
    const uint32_t row0 = uniform(t[1]), nrows = uniform(t[2]), c0 = nt * kGateUpCols;
    const int32_t *pp = v.pair_of_pos;
    if (c0 + kGateUpCols / 2 >= a.I) { // 64 h columns left: the half-width tile, whose
        // two wave rows split the token rows (an odd block count runs one block more)
        switch ((blocks + 1) / 2) {
        case 4: gateup_tile<8, true>(a, lds, pp, e, row0, nrows, c0); break;
        case 3: gateup_tile<6, true>(a, lds, pp, e, row0, nrows, c0); break;
        case 2: gateup_tile<4, true>(a, lds, pp, e, row0, nrows, c0); break;
        default: gateup_tile<2, true>(a, lds, pp, e, row0, nrows, c0); break;
        }
        return;
    }
    switch (blocks) {
    case 8: gateup_tile<8, false>(a, lds, pp, e, row0, nrows, c0); break;
    case 7: gateup_tile<7, false>(a, lds, pp, e, row0, nrows, c0); break;
    case 6: gateup_tile<6, false>(a, lds, pp, e, row0, nrows, c0); break;
    case 5: gateup_tile<5, false>(a, lds, pp, e, row0, nrows, c0); break;
    case 4: gateup_tile<4, false>(a, lds, pp, e, row0, nrows, c0); break;
    case 3: gateup_tile<3, false>(a, lds, pp, e, row0, nrows, c0); break;
    case 2: gateup_tile<2, false>(a, lds, pp, e, row0, nrows, c0); break;
    default: gateup_tile<1, false>(a, lds, pp, e, row0, nrows, c0); break;
    }
}

template <int MT>
__device__ __forceinline__ void down_tile(const MoeArgs &a, uint8_t *lds, int e, uint32_t row0,
                                          uint32_t nrows, uint32_t n0) {
    const uint32_t H = a.H, I = a.I, P = a.T * a.k;
    const uint8_t *slot = a.slots.base + (size_t)e * a.slots.stride;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(a.h, P * I * 2);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(slot, (uint32_t)a.slots.stride);
    const uint32_t dw = (uint32_t)a.slots.down_w, ds = (uint32_t)a.slots.down_s;
    auto a_row = [=](int r) { return (uint32_t)r < nrows ? (row0 + r) * I * 2 : kOut; };
    auto w_code = [=](int r) { return n0 + r < H ? dw + (n0 + r) * (I / 2) : kOut; };
    auto w_scale = [=](int r) { return n0 + r < H ? ds + (n0 + r) * (I / 16) : kOut; };
    const __amdgpu_buffer_rsrc_t rw2[2] = {rw, rw};
    Acc<MT, 4> acc;
    gemm_tile<MT, 4>(lds, ra, rw2, rw2, I, a_row, w_code, w_scale, acc);
    // Whole-row stores staged through the drained LDS ring: 3% faster than the direct
    // 16-byte pieces on this short-K GEMM (the GeGLU gate/up epilogue was 5% slower
    // staged, so it stores directly).
    store_tile_bf16_lds<MT>(acc, lds, a.d + (size_t)row0 * H, H, 0, n0, nrows, H, 1.0f);
}

// Down GEMM over the gate/up GEMM's m-tiles (up to 256 rows: 1-8 blocks of 32), one
// workgroup per CU on the chunked-W tile core, tiles dealt as the gate/up GEMM's
// (xcd_tile).  Measured against 128-row halves at two workgroups per CU (the previous
// form, whose 3-stage per-stage W ring fit two in the LDS but left W one stage of
// latency cover): the same 178 us (fastest of ~100 launches) and 185 vs 189 us on
// average, with one tile list for both GEMMs.
__global__ __launch_bounds__(kThreads) void moe_down_gemm_kernel(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t E = a.E, P = a.T * a.k;
    const PlanView v = plan_view(a.plan, E, P);
    const uint32_t nn = (a.H + BN - 1) / BN;
    uint32_t mt, nt;
    xcd_tile(nn, mt, nt);
    if (mt >= uniform(v.hdr[1]))
        return;
    const int32_t *t = v.tiles + 4 * mt;
    const int e = uniform(t[0]);
    const uint32_t row0 = uniform(t[1]), nrows = uniform(t[2]);
    const uint32_t n0 = nt * BN;
    switch ((nrows + 31) / 32) {
    case 8: down_tile<8>(a, lds, e, row0, nrows, n0); break;
    case 7: down_tile<7>(a, lds, e, row0, nrows, n0); break;
    case 6: down_tile<6>(a, lds, e, row0, nrows, n0); break;
    case 5: down_tile<5>(a, lds, e, row0, nrows, n0); break;
    case 4: down_tile<4>(a, lds, e, row0, nrows, n0); break;
    case 3: down_tile<3>(a, lds, e, row0, nrows, n0); break;
    case 2: down_tile<2>(a, lds, e, row0, nrows, n0); break;
    default: down_tile<1>(a, lds, e, row0, nrows, n0); break;
    }
}

// y[t] = sum_j w[t,j] d[pos(t,j)], slot order, fp32; 8 columns per thread.  Workgroup
// (t, c) covers columns [2048 c, 2048 c + 2048) of token t; the k pairs' rows are
// loaded 8 at a time (slots past k read zeros with weight 0) so the loads overlap.
constexpr uint32_t kCombineCols = 256 * 8;

__global__ __launch_bounds__(256) void moe_combine_kernel(MoeArgs a) {
    const uint32_t t = blockIdx.x;
    const uint32_t E = a.E, P = a.T * a.k, H = a.H, k = a.k;
    const PlanView v = plan_view(a.plan, E, P);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.d, P * H * 2);
    const uint32_t c = blockIdx.y * kCombineCols + threadIdx.x * 8;
    if (c >= H)
        return;
    float acc[8] = {};
    for (uint32_t j0 = 0; j0 < k; j0 += 8) {
        u32x4_t dv[8];
        float wt[8];
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) {
            const uint32_t j = j0 + jj;
            const bool ok = j < k;
            const uint32_t pair = t * k + (ok ? j : 0);
            wt[jj] = ok ? uniform_f(a.w[pair]) : 0.0f;
            const uint32_t pos = uniform(v.pos_of_pair[pair]);
            // streaming policy: every d row is read once (33.2 vs 34.2 us at 4096 tokens)
            dv[jj] = load_b128<APEX_WEIGHT_CPOL>(rd, ok ? (pos * H + c) * 2 : kOutOfRange);
        }
#pragma unroll
        for (int jj = 0; jj < 8; ++jj)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] += wt[jj] * bf16_bits_to_f32(dv[jj][q] & 0xFFFFu);
                acc[2 * q + 1] += wt[jj] * bf16_bits_to_f32(dv[jj][q] >> 16);
            }
    }
    u32x4_t o;
#pragma unroll
    for (int q = 0; q < 4; ++q)
        o[q] = (uint32_t)f32_to_bf16_bits(acc[2 * q]) |
               ((uint32_t)f32_to_bf16_bits(acc[2 * q + 1]) << 16);
    *reinterpret_cast<u32x4_t *>(a.y + (size_t)t * H + c) = o;
}

template <typename F> hipError_t set_lds(F *kernel, size_t bytes, std::atomic<uint64_t> &done) {
    return allow_dynamic_lds(kernel, bytes, done);
}

uint32_t gemv_slots(uint32_t K, int G) { return (K / 32 + G - 1) / G; }

// Decode down GEMV by token groups (moe_down_group_kernel): 8-lane row groups, one row
// set (8 rows) per item -- two row sets per item exceed the register budget of 16
// waves per CU with the second in-flight set.  Segments: the fewest S with
// ceil(P / S) + 10 staged rows within the LDS budget.  The decode path's limits
// (I <= 1024, P <= kMoeGemvMaxPairs) always leave one: 4 slots at most, and 16
// segments fit even the largest I.
constexpr int kDownGroupLanes = 8;
constexpr int kDownGroupNB = 1;
constexpr uint32_t kDownGroupMaxSlots = 4;
static_assert((1024 / 32 + kDownGroupLanes - 1) / kDownGroupLanes <= kDownGroupMaxSlots &&
                  (kMoeGemvMaxPairs + 15) / 16 + 10 <= kXLdsBytes / ((1024 / 32 + 1) * 64),
              "every decode shape (I <= 1024, P <= 256) has a segment count");

uint32_t down_group_segments(uint32_t P, uint32_t I, uint32_t &rows) {
    const uint32_t hrow = (I / 32 + 1) * 64;
    const uint32_t cap = kXLdsBytes / hrow;
    if (gemv_slots(I, kDownGroupLanes) > kDownGroupMaxSlots)
        return 0;
    for (uint32_t S = 1; S <= 16 && S <= (uint32_t)num_cus(); ++S)
        if ((P + S - 1) / S + 10 <= cap) {
            rows = (P + S - 1) / S + 10 < P ? (P + S - 1) / S + 10 : P;
            return S;
        }
    return 0;
}

template <int SLOTS, int NB>
hipError_t launch_down_group(const MoeArgs &a, uint32_t S, uint32_t rows, hipStream_t stream) {
    static std::atomic<uint64_t> attr{0};
    const hipError_t err = set_lds(moe_down_group_kernel<kDownGroupLanes, SLOTS, NB>, kXLdsBytes, attr);
    if (err != hipSuccess)
        return err;
    const size_t bytes = (size_t)rows * (a.I / 32 + 1) * 64;
    hipLaunchKernelGGL((moe_down_group_kernel<kDownGroupLanes, SLOTS, NB>), dim3((uint32_t)num_cus()),
                       dim3(kXLdsThreads), bytes, stream, a, S, rows);
    return hipSuccess;
}

hipError_t down_group_by_slots(const MoeArgs &a, uint32_t S, uint32_t rows, hipStream_t stream) {
    switch (gemv_slots(a.I, kDownGroupLanes)) {
    case 1: return launch_down_group<1, kDownGroupNB>(a, S, rows, stream);
    case 2: return launch_down_group<2, kDownGroupNB>(a, S, rows, stream);
    case 3: return launch_down_group<3, kDownGroupNB>(a, S, rows, stream);
    default: return launch_down_group<4, kDownGroupNB>(a, S, rows, stream);
    }
}

} // namespace

bool moe_supported(const MoeArgs &a, bool gemm, const char **why) {
    auto no = [&](const char *m) {
        *why = m;
        return false;
    };
    const uint64_t P = (uint64_t)a.T * a.k;
    const MoeSlots &s = a.slots;
    if (a.E == 0 || a.E > kMoeMaxExperts)
        return no("experts must be in [1, 256]");
    if (a.k == 0 || a.k > kMoeMaxTopK || a.k > a.E)
        return no("top_k must be in [1, min(16, experts)]");
    if (a.H % 64 || a.I % 64 || a.H == 0 || a.I == 0)
        return no("hidden and intermediate sizes must be multiples of 64");
    if ((uintptr_t)s.base % 16 || s.stride % 16 || s.gate_w % 16 || s.up_w % 16 || s.down_w % 16)
        return no("expert slots: base, stride and code offsets must be 16-byte aligned");
    if (s.gate_s % 4 || s.up_s % 4 || s.down_s % 4)
        return no("expert slots: scale offsets must be 4-byte aligned");
    const uint64_t gw = (uint64_t)a.I * a.H / 2, gsz = (uint64_t)a.I * a.H / 16;
    if (s.gate_w + gw > s.stride || s.up_w + gw > s.stride || s.down_w + gw > s.stride ||
        s.gate_s + gsz > s.stride || s.up_s + gsz > s.stride || s.down_s + gsz > s.stride)
        return no("expert slots: a piece extends past the slot stride");
    if (s.stride >= (1ull << 31) || (uint64_t)a.T * a.H * 2 >= (1ull << 31) ||
        P * a.H * 2 >= (1ull << 31) || P * a.I * 2 >= (1ull << 31))
        return no("operands must stay below 2 GiB");
    if ((uintptr_t)a.x % 16 || (uintptr_t)a.y % 16)
        return no("x and y must be 16-byte aligned");
    if (!gemm) {
        if (a.T > kMoeGemvMaxTokens || P > kMoeGemvMaxPairs)
            return no("the grouped-GEMV path takes at most 32 tokens and 256 (token, expert) pairs");
        if (gemv_slots(a.H, 32) > 3 || gemv_slots(a.I, 32) > 1)
            return no("the grouped-GEMV path takes hidden <= 3072 and intermediate <= 1024");
    }
    return true;
}

hipError_t moe_route_launch(const uint16_t *logits, uint32_t T, uint32_t E, uint32_t k,
                            int32_t *ids, float *w, hipStream_t stream) {
    if (T == 0)
        return hipSuccess;
    hipLaunchKernelGGL(moe_route_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, logits, T, E, k,
                       ids, w);
    return hipGetLastError();
}

hipError_t moe_route_f32_launch(const float *logits, const uint16_t *pes, uint32_t T, uint32_t E,
                                uint32_t k, int32_t *ids, float *w, hipStream_t stream) {
    if (T == 0)
        return hipSuccess;
    hipLaunchKernelGGL(moe_route_f32_kernel, dim3((T + 3) / 4), dim3(256), 0, stream, logits, pes,
                       T, E, k, ids, w);
    return hipGetLastError();
}

bool moe_router_supported(const MoeRouterArgs &a, const char **why) {
    auto no = [&](const char *m) {
        *why = m;
        return false;
    };
    if (a.E == 0 || a.E > kMoeMaxExperts)
        return no("experts must be in [1, 256]");
    if (a.H == 0 || a.H % kQGroup || a.H > kRouterMaxHidden)
        return no("hidden must be a positive multiple of 64, at most 4096");
    if ((uint64_t)a.E * a.H >= (1ull << 31))
        return no("router weights must be below 2 GiB");
    if ((uintptr_t)a.qw % 16)
        return no("router weights must be 16-byte aligned");
    return true;
}

// The largest dynamic LDS an instantiation can be launched with (hidden <= 4096,
// experts <= 256, and never above kMaxDynLds: larger shapes take another tile size).
// The kernel's limit is raised to it once, whatever the first call's shape.
template <int TT, int WAVES> constexpr size_t router_lds_max() {
    const size_t m = 4 * ((size_t)TT * kRouterMaxHidden + (size_t)TT * (kRouterMaxHidden / kQGroup) +
                          (size_t)WAVES * TT * kMoeMaxExperts);
    return m < kMaxDynLds ? m : kMaxDynLds;
}

template <int TT, int EPL, int WAVES>
hipError_t router_launch(const MoeRouterArgs &a, hipStream_t stream) {
    static std::atomic<uint64_t> set{0};
    const size_t lds = router_lds<TT, WAVES>(a);
    if (lds > router_lds_max<TT, WAVES>())
        return hipErrorInvalidValue;
    hipError_t e = set_lds(moe_router_kernel<TT, EPL, WAVES>, router_lds_max<TT, WAVES>(), set);
    if (e != hipSuccess)
        return e;
    hipLaunchKernelGGL((moe_router_kernel<TT, EPL, WAVES>), dim3((a.T + TT - 1) / TT),
                       dim3(64 * WAVES), lds, stream, a);
    return hipGetLastError();
}

// The most waves a workgroup of the router can have without spilling: per owned expert
// a lane holds two groups of codes (32 registers), 2 * TT partial logits, 4 decoded
// codes and 3 offsets / scales, plus about 40 of its own; a SIMD's 512 registers are
// shared by WAVES / 4 waves.
constexpr int router_waves(int TT, int EPL, int want) {
    const int need = EPL * (32 + 2 * TT + 7) + 40;
    int w = want;
    while (w > 4 && need > 512 / (w / 4))
        w /= 2;
    return w;
}

template <int TT, int WAVES>
hipError_t router_launch_epl(const MoeRouterArgs &a, hipStream_t stream) {
    switch ((a.E + 63) / 64) {
    case 1: return router_launch<TT, 1, router_waves(TT, 1, WAVES)>(a, stream);
    case 2: return router_launch<TT, 2, router_waves(TT, 2, WAVES)>(a, stream);
    case 3: return router_launch<TT, 3, router_waves(TT, 3, WAVES)>(a, stream);
    default: return router_launch<TT, 4, router_waves(TT, 4, WAVES)>(a, stream);
    }
}

namespace {

// Router logits, fused prefill form: one workgroup per block of kRfTokens tokens and
// kRfExperts experts reads the tokens' fp32 rows once and produces their logits, with
// no pass over the rows before it and no partials after it.  The RMSNorm's per-token
// factor is taken out of the sums:
//   logits[t][e] = inv[t] * sum_g (s[e][g] * sum_{k in g} q[e][k] x'[t][k]
//                                  + b[e][g] * sum_{k in g} x'[t][k]),
// x' = h * router.scale, inv = 1 / sqrt(mean(h^2) + eps) -- the reference's product
// (orc_moe_router_logits_q8) regrouped, a few fp32 roundings apart.
//   K advances in chunks of kRfGroups 64-column groups.  Four waves produce: thread p
// owns token p / 16 and 4 columns of every group of every chunk, with kRfDepth
// chunks' loads in flight (register ring); it multiplies by router.scale, adds h^2
// into the token's sum of squares, splits x' into bf16 hi + lo (x' - hi: ~16
// significant bits) straight into the MFMA operand layout in LDS, sums x' over each
// group (16 lanes), and stages the chunk's group scales (p < 128) or biases.
//   Four waves consume: consumer w takes group w of every chunk for all the block's
// experts (4 tiles of 32), so no two waves read the same operands from LDS.  x is the
// MFMA's first operand and the codes (exact in bf16, straight from L2 into registers,
// one chunk ahead) its second, so each lane's accumulators are one expert's, for 16
// tokens (of which rows 16..31 are zero padding and skipped): its group's scale and
// bias are two scalars, and s * acc + b * sum(x') folds the group into the totals.
// The four waves' totals are summed in wave order at the end.
//   The roles meet at one barrier per chunk (LDS double-buffered); each keeps its own
// loads in flight across it (a bare s_barrier: __syncthreads would wait for them).
// Both run the same padded count of chunks (columns past H read zeros), so their
// barriers pair up.
//   At 4096 tokens x 128 experts x 2816: 24.8 us, against 53 us for a split pass
// (normed rows -> bf16 hi + lo in HBM), an MFMA kernel on 128-token tiles with split
// K and a partials sum.  The small scattered loads weigh most: the codes as 16-byte
// pieces (32.7 -> 26.0 us against 8-byte ones) and the scales as one 8-byte load per
// chunk (-> 24.8 us against four 2-byte ones).
constexpr uint32_t kRfTokens = 16;
constexpr uint32_t kRfGroups = 4;
constexpr uint32_t kRfChunk = kRfGroups * kQGroup;
constexpr uint32_t kRfSteps = kRfChunk / 16; // 32x32x16 k-steps per chunk
constexpr uint32_t kRfDepth = 4;
constexpr uint32_t kRfThreads = 512;
constexpr uint32_t kRfExperts = 128;

// SB4: the group count H / 64 is a multiple of 4, so a chunk's 4 group scales (and
// biases) of an expert are one aligned 8-byte load instead of four 2-byte loads.
template <bool SB4>
__global__ __launch_bounds__(kRfThreads) void moe_router_fused_kernel(MoeRouterArgs a) {
    typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
    typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
    typedef float f32x2_v __attribute__((ext_vector_type(2)));
    typedef float f32x4_v __attribute__((ext_vector_type(4)));
    typedef uint32_t u32x2_v __attribute__((ext_vector_type(2)));
    // [buffer][hi, lo][k-step ks][slot l ^ ks]: the MFMA's first operand, lane l = token
    // l % 32; k-step kk of a group holds its columns 32 (l / 32) + 8 kk .. +7 (a
    // permutation of the group's columns, applied to x and the codes alike, so a lane's
    // codes of a group are 32 contiguous bytes); tokens 16..31 stay zero.  The XOR
    // spreads a producer store instruction over the banks.  After the last chunk it
    // holds the consumer waves' totals.
    __shared__ u32x4_t s_x[2][2][kRfSteps][64];
    __shared__ f32x2_v s_sb[2][kRfGroups][kRfExperts]; // [buffer][group][expert]: scale, bias
    __shared__ float s_sx[2][kRfGroups][32];            // [buffer][group][token]: sum of x'
    __shared__ float s_inv[kRfTokens];
    const uint32_t T = a.T, E = a.E, H = a.H, NG = H / kQGroup;
    const uint32_t nc = (H + kRfChunk - 1) / kRfChunk;
    const uint32_t ncp = (nc + kRfDepth - 1) / kRfDepth * kRfDepth; // a multiple of 2 as well
    const uint32_t t0 = blockIdx.x * kRfTokens, e0 = blockIdx.y * kRfExperts;
    const uint32_t wave = uniform(threadIdx.x >> 6);
    const uint32_t lane = threadIdx.x & 63;
    auto barrier = [] {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    // Roles by SIMD (wave w runs on SIMD w % 4): waves 0, 1, 4, 5 produce and 2, 3, 6, 7
    // consume, so no SIMD runs both (sharing one, the roles' instruction streams slowed
    // each other down: 35.6 us at 4096 tokens against 9.9 and 9.3 for each alone).
    const uint32_t ri = (wave >> 2) * 2 + (wave & 1); // index within the role, 0..3
    if ((wave & 2) == 0) {
        // ---- producers ----
        const uint32_t p = ri * 64 + lane, tk = p >> 4, m = p & 15;
        const __amdgpu_buffer_rsrc_t rh = make_rsrc(a.h, T * H * 4);
        const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.norm_w, H * 2);
        // p < 128 stage the group scales, the others the biases, of expert e0 + p % 128
        const __amdgpu_buffer_rsrc_t rsb = make_rsrc(ri < 2 ? a.qs : a.qb, E * NG * 2);
        const uint32_t xrow = t0 + tk < T ? (t0 + tk) * H * 4 : kOutOfRange;
        const uint32_t se = e0 + (p & (kRfExperts - 1));
        // Load j of a chunk: thread p reads 16-byte piece pc = p % 16 + 16 j of its
        // token's row segment (columns 4 pc .. +3, all in group j), so one load
        // instruction reads 256 contiguous bytes of each of the wave's 4 rows.
        struct Slot {
            u32x4_t x[4];
            u32x2_v w[4];
            uint32_t sb[kRfGroups];
        };
        // chunk c's loads; columns past H, tokens past T and experts past E read zeros
        auto issue = [&](Slot &s, uint32_t c) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const uint32_t k = c * kRfChunk + 4 * (m + 16 * j);
                s.x[j] = load_b128<APEX_WEIGHT_CPOL>(rh, k < H && xrow != kOutOfRange ? xrow + k * 4 : kOutOfRange);
                s.w[j] = __builtin_bit_cast(
                    u32x2_v, __builtin_amdgcn_raw_buffer_load_b64(rw, (int)(k < H ? k * 2 : kOutOfRange), 0, 0));
            }
            if constexpr (SB4) {
                const uint32_t g = kRfGroups * c;
                uint32_t off = se < E && g < NG ? (se * NG + g) * 2 : kOutOfRange;
                asm volatile("" : "+v"(off)); // no branch around the load (see issue_codes)
                const u32x2_v v2 = __builtin_bit_cast(u32x2_v, __builtin_amdgcn_raw_buffer_load_b64(rsb, (int)off, 0, 0));
                s.sb[0] = v2[0];
                s.sb[1] = v2[1];
            } else {
#pragma unroll
                for (uint32_t j = 0; j < kRfGroups; ++j) {
                    const uint32_t g = kRfGroups * c + j;
                    uint32_t off = se < E && g < NG ? (se * NG + g) * 2 : kOutOfRange;
                    asm volatile("" : "+v"(off)); // no branch around the load (see issue_codes)
                    s.sb[j] = load_u16(rsb, off);
                }
            }
        };
        float ss = 0.0f;
        auto split = [&](const Slot &s, int b) {
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                float sx = 0.0f;
                u32x2_v hi, lo;
#pragma unroll
                for (int q = 0; q < 2; ++q) {
                    const float h0 = __uint_as_float(s.x[j][2 * q]), h1 = __uint_as_float(s.x[j][2 * q + 1]);
                    const uint32_t ww = s.w[j][q];
                    const float v0 = h0 * __uint_as_float(ww << 16);
                    const float v1 = h1 * __uint_as_float(ww & 0xFFFF0000u);
                    ss = __builtin_fmaf(h0, h0, ss);
                    ss = __builtin_fmaf(h1, h1, ss);
                    sx += v0;
                    sx += v1;
                    const uint32_t hb = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_v{v0, v1}, bf16x2_v));
                    const float r0 = v0 - __uint_as_float(hb << 16), r1 = v1 - __uint_as_float(hb & 0xFFFF0000u);
                    hi[q] = hb;
                    lo[q] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_v{r0, r1}, bf16x2_v));
                }
                // group columns 4 m .. +3: k-step 4 j + (m / 2) % 4, lane half m / 8,
                // 8-byte quarter m % 2 (the group's column order, see s_x)
                const uint32_t ks = 4 * j + ((m >> 1) & 3);
                const uint32_t slot = (tk + 32 * (m >> 3)) ^ ks;
                *reinterpret_cast<u32x2_v *>(reinterpret_cast<uint8_t *>(&s_x[b][0][ks][slot]) + 8 * (m & 1)) = hi;
                *reinterpret_cast<u32x2_v *>(reinterpret_cast<uint8_t *>(&s_x[b][1][ks][slot]) + 8 * (m & 1)) = lo;
                sx = group_sum<16>(sx); // the token's 16 lanes hold group j
                if (m == 0)
                    s_sx[b][j][tk] = sx;
            }
#pragma unroll
            for (uint32_t j = 0; j < kRfGroups; ++j) {
                const uint32_t bits = SB4 ? ((j & 1) ? s.sb[j >> 1] & 0xFFFF0000u : s.sb[j >> 1] << 16)
                                          : s.sb[j] << 16;
                reinterpret_cast<float *>(&s_sb[b][j][p & (kRfExperts - 1)])[p >> 7] = __uint_as_float(bits);
            }
        };
        // Each slot's loads go out together and in slot order (compiler barriers: it
        // would otherwise group the prologue's loads by kind, and the waits for slot 0
        // would then cover the later slots' loads too).
        Slot ring[kRfDepth];
#pragma unroll
        for (uint32_t d = 0; d < kRfDepth; ++d) {
            issue(ring[d], d);
            asm volatile("" ::: "memory");
        }
        // token columns 16..31 of both x buffers: never written, read as zeros
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const uint32_t q = p + 256 * i, r = q >> 5; // r: buffer, hi/lo, k-step
            s_x[r >> 5][(r >> 4) & 1][r & 15][16 + (q & 15) + 32 * ((q >> 4) & 1)] = u32x4_t{0, 0, 0, 0};
        }
        barrier();
        for (uint32_t c0 = 0; c0 < ncp; c0 += kRfDepth) {
#pragma unroll
            for (uint32_t d = 0; d < kRfDepth; ++d) {
                split(ring[d], d & 1);
                asm volatile("" ::: "memory");
                issue(ring[d], c0 + d + kRfDepth);
                asm volatile("" ::: "memory");
                barrier();
            }
        }
        ss = group_sum<16>(ss); // the token's 16 lanes
        if (m == 0)
            s_inv[tk] = 1.0f / sqrtf(ss / (float)H + a.eps);
        barrier();
        barrier(); // the consumers' totals are in LDS
        return;
    }

    // ---- consumers ----
    const uint32_t gl = ri, er = lane & 31, kh = lane >> 5;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qw, E * H);
    // codes of chunk c, this wave's group: tile i (experts e0 + 32 i ..), lane: expert
    // e0 + 32 i + er; its four k-steps of the group are the expert's 32 code bytes
    // 32 kh .. +31 (two 16-byte loads)
    auto issue_codes = [&](u32x4_t (&cd)[4][2], uint32_t c) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t e = e0 + 32 * i + er;
#pragma unroll
            for (uint32_t hh = 0; hh < 2; ++hh) {
                const uint32_t k = c * kRfChunk + kQGroup * gl + 32 * kh + 16 * hh;
                uint32_t off = e < E && k < H ? e * H + k : kOutOfRange;
                // opaque to the compiler: it would otherwise branch around the load
                // for the out-of-range lanes instead of letting the descriptor drop it
                asm volatile("" : "+v"(off));
                cd[i][hh] = load_b128(rq, off);
            }
        }
    };
    // 8 codes (bytes, low first) -> bf16, exact
    auto cvt8 = [](u32x2_v w) {
        u32x4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t word = w[j >> 1], sh = 16 * (j & 1);
            const float f0 = (float)((word >> sh) & 0xFFu), f1 = (float)((word >> (sh + 8)) & 0xFFu);
            o[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_v{f0, f1}, bf16x2_v));
        }
        return __builtin_bit_cast(bf16x8_t, o);
    };
    // accumulator element el of a lane: expert column er, token row
    // 8 (el / 4) + 4 kh + el % 4; rows 16..31 (el >= 8) are padding
    float tot[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int el = 0; el < 8; ++el)
            tot[i][el] = 0.0f;
    // The chunk's LDS operands are read in one batch (read one by one right before
    // their MFMAs, each waited out the LDS latency); four independent accumulator
    // chains (one per tile) are interleaved.
    auto consume = [&](const u32x4_t (&cd)[4][2], int b) {
        u32x4_t xv[2][4];
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            xv[0][kk] = s_x[b][0][4 * gl + kk][lane ^ (4 * gl + kk)];
            xv[1][kk] = s_x[b][1][4 * gl + kk][lane ^ (4 * gl + kk)];
        }
        f32x2_v sb[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
            sb[i] = s_sb[b][gl][32 * i + er];
        const f32x4_v sx0 = *reinterpret_cast<const f32x4_v *>(&s_sx[b][gl][4 * kh]);
        const f32x4_v sx1 = *reinterpret_cast<const f32x4_v *>(&s_sx[b][gl][8 + 4 * kh]);
        asm volatile("" ::: "memory");
        f32x16_t acc[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int el = 0; el < 16; ++el)
                acc[i][el] = 0.0f;
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
            bf16x8_t q[4];
#pragma unroll
            for (int i = 0; i < 4; ++i)
                q[i] = cvt8(u32x2_v{cd[i][kk >> 1][2 * (kk & 1)], cd[i][kk >> 1][2 * (kk & 1) + 1]});
#pragma unroll
            for (int hl = 0; hl < 2; ++hl)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8_t, xv[hl][kk]), q[i], acc[i], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int el = 0; el < 8; ++el)
                tot[i][el] += sb[i][0] * acc[i][el] + sb[i][1] * (el < 4 ? sx0[el] : sx1[el - 4]);
    };
    u32x4_t code[2][4][2];
    issue_codes(code[0], 0);
    if (ri * 64 + lane < 2 * kRfGroups * 32)
        (&s_sx[0][0][0])[ri * 64 + lane] = 0.0f;
    barrier();
    for (uint32_t c0 = 0; c0 < ncp; c0 += 2) {
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            issue_codes(code[d ^ 1], c0 + d + 1);
            asm volatile("" ::: "memory");
            barrier();
            consume(code[d], d);
        }
    }
    barrier(); // s_inv is written; every wave is past its last read of s_x
    // totals -> LDS [wave][tile][el][lane], summed in wave order by the wave owning the tile
    float *red = reinterpret_cast<float *>(&s_x[0][0][0][0]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int el = 0; el < 8; ++el)
            red[((gl * 4 + i) * 8 + el) * 64 + lane] = tot[i][el];
    barrier();
    const uint32_t e = e0 + 32 * gl + er;
    if (e >= E)
        return;
#pragma unroll
    for (int el = 0; el < 8; ++el) {
        const uint32_t tk = 8 * (el >> 2) + 4 * kh + (el & 3), t = t0 + tk;
        float v = 0.0f;
#pragma unroll
        for (uint32_t w = 0; w < 4; ++w)
            v += red[((w * 4 + gl) * 8 + el) * 64 + lane];
        if (t < T)
            a.logits[(size_t)t * E + e] = v * s_inv[tk];
    }
}

} // namespace

bool moe_router_fused_fits(const MoeRouterArgs &a) {
    return a.E <= kMoeMaxExperts && a.H <= kRouterMaxHidden && a.H % kQGroup == 0 &&
           (uint64_t)a.T * a.H * 4 < (1ull << 31);
}

hipError_t moe_router_fused_launch(const MoeRouterArgs &a, hipStream_t stream) {
    if (a.T == 0)
        return hipSuccess;
    if (!moe_router_fused_fits(a))
        return hipErrorInvalidValue;
    // experts in blocks of kRfExperts (a second block re-reads the rows)
    const dim3 grid((a.T + kRfTokens - 1) / kRfTokens, (a.E + kRfExperts - 1) / kRfExperts);
    // 8-byte scale / bias loads: 4 groups per expert row chunk, 8-byte aligned tables
    if ((a.H / kQGroup) % kRfGroups == 0 && ((uintptr_t)a.qs | (uintptr_t)a.qb) % 8 == 0)
        hipLaunchKernelGGL(moe_router_fused_kernel<true>, grid, dim3(kRfThreads), 0, stream, a);
    else
        hipLaunchKernelGGL(moe_router_fused_kernel<false>, grid, dim3(kRfThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t moe_router_logits_launch(const MoeRouterArgs &a, hipStream_t stream) {
    if (a.T == 0)
        return hipSuccess;
    // decode sizes: a workgroup per (token, 16 experts); up to 256 tokens one token per
    // workgroup of 16 waves (parallelism over tokens and K); more: tiles of 8 (or, for
    // the widest shapes, 4) tokens share the weight reads
    if (a.T <= kRouterSmallTokens) {
        hipLaunchKernelGGL(moe_router_small_kernel,
                           dim3(a.T, (a.E + kRouterSmallExperts - 1) / kRouterSmallExperts),
                           dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    if (a.T <= 256)
        return router_launch_epl<1, 16>(a, stream);
    if (router_lds<8, 8>(a) <= kMaxDynLds)
        return router_launch_epl<8, 8>(a, stream);
    return router_launch_epl<4, 8>(a, stream);
}

// The decode path's fixed workspace (moe_static_workspace).  Host code never names the
// array in a launch or copy: its device address is looked up per device and passed on.
static __device__ __align__(256) uint8_t scratch[kMoeStaticWorkspaceBytes];

hipError_t moe_static_workspace(void **ptr) {
    constexpr int kMaxDevices = 64;
    static std::atomic<void *> addr[kMaxDevices] = {};
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess)
        return e;
    if (dev < 0 || dev >= kMaxDevices)
        return hipErrorInvalidDevice;
    void *p = addr[dev].load(std::memory_order_acquire);
    if (!p) {
        // with the device current: each device holds its own copy of the array
        if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
            return e;
        if (!p)
            return hipErrorInvalidSymbol;
        addr[dev].store(p, std::memory_order_release);
    }
    *ptr = p;
    return hipSuccess;
}

hipError_t moe_ffn_launch(const MoeArgs &a, bool gemm, hipStream_t stream) {
    if (a.T == 0)
        return hipSuccess;
    if (!gemm) {
        const dim3 grid((uint32_t)num_cus() * kGemvBlocksPerCU), block(256);
        // gate/up: 32 lanes per row; x staged in LDS when it fits (one workgroup per
        // CU, which also routes and plans), else route+plan by its own launch and x
        // read per token from global memory
        const uint32_t xbytes = a.T * (a.H / 32 + 1) * 64;
        if (xbytes <= kXLdsBytes) {
            static std::atomic<uint64_t> attr[3] = {};
            const dim3 lgrid((uint32_t)num_cus()), lblock(kXLdsThreads);
            hipError_t err = hipSuccess;
            switch (gemv_slots(a.H, 32)) {
            case 1:
                err = set_lds(moe_gemv_kernel<32, 1, 2, true, 1, true>, kXLdsBytes, attr[0]);
                hipLaunchKernelGGL((moe_gemv_kernel<32, 1, 2, true, 1, true>), lgrid, lblock, xbytes,
                                   stream, a);
                break;
            case 2:
                err = set_lds(moe_gemv_kernel<32, 2, 1, true, kTokenGroup, true>, kXLdsBytes, attr[1]);
                hipLaunchKernelGGL((moe_gemv_kernel<32, 2, 1, true, kTokenGroup, true>), lgrid, lblock,
                                   xbytes, stream, a);
                break;
            default:
                err = set_lds(moe_gemv_kernel<32, 3, 1, true, kTokenGroup, true>, kXLdsBytes, attr[2]);
                hipLaunchKernelGGL((moe_gemv_kernel<32, 3, 1, true, kTokenGroup, true>), lgrid, lblock,
                                   xbytes, stream, a);
                break;
            }
            if (err != hipSuccess)
                return err;
        } else {
            hipLaunchKernelGGL(moe_route_plan_kernel, dim3(1), dim3(1024), 0, stream, a);
            switch (gemv_slots(a.H, 32)) {
            case 1: hipLaunchKernelGGL((moe_gemv_kernel<32, 1, 2, false, 1>), grid, block, 0, stream, a); break;
            case 2: hipLaunchKernelGGL((moe_gemv_kernel<32, 2, 2, false, 1>), grid, block, 0, stream, a); break;
            default: hipLaunchKernelGGL((moe_gemv_kernel<32, 3, 1, false, 1>), grid, block, 0, stream, a); break;
            }
        }
        uint32_t rows = 0;
        const uint32_t S = down_group_segments(a.T * a.k, a.I, rows);
        if (S == 0)
            return hipErrorInvalidValue; // excluded by moe_supported's limits
        const hipError_t err = down_group_by_slots(a, S, rows, stream);
        if (err != hipSuccess)
            return err;
        hipLaunchKernelGGL(moe_combine_kernel, dim3(a.T, (a.H + kCombineCols - 1) / kCombineCols),
                           dim3(256), 0, stream, a);
        return hipGetLastError();
    }
    static std::atomic<uint64_t> lds_gateup{0}, lds_down{0};
    hipError_t err = set_lds(moe_gateup_gemm_kernel, kMaxLds, lds_gateup);
    if (err == hipSuccess)
        err = set_lds(moe_down_gemm_kernel, kMaxLds, lds_down);
    if (err != hipSuccess)
        return err;
    const uint32_t nb = (a.T + kRouteBlockTokens - 1) / kRouteBlockTokens;
    hipLaunchKernelGGL(moe_route_hist_kernel, dim3(nb), dim3(64 * kRouteWaves), 0, stream, a);
    hipLaunchKernelGGL(moe_hist_scan_kernel, dim3((a.E + 63) / 64, kScanChunks), dim3(64 * kScanWaves), 0,
                       stream, a);
    hipLaunchKernelGGL(moe_place_kernel, dim3(nb), dim3(256), 0, stream, a);
    const uint32_t mt8 = 8 * ((a.max_tiles + 7) / 8); // m-tiles rounded to whole XCD turns
    const uint32_t nn_gu = (a.I + kGateUpCols - 1) / kGateUpCols;
    hipLaunchKernelGGL(moe_gateup_gemm_kernel, dim3(mt8 * nn_gu), dim3(kThreads), kMaxLds, stream,
                       a);
    const uint32_t nn_d = (a.H + BN - 1) / BN;
    hipLaunchKernelGGL(moe_down_gemm_kernel, dim3(mt8 * nn_d), dim3(kThreads), kMaxLds, stream, a);
    hipLaunchKernelGGL(moe_combine_kernel, dim3(a.T, (a.H + kCombineCols - 1) / kCombineCols),
                       dim3(256), 0, stream, a);
    return hipGetLastError();
}

} // namespace apex_hip
