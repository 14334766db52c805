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
//   gate/up  persistent waves over (active expert, row pair) units: both gate and up
//            rows of the unit stream once and serve every token routed to the
//            expert; GeGLU in registers -> h[pos] (bf16).
//   down     one workgroup per 8 output rows; its 8 waves split the active experts,
//            stream the experts' 8 down rows and dot them with h of each routed
//            token; router-weighted partial sums meet in LDS and are added in a fixed
//            wave order (no float atomics): a deterministic combine.
// Prefill regime: MFMA grouped GEMMs on the gemm_core tile (bf16 MFMA on exactly
// dequantised weights).
//   m-tiles  per expert, 256-row tiles plus one tail tile of 256, 128 or 64 rows, big
//            tiles first; token rows are gathered through the pair list by the
//            A-tile DMA loads (no permuted copy of x).
//   gate/up  each 256-wide W tile holds 128 gate rows and the same 128 up rows, placed
//            so that a lane's two accumulator sets are gate and up of one h column:
//            GeGLU epilogue in registers -> h[pos] (bf16).
//   down     h rows are contiguous per expert -> d[pos] (bf16).
//   combine  y[t] = sum_j w[t,j] d[pos(t,j)] in slot order j, fp32 -> bf16.
#include "gemm_core.h"
#include "gemv_kernels.h"
#include "moe.h"

namespace apex_hip {

int kMoePath = 0;

namespace {

using gemv_detail::chunk_dot;
using gemv_detail::chunk_scales;
using gemv_detail::load_row;
using gemv_detail::RowRegs;
using gemv_detail::XChunk;

constexpr uint32_t kOutOfRange = 0x80000000u;

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

struct PlanView {
    int32_t *hdr, *cnt, *off, *act, *pos_of_pair, *pair_of_pos, *tiles;
};

__host__ __device__ inline PlanView plan_view(int32_t *plan, uint32_t E, uint32_t P) {
    PlanView v;
    v.hdr = plan;
    v.cnt = plan + kMoePlanHeader;
    v.off = v.cnt + E;
    v.act = v.off + E + 1;
    v.pos_of_pair = v.act + E;
    v.pair_of_pos = v.pos_of_pair + P;
    v.tiles = v.pair_of_pos + P;
    return v;
}

// ---------------------------------------------------------------------------------
// Routing
// ---------------------------------------------------------------------------------

// Top-k of one token's E logits (E <= 256) by wave 0..63 lanes, then softmax over the
// k; lane j < k returns slot j's expert id and weight.  Keys order by logit, then by
// lower expert id (the reference tie-break), and are unique per expert.
__device__ __forceinline__ void route_token(const uint16_t *logits, uint32_t E, uint32_t k,
                                            int lane, int32_t &my_id, float &my_w) {
    uint64_t key[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint32_t e = lane + 64 * q;
        if (e < E) {
            const uint32_t u = (uint32_t)logits[e] << 16;
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
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) {
            const uint32_t lo = __shfl_xor((uint32_t)best, o, 64);
            const uint32_t hi = __shfl_xor((uint32_t)(best >> 32), o, 64);
            const uint64_t other = ((uint64_t)hi << 32) | lo;
            best = other > best ? other : best;
        }
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
    const float vmax = __shfl(my_v, 0, 64); // slot 0 holds the largest logit
    float p = (uint32_t)lane < k ? expf(my_v - vmax) : 0.0f;
    float z = p;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1)
        z += __shfl_xor(z, o, 64);
    my_w = p / z;
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

// Grouping of the P = T*k pairs by expert (one workgroup of 1024 threads).  With
// `tiles`, also the m-tile list of the grouped GEMMs: entries (expert, first pos,
// rows, class) with class 0/1/2 = 256/128/64-row tiles, all class-0 tiles first.
__device__ void plan_block(const MoeArgs &a, const int32_t *ids, bool tiles) {
    __shared__ int cnt[kMoeMaxExperts], cur[kMoeMaxExperts + 1];
    const uint32_t E = a.E, P = a.T * a.k;
    PlanView v = plan_view(a.plan, E, P);
    const int tid = threadIdx.x;
    for (uint32_t e = tid; e < E; e += blockDim.x)
        cnt[e] = 0;
    __syncthreads();
    for (uint32_t p = tid; p < P; p += blockDim.x)
        atomicAdd(&cnt[ids[p]], 1);
    __syncthreads();
    if (tid == 0) {
        int off = 0, U = 0;
        for (uint32_t e = 0; e < E; ++e) {
            cur[e] = off;
            v.off[e] = off;
            v.cnt[e] = cnt[e];
            off += cnt[e];
            if (cnt[e] > 0)
                v.act[U++] = (int32_t)e;
        }
        v.off[E] = off;
        v.hdr[0] = U;
        if (tiles) {
            int n = 0, big = 0;
            for (int cls = 0; cls < 3; ++cls) {
                for (int i = 0; i < U; ++i) {
                    const int e = v.act[i];
                    const int c = cnt[e], full = c / 256, rem = c % 256;
                    int rows = 0, tile_cls = -1;
                    if (cls == 0) {
                        for (int f = 0; f < full; ++f) {
                            int32_t *t = v.tiles + 4 * n++;
                            t[0] = e, t[1] = cur[e] + 256 * f, t[2] = 256, t[3] = 0;
                        }
                        if (rem > 128)
                            rows = rem, tile_cls = 0;
                    } else if (cls == 1 && rem > 64 && rem <= 128) {
                        rows = rem, tile_cls = 1;
                    } else if (cls == 2 && rem > 0 && rem <= 64) {
                        rows = rem, tile_cls = 2;
                    }
                    if (tile_cls >= 0) {
                        int32_t *t = v.tiles + 4 * n++;
                        t[0] = e, t[1] = cur[e] + 256 * full, t[2] = rows, t[3] = tile_cls;
                    }
                }
                if (cls == 0)
                    big = n;
            }
            v.hdr[1] = n;
            v.hdr[2] = big;
        }
    }
    __syncthreads();
    for (uint32_t p = tid; p < P; p += blockDim.x) {
        const int pos = atomicAdd(&cur[ids[p]], 1);
        v.pos_of_pair[p] = pos;
        v.pair_of_pos[pos] = (int32_t)p;
    }
}

__global__ __launch_bounds__(1024) void moe_plan_kernel(MoeArgs a) { plan_block(a, a.ids, true); }

// Decode: route all T <= 32 tokens (two per wave) and plan, in one workgroup.
__global__ __launch_bounds__(1024) void moe_route_plan_kernel(MoeArgs a) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    for (uint32_t t = wave; t < a.T; t += blockDim.x / 64) {
        int32_t id;
        float wt;
        route_token(a.logits + (size_t)t * a.E, a.E, a.k, lane, id, wt);
        if ((uint32_t)lane < a.k) {
            a.ids[t * a.k + lane] = id;
            a.w[t * a.k + lane] = wt;
        }
    }
    __threadfence_block();
    __syncthreads();
    plan_block(a, a.ids, false);
}

// ---------------------------------------------------------------------------------
// Decode: grouped GEMVs
// ---------------------------------------------------------------------------------

// x chunks c = gl + s*G of one bf16 row at byte offset `row_off` (chunks past the row
// read zeros).
template <int G, int SLOTS>
__device__ __forceinline__ void load_x(XChunk<uint16_t> (&xc)[SLOTS], __amdgpu_buffer_rsrc_t r,
                                       uint32_t row_off, int gl, int nchunks) {
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        const int c = gl + s * G;
        const uint32_t off = c < nchunks ? row_off + (uint32_t)c * 64 : kOutOfRange;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            xc[s].p[q] = load_b128(r, off + q * 16);
    }
}

template <int SLOTS>
__device__ __forceinline__ float row_dot(const RowRegs<SLOTS> &r, const XChunk<uint16_t> (&xc)[SLOTS]) {
    float acc = 0.0f;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s)
        chunk_dot(r.codes[s], chunk_scales<true>(r.scales[s]), xc[s], acc);
    return acc;
}

// Gate/up: G = 32 lanes per row, two rows per wave and unit; a persistent grid of
// kGateUpBlocksPerCU workgroups (one wave per SIMD each) per CU.
constexpr int kGateUpBlocksPerCU = 3;

template <int SLOTS>
__global__ __launch_bounds__(256, kGateUpBlocksPerCU) void moe_gateup_gemv_kernel(MoeArgs a) {
    constexpr int G = 32;
    const int lane = threadIdx.x & 63;
    const int sub = lane / G, gl = lane % G;
    const uint32_t E = a.E, P = a.T * a.k, H = a.H, I = a.I;
    const PlanView v = plan_view(a.plan, E, P);
    const uint32_t U = v.hdr[0];
    const uint32_t rpe = (I + 1) / 2;
    const uint32_t units = U * rpe;
    const int nchunks = (int)(H / 32);
    const bool last_ok = gl + (SLOTS - 1) * G < nchunks;
    const uint32_t last_c = last_ok ? (SLOTS - 1) * G * 16 : kOutOfRange;
    const uint32_t last_s = last_ok ? (SLOTS - 1) * G * 2 : kOutOfRange;
    const __amdgpu_buffer_rsrc_t rx = make_rsrc(a.x, a.T * H * 2);
    const uint32_t nw = gridDim.x * 4;
    for (uint32_t u = blockIdx.x * 4 + (threadIdx.x >> 6); u < units; u += nw) {
        const uint32_t ai = u / rpe;
        const uint32_t row = 2 * (u - ai * rpe) + sub;
        const int e = v.act[ai];
        const uint8_t *slot = a.slots.base + (size_t)e * a.slots.stride;
        const uint32_t lrow = row < I ? row : I;
        RowRegs<SLOTS> rg, ru;
        load_row<SLOTS, G>(rg, make_rsrc(slot + a.slots.gate_w, I * H / 2),
                           make_rsrc(slot + a.slots.gate_s, I * H / 16), lrow, gl, H, last_c, last_s);
        load_row<SLOTS, G>(ru, make_rsrc(slot + a.slots.up_w, I * H / 2),
                           make_rsrc(slot + a.slots.up_s, I * H / 16), lrow, gl, H, last_c, last_s);
        const int n = v.cnt[e], p0 = v.off[e];
        for (int i = 0; i < n; ++i) {
            const int pos = p0 + i;
            const uint32_t t = (uint32_t)v.pair_of_pos[pos] / a.k;
            // one slot of x at a time keeps the register footprint at 4 waves per SIMD
            float g = 0.0f, up = 0.0f;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const int c = gl + s * G;
                const uint32_t off = c < nchunks ? t * H * 2 + (uint32_t)c * 64 : kOutOfRange;
                XChunk<uint16_t> xc;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    xc.p[q] = load_b128(rx, off + q * 16);
                chunk_dot(rg.codes[s], chunk_scales<true>(rg.scales[s]), xc, g);
                chunk_dot(ru.codes[s], chunk_scales<true>(ru.scales[s]), xc, up);
            }
            g = group_sum<G>(g);
            up = group_sum<G>(up);
            if (gl == 0 && row < I)
                a.h[(size_t)pos * I + row] = f32_to_bf16_bits(gelu_tanh(g) * up);
        }
    }
}

// Down + combine: workgroup b owns output rows [8b, 8b+8); G = 8 lanes per row.
constexpr int kDownWaves = 8;

template <int SLOTS>
__global__ __launch_bounds__(kDownWaves * 64) void moe_down_gemv_kernel(MoeArgs a) {
    constexpr int G = 8, R = 8;
    __shared__ float part[kDownWaves][kMoeGemvMaxTokens][R];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int sub = lane / G, gl = lane % G;
    const uint32_t E = a.E, P = a.T * a.k, H = a.H, I = a.I;
    const PlanView v = plan_view(a.plan, E, P);
    for (uint32_t q = threadIdx.x; q < kDownWaves * kMoeGemvMaxTokens * R; q += blockDim.x)
        (&part[0][0][0])[q] = 0.0f;
    __syncthreads();
    const uint32_t U = v.hdr[0];
    const uint32_t row = blockIdx.x * R + sub;
    const uint32_t lrow = row < H ? row : H;
    const int nchunks = (int)(I / 32);
    const bool last_ok = gl + (SLOTS - 1) * G < nchunks;
    const uint32_t last_c = last_ok ? (SLOTS - 1) * G * 16 : kOutOfRange;
    const uint32_t last_s = last_ok ? (SLOTS - 1) * G * 2 : kOutOfRange;
    const __amdgpu_buffer_rsrc_t rh = make_rsrc(a.h, P * I * 2);
    // Two experts per step: both experts' rows are in flight before the first dot.
    for (uint32_t ai = wave; ai < U; ai += 2 * kDownWaves) {
        const uint32_t bi = ai + kDownWaves;
        const int e0 = v.act[ai];
        const int e1 = bi < U ? v.act[bi] : e0;
        RowRegs<SLOTS> r[2];
        const int es[2] = {e0, e1};
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint8_t *slot = a.slots.base + (size_t)es[b] * a.slots.stride;
            load_row<SLOTS, G>(r[b], make_rsrc(slot + a.slots.down_w, H * I / 2),
                               make_rsrc(slot + a.slots.down_s, H * I / 16),
                               (b == 1 && bi >= U) ? H : lrow, gl, I, last_c, last_s);
        }
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            if (b == 1 && bi >= U)
                break;
            const int e = es[b];
            const int n = v.cnt[e], p0 = v.off[e];
            for (int i = 0; i < n; ++i) {
                const int pos = p0 + i;
                const uint32_t pair = (uint32_t)v.pair_of_pos[pos];
                const uint32_t t = pair / a.k;
                XChunk<uint16_t> xc[SLOTS];
                load_x<G, SLOTS>(xc, rh, (uint32_t)pos * I * 2, gl, nchunks);
                const float d = group_sum<G>(row_dot(r[b], xc));
                if (gl == 0)
                    part[wave][t][sub] += a.w[pair] * d;
            }
        }
    }
    __syncthreads();
    for (uint32_t q = threadIdx.x; q < a.T * R; q += blockDim.x) {
        const uint32_t t = q / R, rr = q % R;
        const uint32_t orow = blockIdx.x * R + rr;
        if (orow >= H)
            continue;
        float s = 0.0f;
        for (int w = 0; w < kDownWaves; ++w)
            s += part[w][t][rr];
        a.y[(size_t)t * H + orow] = f32_to_bf16_bits(s);
    }
}

// ---------------------------------------------------------------------------------
// Prefill: grouped GEMMs
// ---------------------------------------------------------------------------------

using namespace gemm_core;
constexpr int kGateUpCols = BN / 2; // h columns per gate/up tile

template <int MT>
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
    Acc<MT> acc;
    gemm_tile<MT>(lds, ra, rw, rw, H, a_row, w_code, w_scale, acc);
    const int lane = threadIdx.x & 63;
    const uint32_t col = c0 + 32 * (threadIdx.x >> 6) + (lane & 31);
    const uint32_t rb = 4 * (lane >> 5);
    if (col >= I)
        return;
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const uint32_t r = rb + 32 * i + 8 * (q >> 2) + (q & 3);
            if (r < nrows)
                a.h[(size_t)(row0 + r) * I + col] =
                    f32_to_bf16_bits(gelu_tanh(acc[i][0][q]) * acc[i][1][q]);
        }
}

__global__ __launch_bounds__(kThreads) void moe_gateup_gemm_kernel(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t E = a.E, P = a.T * a.k;
    const PlanView v = plan_view(a.plan, E, P);
    const uint32_t nn = (a.I + kGateUpCols - 1) / kGateUpCols;
    const uint32_t mt = blockIdx.x / nn, nt = blockIdx.x % nn;
    if (mt >= (uint32_t)v.hdr[1])
        return;
    const int32_t *t = v.tiles + 4 * mt;
    const int e = t[0], cls = t[3];
    const uint32_t row0 = t[1], nrows = t[2], c0 = nt * kGateUpCols;
    if (cls == 0)
        gateup_tile<8>(a, lds, v.pair_of_pos, e, row0, nrows, c0);
    else if (cls == 1)
        gateup_tile<4>(a, lds, v.pair_of_pos, e, row0, nrows, c0);
    else
        gateup_tile<2>(a, lds, v.pair_of_pos, e, row0, nrows, c0);
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
    Acc<MT> acc;
    gemm_tile<MT>(lds, ra, rw, rw, I, a_row, w_code, w_scale, acc);
    const int lane = threadIdx.x & 63;
    const uint32_t cn = n0 + 64 * (threadIdx.x >> 6) + (lane & 31);
    const uint32_t rb = 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < MT; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                const uint32_t r = rb + 32 * i + 8 * (q >> 2) + (q & 3);
                const uint32_t n = cn + 32 * j;
                if (r < nrows && n < H)
                    a.d[(size_t)(row0 + r) * H + n] = f32_to_bf16_bits(acc[i][j][q]);
            }
}

__global__ __launch_bounds__(kThreads) void moe_down_gemm_kernel(MoeArgs a) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const uint32_t E = a.E, P = a.T * a.k;
    const PlanView v = plan_view(a.plan, E, P);
    const uint32_t nn = (a.H + BN - 1) / BN;
    const uint32_t mt = blockIdx.x / nn, nt = blockIdx.x % nn;
    if (mt >= (uint32_t)v.hdr[1])
        return;
    const int32_t *t = v.tiles + 4 * mt;
    const int e = t[0], cls = t[3];
    const uint32_t row0 = t[1], nrows = t[2], n0 = nt * BN;
    if (cls == 0)
        down_tile<8>(a, lds, e, row0, nrows, n0);
    else if (cls == 1)
        down_tile<4>(a, lds, e, row0, nrows, n0);
    else
        down_tile<2>(a, lds, e, row0, nrows, n0);
}

// y[t] = sum_j w[t,j] d[pos(t,j)], slot order, fp32; 8 columns per thread.
__global__ __launch_bounds__(256) void moe_combine_kernel(MoeArgs a) {
    const uint32_t t = blockIdx.x;
    const uint32_t E = a.E, P = a.T * a.k, H = a.H, k = a.k;
    const PlanView v = plan_view(a.plan, E, P);
    const __amdgpu_buffer_rsrc_t rd = make_rsrc(a.d, P * H * 2);
    for (uint32_t c = threadIdx.x * 8; c < H; c += blockDim.x * 8) {
        float acc[8] = {};
        for (uint32_t j = 0; j < k; ++j) {
            const uint32_t pair = t * k + j;
            const uint32_t pos = (uint32_t)v.pos_of_pair[pair];
            const float wt = a.w[pair];
            const u32x4_t dv = load_b128(rd, (pos * H + c) * 2);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[2 * q] += wt * bf16_bits_to_f32(dv[q] & 0xFFFFu);
                acc[2 * q + 1] += wt * bf16_bits_to_f32(dv[q] >> 16);
            }
        }
        u32x4_t o;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = (uint32_t)f32_to_bf16_bits(acc[2 * q]) |
                   ((uint32_t)f32_to_bf16_bits(acc[2 * q + 1]) << 16);
        *reinterpret_cast<u32x4_t *>(a.y + (size_t)t * H + c) = o;
    }
}

template <typename F> hipError_t set_lds(F *kernel, size_t bytes, bool &done) {
    if (done)
        return hipSuccess;
    const hipError_t e =
        hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e == hipSuccess)
        done = true;
    return e;
}

uint32_t gemv_slots(uint32_t K, int G) { return (K / 32 + G - 1) / G; }

} // namespace

MoeWorkspace moe_workspace(uint32_t T, uint32_t E, uint32_t k, uint32_t H, uint32_t I, bool gemm) {
    MoeWorkspace w{};
    const size_t P = (size_t)T * k;
    w.max_tiles = (uint32_t)(P / 256 + (P < E ? P : E) + 1);
    size_t off = 0;
    w.ids = off;
    off = align256(off + P * 4);
    w.w = off;
    off = align256(off + P * 4);
    w.plan = off;
    off = align256(off + 4 * ((size_t)kMoePlanHeader + 3 * E + 1 + 2 * P + 4 * (size_t)w.max_tiles));
    w.h = off;
    off = align256(off + P * I * 2);
    w.d = off;
    if (gemm)
        off = align256(off + P * H * 2);
    w.total = off;
    return w;
}

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
        if (gemv_slots(a.H, 32) > 3 || gemv_slots(a.I, 8) > 4)
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

hipError_t moe_ffn_launch(const MoeArgs &a, bool gemm, hipStream_t stream) {
    if (a.T == 0)
        return hipSuccess;
    if (!gemm) {
        hipLaunchKernelGGL(moe_route_plan_kernel, dim3(1), dim3(1024), 0, stream, a);
        const uint32_t grid = (uint32_t)kNumCUs * kGateUpBlocksPerCU;
        switch (gemv_slots(a.H, 32)) {
        case 1: hipLaunchKernelGGL(moe_gateup_gemv_kernel<1>, dim3(grid), dim3(256), 0, stream, a); break;
        case 2: hipLaunchKernelGGL(moe_gateup_gemv_kernel<2>, dim3(grid), dim3(256), 0, stream, a); break;
        default: hipLaunchKernelGGL(moe_gateup_gemv_kernel<3>, dim3(grid), dim3(256), 0, stream, a); break;
        }
        const dim3 dgrid((a.H + 7) / 8), dblock(kDownWaves * 64);
        switch (gemv_slots(a.I, 8)) {
        case 1: hipLaunchKernelGGL(moe_down_gemv_kernel<1>, dgrid, dblock, 0, stream, a); break;
        case 2: hipLaunchKernelGGL(moe_down_gemv_kernel<2>, dgrid, dblock, 0, stream, a); break;
        case 3: hipLaunchKernelGGL(moe_down_gemv_kernel<3>, dgrid, dblock, 0, stream, a); break;
        default: hipLaunchKernelGGL(moe_down_gemv_kernel<4>, dgrid, dblock, 0, stream, a); break;
        }
        return hipGetLastError();
    }
    static bool lds_gateup = false, lds_down = false;
    hipError_t err = set_lds(moe_gateup_gemm_kernel, kMaxLds, lds_gateup);
    if (err == hipSuccess)
        err = set_lds(moe_down_gemm_kernel, kMaxLds, lds_down);
    if (err != hipSuccess)
        return err;
    hipLaunchKernelGGL(moe_route_kernel, dim3((a.T + 3) / 4), dim3(256), 0, stream, a.logits, a.T,
                       a.E, a.k, a.ids, a.w);
    hipLaunchKernelGGL(moe_plan_kernel, dim3(1), dim3(1024), 0, stream, a);
    const uint32_t nn_gu = (a.I + kGateUpCols - 1) / kGateUpCols;
    hipLaunchKernelGGL(moe_gateup_gemm_kernel, dim3(a.max_tiles * nn_gu), dim3(kThreads), kMaxLds,
                       stream, a);
    const uint32_t nn_d = (a.H + BN - 1) / BN;
    hipLaunchKernelGGL(moe_down_gemm_kernel, dim3(a.max_tiles * nn_d), dim3(kThreads), kMaxLds,
                       stream, a);
    hipLaunchKernelGGL(moe_combine_kernel, dim3(a.T), dim3(256), 0, stream, a);
    return hipGetLastError();
}

} // namespace apex_hip
