// C++ checks of apex::HipBackend and the ops.h helpers against the CPU oracle, in the
// style of the reference's own harness (src/tests/dense_mlp.cpp: fill buffers through
// contents(), queue ops, sync(), compare with the CPU result by rel L2).
//
//   test_host            run every check on device 0 (needs a GPU)
//   test_host --no-gpu   checks that need no GPU (constructor error path)
//
// Test infrastructure: links the oracle (oracle/liboracle.so).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <stdexcept>
#include <string>
#include <vector>

#include "apex_hip.h"
#include "hip_backend.h"
#include "model_info.h"
#include "model_loader.h"
#include "nvfp4_oracle.h"
#include "ops.h"
#include "profiling.h"

using namespace apex;

namespace {

int g_failures = 0;

void report(const std::string &name, bool ok, const std::string &detail = "") {
    std::printf("%s %s%s%s\n", ok ? "PASS" : "FAIL", name.c_str(), detail.empty() ? "" : ": ",
                detail.c_str());
    std::fflush(stdout);
    if (!ok)
        ++g_failures;
}

// splitmix64: the test's own deterministic generator.
struct Rng {
    uint64_t s;
    uint64_t next() {
        uint64_t z = (s += 0x9E3779B97F4A7C15ull);
        z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
        z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
        return z ^ (z >> 31);
    }
    float normal() { // Box-Muller
        const double u1 = ((next() >> 11) + 1.0) / 9007199254740993.0;
        const double u2 = (next() >> 11) / 9007199254740992.0;
        return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
    }
};

struct HostMatrix {
    std::vector<uint32_t> codes;
    std::vector<uint8_t> scales;
    uint32_t rows, K;
};

HostMatrix random_matrix(Rng &rng, uint32_t rows, uint32_t K) {
    HostMatrix m{std::vector<uint32_t>((size_t)rows * K / 8), std::vector<uint8_t>((size_t)rows * K / 16),
                 rows, K};
    for (auto &c : m.codes)
        c = (uint32_t)rng.next();
    for (auto &s : m.scales)
        s = orc_e4m3_from_float(std::fabs(rng.normal()) * 0.05f);
    return m;
}

double rel_l2(const float *a, const float *b, size_t n) {
    double mx, rel;
    orc_diff(a, b, n, &mx, &rel);
    return rel;
}

// Copy host bytes into a fresh backend buffer through contents().
Buffer *upload(HipBackend &be, const void *src, size_t bytes, const char *cat) {
    Buffer *b = be.allocate(bytes, cat);
    std::memcpy(be.contents(b), src, bytes);
    return b;
}

// Weights for one matrix in one buffer: codes then scales (as core.bin places them).
struct DevMatrix {
    Buffer *buf;
    Nvfp4Matrix m;
};

DevMatrix upload_matrix(HipBackend &be, const HostMatrix &h) {
    const size_t cb = h.codes.size() * 4, sb = h.scales.size();
    Buffer *b = be.allocate(cb + sb, "core_weights");
    auto *p = static_cast<uint8_t *>(be.contents(b));
    std::memcpy(p, h.codes.data(), cb);
    std::memcpy(p + cb, h.scales.data(), sb);
    return {b, Nvfp4Matrix{b, 0, b, cb, h.rows, h.K}};
}

uint16_t to_bf16(float f) { return orc_float_to_bf16(f); }
float from_bf16(uint16_t b) { return orc_bf16_to_float(b); }

void test_dense_mlp(HipBackend &be) {
    // src/tests/dense_mlp.cpp:148-182 composition at a small dense shape, fp32 contract.
    Rng rng{1};
    const uint32_t H = 512, I = 256, T = 3;
    HostMatrix g = random_matrix(rng, I, H), u = random_matrix(rng, I, H), d = random_matrix(rng, H, I);
    std::vector<float> x((size_t)T * H);
    for (auto &v : x)
        v = rng.normal();
    std::vector<float> want((size_t)T * H);
    orc_dense_mlp(g.codes.data(), g.scales.data(), u.codes.data(), u.scales.data(), d.codes.data(),
                  d.scales.data(), x.data(), want.data(), T, H, I);

    DevMatrix dg = upload_matrix(be, g), du = upload_matrix(be, u), dd = upload_matrix(be, d);
    Buffer *in = upload(be, x.data(), x.size() * 4, "scratch");
    Buffer *gate_tmp = be.allocate((size_t)T * I * 4, "scratch");
    Buffer *up_tmp = be.allocate((size_t)T * I * 4, "scratch");
    Buffer *out = be.allocate((size_t)T * H * 4, "scratch");
    denseMlp(be, in, dg.m, du.m, dd.m, gate_tmp, up_tmp, out, T);
    be.sync();
    const double r = rel_l2(static_cast<float *>(be.contents(out)), want.data(), want.size());
    // the reference harness's gate for fp32 outputs (src/tests/dense_mlp.cpp:113)
    report("denseMlp fp32 (4 launches) vs oracle", r < 1e-5, "rel_l2 " + std::to_string(r));

    // fused gate/up + down
    Buffer *h_tmp = be.allocate((size_t)T * I * 4, "scratch");
    Buffer *out2 = be.allocate((size_t)T * H * 4, "scratch");
    denseMlpFused(be, in, dg.m, du.m, dd.m, h_tmp, out2, T);
    be.sync();
    const double r2 = rel_l2(static_cast<float *>(be.contents(out2)), want.data(), want.size());
    report("denseMlpFused fp32 (2 launches) vs oracle", r2 < 1e-5, "rel_l2 " + std::to_string(r2));

    // re-run after rewriting the input through contents(): the mirror must be uploaded
    for (auto &v : x)
        v = -v;
    std::memcpy(be.contents(in), x.data(), x.size() * 4);
    denseMlp(be, in, dg.m, du.m, dd.m, gate_tmp, up_tmp, out, T);
    be.sync();
    orc_dense_mlp(g.codes.data(), g.scales.data(), u.codes.data(), u.scales.data(), d.codes.data(),
                  d.scales.data(), x.data(), want.data(), T, H, I);
    const double r3 = rel_l2(static_cast<float *>(be.contents(out)), want.data(), want.size());
    report("contents() write before run is uploaded", r3 < 1e-5, "rel_l2 " + std::to_string(r3));

    // rmsNorm fused into the gate/up GEMV (norm weights at an offset in a core buffer)
    const size_t woff = 512;
    std::vector<uint8_t> core(woff + H * 2);
    for (uint32_t i = 0; i < H; ++i) {
        const uint16_t w = to_bf16(1.0f + 0.1f * rng.normal());
        std::memcpy(core.data() + woff + 2 * i, &w, 2);
    }
    Buffer *cb = upload(be, core.data(), core.size(), "core_weights");
    const float eps = 1e-6f;
    gegluNvfp4RmsNorm(be, in, cb, woff, eps, dg.m, du.m, h_tmp, T);
    matmulNvfp4(be, h_tmp, dd.m, out2, T);
    be.sync();
    std::vector<float> xn(x.size());
    orc_rms_norm(x.data(), reinterpret_cast<const uint16_t *>(core.data() + woff), xn.data(), T, H,
                 eps);
    orc_dense_mlp(g.codes.data(), g.scales.data(), u.codes.data(), u.scales.data(), d.codes.data(),
                  d.scales.data(), xn.data(), want.data(), T, H, I);
    const double r4 = rel_l2(static_cast<float *>(be.contents(out2)), want.data(), want.size());
    report("gegluNvfp4RmsNorm + matmulNvfp4 vs rmsNorm + denseMlp oracle", r4 < 1e-5,
           "rel_l2 " + std::to_string(r4));

    for (Buffer *b : {dg.buf, du.buf, dd.buf, in, gate_tmp, up_tmp, out, h_tmp, out2, cb})
        be.release(b);
}

// MFMA GEMM launches (plain and split-K) made by the library so far.
uint64_t gemm_launches() {
    uint64_t c[4] = {};
    if (apex_hip_dense_dispatch_counts(c) != APEX_HIP_OK)
        return 0;
    return c[1] + c[2];
}

// The reference-named launches at prefill token counts: denseMlp queues matmul_nvfp4
// with the reference's grid (src/ops.h:34-46, 61-69), which covers every row, so each
// of its three products runs as an MFMA GEMM (fp32 x through its bf16 hi + lo split;
// split-K for these few tiles), checked by the library's launch counts, at the same
// reference gate as the decode sizes.
void test_dense_prefill(HipBackend &be) {
    Rng rng{11};
    const uint32_t H = 1024, I = 512;
    HostMatrix g = random_matrix(rng, I, H), u = random_matrix(rng, I, H), d = random_matrix(rng, H, I);
    DevMatrix dg = upload_matrix(be, g), du = upload_matrix(be, u), dd = upload_matrix(be, d);
    for (uint32_t T : {128u, 512u}) {
        std::vector<float> x((size_t)T * H);
        for (auto &v : x)
            v = rng.normal();
        std::vector<float> want((size_t)T * H);
        orc_dense_mlp(g.codes.data(), g.scales.data(), u.codes.data(), u.scales.data(),
                      d.codes.data(), d.scales.data(), x.data(), want.data(), T, H, I);
        Buffer *in = upload(be, x.data(), x.size() * 4, "activations");
        Buffer *gate_tmp = be.allocate((size_t)T * I * 4, "scratch");
        Buffer *up_tmp = be.allocate((size_t)T * I * 4, "scratch");
        Buffer *out = be.allocate((size_t)T * H * 4, "scratch");
        const std::string tag = " at " + std::to_string(T) + " tokens";
        uint64_t n0 = gemm_launches();
        denseMlp(be, in, dg.m, du.m, dd.m, gate_tmp, up_tmp, out, T);
        be.sync();
        double r = rel_l2(static_cast<float *>(be.contents(out)), want.data(), want.size());
        report("denseMlp fp32" + tag + " vs oracle", r < 1e-5, "rel_l2 " + std::to_string(r));
        uint64_t n = gemm_launches() - n0;
        report("denseMlp" + tag + ": matmul_nvfp4 ran 3 MFMA GEMMs", n == 3,
               std::to_string(n) + " GEMM launches");
        n0 = gemm_launches();
        denseMlpFused(be, in, dg.m, du.m, dd.m, gate_tmp, out, T);
        be.sync();
        r = rel_l2(static_cast<float *>(be.contents(out)), want.data(), want.size());
        report("denseMlpFused fp32" + tag + " vs oracle", r < 1e-5, "rel_l2 " + std::to_string(r));
        n = gemm_launches() - n0;
        report("denseMlpFused" + tag + ": 2 MFMA GEMMs", n == 2, std::to_string(n) + " GEMM launches");
        for (Buffer *b : {in, gate_tmp, up_tmp, out})
            be.release(b);
    }
    for (Buffer *b : {dg.buf, du.buf, dd.buf})
        be.release(b);
}

void test_bf16_ops(HipBackend &be) {
    Rng rng{2};
    const uint32_t K = 1024, N = 384;
    HostMatrix w = random_matrix(rng, N, K);
    DevMatrix dw = upload_matrix(be, w);
    HostMatrix u = random_matrix(rng, N, K);
    DevMatrix du = upload_matrix(be, u);
    for (uint32_t T : {1u, 5u, 96u}) { // GEMV for few tokens, MFMA GEMM for 96
        std::vector<uint16_t> xb((size_t)T * K);
        std::vector<float> xf((size_t)T * K);
        for (size_t i = 0; i < xb.size(); ++i) {
            xb[i] = to_bf16(rng.normal());
            xf[i] = from_bf16(xb[i]);
        }
        std::vector<float> want((size_t)T * N);
        orc_matvec_nvfp4(w.codes.data(), w.scales.data(), xf.data(), want.data(), T, N, K, 1.0f);
        Buffer *in = upload(be, xb.data(), xb.size() * 2, "scratch");
        Buffer *out = be.allocate((size_t)T * N * 2, "scratch");
        matmulNvfp4Bf16(be, in, dw.m, out, T);
        be.sync();
        const uint16_t *ob = static_cast<const uint16_t *>(be.contents(out));
        std::vector<float> got((size_t)T * N);
        for (size_t i = 0; i < got.size(); ++i)
            got[i] = from_bf16(ob[i]);
        const double r = rel_l2(got.data(), want.data(), want.size());
        report("matmulNvfp4Bf16 T=" + std::to_string(T), r < 1e-2, "rel_l2 " + std::to_string(r));
        // fused GeGLU through the registry (gate = w, up = u), bf16 in and out
        std::vector<float> upv((size_t)T * N);
        orc_matvec_nvfp4(u.codes.data(), u.scales.data(), xf.data(), upv.data(), T, N, K, 1.0f);
        orc_geglu(want.data(), upv.data(), want.data(), want.size());
        gegluNvfp4(be, in, dw.m, du.m, out, T, /*bf16=*/true);
        be.sync();
        ob = static_cast<const uint16_t *>(be.contents(out));
        for (size_t i = 0; i < got.size(); ++i)
            got[i] = from_bf16(ob[i]);
        const double rg = rel_l2(got.data(), want.data(), want.size());
        report("gegluNvfp4 bf16 T=" + std::to_string(T), rg < 1e-2, "rel_l2 " + std::to_string(rg));
        be.release(in);
        be.release(out);
    }
    be.release(dw.buf);
    be.release(du.buf);
}

void test_moe(HipBackend &be) {
    Rng rng{3};
    const uint32_t T = 5, E = 12, k = 3, H = 256, I = 128;
    orc_expert_layout L{};
    L.gate_w = 0;
    L.gate_s = L.gate_w + (size_t)I * H / 2;
    L.up_w = L.gate_s + (size_t)I * H / 16;
    L.up_s = L.up_w + (size_t)I * H / 2;
    L.down_w = L.up_s + (size_t)I * H / 16;
    L.down_s = L.down_w + (size_t)H * I / 2;
    L.slot_stride = (L.down_s + (size_t)H * I / 16 + 16383) / 16384 * 16384;
    std::vector<uint8_t> slots((size_t)E * L.slot_stride, 0);
    for (uint32_t e = 0; e < E; ++e) {
        uint8_t *s = slots.data() + (size_t)e * L.slot_stride;
        struct P {
            size_t w, s;
            uint32_t rows, K;
        } pieces[3] = {{L.gate_w, L.gate_s, I, H}, {L.up_w, L.up_s, I, H}, {L.down_w, L.down_s, H, I}};
        for (const P &p : pieces) {
            HostMatrix m = random_matrix(rng, p.rows, p.K);
            std::memcpy(s + p.w, m.codes.data(), m.codes.size() * 4);
            std::memcpy(s + p.s, m.scales.data(), m.scales.size());
        }
    }
    std::vector<uint16_t> xb((size_t)T * H), lb((size_t)T * E);
    std::vector<float> xf(xb.size()), lf(lb.size());
    for (size_t i = 0; i < xb.size(); ++i)
        xf[i] = from_bf16(xb[i] = to_bf16(rng.normal()));
    for (size_t i = 0; i < lb.size(); ++i)
        lf[i] = from_bf16(lb[i] = to_bf16(rng.normal()));
    std::vector<int32_t> ids((size_t)T * k);
    std::vector<float> w((size_t)T * k), want((size_t)T * H);
    orc_moe_route(lf.data(), T, E, k, ids.data(), w.data());
    orc_moe_ffn(slots.data(), &L, xf.data(), ids.data(), w.data(), want.data(), T, k, H, I);

    Buffer *dx = upload(be, xb.data(), xb.size() * 2, "scratch");
    Buffer *dl = upload(be, lb.data(), lb.size() * 2, "scratch");
    Buffer *ds = upload(be, slots.data(), slots.size(), "expert_slots");
    Buffer *dy = be.allocate((size_t)T * H * 2, "scratch");
    Buffer *ws = be.allocate(moeWorkspaceBytes(T, E, k, H, I), "scratch");
    ExpertSlots es{ds, (uint32_t)L.slot_stride, (uint32_t)L.gate_w, (uint32_t)L.gate_s, (uint32_t)L.up_w,
                   (uint32_t)L.up_s, (uint32_t)L.down_w, (uint32_t)L.down_s};
    moeFfn(be, dx, dl, es, dy, ws, T, E, k, H, I);
    be.sync();
    const auto *yb = static_cast<const uint16_t *>(be.contents(dy));
    std::vector<float> got((size_t)T * H);
    for (size_t i = 0; i < got.size(); ++i)
        got[i] = from_bf16(yb[i]);
    const double r = rel_l2(got.data(), want.data(), want.size());
    report("moeFfn vs oracle", r < 1e-2, "rel_l2 " + std::to_string(r));
    for (Buffer *b : {dx, dl, ds, dy, ws})
        be.release(b);
}

// src/tests/test_norm.cpp:70-101 pattern: weights at an offset inside a shared
// "core" buffer, rmsNorm over every token row, compared by rel L2 (tolerance 1e-5).
void test_norms(HipBackend &be) {
    Rng rng{7};
    const uint32_t T = 5, H = 2816;
    std::vector<float> x((size_t)T * H);
    for (auto &v : x)
        v = rng.normal();
    const size_t woff = 4096; // bytes before the weights inside the core buffer
    std::vector<uint8_t> core(woff + H * 2);
    for (uint32_t i = 0; i < H; ++i) {
        const uint16_t w = to_bf16(1.0f + 0.1f * rng.normal());
        std::memcpy(core.data() + woff + 2 * i, &w, 2);
    }
    Buffer *cb = upload(be, core.data(), core.size(), "core_weights");
    Buffer *in = upload(be, x.data(), x.size() * 4, "activations");
    Buffer *out = be.allocate(x.size() * 4, "activations");
    const float eps = 1e-6f;
    rmsNorm(be, in, cb, woff, out, T, H, eps);
    be.sync();
    std::vector<float> want(x.size());
    orc_rms_norm(x.data(), reinterpret_cast<const uint16_t *>(core.data() + woff), want.data(), T,
                 H, eps);
    double r = rel_l2(static_cast<const float *>(be.contents(out)), want.data(), want.size());
    report("rmsNorm vs oracle", r < 1e-5, "rel_l2 " + std::to_string(r));

    // per-head norm + RoPE: 3 tokens x 8 heads x 256, 128 rotated pairs, output placed
    // into a wider buffer (token stride 2 * heads * head_dim, at an offset)
    const uint32_t nt = 3, heads = 8, D = 256, pairs = 128, pos0 = 7;
    const uint32_t ts = 2 * heads * D, hs = D;
    const float base = 10000.0f;
    std::vector<float> q((size_t)nt * heads * D);
    for (auto &v : q)
        v = rng.normal();
    std::vector<uint16_t> hw(D);
    for (auto &w : hw)
        w = to_bf16(1.0f + 0.1f * rng.normal());
    Buffer *qb = upload(be, q.data(), q.size() * 4, "activations");
    Buffer *wb = upload(be, hw.data(), hw.size() * 2, "core_weights");
    const size_t out_off = 256; // bytes
    const size_t n_out = (size_t)(nt - 1) * ts + (heads - 1) * hs + D;
    Buffer *ob = be.allocate(out_off + n_out * 4, "activations");
    std::memset(be.contents(ob), 0, out_off + n_out * 4);
    headNormRope(be, qb, wb, 0, true, ob, out_off, nt, heads, D, pairs, base, pos0, ts, hs, eps);
    be.sync();
    std::vector<float> want_q(n_out, 0.0f);
    orc_head_norm_rope(q.data(), hw.data(), 1, want_q.data(), nt, heads, D, pairs, base, pos0, ts,
                       hs, eps);
    const float *got_q =
        reinterpret_cast<const float *>(static_cast<const uint8_t *>(be.contents(ob)) + out_off);
    r = rel_l2(got_q, want_q.data(), n_out);
    report("headNormRope vs oracle", r < 1e-5, "rel_l2 " + std::to_string(r));
    for (Buffer *b : {cb, in, out, qb, wb, ob})
        be.release(b);
}

bool throws(const std::function<void()> &f, const char *needle);

// manifest.json of a packed directory (written by the Python side in the repack
// format): the ModelInfo fields the engine reads.
void test_manifest(const std::string &dir) {
    const ModelInfo m = ModelInfo::load(dir);
    const bool cfg = m.config.hidden_size > 0 && m.config.num_experts > 0 &&
                     m.config.top_k_experts == 8 && m.config.rms_norm_eps > 0 &&
                     m.config.rope_theta_full == 1000000.0 && m.quant_group_size == 64 &&
                     m.quant_bits == 8 && m.quant_mode == "affine" &&
                     (int)m.config.layer_types.size() == m.config.num_hidden_layers;
    report("manifest: config and quantization", cfg);
    bool pieces = m.expert_pieces.size() == 6 && m.expert_slot_size % 16384 == 0;
    uint64_t end = 0;
    for (const char *n : {"gate_proj.weight", "gate_proj.scales", "up_proj.weight",
                          "up_proj.scales", "down_proj.weight", "down_proj.scales"}) {
        const ExpertPiece &p = m.piece(n);
        pieces = pieces && p.offset == end; // contiguous, in the fixed order
        end = p.offset + p.nbytes;
    }
    pieces = pieces && end <= m.expert_slot_size;
    report("manifest: expert slot pieces", pieces);
    bool layers = (int)m.layers.size() == m.config.num_hidden_layers;
    for (const LayerFile &f : m.layers)
        layers = layers && f.stride == m.expert_slot_size &&
                 f.size == (uint64_t)f.num_experts * f.stride &&
                 (int)f.expert_sha256.size() == f.num_experts &&
                 m.layer_file(f.layer) == m.dir + "/" + f.file;
    report("manifest: layer files", layers);
    const TensorInfo &t = m.getTensor("layers.0.router.proj.weight");
    report("manifest: core tensors", t.dtype == "U32" && t.offset % 16384 == 0 &&
                                         t.nbytes == (uint64_t)t.shape[0] * t.shape[1] * 4);
    report("manifest: unknown tensor throws",
           throws([&] { (void)m.getTensor("no.such.tensor"); }, "tensor not found"));
}

// The MoE block of layer 1 from a packed directory loaded to the device: router logits
// and the routed expert FFN over buffers streamed from core.bin and layer_01.bin,
// against the oracle composition on the same files' bytes.
void test_packed_moe(HipBackend &be, const std::string &dir) {
    const ModelInfo m = ModelInfo::load(dir);
    const int layer = 1;
    Buffer *core = loadCore(be, m);
    Buffer *slots = loadExpertLayer(be, m, layer);
    const RouterWeights R = routerWeights(m, core, layer);
    const ExpertSlots S = expertSlots(m, slots);
    const uint32_t T = 5, H = m.config.hidden_size, E = m.config.num_experts,
                   I = m.config.moe_intermediate_size, k = m.config.top_k_experts;
    Rng rng{9};
    std::vector<float> h((size_t)T * H);
    for (auto &v : h)
        v = rng.normal();
    std::vector<uint16_t> x((size_t)T * H);
    for (auto &v : x)
        v = to_bf16(rng.normal());
    Buffer *bh = upload(be, h.data(), h.size() * 4, "activations");
    Buffer *bx = upload(be, x.data(), x.size() * 2, "activations");
    Buffer *lg = be.allocate((size_t)T * E * 4, "activations");
    Buffer *y = be.allocate((size_t)T * H * 2, "activations");
    Buffer *ws = be.allocate(moeWorkspaceBytes(T, E, k, H, I), "scratch");
    moeRouterLogits(be, bh, R, lg, T, (float)m.config.rms_norm_eps);
    moeFfnFromLogits(be, bx, lg, R, S, y, ws, T, k, H, I);
    be.sync();

    // oracle on the files' own bytes
    std::vector<uint8_t> cb(m.core_size), lb(m.layers[layer].size);
    FILE *f = std::fopen((m.dir + "/core.bin").c_str(), "rb");
    bool ok = f && std::fread(cb.data(), 1, cb.size(), f) == cb.size();
    if (f)
        std::fclose(f);
    f = std::fopen(m.layer_file(layer).c_str(), "rb");
    ok = ok && f && std::fread(lb.data(), 1, lb.size(), f) == lb.size();
    if (f)
        std::fclose(f);
    report("packed files read back", ok);
    auto at = [&](const char *name) {
        return cb.data() + m.getTensor("layers.1.router." + std::string(name)).offset;
    };
    std::vector<float> want_lg((size_t)T * E);
    orc_moe_router_logits_q8(h.data(), (const uint16_t *)at("scale"), (float)m.config.rms_norm_eps,
                             (const uint32_t *)at("proj.weight"), (const uint16_t *)at("proj.scales"),
                             (const uint16_t *)at("proj.biases"), T, E, H, want_lg.data());
    const float *got_lg = static_cast<const float *>(be.contents(lg));
    const double r_lg = rel_l2(got_lg, want_lg.data(), want_lg.size());
    report("packed router logits vs oracle", r_lg < 1e-5, "rel_l2 " + std::to_string(r_lg));
    // route on the device's logits (the oracle's top-k on them), scale, dense FFNs
    std::vector<int32_t> ids((size_t)T * k);
    std::vector<float> w((size_t)T * k), xf((size_t)T * H), yf((size_t)T * H), got((size_t)T * H);
    orc_moe_route(got_lg, T, E, k, ids.data(), w.data());
    const uint16_t *pes = (const uint16_t *)at("per_expert_scale");
    for (size_t i = 0; i < ids.size(); ++i)
        w[i] *= from_bf16(pes[ids[i]]);
    for (size_t i = 0; i < xf.size(); ++i)
        xf[i] = from_bf16(x[i]);
    orc_expert_layout L{m.expert_slot_size, S.gate_w, S.gate_s, S.up_w, S.up_s, S.down_w, S.down_s};
    orc_moe_ffn(lb.data(), &L, xf.data(), ids.data(), w.data(), yf.data(), T, k, H, I);
    const uint16_t *gy = static_cast<const uint16_t *>(be.contents(y));
    for (size_t i = 0; i < got.size(); ++i)
        got[i] = from_bf16(gy[i]);
    const double r = rel_l2(got.data(), yf.data(), yf.size());
    report("packed MoE block vs oracle", r < 1e-2, "rel_l2 " + std::to_string(r));
    for (Buffer *b : {core, slots, bh, bx, lg, y, ws})
        be.release(b);
}

bool throws(const std::function<void()> &f, const char *needle) {
    try {
        f();
    } catch (const std::runtime_error &e) {
        return std::strstr(e.what(), needle) != nullptr;
    }
    return false;
}

void test_errors(HipBackend &be) {
    Buffer *b = be.allocate(4096, "scratch");
    report("unknown kernel throws",
           throws([&] { be.run("attention_f32", {Arg::buf(b)}, Dim3{1}, Dim3{256}); },
                  "cannot find kernel"));
    report("threadgroup too large throws",
           throws([&] {
               uint32_t n = 1;
               be.run("geglu_f32", {Arg::buf(b), Arg::buf(b), Arg::buf(b), Arg::val(n)}, Dim3{1},
                      Dim3{2048});
           },
                  "threadgroup too large"));
    report("wrong argument count throws",
           throws([&] { be.run("geglu_f32", {Arg::buf(b)}, Dim3{1}, Dim3{256}); }, "expected 4"));
    alignas(16384) static uint8_t page[32768];
    report("wrapNoCopy rejects a misaligned pointer",
           throws([&] { be.wrapNoCopy(page + 64, 16384); }, "wrapNoCopy"));
    Buffer *w = be.wrapNoCopy(page, 16384);
    report("wrapNoCopy accepts an aligned page", w != nullptr);
    be.release(w);
    const uint64_t before = MemoryTracker::get().category("scratch");
    be.release(b);
    report("release updates the memory tracker",
           MemoryTracker::get().category("scratch") == before - 4096);
}

} // namespace

int main(int argc, char **argv) {
    bool no_gpu = false;
    std::string packed;
    for (int i = 1; i < argc; ++i) {
        if (std::strcmp(argv[i], "--no-gpu") == 0)
            no_gpu = true;
        else if (std::strcmp(argv[i], "--packed") == 0 && i + 1 < argc)
            packed = argv[++i];
    }
    if (!packed.empty())
        test_manifest(packed);
    if (no_gpu) {
        // Without a device, construction fails with the C ABI's message.
        report("HipBackend without a device throws",
               throws([] { HipBackend be(0); }, "HipBackend"));
        Profile::get().add("phase_a", 1.5);
        Profile::get().add("phase_a", 0.25);
        { Timer t("phase_b"); }
        const Profile::Phase a = Profile::get().phase("phase_a");
        report("Profile: calls, total, shortest and longest per phase",
               a.count == 2 && a.total_ns == 1750000 && a.shortest_ns == 250000 &&
                   a.longest_ns == 1500000 && Profile::get().phase("phase_b").count == 1 &&
                   Profile::get().phase("never").count == 0);
        Profile::get().reset();
        return g_failures ? 1 : 0;
    }
    HipBackend be(0);
    std::printf("device: %s\n", be.deviceName());
    test_dense_mlp(be);
    test_dense_prefill(be);
    test_bf16_ops(be);
    test_moe(be);
    test_norms(be);
    if (!packed.empty())
        test_packed_moe(be, packed);
    test_errors(be);
    const Profile::Phase ps = Profile::get().phase("gpu_sync");
    report("Backend::sync timed under gpu_sync", ps.count > 0 && ps.longest_ns >= ps.shortest_ns,
           std::to_string(ps.count) + " calls");
    Profile::get().print(stdout);
    std::printf("%s (%d failure%s)\n", g_failures ? "FAILED" : "OK", g_failures,
                g_failures == 1 ? "" : "s");
    return g_failures ? 1 : 0;
}
