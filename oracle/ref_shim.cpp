// C-ABI shim over the reference's own CPU NVFP4 code, compiled in place from the
// reference sources (src/nvfp4.h, src/tests/cpu_ref.h) into oracle/_ref/.  TEST
// INFRASTRUCTURE ONLY: it lets the tests check the C restatement in
// nvfp4_oracle.c against the reference, and lets bench.py time the reference's
// own matvec as its CPU baseline.  Nothing here is part of the product.
#include <cstddef>
#include <cstdint>
#include <vector>

#include "tests/cpu_ref.h"

extern "C" {

float ref_e2m1_to_float(uint32_t code) { return apex::e2m1ToFloat(code); }

float ref_e4m3_to_float(uint8_t byte) { return apex::e4m3ToFloat(byte); }

void ref_decode_row(const uint32_t *codes, const uint8_t *scales, float *out, size_t K) {
    apex::decodeRowNvfp4(codes, scales, out, K);
}

void ref_matvec_nvfp4(const uint32_t *codes, const uint8_t *scales, const float *in, float *out,
                      size_t tokens, size_t rows, size_t K) {
    matvecNvfp4Cpu(codes, scales, in, out, tokens, rows, K);
}

float ref_gelu_tanh(float g) { return geluTanh(g); }

void ref_rms_norm(const float *x, const uint16_t *w_bf16, float *y, size_t n, float eps) {
    rmsNormCpu(x, w_bf16, y, n, eps);
}

// The gate/up half of the dense FFN with the reference's functions, in the order
// src/tests/dense_mlp.cpp:167-177 runs it: both matvecs over every token, then
// out = geluTanh(gate) * up in float.
void ref_geglu(const uint32_t *gate_codes, const uint8_t *gate_scales, const uint32_t *up_codes,
               const uint8_t *up_scales, const float *in, float *out, size_t tokens, size_t rows,
               size_t K) {
    std::vector<float> up(tokens * rows);
    matvecNvfp4Cpu(gate_codes, gate_scales, in, out, tokens, rows, K);
    matvecNvfp4Cpu(up_codes, up_scales, in, up.data(), tokens, rows, K);
    for (size_t i = 0; i < up.size(); ++i)
        out[i] = geluTanh(out[i]) * up[i];
}

// MoE expert FFN on the CPU with the reference's functions (the reference has no MoE
// code; tools/dump_reference.py:208-219 semantics): each expert's tokens are gathered
// and run through denseMlpCpu's sequence (src/tests/dense_mlp.cpp:167-181: gate and up
// matvecs, geluTanh(gate) * up, down matvec) in one matvecNvfp4Cpu call per matrix, so
// every weight row is decoded once per expert as that function intends; then
// y[t] = float(sum_j double(w[t, j]) * d[t, j]) in slot order j.  Expert e's pieces sit
// at slots + e * stride + the piece offsets (tools/repack.py:180-213).
void ref_moe_ffn(const uint8_t *slots, size_t stride, size_t gate_w, size_t gate_s, size_t up_w,
                 size_t up_s, size_t down_w, size_t down_s, const float *x, const int32_t *ids,
                 const float *w, float *y, size_t tokens, size_t k, size_t experts, size_t H,
                 size_t I) {
    std::vector<float> d(tokens * k * H), xe, g, de;
    std::vector<size_t> pairs;
    for (size_t e = 0; e < experts; ++e) {
        pairs.clear();
        for (size_t p = 0; p < tokens * k; ++p)
            if ((size_t)ids[p] == e)
                pairs.push_back(p);
        const size_t n = pairs.size();
        if (n == 0)
            continue;
        xe.resize(n * H), g.resize(n * I), de.resize(n * H);
        for (size_t i = 0; i < n; ++i)
            for (size_t c = 0; c < H; ++c)
                xe[i * H + c] = x[(pairs[i] / k) * H + c];
        const uint8_t *s = slots + e * stride;
        ref_geglu(reinterpret_cast<const uint32_t *>(s + gate_w), s + gate_s,
                  reinterpret_cast<const uint32_t *>(s + up_w), s + up_s, xe.data(), g.data(), n,
                  I, H);
        matvecNvfp4Cpu(reinterpret_cast<const uint32_t *>(s + down_w), s + down_s, g.data(),
                       de.data(), n, H, I);
        for (size_t i = 0; i < n; ++i)
            for (size_t c = 0; c < H; ++c)
                d[pairs[i] * H + c] = de[i * H + c];
    }
    for (size_t t = 0; t < tokens; ++t)
        for (size_t c = 0; c < H; ++c) {
            double acc = 0.0;
            for (size_t j = 0; j < k; ++j)
                acc += double(w[t * k + j]) * d[(t * k + j) * H + c];
            y[t * H + c] = float(acc);
        }
}

void ref_diff(const float *a, const float *b, size_t n, double *max_abs, double *rel_l2) {
    const Diff d = diff(a, b, n);
    *max_abs = d.max_abs;
    *rel_l2 = d.rel_l2;
}
}
