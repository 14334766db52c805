// C-ABI shim over the reference's own CPU NVFP4 code, compiled in place from the
// reference sources (src/nvfp4.h, src/tests/cpu_ref.h) into oracle/_ref/.  TEST
// INFRASTRUCTURE ONLY: it lets the tests check the C restatement in
// nvfp4_oracle.c against the reference, and lets bench.py time the reference's
// own matvec as its CPU baseline.  Nothing here is part of the product.
#include <cstddef>
#include <cstdint>

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

void ref_diff(const float *a, const float *b, size_t n, double *max_abs, double *rel_l2) {
    const Diff d = diff(a, b, n);
    *max_abs = d.max_abs;
    *rel_l2 = d.rel_l2;
}
}
