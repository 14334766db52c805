/*
 * CPU oracle for the NVFP4 matmul hot path.  TEST INFRASTRUCTURE ONLY: loaded by
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, never by the
 * product path.  Function contracts and the reference lines each one follows are
 * in nvfp4_oracle.h.  Build: gcc -O2 -ffp-contract=off (no FMA contraction, so the
 * float expressions round exactly as written).
 */
#include "nvfp4_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* src/nvfp4.h:10-15 */
float orc_e2m1_to_float(uint32_t code) {
    static const float magnitude[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
    float v = magnitude[code & 7u];
    return (code & 8u) ? -v : v;
}

/* src/nvfp4.h:17-25: exponent field 0 is subnormal (m/512); otherwise
 * (1 + m/8) * 2^(e-7).  No NaN branch: 0x7F decodes to 1.875 * 2^8 = 480. */
float orc_e4m3_to_float(uint8_t byte) {
    uint32_t e = (byte >> 3) & 0xFu;
    uint32_t m = byte & 7u;
    float v = (e == 0) ? (float)m * (1.0f / 512.0f) : ldexpf(1.0f + (float)m * 0.125f, (int)e - 7);
    return (byte & 0x80u) ? -v : v;
}

/* src/nvfp4.h:27-43 */
void orc_decode_row(const uint32_t *codes, const uint8_t *scales, float *out, size_t K) {
    for (size_t blk = 0; blk < K / 16; ++blk) {
        float s = orc_e4m3_to_float(scales[blk]);
        for (size_t i = 0; i < 16; ++i) {
            uint32_t word = codes[2 * blk + i / 8];
            uint32_t code = (word >> (4u * (uint32_t)(i % 8))) & 0xFu;
            out[blk * 16 + i] = orc_e2m1_to_float(code) * s;
        }
    }
}

static float finish(double sum, float tensor_scale) {
    return (float)(sum * (double)tensor_scale);
}

/* src/tests/cpu_ref.h:48-63: decode a row once, then dot with every token. */
void orc_matvec_nvfp4(const uint32_t *codes, const uint8_t *scales, const float *in, float *out,
                      size_t tokens, size_t rows, size_t K, float tensor_scale) {
    float *w = (float *)malloc(K * sizeof(float));
    for (size_t r = 0; r < rows; ++r) {
        orc_decode_row(codes + r * (K / 8), scales + r * (K / 16), w, K);
        for (size_t t = 0; t < tokens; ++t) {
            const float *x = in + t * K;
            double sum = 0.0;
            for (size_t i = 0; i < K; ++i)
                sum += (double)w[i] * (double)x[i];
            out[t * rows + r] = finish(sum, tensor_scale);
        }
    }
    free(w);
}

void orc_matvec_nvfp4_rows(const uint32_t *codes, const uint8_t *scales, const float *in,
                           float *out, size_t tokens, size_t K, const int64_t *row_ids,
                           size_t n_ids, float tensor_scale) {
    float *w = (float *)malloc(K * sizeof(float));
    for (size_t j = 0; j < n_ids; ++j) {
        size_t r = (size_t)row_ids[j];
        orc_decode_row(codes + r * (K / 8), scales + r * (K / 16), w, K);
        for (size_t t = 0; t < tokens; ++t) {
            const float *x = in + t * K;
            double sum = 0.0;
            for (size_t i = 0; i < K; ++i)
                sum += (double)w[i] * (double)x[i];
            out[t * n_ids + j] = finish(sum, tensor_scale);
        }
    }
    free(w);
}

/* src/tests/cpu_ref.h:65-68, float arithmetic in the written order. */
float orc_gelu_tanh(float g) {
    float inner = 0.7978845608028654f * (g + 0.044715f * g * g * g);
    return 0.5f * g * (1.0f + tanhf(inner));
}

void orc_geglu(const float *gate, const float *up, float *out, size_t n) {
    for (size_t i = 0; i < n; ++i)
        out[i] = orc_gelu_tanh(gate[i]) * up[i];
}

/* src/tests/dense_mlp.cpp:170-181 (the part after the RMSNorm). */
void orc_dense_mlp(const uint32_t *gate_codes, const uint8_t *gate_scales,
                   const uint32_t *up_codes, const uint8_t *up_scales,
                   const uint32_t *down_codes, const uint8_t *down_scales, const float *x,
                   float *y, size_t tokens, size_t H, size_t I) {
    float *gate = (float *)malloc(tokens * I * sizeof(float));
    float *up = (float *)malloc(tokens * I * sizeof(float));
    orc_matvec_nvfp4(gate_codes, gate_scales, x, gate, tokens, I, H, 1.0f);
    orc_matvec_nvfp4(up_codes, up_scales, x, up, tokens, I, H, 1.0f);
    orc_geglu(gate, up, gate, tokens * I);
    orc_matvec_nvfp4(down_codes, down_scales, gate, y, tokens, H, I, 1.0f);
    free(gate);
    free(up);
}

/* src/tests/cpu_ref.h:27-46 */
void orc_diff(const float *a, const float *b, size_t n, double *max_abs, double *rel_l2) {
    double num = 0.0, den = 0.0, mx = 0.0;
    for (size_t i = 0; i < n; ++i) {
        if (!isfinite(a[i]) || !isfinite(b[i])) {
            *max_abs = INFINITY;
            *rel_l2 = INFINITY;
            return;
        }
        double e = (double)a[i] - (double)b[i];
        num += e * e;
        den += (double)b[i] * (double)b[i];
        if (fabs(e) > mx)
            mx = fabs(e);
    }
    *max_abs = mx;
    *rel_l2 = den > 0.0 ? sqrt(num / den) : sqrt(num);
}

/* Top-k by repeated selection of the largest remaining logit; a strictly-greater
 * comparison scanning ids upward keeps the lower id on ties. */
void orc_moe_route(const float *logits, size_t T, size_t E, size_t k, int32_t *ids,
                   float *weights) {
    unsigned char *taken = (unsigned char *)malloc(E);
    double *sel = (double *)malloc(k * sizeof(double));
    for (size_t t = 0; t < T; ++t) {
        const float *l = logits + t * E;
        memset(taken, 0, E);
        for (size_t j = 0; j < k; ++j) {
            size_t best = E;
            for (size_t e = 0; e < E; ++e) {
                if (taken[e])
                    continue;
                if (best == E || l[e] > l[best])
                    best = e;
            }
            taken[best] = 1;
            ids[t * k + j] = (int32_t)best;
            sel[j] = (double)l[best];
        }
        double mx = sel[0], z = 0.0;
        for (size_t j = 0; j < k; ++j)
            z += exp(sel[j] - mx);
        for (size_t j = 0; j < k; ++j)
            weights[t * k + j] = (float)(exp(sel[j] - mx) / z);
    }
    free(taken);
    free(sel);
}

void orc_moe_ffn(const uint8_t *slots, const orc_expert_layout *L, const float *x,
                 const int32_t *ids, const float *weights, float *y, size_t T, size_t k,
                 size_t H, size_t I) {
    float *d = (float *)malloc(k * H * sizeof(float));
    for (size_t t = 0; t < T; ++t) {
        for (size_t j = 0; j < k; ++j) {
            const uint8_t *s = slots + (size_t)ids[t * k + j] * L->slot_stride;
            orc_dense_mlp((const uint32_t *)(s + L->gate_w), s + L->gate_s,
                          (const uint32_t *)(s + L->up_w), s + L->up_s,
                          (const uint32_t *)(s + L->down_w), s + L->down_s, x + t * H,
                          d + j * H, 1, H, I);
        }
        for (size_t h = 0; h < H; ++h) {
            double acc = 0.0;
            for (size_t j = 0; j < k; ++j)
                acc += (double)weights[t * k + j] * (double)d[j * H + h];
            y[t * H + h] = (float)acc;
        }
    }
    free(d);
}

/* Round to nearest even on the E4M3 grid: spacing 2^-9 below 2^-6 (subnormals),
 * 2^(e-3) in binade [2^e, 2^(e+1)); saturate at 448 (0x7E). */
uint8_t orc_e4m3_from_float(float v) {
    uint8_t sign = signbit(v) ? 0x80 : 0x00;
    double a = fabs((double)v);
    if (!(a == a))
        return 0x7E | sign;
    if (a >= 464.0) /* halfway between 448 and the (absent) 480 rounds to even: 448 */
        return 0x7E | sign;
    if (a < 0.015625) { /* subnormal range */
        double q = nearbyint(a * 512.0); /* default rounding mode: to nearest even */
        return (uint8_t)(sign | (uint8_t)q); /* q == 8 is exactly the min normal 0x08 */
    }
    int e;
    double f = frexp(a, &e); /* a = f * 2^e, f in [0.5, 1) */
    int ex = e - 1;          /* a = (2f) * 2^ex, 2f in [1, 2) */
    double m = nearbyint((2.0 * f - 1.0) * 8.0);
    if (m == 8.0) {
        m = 0.0;
        ex += 1;
    }
    if (ex + 7 > 15 || (ex + 7 == 15 && m == 7.0))
        return 0x7E | sign;
    return (uint8_t)(sign | (uint8_t)((ex + 7) << 3) | (uint8_t)m);
}

float orc_bf16_to_float(uint16_t b) {
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

uint16_t orc_float_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u && (u & 0x007FFFFFu)) /* NaN stays NaN */
        return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* src/tests/cpu_ref.h:10-22 (rmsNormCpu): fp64 sum of squares in index order,
 * inv = 1 / sqrt(float(ss / n) + eps) in float, y = x * inv * w in float. */
void orc_rms_norm(const float *x, const uint16_t *w_bf16, float *y, size_t rows, size_t n,
                  float eps) {
    for (size_t r = 0; r < rows; ++r) {
        const float *xr = x + r * n;
        float *yr = y + r * n;
        double ss = 0.0;
        for (size_t i = 0; i < n; ++i)
            ss += (double)xr[i] * xr[i];
        const float inv = 1.0f / sqrtf((float)(ss / (double)n) + eps);
        for (size_t i = 0; i < n; ++i)
            yr[i] = xr[i] * inv * orc_bf16_to_float(w_bf16[i]);
    }
}

/* shaders/head_norm_rope.metal:5-72 (no CPU reference exists): per (token, head) the
 * rmsNormCpu arithmetic above over head_dim values (times w when has_weight), then
 * pairs (i, half + i), i < rope_pairs, rotated by the angle the shader forms in fp32:
 * pos = float(abs_pos + token), angle = pos * powf(rope_base, -2.0f * i / head_dim)
 * (head_norm_rope.metal:53-55); cos, sin and the rotation in fp64, cast once. */
void orc_head_norm_rope(const float *x, const uint16_t *w_bf16, int has_weight, float *y,
                        size_t tokens, size_t heads, size_t head_dim, size_t rope_pairs,
                        float rope_base, uint32_t abs_pos, size_t out_token_stride,
                        size_t out_head_stride, float eps) {
    const size_t half = head_dim / 2;
    float *row = (float *)malloc(head_dim * sizeof(float));
    for (size_t t = 0; t < tokens; ++t)
        for (size_t h = 0; h < heads; ++h) {
            const float *xr = x + (t * heads + h) * head_dim;
            float *yr = y + t * out_token_stride + h * out_head_stride;
            double ss = 0.0;
            for (size_t i = 0; i < head_dim; ++i)
                ss += (double)xr[i] * xr[i];
            const float inv = 1.0f / sqrtf((float)(ss / (double)head_dim) + eps);
            for (size_t i = 0; i < head_dim; ++i)
                row[i] = xr[i] * inv * (has_weight ? orc_bf16_to_float(w_bf16[i]) : 1.0f);
            const float pos = (float)(abs_pos + (uint32_t)t);
            for (size_t i = 0; i < rope_pairs; ++i) {
                const float angle = pos * powf(rope_base, -2.0f * (float)i / (float)head_dim);
                const double c = cos((double)angle), sn = sin((double)angle);
                const double a = row[i], b = row[half + i];
                row[i] = (float)(a * c - b * sn);
                row[half + i] = (float)(a * sn + b * c);
            }
            for (size_t i = 0; i < head_dim; ++i)
                yr[i] = row[i];
        }
    free(row);
}

/* docs/B6_3_attention.md:721-725: rmsNormCpu arithmetic (above) with the router.scale
 * weights, then the affine 8-bit projection w[e][k] = scale[e][g] * q[e][k] + bias[e][g],
 * q = byte k % 4 (least significant first) of word k / 4, g = k / 64; the sum runs in
 * fp64 per group (scale * sum xn q + bias * sum xn) and over groups in index order. */
void orc_moe_router_logits_q8(const float *h, const uint16_t *norm_w, float eps,
                              const uint32_t *qw, const uint16_t *qs, const uint16_t *qb,
                              size_t T, size_t E, size_t H, float *logits) {
    float *xn = (float *)malloc(H * sizeof(float));
    const size_t NG = H / 64;
    for (size_t t = 0; t < T; ++t) {
        orc_rms_norm(h + t * H, norm_w, xn, 1, H, eps);
        for (size_t e = 0; e < E; ++e) {
            const uint8_t *q = (const uint8_t *)(qw + e * (H / 4));
            double acc = 0.0;
            for (size_t g = 0; g < NG; ++g) {
                double sq = 0.0, sx = 0.0;
                for (size_t j = 0; j < 64; ++j) {
                    const size_t k = 64 * g + j;
                    sq += (double)xn[k] * (double)q[k];
                    sx += (double)xn[k];
                }
                acc += (double)orc_bf16_to_float(qs[e * NG + g]) * sq +
                       (double)orc_bf16_to_float(qb[e * NG + g]) * sx;
            }
            logits[t * E + e] = (float)acc;
        }
    }
    free(xn);
}
