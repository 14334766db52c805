/*
 * CPU oracle for the NVFP4 matmul hot path.  TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C restatement of the reference's CPU implementation of the
 * NVFP4 dequant + matvec, GeLU-tanh and dense GeGLU FFN, plus the MoE expert-FFN
 * composition the reference describes but does not implement.  It exists to check
 * the HIP kernels: only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product path never calls it.
 *
 * Arithmetic follows the reference exactly: every weight is dequantised to fp32
 * as e2m1(code) * e4m3(scale) (exact), dot products accumulate in fp64 in index
 * order, and each output is cast to float once at the end.
 *
 * Parity pins (what checks each function; see tests/test_oracle.py):
 *   orc_e2m1_to_float   closed form over all 16 codes + compiled reference
 *   orc_e4m3_to_float   closed form over all 256 codes + torch.float8_e4m3fn on
 *                       254 codes + compiled reference (0x7F/0xFF -> +-480)
 *   orc_decode_row      compiled reference, bit-exact; product exactness invariant
 *   orc_matvec_nvfp4    golden vectors from the compiled reference; brute-force
 *                       fp64 on tiny inputs; linearity in x; sign symmetry
 *   orc_gelu_tanh       closed form (math.tanh) + compiled reference
 *   orc_dense_mlp       composition of the above; compiled reference composition
 *   orc_moe_route       brute-force sort on tiny inputs, softmax invariants
 *   orc_moe_ffn         equals a per-(token, expert) dense FFN loop; linearity in
 *                       the routing weights.  Parity vs mlx-lm: UNPINNED (mlx-lm
 *                       is not importable; see the MoE section of the design notes)
 *   orc_e4m3_from_float round-to-nearest-even, checked against torch.float8_e4m3fn
 *   orc_rms_norm        compiled reference rmsNormCpu (bit-exact), scale invariance
 *   orc_moe_router_logits_q8  fp64 matvec with the explicitly dequantised weights
 *                       (numpy); byte order on one-hot codes; the norm is orc_rms_norm.
 *                       Parity vs mlx-lm's router: UNPINNED (not importable)
 *   orc_head_norm_rope  rope_pairs = 0 / position 0 reduce to orc_rms_norm per head;
 *                       recovered rotation angles equal pos * base^(-2i/d) (numpy);
 *                       pair norms preserved; relative-position invariance of q.k
 */
#ifndef APEX_NVFP4_ORACLE_H
#define APEX_NVFP4_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/nvfp4.h:10-15 -- 4-bit E2M1 code, sign in bit 3.  Code 8 -> -0.0f. */
float orc_e2m1_to_float(uint32_t code);

/* src/nvfp4.h:17-25 -- FP8 E4M3 (bias 7, subnormal m/512, no NaN: 0x7F -> 480). */
float orc_e4m3_to_float(uint8_t byte);

/* src/nvfp4.h:27-43 -- dequantise one row: element k is nibble k%8 (LSB first) of
 * uint32 word k/8 times scale byte k/16.  K must be a multiple of 16. */
void orc_decode_row(const uint32_t *codes, const uint8_t *scales, float *out, size_t K);

/* src/tests/cpu_ref.h:48-63 -- out[t*rows + r] = float(sum_i double(w_r[i]) * in[t*K+i]),
 * rows outer, tokens inner, fp64 accumulation in index order.
 * tensor_scale is this build's per-tensor FP32 scale extension: the fp64 sum is
 * multiplied by double(tensor_scale) before the float cast (1.0 = reference). */
void orc_matvec_nvfp4(const uint32_t *codes, const uint8_t *scales, const float *in, float *out,
                      size_t tokens, size_t rows, size_t K, float tensor_scale);

/* Same as orc_matvec_nvfp4 restricted to the rows listed in row_ids (out is
 * [tokens, n_ids], token-major); used to check full-size GEMMs on a row sample. */
void orc_matvec_nvfp4_rows(const uint32_t *codes, const uint8_t *scales, const float *in,
                           float *out, size_t tokens, size_t K, const int64_t *row_ids,
                           size_t n_ids, float tensor_scale);

/* src/tests/cpu_ref.h:65-68 -- 0.5 g (1 + tanh(0.7978845608028654 (g + 0.044715 g^3))),
 * evaluated in float like the reference. */
float orc_gelu_tanh(float g);

/* shaders/geglu.metal:6-24 / src/tests/dense_mlp.cpp:176-178 -- out[i] = gelu(gate[i]) * up[i]. */
void orc_geglu(const float *gate, const float *up, float *out, size_t n);

/* src/tests/dense_mlp.cpp:148-182 without the RMSNorm: gate/up matvec, GeGLU, down matvec.
 * gate/up are [I, H], down is [H, I]; x is [T, H] fp32; y is [T, H] fp32. */
void orc_dense_mlp(const uint32_t *gate_codes, const uint8_t *gate_scales,
                   const uint32_t *up_codes, const uint8_t *up_scales,
                   const uint32_t *down_codes, const uint8_t *down_scales, const float *x,
                   float *y, size_t tokens, size_t H, size_t I);

/* src/tests/cpu_ref.h:27-46 -- max |a-b| and ||a-b|| / ||b||; +inf if any value is
 * non-finite. */
void orc_diff(const float *a, const float *b, size_t n, double *max_abs, double *rel_l2);

/* MoE router (no reference code; semantics of the mlx-lm call at
 * tools/dump_reference.py:213 with synthetic logits): per token, the k largest of
 * E logits (ties -> lower expert id), sorted by descending logit, then softmax over
 * those k in fp64, stored as float. */
void orc_moe_route(const float *logits, size_t T, size_t E, size_t k, int32_t *ids,
                   float *weights);

/* MoE expert FFN (no reference code; tools/dump_reference.py:212-216 semantics):
 *   y[t] = sum_j w[t,j] * down_e( gelu(gate_e x_t) (*) up_e x_t ),  e = ids[t,j]
 * Each expert's gate/up/down is an NVFP4 matrix inside a slot of slot_stride bytes
 * at the piece offsets given (the tools/repack.py:180-213 slot format).  Each
 * (token, expert) pair runs orc_dense_mlp's arithmetic (float gate/up/h, float down
 * output); the router-weighted sum over j then runs in fp64 in slot order
 * j = 0..k-1 and is cast to float once. */
typedef struct {
    size_t slot_stride;
    size_t gate_w, gate_s, up_w, up_s, down_w, down_s; /* byte offsets inside a slot */
} orc_expert_layout;

void orc_moe_ffn(const uint8_t *slots, const orc_expert_layout *layout, const float *x,
                 const int32_t *ids, const float *weights, float *y, size_t T, size_t k,
                 size_t H, size_t I);

/* src/tests/cpu_ref.h:10-22 (rmsNormCpu) over `rows` rows of n values: fp64 sum of
 * squares, inv = 1 / sqrt(float(ss / n) + eps), y = x * inv * bf16 weight. */
void orc_rms_norm(const float *x, const uint16_t *w_bf16, float *y, size_t rows, size_t n,
                  float eps);

/* shaders/head_norm_rope.metal:5-72: per (token, head) the RMSNorm above (weights
 * optional), then RoPE on pairs (i, head_dim/2 + i), i < rope_pairs, with the fp32
 * angle float(abs_pos + token) * powf(rope_base, -2i/head_dim) of the shader and the
 * rotation in fp64.  Output head (t, h) at y + t*out_token_stride + h*out_head_stride. */
void orc_head_norm_rope(const float *x, const uint16_t *w_bf16, int has_weight, float *y,
                        size_t tokens, size_t heads, size_t head_dim, size_t rope_pairs,
                        float rope_base, uint32_t abs_pos, size_t out_token_stride,
                        size_t out_head_stride, float eps);

/* Gemma-4 router logits (docs/B6_3_attention.md:721-725): xn = rmsNormCpu(h, norm_w),
 * logits[t][e] = sum_k xn[k] * (scale[e][k/64] * q[e][k] + bias[e][k/64]) with q byte
 * k % 4 (LSB first) of qw[e][k/4]; per group scale * sum(xn q) + bias * sum(xn) in fp64. */
void orc_moe_router_logits_q8(const float *h, const uint16_t *norm_w, float eps,
                              const uint32_t *qw, const uint16_t *qs, const uint16_t *qb,
                              size_t T, size_t E, size_t H, float *logits);

/* Round-to-nearest-even float -> FP8 E4M3 byte, saturating to +-448 (never emits
 * 0x7F/0xFF).  The synthetic generator's scale rounding, restated for checking. */
uint8_t orc_e4m3_from_float(float v);

/* bf16 helpers: exact widening, and round-to-nearest-even narrowing. */
float orc_bf16_to_float(uint16_t b);
uint16_t orc_float_to_bf16(float f);

#ifdef __cplusplus
}
#endif
#endif
