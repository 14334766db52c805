// Kernel-launch helpers over the Backend interface, as src/ops.h provides them for the
// engine: the reference's ops under their reference names and argument order
// (rmsNorm, matmulNvfp4, geglu, denseMlp, headNormRope: src/ops.h:7-118), plus the HIP backend's
// additional ops -- bf16 activations, the fused GeGLU projection, the MFMA prefill
// GEMM and the MoE expert FFN.  Every helper only queues work (Backend::run); results
// are visible after Backend::sync().
#pragma once
#include <cstdint>

#include "apex_hip.h"
#include "backend.h"

namespace apex {

// An NVFP4 matrix [w_rows, hidden_dim] in GPU memory; codes and scales may share one
// buffer at different offsets (src/ops.h:7-16).
struct Nvfp4Matrix {
    Buffer *weights;
    size_t weights_offset; // uint32 [w_rows, hidden_dim / 8]
    Buffer *scales;
    size_t scales_offset;  // uint8  [w_rows, hidden_dim / 16]
    uint32_t w_rows;
    uint32_t hidden_dim;
};

// RMSNorm of fp32 rows with bf16 weights (src/ops.h:18-26): one threadgroup per row.
inline void rmsNorm(Backend &backend, Buffer *input, Buffer *weights, size_t weight_offset,
                    Buffer *result, uint32_t rows, uint32_t hidden_dim, float eps) {
    constexpr uint32_t kThreads = 256;
    backend.run("rms_norm_f32",
                {Arg::buf(input), Arg::buf(weights, weight_offset), Arg::buf(result),
                 Arg::val(hidden_dim), Arg::val(eps)},
                Dim3{rows}, Dim3{kThreads});
}

// Per-head RMSNorm, optional learned scaling and RoPE on the first rope_pairs pairs
// (src/ops.h:71-118): input [tokens, heads, head_dim] fp32; head (t, h) is written at
// output + output_offset + (t * out_token_stride + h * out_head_stride) floats.
inline void headNormRope(Backend &backend, Buffer *input, Buffer *weights, size_t weights_offset,
                         bool has_weights, Buffer *output, size_t output_offset, uint32_t tokens,
                         uint32_t heads, uint32_t head_dim, uint32_t rope_pairs, float rope_base,
                         uint32_t abs_pos, uint32_t out_token_stride, uint32_t out_head_stride,
                         float eps) {
    constexpr uint32_t kThreads = 256;
    const uint32_t weight_flag = has_weights ? 1u : 0u;
    backend.run("head_norm_rope_f32",
                {Arg::buf(input), Arg::buf(weights, weights_offset),
                 Arg::buf(output, output_offset), Arg::val(heads), Arg::val(head_dim),
                 Arg::val(weight_flag), Arg::val(rope_pairs), Arg::val(rope_base),
                 Arg::val(abs_pos), Arg::val(out_token_stride), Arg::val(out_head_stride),
                 Arg::val(eps)},
                Dim3{tokens, heads}, Dim3{kThreads});
}

// fp32 [tokens, hidden_dim] -> fp32 [tokens, w_rows] (src/ops.h:34-46): the reference
// launch shape, rows in groups of 8 and tokens on the grid's y axis.
inline void matmulNvfp4(Backend &backend, Buffer *input, const Nvfp4Matrix &W, Buffer *output,
                        uint32_t tokens) {
    constexpr uint32_t kRowsPerGroup = 8, kThreads = 256;
    const uint32_t row_groups = (W.w_rows + kRowsPerGroup - 1) / kRowsPerGroup;
    backend.run("matmul_nvfp4",
                {Arg::buf(input), Arg::buf(W.weights, W.weights_offset),
                 Arg::buf(W.scales, W.scales_offset), Arg::buf(output), Arg::val(W.hidden_dim),
                 Arg::val(W.w_rows)},
                Dim3{row_groups, tokens}, Dim3{kThreads});
}

// output[i] = gelu_tanh(gate[i]) * up[i], fp32, in place allowed (src/ops.h:48-55).
inline void geglu(Backend &backend, Buffer *gate, Buffer *up, Buffer *output, uint32_t count) {
    constexpr uint32_t kThreads = 256;
    backend.run("geglu_f32", {Arg::buf(gate), Arg::buf(up), Arg::buf(output), Arg::val(count)},
                Dim3{(count + kThreads - 1) / kThreads}, Dim3{kThreads});
}

// GeGLU FFN with fp32 intermediates, four launches (src/ops.h:57-69).
inline void denseMlp(Backend &backend, Buffer *input, const Nvfp4Matrix &gate_weights,
                     const Nvfp4Matrix &up_weights, const Nvfp4Matrix &down_weights,
                     Buffer *gate_tmp, Buffer *up_tmp, Buffer *output, uint32_t tokens) {
    matmulNvfp4(backend, input, gate_weights, gate_tmp, tokens);
    matmulNvfp4(backend, input, up_weights, up_tmp, tokens);
    geglu(backend, gate_tmp, up_tmp, gate_tmp, tokens * gate_weights.w_rows);
    matmulNvfp4(backend, gate_tmp, down_weights, output, tokens);
}

// ---- additional ops of the HIP backend ------------------------------------------------

// bf16 [tokens, hidden_dim] -> bf16 [tokens, w_rows], fp32 accumulation.  Few tokens
// run as the bandwidth-bound GEMV, more as the MFMA GEMM (apex_hip_set_gemm_min_tokens);
// matmulNvfp4 and gegluNvfp4 switch the same way.
inline void matmulNvfp4Bf16(Backend &backend, Buffer *input, const Nvfp4Matrix &W, Buffer *output,
                            uint32_t tokens, float tensor_scale = 1.0f) {
    backend.run("matmul_nvfp4_bf16",
                {Arg::buf(input), Arg::buf(W.weights, W.weights_offset),
                 Arg::buf(W.scales, W.scales_offset), Arg::buf(output), Arg::val(W.hidden_dim),
                 Arg::val(W.w_rows), Arg::val(tokens), Arg::val(tensor_scale)},
                Dim3{1}, Dim3{256});
}

// gelu_tanh(gate . x) * (up . x) in one pass over both weight matrices: the gate/up
// half of denseMlp fused (no fp32 round trip).  x and output are bf16 if `bf16`,
// else fp32.
inline void gegluNvfp4(Backend &backend, Buffer *input, const Nvfp4Matrix &gate,
                       const Nvfp4Matrix &up, Buffer *output, uint32_t tokens, bool bf16,
                       float gate_scale = 1.0f, float up_scale = 1.0f) {
    backend.run(bf16 ? "geglu_nvfp4_bf16" : "geglu_nvfp4_f32",
                {Arg::buf(input), Arg::buf(gate.weights, gate.weights_offset),
                 Arg::buf(gate.scales, gate.scales_offset), Arg::buf(up.weights, up.weights_offset),
                 Arg::buf(up.scales, up.scales_offset), Arg::buf(output), Arg::val(gate.hidden_dim),
                 Arg::val(gate.w_rows), Arg::val(tokens), Arg::val(gate_scale),
                 Arg::val(up_scale)},
                Dim3{1}, Dim3{256});
}

// rmsNorm of each fp32 input row (bf16 weights at norm_weights + norm_offset) fused into
// the fp32 gate/up GeGLU GEMV: one launch in place of rmsNorm + gegluNvfp4.  Needs
// hidden_dim % 32 == 0 and a 16-byte aligned input.
inline void gegluNvfp4RmsNorm(Backend &backend, Buffer *input, Buffer *norm_weights,
                              size_t norm_offset, float eps, const Nvfp4Matrix &gate,
                              const Nvfp4Matrix &up, Buffer *output, uint32_t tokens,
                              float gate_scale = 1.0f, float up_scale = 1.0f) {
    backend.run("geglu_nvfp4_rms_norm_f32",
                {Arg::buf(input), Arg::buf(norm_weights, norm_offset),
                 Arg::buf(gate.weights, gate.weights_offset),
                 Arg::buf(gate.scales, gate.scales_offset), Arg::buf(up.weights, up.weights_offset),
                 Arg::buf(up.scales, up.scales_offset), Arg::buf(output), Arg::val(gate.hidden_dim),
                 Arg::val(gate.w_rows), Arg::val(tokens), Arg::val(gate_scale),
                 Arg::val(up_scale), Arg::val(eps)},
                Dim3{1}, Dim3{256});
}

// Prefill GEMM: bf16 A [M, K] x NVFP4 W [N, K]^T -> bf16 C [M, N] on bf16 MFMA.
inline void gemmNvfp4Bf16(Backend &backend, Buffer *A, const Nvfp4Matrix &W, Buffer *C, uint32_t M,
                          float tensor_scale = 1.0f) {
    backend.run("gemm_nvfp4_bf16",
                {Arg::buf(A), Arg::buf(W.weights, W.weights_offset),
                 Arg::buf(W.scales, W.scales_offset), Arg::buf(C), Arg::val(M), Arg::val(W.w_rows),
                 Arg::val(W.hidden_dim), Arg::val(tensor_scale)},
                Dim3{1}, Dim3{256});
}

// Dense GeGLU FFN with the fused gate/up projection: two launches instead of four.
inline void denseMlpFused(Backend &backend, Buffer *input, const Nvfp4Matrix &gate_weights,
                          const Nvfp4Matrix &up_weights, const Nvfp4Matrix &down_weights,
                          Buffer *h_tmp, Buffer *output, uint32_t tokens) {
    gegluNvfp4(backend, input, gate_weights, up_weights, h_tmp, tokens, false);
    matmulNvfp4(backend, h_tmp, down_weights, output, tokens);
}

// Expert slots: expert e's six pieces at slots + e * stride + offset
// (tools/repack.py:180-213 slot format).
struct ExpertSlots {
    Buffer *slots;
    uint32_t stride;
    uint32_t gate_w, gate_s, up_w, up_s, down_w, down_s;
};

// Device workspace the MoE op needs for these sizes.
inline size_t moeWorkspaceBytes(uint32_t tokens, uint32_t experts, uint32_t top_k, uint32_t hidden,
                                uint32_t inter) {
    return apex_moe_workspace_bytes(tokens, experts, top_k, hidden, inter);
}

// MoE expert FFN: router top-k + softmax over bf16 logits [tokens, experts], then
// y = sum_j w_j * down_e(gelu(gate_e x) * up_e x) for bf16 x, y [tokens, hidden].
inline void moeFfn(Backend &backend, Buffer *x, Buffer *logits, const ExpertSlots &E, Buffer *y,
                   Buffer *workspace, uint32_t tokens, uint32_t experts, uint32_t top_k,
                   uint32_t hidden, uint32_t inter) {
    backend.run("moe_ffn_nvfp4_bf16",
                {Arg::buf(x), Arg::buf(logits), Arg::buf(E.slots), Arg::buf(y), Arg::buf(workspace),
                 Arg::val(tokens), Arg::val(experts), Arg::val(top_k), Arg::val(hidden),
                 Arg::val(inter), Arg::val(E.stride), Arg::val(E.gate_w), Arg::val(E.gate_s),
                 Arg::val(E.up_w), Arg::val(E.up_s), Arg::val(E.down_w), Arg::val(E.down_s)},
                Dim3{1}, Dim3{256});
}

// Gemma-4 router (docs/B6_3_attention.md:721-725), the tensors of tools/out.txt:247-290:
// router.scale (RMSNorm weights, bf16 [hidden]), router.proj (affine 8-bit: u32 codes
// [experts, hidden/4], bf16 scales and biases [experts, hidden/64]) and
// router.per_expert_scale (bf16 [experts]), each at an offset in a weights buffer.
struct RouterWeights {
    Buffer *buffer;
    size_t norm_offset, codes_offset, scales_offset, biases_offset, per_expert_scale_offset;
    uint32_t experts, hidden;
};

// Router logits fp32 [tokens, experts] from the raw hidden h fp32 [tokens, hidden].
inline void moeRouterLogits(Backend &backend, Buffer *h, const RouterWeights &R, Buffer *logits,
                            uint32_t tokens, float eps) {
    backend.run("moe_router_logits_q8_f32",
                {Arg::buf(h), Arg::buf(R.buffer, R.norm_offset), Arg::buf(R.buffer, R.codes_offset),
                 Arg::buf(R.buffer, R.scales_offset), Arg::buf(R.buffer, R.biases_offset),
                 Arg::buf(logits), Arg::val(tokens), Arg::val(R.experts), Arg::val(R.hidden),
                 Arg::val(eps)},
                Dim3{1}, Dim3{256});
}

// Top-k of fp32 logits, softmax over the k, times router.per_expert_scale:
// ids i32 / weights f32 [tokens, top_k].
inline void moeRoute(Backend &backend, Buffer *logits, const RouterWeights &R, Buffer *ids,
                     Buffer *weights, uint32_t tokens, uint32_t top_k) {
    const uint32_t has_scale = 1;
    backend.run("moe_route_f32",
                {Arg::buf(logits), Arg::buf(R.buffer, R.per_expert_scale_offset), Arg::buf(ids),
                 Arg::buf(weights), Arg::val(tokens), Arg::val(R.experts), Arg::val(top_k),
                 Arg::val(has_scale)},
                Dim3{1}, Dim3{256});
}

// The MoE block after the router projection: routing from the fp32 logits (times
// router.per_expert_scale) and the expert FFN, bf16 x, y [tokens, hidden].
inline void moeFfnFromLogits(Backend &backend, Buffer *x, Buffer *logits, const RouterWeights &R,
                             const ExpertSlots &E, Buffer *y, Buffer *workspace, uint32_t tokens,
                             uint32_t top_k, uint32_t hidden, uint32_t inter) {
    const uint32_t has_scale = 1;
    backend.run("moe_ffn_f32logits_nvfp4_bf16",
                {Arg::buf(x), Arg::buf(logits), Arg::buf(R.buffer, R.per_expert_scale_offset),
                 Arg::buf(E.slots), Arg::buf(y), Arg::buf(workspace), Arg::val(tokens),
                 Arg::val(R.experts), Arg::val(top_k), Arg::val(hidden), Arg::val(inter),
                 Arg::val(E.stride), Arg::val(E.gate_w), Arg::val(E.gate_s), Arg::val(E.up_w),
                 Arg::val(E.up_s), Arg::val(E.down_w), Arg::val(E.down_s), Arg::val(has_scale)},
                Dim3{1}, Dim3{256});
}

} // namespace apex
