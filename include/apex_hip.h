/*
 * apex_hip.h -- C ABI of the MI355X (gfx950) HIP backend for APEX's NVFP4 matmul path.
 *
 * Three layers, all plain C (pointers, sizes, no HIP or C++ types):
 *
 *  1. The backend object.  One-for-one with the reference's apex::Backend interface
 *     (src/backend/backend.h:39-63) and its Metal implementation
 *     (src/backend/metal_backend.{h,cpp}); the C++ class apex::HipBackend
 *     (apex_amd/host/hip_backend.h) is a thin adapter over these calls, and the
 *     reference's src/ops.h calls it unchanged.  Kernels are selected by name as in
 *     metal_backend.cpp:54-82 and bound by position as in metal_backend.cpp:162-167.
 *  2. Direct entry points on device pointers and a stream, for hosts that manage
 *     their own device memory.  The backend's kernels call the same code.
 *  3. Plumbing (device memory, copies, streams, events) for hosts without their own
 *     HIP runtime, e.g. Python through ctypes.
 *
 * Every function returns APEX_HIP_OK (0) on success or a nonzero APEX_HIP_E_* code;
 * apex_hip_last_error() then describes the failure (per calling thread).  The
 * reference throws std::runtime_error in the same places (metal_backend.cpp:18-34,
 * 61-76, 91-93, 117-119, 169-171); apex::HipBackend turns nonzero codes back into
 * std::runtime_error.  A backend object is not thread-safe (one stream, one host
 * thread), like MetalBackend.
 */
#ifndef APEX_HIP_H
#define APEX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define APEX_HIP_ABI_VERSION 1

enum {
    APEX_HIP_OK = 0,
    APEX_HIP_E_INVALID = 1,        /* bad argument value or shape */
    APEX_HIP_E_UNKNOWN_KERNEL = 2, /* metal_backend.cpp:61-64 "cannot find function" */
    APEX_HIP_E_ARGS = 3,           /* wrong argument count or kind for a kernel */
    APEX_HIP_E_ALIGN = 4,          /* metal_backend.cpp:89-93 wrapNoCopy alignment */
    APEX_HIP_E_DEVICE = 5,         /* HIP runtime error or no device */
    APEX_HIP_E_OOM = 6,            /* allocation failed (metal_backend.cpp:117-119) */
    APEX_HIP_E_THREADGROUP = 7     /* metal_backend.cpp:169-171 "threadgroup too large" */
};

typedef struct apex_hip_backend apex_hip_backend;
typedef struct apex_hip_buffer apex_hip_buffer;

/* src/backend/backend.h:15-29 (Arg): a buffer plus byte offset, or `size` value bytes
 * at `bytes` (copied when the kernel is queued, so temporaries are fine). */
typedef struct {
    apex_hip_buffer *buffer;
    size_t offset;
    const void *bytes;
    size_t size;
} apex_hip_arg;

/* src/backend/backend.h:33-37 (Dim3). */
typedef struct {
    uint32_t x, y, z;
} apex_hip_dim3;

/* Description of the failure of the last call that returned nonzero on this thread. */
const char *apex_hip_last_error(void);
int apex_hip_abi_version(void);

/* ---------------------------------------------------------------------------------
 * 1. Backend object
 * -------------------------------------------------------------------------------*/

/* MetalBackend::MetalBackend (metal_backend.cpp:14-35): opens `device` and creates
 * one in-order stream.  The kernels are linked in, so there is no library path. */
int apex_hip_backend_create(int device, apex_hip_backend **out);

/* MetalBackend::~MetalBackend (metal_backend.cpp:37-45). */
void apex_hip_backend_destroy(apex_hip_backend *backend);

/* MetalBackend::deviceName (metal_backend.cpp:47-49): gcnArchName of the device. */
int apex_hip_device_name(apex_hip_backend *backend, char *buf, size_t len);

/* Backend::wrapNoCopy (backend.h:45-46, metal_backend.cpp:88-107).  `host` and
 * `bytes` must be multiples of 16384, as in the reference.  HBM is not the host's
 * memory, so the bytes are uploaded once, before the first kernel that reads the
 * buffer; `host` must stay valid until release.  Not counted by any tracker. */
int apex_hip_wrap_no_copy(apex_hip_backend *backend, void *host, size_t bytes,
                          apex_hip_buffer **out);

/* Backend::allocate (backend.h:48-49, metal_backend.cpp:113-126): `bytes` of
 * zero-filled device memory.  `category` is kept for the caller's memory tracker. */
int apex_hip_allocate(apex_hip_backend *backend, size_t bytes, const char *category,
                      apex_hip_buffer **out);

/* Backend::contents (backend.h:51-52, metal_backend.cpp:131): a host pointer to the
 * buffer's bytes.  The reference's memory is unified; here the buffer has a host
 * mirror: this call waits for queued kernels if the device copy is newer, downloads
 * it, and marks the host copy as the one to upload before the next kernel that uses
 * the buffer.  Do not call it inside timed regions. */
int apex_hip_contents(apex_hip_backend *backend, apex_hip_buffer *buffer, void **out);

/* Backend::release (backend.h:54-55, metal_backend.cpp:136-149). */
int apex_hip_release(apex_hip_backend *backend, apex_hip_buffer *buffer);

/* Backend::run (backend.h:57-60, metal_backend.cpp:151-174): queue kernel `kernel`
 * with positional arguments.  Returns once the kernels are queued; they run in queue
 * order.  The dense ops that run as an MFMA GEMM at prefill token counts (matmul_nvfp4
 * with a full grid, matmul_nvfp4_bf16, the geglu_nvfp4 kernels, gemm_nvfp4_bf16) use the
 * device's GEMM scratch when their activations are fp32 (the bf16 hi / lo split) or
 * their grid has few tiles (split-K partials).  A call needing more scratch than any
 * before grows it: that call allocates device memory and waits for the scratch's
 * earlier users, so it does not return at once and cannot run under graph capture.
 * Keep the GEMV with apex_hip_set_gemm_min_tokens, or make one warm-up call at the
 * largest shape first.
 * Kernels and argument lists (B = buffer, U = uint32 value, F = float value):
 *   matmul_nvfp4      B input f32 [T,K], B weights u32 [rows,K/8], B scales u8
 *                     [rows,K/16], B output f32 [T,w_rows], U hidden_dim K, U w_rows.
 *                     T = threadgroups.y and rows covered = min(w_rows,
 *                     threadgroups.x * threads/32), as the reference launch
 *                     (src/ops.h:34-46, shaders/matmul.metal:14-18) implies.  A grid
 *                     covering every row (the reference's ceil(w_rows/8) x 256) runs
 *                     apex_nvfp4_matmul_f32: an MFMA GEMM at prefill token counts
 *                     (on the GEMM scratch, see above), a GEMV below them; a grid
 *                     covering fewer rows runs the GEMV on those rows (output rows
 *                     strided by w_rows).
 *   geglu_f32         B gate, B up, B output, U count (in place allowed);
 *                     src/ops.h:48-55, shaders/geglu.metal:6-24.
 *   matmul_nvfp4_bf16 B input bf16 [T,K], B weights, B scales, B output bf16 [T,rows],
 *                     U hidden_dim, U w_rows, U tokens, F tensor_scale.
 *   geglu_nvfp4_f32   B input f32, B gate weights, B gate scales, B up weights,
 *   geglu_nvfp4_bf16  B up scales, B output [T,rows], U hidden_dim, U w_rows,
 *                     U tokens, F gate tensor_scale, F up tensor_scale:
 *                     gelu_tanh(gate.x) * (up.x) in one pass (src/ops.h:65-67 fused).
 *   geglu_nvfp4_rms_norm_f32 B input f32 [T,K], B norm weights bf16 [K], B gate
 *                     weights, B gate scales, B up weights, B up scales, B output f32
 *                     [T,rows], U hidden_dim, U w_rows, U tokens, F gate tensor_scale,
 *                     F up tensor_scale, F eps: rms_norm_f32 of x, then geglu_nvfp4_f32
 *                     (apex_nvfp4_geglu_rms_norm_f32).
 *   gemm_nvfp4_bf16   B A bf16 [M,K], B weights [N,K/8], B scales [N,K/16], B C bf16
 *                     [M,N], U M, U N, U K, F tensor_scale (apex_nvfp4_gemm_bf16).
 *   dequant_nvfp4_f32 B weights, B scales, B output [rows,K], U hidden_dim,
 *   dequant_nvfp4_bf16 U w_rows, F tensor_scale (src/nvfp4.h:27-43 on the device).
 *   moe_ffn_nvfp4_bf16 B x bf16 [T,H], B logits bf16 [T,E], B expert slots, B y bf16
 *                     [T,H], B workspace (apex_moe_workspace_bytes), U T, U E, U top_k,
 *                     U H, U I, U slot stride, U gate_w, U gate_s, U up_w, U up_s,
 *                     U down_w, U down_s (apex_moe_ffn_bf16).
 *   moe_route_bf16    B logits bf16 [T,E], B ids i32 [T,k], B weights f32 [T,k], U T,
 *                     U E, U top_k (apex_moe_route_bf16).
 *   moe_router_logits_q8_f32 B h f32 [T,H], B router.scale bf16 [H], B proj weights
 *                     u32 [E,H/4], B proj scales bf16 [E,H/64], B proj biases, B logits f32
 *                     [T,E], U T, U E, U H, F eps (apex_moe_router_logits_q8).
 *   moe_route_f32     B logits f32 [T,E], B per-expert scale bf16 [E], B ids, B weights,
 *                     U T, U E, U top_k, U has_scale (apex_moe_route_f32).
 *   moe_ffn_f32logits_nvfp4_bf16 B x bf16, B logits f32, B per-expert scale, B expert
 *                     slots, B y bf16, B workspace, U T, U E, U top_k, U H, U I, U slot
 *                     stride, the six U piece offsets, U has_scale
 *                     (apex_moe_ffn_f32logits_bf16).
 *   rms_norm_f32      B input f32 [rows,n], B weights bf16 [n], B result f32 [rows,n],
 *                     U hidden_dim n, F eps; rows = threadgroups.x (src/ops.h:18-26,
 *                     shaders/norm.metal:33-81).
 *   head_norm_rope_f32 B input f32 [T,heads,head_dim], B weights bf16 [head_dim], B
 *                     output, U heads, U head_dim, U has_weight, U rope_pairs, F
 *                     rope_base, U abs_pos, U out_token_stride, U out_head_stride, F eps;
 *                     T = threadgroups.x, threadgroups.y = heads (src/ops.h:88-118,
 *                     shaders/head_norm_rope.metal:5-72).  head_dim even, <= 512.
 * For the kernels after geglu_f32 the launch shape is chosen by the backend; the
 * caller's threadgroups/threads must only be nonzero (the norms read T / rows from
 * threadgroups as the reference launches do). */
int apex_hip_run(apex_hip_backend *backend, const char *kernel, const apex_hip_arg *args,
                 size_t nargs, apex_hip_dim3 threadgroups, apex_hip_dim3 threads_per_group);

/* Backend::sync (backend.h:62-63, metal_backend.cpp:176-184): wait for all queued
 * kernels. */
int apex_hip_sync(apex_hip_backend *backend);

/* No reference counterpart (the reference maps files into unified memory, src/file.h:
 * 27-73, and wraps the mapping with Backend::wrapNoCopy): bytes [file_offset,
 * file_offset + bytes) of the file at `path` are streamed into `buffer` at
 * buffer_offset through pinned staging buffers (pread overlapped with host-to-device
 * copies on the backend's stream); returns when they are on the device.  The rest of
 * the buffer keeps its contents. */
int apex_hip_load_file(apex_hip_backend *backend, apex_hip_buffer *buffer, uint64_t buffer_offset,
                       const char *path, uint64_t file_offset, uint64_t bytes);

/* No reference counterpart (the reference's buffers are host-visible): the device
 * address of a buffer (valid until release), its length, and the backend's stream
 * (a hipStream_t) for hosts mixing backend kernels with direct entry points. */
int apex_hip_buffer_device_ptr(apex_hip_buffer *buffer, void **out);
size_t apex_hip_buffer_length(apex_hip_buffer *buffer);
void *apex_hip_backend_stream(apex_hip_backend *backend);

/* Registry introspection and argument validation (host only, no device needed):
 * the checks apex_hip_run applies before anything touches the GPU. */
int apex_hip_kernel_count(void);
const char *apex_hip_kernel_name(int index);
const char *apex_hip_kernel_signature(const char *kernel);
int apex_hip_validate_run(const char *kernel, const apex_hip_arg *args, size_t nargs,
                          apex_hip_dim3 threadgroups, apex_hip_dim3 threads_per_group);

/* ---------------------------------------------------------------------------------
 * 2. Direct entry points: device pointers, `stream` is a hipStream_t (NULL = default).
 *    W is NVFP4 [rows, K]: codes uint32 [rows, K/8], scales E4M3 [rows, K/16];
 *    K % 16 == 0.  tensor_scale multiplies every weight (1.0 = reference).
 * -------------------------------------------------------------------------------*/

/* shaders/matmul.metal:4-53 / src/tests/cpu_ref.h:48-63: out[t, r] = sum_k W[r,k] x[t,k]
 * with fp32 activations and outputs.  A GEMV for few tokens; for more (K % 64 == 0,
 * apex_hip_set_gemm_min_tokens) an MFMA GEMM on x split into bf16 hi + lo halves
 * (|x - hi - lo| <= 2^-17 |x|) held in the device's GEMM scratch (tokens * K * 4
 * bytes). */
int apex_nvfp4_matmul_f32(const float *x, const uint32_t *codes, const uint8_t *scales,
                          float tensor_scale, float *out, uint32_t tokens, uint32_t rows,
                          uint32_t K, void *stream);

/* Same product with bf16 activations and bf16 outputs (fp32 accumulation): a GEMV
 * for few tokens, the MFMA GEMM below for more (K % 64 == 0,
 * apex_hip_set_gemm_min_tokens). */
int apex_nvfp4_matmul_bf16(const uint16_t *x, const uint32_t *codes, const uint8_t *scales,
                           float tensor_scale, uint16_t *out, uint32_t tokens, uint32_t rows,
                           uint32_t K, void *stream);

/* Prefill GEMM (no reference counterpart: the reference runs prefill as one GEMV per
 * token, src/ops.h:44): C[M, N] = tensor_scale * A[M, K] . W[N, K]^T with A, C bf16
 * row-major (C row stride N), W NVFP4, bf16 MFMA on W dequantised exactly to bf16.
 * Requires K % 64 == 0. */
int apex_nvfp4_gemm_bf16(const uint16_t *A, const uint32_t *codes, const uint8_t *scales,
                         float tensor_scale, uint16_t *C, uint32_t M, uint32_t N, uint32_t K,
                         void *stream);

/* src/ops.h:65-67 fused: out[t, r] = gelu_tanh(Wg[r].x_t) * (Wu[r].x_t).  Like the
 * matmuls: a GEMV for few tokens, for more (K % 64 == 0) one MFMA GEMM whose tiles hold
 * gate and up rows of the same outputs (fp32 x: through its bf16 hi + lo split). */
int apex_nvfp4_geglu_f32(const float *x, const uint32_t *gate_codes, const uint8_t *gate_scales,
                         float gate_tensor_scale, const uint32_t *up_codes,
                         const uint8_t *up_scales, float up_tensor_scale, float *out,
                         uint32_t tokens, uint32_t rows, uint32_t K, void *stream);
/* The same after an RMSNorm of each x row (the step before the MLP in the reference's
 * model, src/ops.h:18-26 rmsNorm then 65-67): x_t * (1 / sqrt(mean(x_t^2) + eps)) * w,
 * computed inside the GEMV's x staging (or the GEMM's split pass) instead of a
 * separate launch and buffer.  norm_w is bf16 [K]; the GEMV form needs K % 32 == 0,
 * K <= 8192, x and codes 16-byte aligned. */
int apex_nvfp4_geglu_rms_norm_f32(const float *x, const uint16_t *norm_w, float eps,
                                  const uint32_t *gate_codes, const uint8_t *gate_scales,
                                  float gate_tensor_scale, const uint32_t *up_codes,
                                  const uint8_t *up_scales, float up_tensor_scale, float *out,
                                  uint32_t tokens, uint32_t rows, uint32_t K, void *stream);
int apex_nvfp4_geglu_bf16(const uint16_t *x, const uint32_t *gate_codes,
                          const uint8_t *gate_scales, float gate_tensor_scale,
                          const uint32_t *up_codes, const uint8_t *up_scales,
                          float up_tensor_scale, uint16_t *out, uint32_t tokens, uint32_t rows,
                          uint32_t K, void *stream);

/* shaders/geglu.metal:6-24: out[i] = gelu_tanh(gate[i]) * up[i]; out may alias gate. */
int apex_geglu_f32(const float *gate, const float *up, float *out, uint32_t count,
                   void *stream);

/* shaders/norm.metal:33-81 (src/ops.h:18-26 rmsNorm): per row of x [rows, hidden_dim]
 * fp32, y = x * (1 / sqrt(mean(x^2) + eps)) * w with w bf16 [hidden_dim]; fp32 sums.
 * y may alias x. */
int apex_rms_norm_f32(const float *x, const uint16_t *weights, float *y, uint32_t rows,
                      uint32_t hidden_dim, float eps, void *stream);

/* shaders/head_norm_rope.metal:5-72 (src/ops.h:88-118 headNormRope): per token t and
 * head h of x [tokens, heads, head_dim] fp32, RMS-normalise the head (times w bf16
 * [head_dim] if has_weights), then rotate pairs (i, head_dim/2 + i) for i < rope_pairs
 * by (abs_pos + t) * rope_base^(-2 i / head_dim); write head (t, h) at
 * y + t * out_token_stride + h * out_head_stride.  head_dim even and <= 512. */
int apex_head_norm_rope_f32(const float *x, const uint16_t *weights, int has_weights, float *y,
                            uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t rope_pairs,
                            float rope_base, uint32_t abs_pos, uint32_t out_token_stride,
                            uint32_t out_head_stride, float eps, void *stream);

/* src/nvfp4.h:27-43 on the device: out[r, k] = e2m1 * e4m3 * tensor_scale. */
int apex_nvfp4_dequant_f32(const uint32_t *codes, const uint8_t *scales, float tensor_scale,
                           float *out, uint32_t rows, uint32_t K, void *stream);
int apex_nvfp4_dequant_bf16(const uint32_t *codes, const uint8_t *scales, float tensor_scale,
                            uint16_t *out, uint32_t rows, uint32_t K, void *stream);

/* ---------------------------------------------------------------------------------
 * 3. Plumbing (no reference counterpart).
 * -------------------------------------------------------------------------------*/
int apex_hip_device_count(int *out);
int apex_hip_set_device(int device);
int apex_hip_malloc(size_t bytes, void **out);
int apex_hip_free(void *ptr);
int apex_hip_memcpy_h2d(void *dst, const void *src, size_t bytes);
int apex_hip_memcpy_d2h(void *dst, const void *src, size_t bytes);
int apex_hip_memcpy_d2d(void *dst, const void *src, size_t bytes);
int apex_hip_memset(void *dst, int value, size_t bytes);
/* Free and total device memory of the current device (hipMemGetInfo). */
int apex_hip_mem_info(size_t *free_bytes, size_t *total_bytes);
int apex_hip_device_synchronize(void);
int apex_hip_stream_create(void **out);
int apex_hip_stream_destroy(void *stream);
int apex_hip_stream_synchronize(void *stream);
int apex_hip_event_create(void **out);
int apex_hip_event_destroy(void *event);
int apex_hip_event_record(void *event, void *stream);
int apex_hip_event_synchronize(void *event);
int apex_hip_event_elapsed_ms(void *start, void *stop, float *ms);

/* Streaming-read probe: reads [ptr, ptr+bytes) once with 16-byte buffer loads
 * (bytes < 2 GiB); `sink` must hold apex_hip_read_probe_sink_words() words.  Used by
 * the benchmark to measure the achievable HBM read rate beside the spec peak. */
int apex_hip_read_probe(const void *ptr, size_t bytes, uint32_t *sink, void *stream);
int apex_hip_read_probe_sink_words(void);

/* Launch tuning of the GEMV kernels: target resident waves per CU (default 8). */
int apex_hip_set_gemv_waves_per_cu(int waves);

/* Tokens from which apex_nvfp4_matmul_* and apex_nvfp4_geglu_* (and their registry
 * kernels) run as MFMA GEMMs instead of GEMVs, for bf16 and for fp32 activations
 * (0 = by size, the default: GeGLU from 16 tokens, matmul from 16 when the GEMM has at
 * least 64 tiles of 256 tokens x 256 outputs, else from 32).
 * Process-wide; results agree within the stated tolerances either way.  The GEMMs'
 * scratch (fp32 split, split-K partials) is device memory the library keeps per
 * device, grown on demand (growing synchronises the calling stream) and held until the
 * process ends; uses from different streams are ordered on the GPU by an event. */
int apex_hip_set_gemm_min_tokens(uint32_t bf16_tokens, uint32_t f32_tokens);

/* Dense-product launches this process has made, by form, counted when the matmul and
 * GeGLU entry points and registry kernels (matmul_nvfp4, geglu_nvfp4_*, ...) enqueue
 * them: counts[0] GEMVs, [1] MFMA GEMMs, [2] split-K MFMA GEMMs, [3] fp32 hi + lo split
 * passes.  Lets a host see which form a call took; no device needed. */
int apex_hip_dense_dispatch_counts(uint64_t counts[4]);

/* How the MFMA GEMM covers an M x N output (N: output columns; GeGLU: h columns) on
 * `ncu` CUs (0: the current device's): out[0] = n-tiles of whole tiles (256 x 256, GeGLU
 * 256 x 128 h columns); the columns past them fill the last round's CUs either as
 * narrow tiles of out[1] W blocks (32 rows) each or as out[2] short tiles (full width,
 * at most 6 32-row blocks of one column each); out[1] = out[2] = 0: whole tiles only.
 * No launch. */
int apex_hip_gemm_tail_plan(uint32_t m, uint32_t n, int geglu, uint32_t ncu, uint32_t out[3]);

/* ---- MoE expert FFN (no reference kernel) ------------------------------------------
 * Semantics: tools/dump_reference.py:208-219 (router top-k, experts combined with the
 * router weights) with each expert the dense GeGLU FFN of src/ops.h:57-69
 * (gate/up [I, H], down [H, I], all NVFP4), stored in the fixed-stride slot format of
 * tools/repack.py:180-213 / src/model_info.h:189-204.  These entry points extend the
 * ops.h surface for the MoE layer the reference plans (docs/B6_3_attention.md:721-725). */

/* One expert slot layout: expert e's pieces start at base + e * stride + offset. */
typedef struct {
    const void *base;   /* device pointer to expert 0's slot (16-byte aligned) */
    uint64_t stride;    /* bytes between consecutive slots (multiple of 16, < 2 GiB) */
    uint64_t gate_w, gate_s, up_w, up_s, down_w, down_s; /* piece offsets in a slot */
} apex_moe_slots;

/* Router: per token the top_k of `experts` bf16 logits (ties to the lower expert id),
 * in descending order, and softmax weights over those k (fp32).  ids/weights are
 * [tokens, top_k].  experts <= 256, top_k <= 16. */
int apex_moe_route_bf16(const uint16_t *logits, uint32_t tokens, uint32_t experts, uint32_t top_k,
                        int32_t *ids, float *weights, void *stream);

/* Gemma-4 router logits (docs/B6_3_attention.md:721-725; tensors router.scale,
 * router.proj.{weight,scales,biases} of tools/out.txt:247-290): per token, RMSNorm of
 * the raw hidden h fp32 [tokens, hidden] with norm_weights bf16 [hidden] (rmsNormCpu
 * arithmetic), then logits[t, e] = sum_k xn[t, k] * (scale[e, g] * q[e, k] + bias[e, g])
 * with q the unsigned byte (k % 4) of proj_weights[e, k / 4] (u32 [experts, hidden/4]),
 * g = k / 64 and scales/biases bf16 [experts, hidden/64]; fp32 out [tokens, experts].
 * experts <= 256, hidden a multiple of 64 and at most 4096.  From 512 tokens the
 * product runs on bf16 MFMA in one kernel with no scratch (h * norm_weights split into
 * bf16 hi + lo on the fly, codes exact in bf16, group scale and bias in fp32, the
 * RMSNorm's per-token factor applied to the finished sums). */
int apex_moe_router_logits_q8(const float *h, const uint16_t *norm_weights, float eps,
                              const uint32_t *proj_weights, const uint16_t *proj_scales,
                              const uint16_t *proj_biases, uint32_t tokens, uint32_t experts,
                              uint32_t hidden, float *logits, void *stream);

/* apex_moe_route_bf16 on fp32 logits, each routing weight then multiplied by the bf16
 * per_expert_scale[expert] (router.per_expert_scale; null: no scale). */
int apex_moe_route_f32(const float *logits, const uint16_t *per_expert_scale, uint32_t tokens,
                       uint32_t experts, uint32_t top_k, int32_t *ids, float *weights,
                       void *stream);

/* Packed weight files (tools/repack.py:180-257: core.bin, layer_NN.bin with 128 expert
 * slots at a fixed stride) into device memory.  apex_file_to_device copies bytes
 * [file_offset, file_offset + bytes) to dst; apex_experts_to_device copies slot
 * experts[i] (file bytes [experts[i] * stride, + slot_bytes)) to dst + i * dst_stride
 * for i < n_experts (experts is a host array).  Both read chunk_bytes at a time into
 * n_buffers pinned host buffers (n_buffers / 2 reader threads, two buffers each) while
 * earlier chunks' host-to-device copies run on `stream` (0: 8 MiB, 8 buffers), and
 * return once every copy has completed.  The pinned buffers are kept for the process
 * and reused by later calls of the same shape; calls are serialised. */
int apex_file_to_device(const char *path, uint64_t file_offset, uint64_t bytes, void *dst,
                        uint64_t chunk_bytes, uint32_t n_buffers, void *stream);
int apex_experts_to_device(const char *path, uint64_t stride, uint64_t slot_bytes,
                           const int32_t *experts, uint32_t n_experts, void *dst,
                           uint64_t dst_stride, uint64_t chunk_bytes, uint32_t n_buffers,
                           void *stream);

/* Device workspace (bytes) apex_moe_ffn_bf16 needs for these sizes (either path). */
size_t apex_moe_workspace_bytes(uint32_t tokens, uint32_t experts, uint32_t top_k, uint32_t hidden,
                                uint32_t inter);

/* No counterpart in the reference (for inspection and tests): byte offset, inside the
 * workspace of apex_moe_ffn_bf16 for these sizes, of the grouping plan a call leaves
 * there: int32 header[16] | cnt[E] | off[E + 1] | act[E] | pos_of_pair[P] |
 * pair_of_pos[P], P = tokens * top_k, pair p = t * top_k + j.  Pairs are grouped by
 * expert, experts ascending, each expert's tokens ascending; header[0] is the number of
 * experts with pairs.  The rest of the workspace is internal. */
size_t apex_moe_workspace_plan_offset(uint32_t tokens, uint32_t experts, uint32_t top_k,
                                      uint32_t hidden, uint32_t inter);

/* y[t] = sum_j w[t,j] * down_e(gelu_tanh(gate_e x_t) * up_e x_t), e = ids[t,j], for
 * x, y bf16 [tokens, hidden] and logits bf16 [tokens, experts].  Up to 32 tokens (and
 * 256 token-expert pairs, hidden <= 3072, inter <= 1024) run as grouped GEMVs, the
 * rest as grouped bf16-MFMA GEMMs; the
 * combine is deterministic (fixed summation order, no float atomics).  hidden and
 * inter must be multiples of 64.  `workspace` is device memory of at least
 * apex_moe_workspace_bytes(), 256-byte aligned; calls sharing one workspace must not
 * overlap. */
int apex_moe_ffn_bf16(const uint16_t *x, const uint16_t *logits, const apex_moe_slots *slots,
                      uint16_t *y, uint32_t tokens, uint32_t experts, uint32_t top_k,
                      uint32_t hidden, uint32_t inter, void *workspace, size_t workspace_bytes,
                      void *stream);

/* No counterpart in the reference: apex_moe_ffn_bf16's decode path (grouped GEMVs) for
 * callers that cannot allocate device memory -- code under HIP graph capture, tight
 * serving loops, harnesses that forbid hipMalloc.  The workspace is a fixed device
 * array of 2.25 MiB inside the library (each GPU the library runs on holds its own
 * copy until the process ends); the call allocates nothing and takes no workspace
 * argument.  Limits: tokens <= 32, tokens * top_k <= 256, experts <= 256, hidden <= 3072,
 * inter <= 1024 (larger shapes return APEX_HIP_E_INVALID).  Results are identical to
 * apex_moe_ffn_bf16 on the same shapes.  Every call on one GPU shares that GPU's array:
 * callers must serialise their calls on one stream per GPU -- calls whose kernels
 * overlap on one GPU (different streams) race.  A call made while another thread is
 * still enqueuing one on the same GPU returns APEX_HIP_E_INVALID without launching. */
int apex_moe_ffn_bf16_noalloc(const uint16_t *x, const uint16_t *logits,
                              const apex_moe_slots *slots, uint16_t *y, uint32_t tokens,
                              uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                              void *stream);

/* Path selection of apex_moe_ffn_bf16: 0 by size (default), 1 grouped GEMV, 2 grouped GEMM. */
int apex_hip_set_moe_path(int path);

/* apex_moe_ffn_bf16 routed from fp32 router logits [tokens, experts] (as
 * apex_moe_router_logits_q8 writes them), each routing weight times the bf16
 * per_expert_scale[expert] when one is given: the whole Gemma-4 MoE block after the
 * router projection.  Same workspace and limits as apex_moe_ffn_bf16. */
int apex_moe_ffn_f32logits_bf16(const uint16_t *x, const float *logits,
                                const uint16_t *per_expert_scale, const apex_moe_slots *slots,
                                uint16_t *y, uint32_t tokens, uint32_t experts, uint32_t top_k,
                                uint32_t hidden, uint32_t inter, void *workspace,
                                size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif
#endif /* APEX_HIP_H */
