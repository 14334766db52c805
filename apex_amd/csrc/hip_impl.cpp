// The one translation unit holding the HIP C-ABI glue of the APEX backend
// (the role src/metal_impl.cpp + src/backend/metal_backend.cpp play for Metal).
// Declarations and contracts: include/apex_hip.h.
#include "apex_hip.h"

#include <hip/hip_runtime.h>

#include <atomic>
#include <map>
#include <memory>
#include <mutex>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>

#include "gemm.h"
#include "gemv.h"
#include "moe.h"
#include "norm.h"
#include "file_io.h"

namespace {

thread_local std::string g_last_error;

struct ApexError : std::runtime_error {
    int code;
    ApexError(int c, const std::string &m) : std::runtime_error(m), code(c) {}
};

[[noreturn]] void fail(int code, const std::string &msg) { throw ApexError(code, msg); }

void hip_check(hipError_t e, const char *what) {
    if (e != hipSuccess)
        fail(APEX_HIP_E_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

template <class F> int guard(F &&f) {
    try {
        f();
        return APEX_HIP_OK;
    } catch (const ApexError &e) {
        g_last_error = e.what();
        return e.code;
    } catch (const std::exception &e) {
        g_last_error = e.what();
        return APEX_HIP_E_INVALID;
    }
}

// CU count of the current device, read once per process for launch sizing.
void init_device_tuning() {
    static std::atomic<bool> done{false};
    if (done.load())
        return;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess &&
        cus > 0)
        apex_hip::kNumCUs.store(cus, std::memory_order_relaxed);
    done = true;
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

void require(bool ok, const char *msg) {
    if (!ok)
        fail(APEX_HIP_E_INVALID, msg);
}

void check_nvfp4_shape(uint32_t rows, uint32_t K) {
    (void)rows;
    require(K % 16 == 0, "hidden_dim (K) must be a multiple of 16");
    require(K > 0, "hidden_dim (K) must be positive");
}

// ------------------------------------------------------------------------------------
// Direct-entry implementations (shared by the registry launchers)
// ------------------------------------------------------------------------------------

// Tokens from which the dense products (matmul, GeGLU) run as MFMA GEMMs instead of
// GEMVs, [bf16 activations, fp32 activations]; 0 = by size (use_dense_gemm).  Set by
// apex_hip_set_gemm_min_tokens; atomic because a setter may run while other threads
// dispatch.
std::atomic<uint32_t> g_gemm_min_tokens[2] = {0, 0};

// Dense-product launches of this process by form (apex_hip_dense_dispatch_counts).
enum DispatchKind { kDispGemv = 0, kDispGemm = 1, kDispSplitK = 2, kDispSplit = 3, kDispKinds };
std::atomic<uint64_t> g_dispatch[kDispKinds] = {};
void count_dispatch(DispatchKind k) { g_dispatch[k].fetch_add(1, std::memory_order_relaxed); }

// Pinned staging for file -> device streaming: 8 buffers of 8 MiB, i.e. 4 reader threads
// with a read and a copy in flight each (64 MiB pinned, kept between calls); measured
// best of 16 MiB x 4 / x 8, 8 MiB x 8 / x 16, 4 MiB x 16 and 32 MiB x 8.
constexpr uint64_t kFileChunk = 8ull << 20;
constexpr uint32_t kFileBuffers = 8;

// Scratch of the dense GEMMs (slot 0: the fp32 split, slot 1: split-K partials), one
// set per device, grown on demand and held until the process ends.  A call holds the
// device's lease while it enqueues the kernels that use the scratch; at the end it
// records an event on its stream, and the next call makes its stream wait for that
// event first (on the GPU, no host synchronisation), so uses from any streams and
// threads run one after another.  Growing synchronises the calling stream (which
// already waits for the last use), frees the old buffer and allocates the new one.
// (Stream-ordered
// hipMallocAsync / hipFreeAsync per call measured 40-330 us of host time per call
// once two sizes alternate.)
struct DeviceScratch {
    std::mutex mu;
    void *p[2] = {nullptr, nullptr};
    size_t bytes[2] = {0, 0};
    hipEvent_t done = nullptr;        // recorded after the last use
    bool used = false;
};

DeviceScratch &device_scratch(int dev) {
    static std::mutex mu;
    static std::map<int, std::unique_ptr<DeviceScratch>> all;
    std::lock_guard<std::mutex> lock(mu);
    auto &e = all[dev];
    if (!e)
        e = std::make_unique<DeviceScratch>();
    return *e;
}

class ScratchLease {
  public:
    // The device's scratch is locked, and the stream made to wait for its last use,
    // only when a call takes scratch (the first get()): calls that need none, such as
    // a bf16 GEMM without split-K, are not ordered behind other streams' GEMMs.
    explicit ScratchLease(hipStream_t stream) : s_(stream) {}
    void *get(int slot, size_t bytes) {
        acquire();
        if (d_->bytes[slot] < bytes) {
            if (d_->p[slot]) {
                hip_check(hipStreamSynchronize(s_), "GEMM scratch resize: stream sync");
                hip_check(hipFree(d_->p[slot]), "GEMM scratch resize: free");
                d_->p[slot] = nullptr;
                d_->bytes[slot] = 0;
            }
            const size_t want = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
            hip_check(hipMalloc(&d_->p[slot], want), "GEMM scratch allocation");
            d_->bytes[slot] = want;
        }
        return d_->p[slot];
    }
    ~ScratchLease() {
        if (d_ && hipEventRecord(d_->done, s_) == hipSuccess)
            d_->used = true;
    }

  private:
    void acquire() {
        if (d_)
            return;
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        DeviceScratch *d = &device_scratch(dev);
        lock_ = std::unique_lock<std::mutex>(d->mu);
        if (!d->done)
            hip_check(hipEventCreateWithFlags(&d->done, hipEventDisableTiming),
                      "GEMM scratch event");
        // always, also when the last use was on this stream's handle: a destroyed
        // stream's handle value can come back for a new stream
        if (d->used)
            hip_check(hipStreamWaitEvent(s_, d->done, 0), "GEMM scratch: wait for last use");
        d_ = d;
    }
    hipStream_t s_;
    DeviceScratch *d_ = nullptr; // set once the lease holds the device's scratch
    std::unique_lock<std::mutex> lock_;
};

// The MFMA GEMM for matmul (geglu false: W = c0/s0) or GeGLU (gate c0/s0, up c1/s1):
// bf16 x directly; fp32 x (optionally RMS-normalised by norm_w first) through its
// bf16 hi / lo split, held in the device's GEMM scratch.  Grids of few tiles run
// split-K (fp32 partials, likewise in that scratch).
void dense_gemm(const void *x, bool bf16, const uint16_t *norm_w, float eps, bool geglu,
                const uint32_t *c0, const uint8_t *s0, float ts0, const uint32_t *c1,
                const uint8_t *s1, float ts1, void *out, uint32_t M, uint32_t N, uint32_t K,
                hipStream_t stream) {
    apex_hip::GemmArgs g{};
    g.codes[0] = c0;
    g.scales[0] = s0;
    g.codes[1] = geglu ? c1 : c0;
    g.scales[1] = geglu ? s1 : s0;
    g.tensor_scale[0] = ts0;
    g.tensor_scale[1] = ts1;
    g.C = out;
    g.M = M;
    g.N = N;
    g.K = K;
    g.ldc = N;
    g.geglu = geglu;
    g.out_f32 = !bf16;
    ScratchLease scratch(stream);
    if (bf16) {
        g.A = static_cast<const uint16_t *>(x);
        g.a_k = K;
    } else {
        auto *split =
            static_cast<uint16_t *>(scratch.get(0, apex_hip::gemm_split_bytes(M, K)));
        hip_check(apex_hip::gemm_split_launch(static_cast<const float *>(x), norm_w, eps, split,
                                              M, K, stream),
                  "fp32 GEMM split launch");
        count_dispatch(kDispSplit);
        g.A = split;
        g.a_k = 2 * K;
    }
    const uint32_t splits = apex_hip::gemm_splitk_splits(g);
    if (splits > 1) {
        auto *part = static_cast<float *>(scratch.get(1, apex_hip::gemm_splitk_bytes(g, splits)));
        hip_check(apex_hip::gemm_splitk_launch(g, splits, part, stream),
                  "gemm_nvfp4 split-K launch");
        count_dispatch(kDispSplitK);
        return;
    }
    hip_check(apex_hip::gemm_launch(g, stream), "gemm_nvfp4 launch");
    count_dispatch(kDispGemm);
}

void gemm_impl(const uint16_t *A, const uint32_t *codes, const uint8_t *scales, float ts,
               uint16_t *C, uint32_t M, uint32_t N, uint32_t K, hipStream_t stream) {
    check_nvfp4_shape(N, K);
    if (M == 0 || N == 0)
        return;
    require(A && codes && scales && C, "null pointer");
    require(apex_hip::gemm_supported(M, N, K, K, false),
            "gemm: K must be a multiple of 64 and operands below 2 GiB");
    init_device_tuning();
    dense_gemm(A, true, nullptr, 0.0f, false, codes, scales, ts, nullptr, nullptr, 1.0f, C, M, N, K,
               stream);
}

// Whether a dense product of `tokens` rows runs as an MFMA GEMM.  The GEMV streams W
// once per block of up to 8 tokens; the GEMM's cost is set by its tiles (grids of few
// tiles run split-K).  Measured crossovers (gfx950, split-K in place): GeGLU from 16
// tokens (2112 x 2816 bf16: 21.5 vs 22.4 us at 16, 39.6 vs 23.4 at 32); matmul from 16
// with at least 64 tiles (21504 x 5376: 106 vs 75 us) and from 32 with fewer
// (2112 x 2816: 14.1 vs 21.7 us at 16, 24.5 vs 21.8 at 32).
bool use_dense_gemm(uint32_t tokens, uint32_t rows, uint32_t K, bool bf16, bool geglu) {
    if (!apex_hip::gemm_supported(tokens, rows, K, bf16 ? K : 2 * K, !bf16))
        return false;
    if (const uint32_t fixed = g_gemm_min_tokens[bf16 ? 0 : 1].load(std::memory_order_relaxed))
        return tokens >= fixed;
    if (geglu)
        return tokens >= 16;
    const uint64_t tiles = (uint64_t)((tokens + 255) / 256) * ((rows + 255) / 256);
    return tokens >= (tiles >= 64 ? 16u : 32u);
}

void matmul_impl(const void *x, bool bf16, const uint32_t *codes, const uint8_t *scales,
                 float ts, void *out, uint32_t tokens, uint32_t rows, uint32_t K,
                 hipStream_t stream) {
    check_nvfp4_shape(rows, K);
    if (tokens == 0 || rows == 0)
        return;
    require(x && codes && scales && out, "null pointer");
    init_device_tuning();
    if (use_dense_gemm(tokens, rows, K, bf16, false)) {
        dense_gemm(x, bf16, nullptr, 0.0f, false, codes, scales, ts, nullptr, nullptr, 1.0f, out,
                   tokens, rows, K, stream);
        return;
    }
    apex_hip::GemvArgs a{};
    a.x = x;
    a.codes[0] = a.codes[1] = codes;
    a.scales[0] = a.scales[1] = scales;
    a.tensor_scale[0] = a.tensor_scale[1] = ts;
    a.out = out;
    a.rows = rows;
    a.K = K;
    a.tokens = tokens;
    a.out_stride = rows;
    hip_check(apex_hip::gemv_launch(a, bf16 ? apex_hip::GemvMode::PlainBF16
                                            : apex_hip::GemvMode::PlainF32,
                                    bf16, stream),
              "matmul_nvfp4 launch");
    count_dispatch(kDispGemv);
}

// norm_w (fp32 x only): RMS-normalise each x row first (x * inv * norm_w, eps norm_eps).
void geglu_impl(const void *x, bool bf16, const uint32_t *gc, const uint8_t *gs, float gts,
                const uint32_t *uc, const uint8_t *us, float uts, void *out, uint32_t tokens,
                uint32_t rows, uint32_t K, hipStream_t stream, const uint16_t *norm_w = nullptr,
                float norm_eps = 0.0f) {
    check_nvfp4_shape(rows, K);
    if (tokens == 0 || rows == 0)
        return;
    require(x && gc && gs && uc && us && out, "null pointer");
    require(!(norm_w && bf16), "geglu with RMSNorm: fp32 x only");
    init_device_tuning();
    if (use_dense_gemm(tokens, rows, K, bf16, true)) {
        dense_gemm(x, bf16, norm_w, norm_eps, true, gc, gs, gts, uc, us, uts, out, tokens, rows,
                   K, stream);
        return;
    }
    if (norm_w)
        require(K % 32 == 0 && K <= 8192 && (uintptr_t)x % 16 == 0 &&
                    (uintptr_t)gc % 16 == 0 && (uintptr_t)uc % 16 == 0 &&
                    (uintptr_t)gs % 2 == 0 && (uintptr_t)us % 2 == 0,
                "geglu with RMSNorm: fp32 x, K a multiple of 32 up to 8192, x and codes "
                "16-byte aligned, scales 2-byte aligned");
    apex_hip::GemvArgs a{};
    a.norm_w = norm_w;
    a.norm_eps = norm_eps;
    a.x = x;
    a.codes[0] = gc;
    a.codes[1] = uc;
    a.scales[0] = gs;
    a.scales[1] = us;
    a.tensor_scale[0] = gts;
    a.tensor_scale[1] = uts;
    a.out = out;
    a.rows = rows;
    a.K = K;
    a.tokens = tokens;
    a.out_stride = rows;
    hip_check(apex_hip::gemv_launch(a, bf16 ? apex_hip::GemvMode::GegluBF16
                                            : apex_hip::GemvMode::GegluF32,
                                    bf16, stream),
              "geglu_nvfp4 launch");
    count_dispatch(kDispGemv);
}

bool moe_use_gemm(uint32_t T, uint32_t k, uint32_t H, uint32_t I) {
    const int path = apex_hip::kMoePath.load(std::memory_order_relaxed);
    if (path == 1)
        return false;
    if (path == 2)
        return true;
    return !(T <= apex_hip::kMoeGemvMaxTokens && (uint64_t)T * k <= apex_hip::kMoeGemvMaxPairs &&
             H <= 3072 && I <= 1024);
}

// Router logits arrive as bf16 (`logits`) or fp32 (`logits_f32`, with an optional
// bf16 per-expert scale on the routing weights); exactly one is given.  `ws` null: the
// decode path on the library's fixed workspace (no allocation; decode shapes only).
void moe_impl(const uint16_t *x, const uint16_t *logits, const float *logits_f32,
              const uint16_t *pes, const apex_moe_slots *slots, uint16_t *y, uint32_t T,
              uint32_t E, uint32_t k, uint32_t H, uint32_t I, void *ws, size_t ws_bytes,
              hipStream_t stream) {
    require(slots != nullptr, "moe_ffn: slots is null");
    if (T == 0)
        return;
    const bool fixed_ws = ws == nullptr;
    require(x && (logits || logits_f32) && slots->base && y, "moe_ffn: null pointer");
    init_device_tuning();
    const bool gemm = !fixed_ws && moe_use_gemm(T, k, H, I);
    apex_hip::MoeArgs a{};
    a.x = x;
    a.logits = logits;
    a.logits_f32 = logits_f32;
    a.pes = pes;
    a.slots = {static_cast<const uint8_t *>(slots->base), slots->stride, slots->gate_w,
               slots->gate_s, slots->up_w, slots->up_s, slots->down_w, slots->down_s};
    a.y = y;
    a.T = T, a.E = E, a.k = k, a.H = H, a.I = I;
    const char *why = nullptr;
    if (!apex_hip::moe_supported(a, gemm, &why))
        fail(APEX_HIP_E_INVALID, std::string(fixed_ws ? "moe_ffn (no-allocation form): "
                                                       : "moe_ffn: ") + why);
    const apex_hip::MoeWorkspace w = apex_hip::moe_workspace(T, E, k, H, I, gemm);
    if (fixed_ws) {
        hip_check(apex_hip::moe_static_workspace(&ws), "moe_ffn: fixed workspace address");
        ws_bytes = apex_hip::kMoeStaticWorkspaceBytes;
    }
    require((uintptr_t)ws % 256 == 0, "moe_ffn: workspace must be 256-byte aligned");
    if (ws_bytes < w.total)
        fail(APEX_HIP_E_INVALID, "moe_ffn: workspace too small (need " + std::to_string(w.total) +
                                     " bytes, have " + std::to_string(ws_bytes) + ")");
    uint8_t *base = static_cast<uint8_t *>(ws);
    a.ids = reinterpret_cast<int32_t *>(base + w.ids);
    a.w = reinterpret_cast<float *>(base + w.w);
    a.plan = reinterpret_cast<int32_t *>(base + w.plan);
    a.h = reinterpret_cast<uint16_t *>(base + w.h);
    a.d = reinterpret_cast<uint16_t *>(base + w.d);
    a.hist = gemm ? reinterpret_cast<int32_t *>(base + w.hist) : nullptr;
    a.rank = gemm ? reinterpret_cast<int32_t *>(base + w.rank) : nullptr;
    a.max_tiles = w.max_tiles;
    hip_check(apex_hip::moe_ffn_launch(a, gemm, stream), "moe_ffn launch");
}

void moe_route_impl(const uint16_t *logits, uint32_t T, uint32_t E, uint32_t k, int32_t *ids,
                    float *w, hipStream_t stream) {
    if (T == 0)
        return;
    require(logits && ids && w, "moe_route: null pointer");
    require(E >= 1 && E <= apex_hip::kMoeMaxExperts, "moe_route: experts must be in [1, 256]");
    require(k >= 1 && k <= apex_hip::kMoeMaxTopK && k <= E,
            "moe_route: top_k must be in [1, min(16, experts)]");
    hip_check(apex_hip::moe_route_launch(logits, T, E, k, ids, w, stream), "moe_route launch");
}

void route_f32_impl(const float *logits, const uint16_t *pes, uint32_t T, uint32_t E, uint32_t k,
                    int32_t *ids, float *w, hipStream_t stream) {
    if (T == 0)
        return;
    require(logits && ids && w, "moe_route: null pointer");
    require(E >= 1 && E <= apex_hip::kMoeMaxExperts, "moe_route: experts must be in [1, 256]");
    require(k >= 1 && k <= apex_hip::kMoeMaxTopK && k <= E,
            "moe_route: top_k must be in [1, min(16, experts)]");
    hip_check(apex_hip::moe_route_f32_launch(logits, pes, T, E, k, ids, w, stream),
              "moe_route launch");
}

void router_impl(const apex_hip::MoeRouterArgs &a, hipStream_t stream) {
    if (a.T == 0)
        return;
    require(a.h && a.norm_w && a.qw && a.qs && a.qb && a.logits, "moe_router: null pointer");
    const char *why = nullptr;
    if (!apex_hip::moe_router_supported(a, &why))
        fail(APEX_HIP_E_INVALID, std::string("moe_router: ") + why);
    init_device_tuning();
    if (a.T >= apex_hip::kRouterMfmaMinTokens && apex_hip::moe_router_fused_fits(a)) {
        // prefill: the fused MFMA form (bf16 hi + lo of the scaled rows made on the fly)
        hip_check(apex_hip::moe_router_fused_launch(a, stream), "moe_router MFMA launch");
        return;
    }
    hip_check(apex_hip::moe_router_logits_launch(a, stream), "moe_router launch");
}

} // namespace

// ------------------------------------------------------------------------------------
// Backend object
// ------------------------------------------------------------------------------------

struct apex_hip_buffer {
    void *dev = nullptr;
    void *host = nullptr;     // pinned mirror (owned) or the wrapped pointer
    size_t length = 0;
    std::string category;
    bool wrapped = false;
    bool host_valid = false;  // host bytes are current
    bool dev_valid = true;    // device bytes are current
};

struct apex_hip_backend {
    int device = 0;
    hipStream_t stream = nullptr;
    std::string name;
};

namespace {

void ensure_device_current(apex_hip_backend *b, apex_hip_buffer *buf) {
    if (buf->dev_valid)
        return;
    hip_check(hipMemcpyAsync(buf->dev, buf->host, buf->length, hipMemcpyHostToDevice, b->stream),
              "upload");
    if (buf->wrapped) // pageable source: make sure the copy has consumed it
        hip_check(hipStreamSynchronize(b->stream), "upload sync");
    buf->dev_valid = true;
}

// ---- registry ---------------------------------------------------------------------

constexpr int kMaxArgs = 24;

struct LaunchCtx {
    void *ptr[kMaxArgs];
    size_t avail[kMaxArgs]; // bytes from the offset to the end of the buffer
    uint32_t u[kMaxArgs];
    float f[kMaxArgs];
    apex_hip_dim3 grid, block;
    hipStream_t stream;
};

using Launcher = void (*)(const LaunchCtx &);

struct KernelSpec {
    const char *name;
    const char *sig;     // one letter per argument: B buffer, U uint32, F float
    uint32_t out_mask;   // bit i set: argument i is written by the kernel
    Launcher launch;
};

void need(const LaunchCtx &c, int i, uint64_t bytes, const char *what) {
    if (bytes > c.avail[i])
        fail(APEX_HIP_E_INVALID, std::string(what) + ": buffer too small (need " +
                                     std::to_string(bytes) + " bytes, have " +
                                     std::to_string(c.avail[i]) + ")");
}

// matmul_nvfp4: reference argument order of src/ops.h:40-45.
void launch_matmul_nvfp4(const LaunchCtx &c) {
    const uint32_t K = c.u[4], w_rows = c.u[5], tokens = c.grid.y;
    const uint64_t simd_per_group = ((uint64_t)c.block.x * c.block.y * c.block.z) / 32;
    const uint64_t covered = (uint64_t)c.grid.x * simd_per_group;
    const uint32_t rows = (uint32_t)(covered < w_rows ? covered : w_rows);
    check_nvfp4_shape(rows, K);
    need(c, 0, (uint64_t)tokens * K * 4, "matmul_nvfp4 input");
    need(c, 1, (uint64_t)rows * K / 2, "matmul_nvfp4 weights");
    need(c, 2, (uint64_t)rows * K / 16, "matmul_nvfp4 scales");
    if (tokens > 0 && rows > 0)
        need(c, 3, (uint64_t)(tokens - 1) * w_rows * 4 + (uint64_t)rows * 4, "matmul_nvfp4 output");
    if (tokens == 0 || rows == 0)
        return;
    if (rows == w_rows) {
        // The launch of src/ops.h:36-45 (ceil(w_rows / 8) groups of 256 threads) covers
        // every row, so the output is a contiguous [T, w_rows]: the product of
        // apex_nvfp4_matmul_f32, an MFMA GEMM at prefill token counts (fp32 x through
        // its bf16 hi + lo split) and a GEMV below them.
        matmul_impl(c.ptr[0], false, (const uint32_t *)c.ptr[1], (const uint8_t *)c.ptr[2], 1.0f,
                    c.ptr[3], tokens, rows, K, c.stream);
        return;
    }
    // A grid covering fewer rows than w_rows: those rows only, output rows strided by
    // w_rows (shaders/matmul.metal:14-18 writes output[token * w_rows + row]).
    init_device_tuning();
    apex_hip::GemvArgs a{};
    a.x = c.ptr[0];
    a.codes[0] = a.codes[1] = (const uint32_t *)c.ptr[1];
    a.scales[0] = a.scales[1] = (const uint8_t *)c.ptr[2];
    a.tensor_scale[0] = a.tensor_scale[1] = 1.0f;
    a.out = c.ptr[3];
    a.rows = rows;
    a.K = K;
    a.tokens = tokens;
    a.out_stride = w_rows;
    hip_check(apex_hip::gemv_launch(a, apex_hip::GemvMode::PlainF32, false, c.stream),
              "matmul_nvfp4 launch");
    count_dispatch(kDispGemv);
}

void rms_norm_impl(const float *x, const uint16_t *w, float *y, uint32_t rows, uint32_t n,
                   float eps, hipStream_t stream) {
    if (rows == 0 || n == 0)
        return;
    require(x && w && y, "null pointer");
    hip_check(apex_hip::rms_norm_launch({x, w, y, rows, n, eps}, stream), "rms_norm_f32 launch");
}

void head_norm_rope_impl(const apex_hip::HeadNormRopeArgs &a, hipStream_t stream) {
    if (a.tokens == 0 || a.heads == 0)
        return;
    require(a.x && a.y && (a.w || !a.has_weight), "null pointer");
    require(a.head_dim > 0 && a.head_dim % 2 == 0 && a.head_dim <= apex_hip::kHeadNormMaxDim,
            "head_norm_rope: head_dim must be even and at most 512");
    require(a.rope_pairs <= a.head_dim / 2, "head_norm_rope: rope_pairs exceeds head_dim / 2");
    hip_check(apex_hip::head_norm_rope_launch(a, stream), "head_norm_rope_f32 launch");
}

// rms_norm_f32: src/ops.h:18-26 (rows = threadgroups.x), shaders/norm.metal:33-44.
void launch_rms_norm(const LaunchCtx &c) {
    const uint32_t rows = c.grid.x, n = c.u[3];
    need(c, 0, (uint64_t)rows * n * 4, "rms_norm_f32 input");
    need(c, 1, (uint64_t)n * 2, "rms_norm_f32 weights");
    need(c, 2, (uint64_t)rows * n * 4, "rms_norm_f32 result");
    rms_norm_impl((const float *)c.ptr[0], (const uint16_t *)c.ptr[1], (float *)c.ptr[2], rows, n,
                  c.f[4], c.stream);
}

// head_norm_rope_f32: src/ops.h:88-118 (tokens = threadgroups.x, heads = threadgroups.y,
// which the reference's launcher sets to the heads argument), shaders/head_norm_rope.metal.
void launch_head_norm_rope(const LaunchCtx &c) {
    apex_hip::HeadNormRopeArgs a{};
    a.x = (const float *)c.ptr[0];
    a.w = (const uint16_t *)c.ptr[1];
    a.y = (float *)c.ptr[2];
    a.tokens = c.grid.x;
    a.heads = c.u[3];
    a.head_dim = c.u[4];
    a.has_weight = c.u[5] != 0;
    a.rope_pairs = c.u[6];
    a.rope_base = c.f[7];
    a.abs_pos = c.u[8];
    a.out_token_stride = c.u[9];
    a.out_head_stride = c.u[10];
    a.eps = c.f[11];
    if (c.grid.y != a.heads)
        fail(APEX_HIP_E_INVALID, "head_norm_rope_f32: threadgroups.y must equal heads");
    if (a.heads == 0)
        return;
    need(c, 0, (uint64_t)a.tokens * a.heads * a.head_dim * 4, "head_norm_rope_f32 input");
    if (a.has_weight)
        need(c, 1, (uint64_t)a.head_dim * 2, "head_norm_rope_f32 weights");
    need(c, 2, ((uint64_t)(a.tokens - 1) * a.out_token_stride +
                (uint64_t)(a.heads - 1) * a.out_head_stride + a.head_dim) * 4,
         "head_norm_rope_f32 output");
    head_norm_rope_impl(a, c.stream);
}

// geglu_f32: src/ops.h:53-54.
void launch_geglu_f32(const LaunchCtx &c) {
    const uint64_t threads = (uint64_t)c.grid.x * c.grid.y * c.grid.z *
                             ((uint64_t)c.block.x * c.block.y * c.block.z);
    const uint32_t count = (uint32_t)(threads < c.u[3] ? threads : c.u[3]);
    need(c, 0, (uint64_t)count * 4, "geglu_f32 gate");
    need(c, 1, (uint64_t)count * 4, "geglu_f32 up");
    need(c, 2, (uint64_t)count * 4, "geglu_f32 output");
    hip_check(apex_hip::geglu_f32_launch((const float *)c.ptr[0], (const float *)c.ptr[1],
                                         (float *)c.ptr[2], count, c.stream),
              "geglu_f32 launch");
}

void launch_matmul_nvfp4_bf16(const LaunchCtx &c) {
    const uint32_t K = c.u[4], rows = c.u[5], tokens = c.u[6];
    check_nvfp4_shape(rows, K);
    need(c, 0, (uint64_t)tokens * K * 2, "matmul_nvfp4_bf16 input");
    need(c, 1, (uint64_t)rows * K / 2, "matmul_nvfp4_bf16 weights");
    need(c, 2, (uint64_t)rows * K / 16, "matmul_nvfp4_bf16 scales");
    need(c, 3, (uint64_t)tokens * rows * 2, "matmul_nvfp4_bf16 output");
    matmul_impl(c.ptr[0], true, (const uint32_t *)c.ptr[1], (const uint8_t *)c.ptr[2], c.f[7],
                c.ptr[3], tokens, rows, K, c.stream);
}

template <bool BF16> void launch_geglu_nvfp4(const LaunchCtx &c) {
    const uint32_t K = c.u[6], rows = c.u[7], tokens = c.u[8];
    const uint64_t es = BF16 ? 2 : 4;
    check_nvfp4_shape(rows, K);
    need(c, 0, (uint64_t)tokens * K * es, "geglu_nvfp4 input");
    need(c, 1, (uint64_t)rows * K / 2, "geglu_nvfp4 gate weights");
    need(c, 2, (uint64_t)rows * K / 16, "geglu_nvfp4 gate scales");
    need(c, 3, (uint64_t)rows * K / 2, "geglu_nvfp4 up weights");
    need(c, 4, (uint64_t)rows * K / 16, "geglu_nvfp4 up scales");
    need(c, 5, (uint64_t)tokens * rows * es, "geglu_nvfp4 output");
    geglu_impl(c.ptr[0], BF16, (const uint32_t *)c.ptr[1], (const uint8_t *)c.ptr[2], c.f[9],
               (const uint32_t *)c.ptr[3], (const uint8_t *)c.ptr[4], c.f[10], c.ptr[5], tokens,
               rows, K, c.stream);
}

// geglu_nvfp4_rms_norm_f32: x, norm_w, gate codes / scales, up codes / scales, out, K,
// rows, tokens, gate / up tensor scales, eps.
void launch_geglu_nvfp4_rms_norm(const LaunchCtx &c) {
    const uint32_t K = c.u[7], rows = c.u[8], tokens = c.u[9];
    check_nvfp4_shape(rows, K);
    need(c, 0, (uint64_t)tokens * K * 4, "geglu_nvfp4_rms_norm input");
    need(c, 1, (uint64_t)K * 2, "geglu_nvfp4_rms_norm norm weights");
    need(c, 2, (uint64_t)rows * K / 2, "geglu_nvfp4_rms_norm gate weights");
    need(c, 3, (uint64_t)rows * K / 16, "geglu_nvfp4_rms_norm gate scales");
    need(c, 4, (uint64_t)rows * K / 2, "geglu_nvfp4_rms_norm up weights");
    need(c, 5, (uint64_t)rows * K / 16, "geglu_nvfp4_rms_norm up scales");
    need(c, 6, (uint64_t)tokens * rows * 4, "geglu_nvfp4_rms_norm output");
    geglu_impl(c.ptr[0], false, (const uint32_t *)c.ptr[2], (const uint8_t *)c.ptr[3], c.f[10],
               (const uint32_t *)c.ptr[4], (const uint8_t *)c.ptr[5], c.f[11], c.ptr[6], tokens,
               rows, K, c.stream, (const uint16_t *)c.ptr[1], c.f[12]);
}

void launch_gemm_nvfp4_bf16(const LaunchCtx &c) {
    const uint32_t M = c.u[4], N = c.u[5], K = c.u[6];
    check_nvfp4_shape(N, K);
    need(c, 0, (uint64_t)M * K * 2, "gemm_nvfp4_bf16 A");
    need(c, 1, (uint64_t)N * K / 2, "gemm_nvfp4_bf16 weights");
    need(c, 2, (uint64_t)N * K / 16, "gemm_nvfp4_bf16 scales");
    need(c, 3, (uint64_t)M * N * 2, "gemm_nvfp4_bf16 output");
    gemm_impl((const uint16_t *)c.ptr[0], (const uint32_t *)c.ptr[1], (const uint8_t *)c.ptr[2],
              c.f[7], (uint16_t *)c.ptr[3], M, N, K, c.stream);
}

template <bool BF16> void launch_dequant(const LaunchCtx &c) {
    const uint32_t K = c.u[3], rows = c.u[4];
    check_nvfp4_shape(rows, K);
    need(c, 0, (uint64_t)rows * K / 2, "dequant weights");
    need(c, 1, (uint64_t)rows * K / 16, "dequant scales");
    need(c, 2, (uint64_t)rows * K * (BF16 ? 2 : 4), "dequant output");
    hip_check(apex_hip::dequant_launch((const uint32_t *)c.ptr[0], (const uint8_t *)c.ptr[1],
                                       c.ptr[2], rows, K, c.f[5], BF16, c.stream),
              "dequant launch");
}

// moe_ffn_nvfp4_bf16: x, logits, expert slots, y, workspace; T, E, k, H, I; slot stride
// and the six piece offsets.
void launch_moe_ffn(const LaunchCtx &c) {
    const uint32_t T = c.u[5], E = c.u[6], k = c.u[7], H = c.u[8], I = c.u[9];
    apex_moe_slots s{c.ptr[2], c.u[10], c.u[11], c.u[12], c.u[13], c.u[14], c.u[15], c.u[16]};
    need(c, 0, (uint64_t)T * H * 2, "moe_ffn x");
    need(c, 1, (uint64_t)T * E * 2, "moe_ffn logits");
    need(c, 2, (uint64_t)E * s.stride, "moe_ffn expert slots");
    need(c, 3, (uint64_t)T * H * 2, "moe_ffn output");
    moe_impl((const uint16_t *)c.ptr[0], (const uint16_t *)c.ptr[1], nullptr, nullptr, &s,
             (uint16_t *)c.ptr[3], T, E, k, H, I, c.ptr[4], c.avail[4], c.stream);
}

// moe_ffn_f32logits_nvfp4_bf16: x, fp32 logits, per-expert scale, expert slots, y,
// workspace; T, E, k, H, I; slot stride and the six piece offsets; has_scale.
void launch_moe_ffn_f32logits(const LaunchCtx &c) {
    const uint32_t T = c.u[6], E = c.u[7], k = c.u[8], H = c.u[9], I = c.u[10];
    const bool has_pes = c.u[18] != 0;
    apex_moe_slots s{c.ptr[3], c.u[11], c.u[12], c.u[13], c.u[14], c.u[15], c.u[16], c.u[17]};
    need(c, 0, (uint64_t)T * H * 2, "moe_ffn x");
    need(c, 1, (uint64_t)T * E * 4, "moe_ffn logits");
    if (has_pes)
        need(c, 2, (uint64_t)E * 2, "moe_ffn per-expert scale");
    need(c, 3, (uint64_t)E * s.stride, "moe_ffn expert slots");
    need(c, 4, (uint64_t)T * H * 2, "moe_ffn output");
    moe_impl((const uint16_t *)c.ptr[0], nullptr, (const float *)c.ptr[1],
             has_pes ? (const uint16_t *)c.ptr[2] : nullptr, &s, (uint16_t *)c.ptr[4], T, E, k, H, I,
             c.ptr[5], c.avail[5], c.stream);
}

// moe_router_logits_q8_f32: h, router.scale, proj weights, scales, biases, logits; T, E,
// H, eps (docs/B6_3_attention.md:721-725).
void launch_moe_router(const LaunchCtx &c) {
    const uint32_t T = c.u[6], E = c.u[7], H = c.u[8];
    need(c, 0, (uint64_t)T * H * 4, "moe_router hidden");
    need(c, 1, (uint64_t)H * 2, "moe_router norm weights");
    need(c, 2, (uint64_t)E * H, "moe_router weights");
    need(c, 3, (uint64_t)E * (H / 64) * 2, "moe_router scales");
    need(c, 4, (uint64_t)E * (H / 64) * 2, "moe_router biases");
    need(c, 5, (uint64_t)T * E * 4, "moe_router logits");
    router_impl({(const float *)c.ptr[0], (const uint16_t *)c.ptr[1], c.f[9],
                 (const uint32_t *)c.ptr[2], (const uint16_t *)c.ptr[3],
                 (const uint16_t *)c.ptr[4], T, E, H, (float *)c.ptr[5]},
                c.stream);
}

// moe_route_f32: fp32 logits, per-expert scale, ids, weights; T, E, k, has_scale.
void launch_moe_route_f32(const LaunchCtx &c) {
    const uint32_t T = c.u[4], E = c.u[5], k = c.u[6];
    const bool has_pes = c.u[7] != 0;
    need(c, 0, (uint64_t)T * E * 4, "moe_route logits");
    if (has_pes)
        need(c, 1, (uint64_t)E * 2, "moe_route per-expert scale");
    need(c, 2, (uint64_t)T * k * 4, "moe_route ids");
    need(c, 3, (uint64_t)T * k * 4, "moe_route weights");
    route_f32_impl((const float *)c.ptr[0], has_pes ? (const uint16_t *)c.ptr[1] : nullptr, T, E, k,
                   (int32_t *)c.ptr[2], (float *)c.ptr[3], c.stream);
}

void launch_moe_route(const LaunchCtx &c) {
    const uint32_t T = c.u[3], E = c.u[4], k = c.u[5];
    need(c, 0, (uint64_t)T * E * 2, "moe_route logits");
    need(c, 1, (uint64_t)T * k * 4, "moe_route ids");
    need(c, 2, (uint64_t)T * k * 4, "moe_route weights");
    moe_route_impl((const uint16_t *)c.ptr[0], T, E, k, (int32_t *)c.ptr[1], (float *)c.ptr[2],
                   c.stream);
}

const KernelSpec kKernels[] = {
    {"matmul_nvfp4", "BBBBUU", 1u << 3, launch_matmul_nvfp4},
    {"geglu_f32", "BBBU", 1u << 2, launch_geglu_f32},
    {"matmul_nvfp4_bf16", "BBBBUUUF", 1u << 3, launch_matmul_nvfp4_bf16},
    {"geglu_nvfp4_f32", "BBBBBBUUUFF", 1u << 5, launch_geglu_nvfp4<false>},
    {"geglu_nvfp4_bf16", "BBBBBBUUUFF", 1u << 5, launch_geglu_nvfp4<true>},
    {"geglu_nvfp4_rms_norm_f32", "BBBBBBBUUUFFF", 1u << 6, launch_geglu_nvfp4_rms_norm},
    {"gemm_nvfp4_bf16", "BBBBUUUF", 1u << 3, launch_gemm_nvfp4_bf16},
    {"dequant_nvfp4_f32", "BBBUUF", 1u << 2, launch_dequant<false>},
    {"dequant_nvfp4_bf16", "BBBUUF", 1u << 2, launch_dequant<true>},
    {"moe_ffn_nvfp4_bf16", "BBBBBUUUUUUUUUUUU", (1u << 3) | (1u << 4), launch_moe_ffn},
    {"moe_route_bf16", "BBBUUU", (1u << 1) | (1u << 2), launch_moe_route},
    {"rms_norm_f32", "BBBUF", 1u << 2, launch_rms_norm},
    {"head_norm_rope_f32", "BBBUUUUFUUUF", 1u << 2, launch_head_norm_rope},
    {"moe_router_logits_q8_f32", "BBBBBBUUUF", 1u << 5, launch_moe_router},
    {"moe_route_f32", "BBBBUUUU", (1u << 2) | (1u << 3), launch_moe_route_f32},
    {"moe_ffn_f32logits_nvfp4_bf16", "BBBBBBUUUUUUUUUUUUU", (1u << 4) | (1u << 5),
     launch_moe_ffn_f32logits},
};
constexpr int kNumKernels = sizeof(kKernels) / sizeof(kKernels[0]);

const KernelSpec *find_kernel(const char *name) {
    if (!name)
        fail(APEX_HIP_E_UNKNOWN_KERNEL, "kernel name is null");
    for (const KernelSpec &k : kKernels)
        if (std::strcmp(k.name, name) == 0)
            return &k;
    fail(APEX_HIP_E_UNKNOWN_KERNEL, std::string("cannot find kernel: ") + name);
}

// Maximum threads per threadgroup accepted, as MTL::ComputePipelineState's
// maxTotalThreadsPerThreadgroup bounds the reference (metal_backend.cpp:169-171).
constexpr uint64_t kMaxThreadsPerGroup = 1024;

const KernelSpec *validate(const char *kernel, const apex_hip_arg *args, size_t nargs,
                           apex_hip_dim3 grid, apex_hip_dim3 block) {
    const KernelSpec *k = find_kernel(kernel);
    const size_t want = std::strlen(k->sig);
    if (nargs != want)
        fail(APEX_HIP_E_ARGS, std::string(kernel) + ": expected " + std::to_string(want) +
                                  " arguments (" + k->sig + "), got " + std::to_string(nargs));
    if (nargs && !args)
        fail(APEX_HIP_E_ARGS, std::string(kernel) + ": argument array is null");
    for (size_t i = 0; i < nargs; ++i) {
        const char kind = k->sig[i];
        const apex_hip_arg &a = args[i];
        if (kind == 'B') {
            if (!a.buffer)
                fail(APEX_HIP_E_ARGS, std::string(kernel) + ": argument " + std::to_string(i) +
                                          " must be a buffer");
        } else {
            if (a.buffer || !a.bytes || a.size != 4)
                fail(APEX_HIP_E_ARGS, std::string(kernel) + ": argument " + std::to_string(i) +
                                          " must be a 4-byte value");
        }
    }
    const uint64_t threads = (uint64_t)block.x * block.y * block.z;
    if (threads > kMaxThreadsPerGroup)
        fail(APEX_HIP_E_THREADGROUP, std::string(kernel) + ": threadgroup too large");
    if (threads == 0 || (uint64_t)grid.x * grid.y * grid.z == 0)
        fail(APEX_HIP_E_INVALID, std::string(kernel) + ": empty grid or threadgroup");
    return k;
}

} // namespace

extern "C" {

const char *apex_hip_last_error(void) { return g_last_error.c_str(); }

int apex_hip_abi_version(void) { return APEX_HIP_ABI_VERSION; }

int apex_hip_backend_create(int device, apex_hip_backend **out) {
    return guard([&] {
        require(out != nullptr, "out is null");
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
            fail(APEX_HIP_E_DEVICE, "HipBackend: no HIP device found");
        if (device < 0 || device >= n)
            fail(APEX_HIP_E_DEVICE, "HipBackend: device index out of range");
        hip_check(hipSetDevice(device), "hipSetDevice");
        auto *b = new apex_hip_backend();
        b->device = device;
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, device) == hipSuccess)
            b->name = p.gcnArchName;
        if (hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking) != hipSuccess) {
            delete b;
            fail(APEX_HIP_E_DEVICE, "HipBackend: failed to create stream");
        }
        init_device_tuning();
        *out = b;
    });
}

void apex_hip_backend_destroy(apex_hip_backend *b) {
    if (!b)
        return;
    if (b->stream) {
        (void)hipStreamSynchronize(b->stream);
        (void)hipStreamDestroy(b->stream);
    }
    delete b;
}

int apex_hip_device_name(apex_hip_backend *b, char *buf, size_t len) {
    return guard([&] {
        require(b && buf && len > 0, "null argument");
        std::snprintf(buf, len, "%s", b->name.c_str());
    });
}

int apex_hip_wrap_no_copy(apex_hip_backend *b, void *host, size_t bytes, apex_hip_buffer **out) {
    return guard([&] {
        require(b && out, "null argument");
        const size_t page = 16384;
        if (reinterpret_cast<uintptr_t>(host) % page || bytes % page || !host)
            fail(APEX_HIP_E_ALIGN, "wrapNoCopy: pointer and length must be page multiples");
        auto *buf = new apex_hip_buffer();
        if (bytes && hipMalloc(&buf->dev, bytes) != hipSuccess) {
            delete buf;
            fail(APEX_HIP_E_OOM, "wrapNoCopy: device allocation failed");
        }
        buf->host = host;
        buf->length = bytes;
        buf->wrapped = true;
        buf->host_valid = true;
        buf->dev_valid = false;
        *out = buf;
    });
}

int apex_hip_allocate(apex_hip_backend *b, size_t bytes, const char *category,
                      apex_hip_buffer **out) {
    return guard([&] {
        require(b && out, "null argument");
        auto *buf = new apex_hip_buffer();
        if (bytes) {
            if (hipMalloc(&buf->dev, bytes) != hipSuccess) {
                delete buf;
                fail(APEX_HIP_E_OOM, "allocate: device allocation failed");
            }
            if (hipMemsetAsync(buf->dev, 0, bytes, b->stream) != hipSuccess) {
                (void)hipFree(buf->dev);
                delete buf;
                fail(APEX_HIP_E_DEVICE, "allocate: zero fill failed");
            }
        }
        buf->length = bytes;
        buf->category = category ? category : "";
        buf->dev_valid = true;
        buf->host_valid = false;
        *out = buf;
    });
}

int apex_hip_contents(apex_hip_backend *b, apex_hip_buffer *buf, void **out) {
    return guard([&] {
        require(b && buf && out, "null argument");
        if (!buf->host) {
            if (buf->length && hipHostMalloc(&buf->host, buf->length, hipHostMallocDefault) != hipSuccess)
                fail(APEX_HIP_E_OOM, "contents: host mirror allocation failed");
            buf->host_valid = false;
        }
        if (!buf->host_valid) {
            hip_check(hipStreamSynchronize(b->stream), "contents: sync");
            if (buf->length)
                hip_check(hipMemcpy(buf->host, buf->dev, buf->length, hipMemcpyDeviceToHost),
                          "contents: download");
            buf->host_valid = true;
        }
        buf->dev_valid = false; // the caller may write through the pointer
        *out = buf->host;
    });
}

int apex_hip_load_file(apex_hip_backend *b, apex_hip_buffer *buf, uint64_t buffer_offset,
                       const char *path, uint64_t file_offset, uint64_t bytes) {
    return guard([&] {
        require(b && buf && path, "null argument");
        require(buffer_offset <= buf->length && bytes <= buf->length - buffer_offset,
                "load_file: range past the end of the buffer");
        if (bytes == 0)
            return;
        ensure_device_current(b, buf); // the rest of the buffer keeps what the host wrote
        const apex_hip::FileRange r{file_offset, bytes, static_cast<char *>(buf->dev) + buffer_offset};
        const apex_hip::FileCopyStatus st =
            apex_hip::copy_file_ranges(path, &r, 1, kFileChunk, kFileBuffers, b->stream);
        if (!st.error.empty())
            fail(APEX_HIP_E_INVALID, "load_file: " + st.error);
        buf->host_valid = false;
        buf->dev_valid = true;
    });
}

int apex_hip_release(apex_hip_backend *b, apex_hip_buffer *buf) {
    return guard([&] {
        if (!buf)
            return;
        if (b && b->stream)
            (void)hipStreamSynchronize(b->stream);
        if (buf->dev)
            (void)hipFree(buf->dev);
        if (buf->host && !buf->wrapped)
            (void)hipHostFree(buf->host);
        delete buf;
    });
}

int apex_hip_run(apex_hip_backend *b, const char *kernel, const apex_hip_arg *args, size_t nargs,
                 apex_hip_dim3 threadgroups, apex_hip_dim3 threads_per_group) {
    return guard([&] {
        require(b != nullptr, "backend is null");
        const KernelSpec *k = validate(kernel, args, nargs, threadgroups, threads_per_group);
        LaunchCtx c{};
        c.grid = threadgroups;
        c.block = threads_per_group;
        c.stream = b->stream;
        for (size_t i = 0; i < nargs; ++i) {
            const apex_hip_arg &a = args[i];
            if (k->sig[i] == 'B') {
                if (a.offset > a.buffer->length)
                    fail(APEX_HIP_E_INVALID, std::string(kernel) + ": offset beyond buffer end");
                ensure_device_current(b, a.buffer);
                c.ptr[i] = static_cast<char *>(a.buffer->dev) + a.offset;
                c.avail[i] = a.buffer->length - a.offset;
            } else if (k->sig[i] == 'U') {
                std::memcpy(&c.u[i], a.bytes, 4);
            } else {
                std::memcpy(&c.f[i], a.bytes, 4);
            }
        }
        k->launch(c);
        for (size_t i = 0; i < nargs; ++i)
            if (k->out_mask & (1u << i))
                args[i].buffer->host_valid = false;
    });
}

int apex_hip_sync(apex_hip_backend *b) {
    return guard([&] {
        require(b != nullptr, "backend is null");
        hip_check(hipStreamSynchronize(b->stream), "sync");
    });
}

int apex_hip_buffer_device_ptr(apex_hip_buffer *buf, void **out) {
    return guard([&] {
        require(buf && out, "null argument");
        *out = buf->dev;
    });
}

size_t apex_hip_buffer_length(apex_hip_buffer *buf) { return buf ? buf->length : 0; }

void *apex_hip_backend_stream(apex_hip_backend *b) { return b ? (void *)b->stream : nullptr; }

int apex_hip_kernel_count(void) { return kNumKernels; }

const char *apex_hip_kernel_name(int index) {
    return (index >= 0 && index < kNumKernels) ? kKernels[index].name : nullptr;
}

const char *apex_hip_kernel_signature(const char *kernel) {
    for (const KernelSpec &k : kKernels)
        if (kernel && std::strcmp(k.name, kernel) == 0)
            return k.sig;
    return nullptr;
}

int apex_hip_validate_run(const char *kernel, const apex_hip_arg *args, size_t nargs,
                          apex_hip_dim3 threadgroups, apex_hip_dim3 threads_per_group) {
    return guard([&] { validate(kernel, args, nargs, threadgroups, threads_per_group); });
}

// ---- direct entry points ----------------------------------------------------------

int apex_nvfp4_matmul_f32(const float *x, const uint32_t *codes, const uint8_t *scales,
                          float tensor_scale, float *out, uint32_t tokens, uint32_t rows,
                          uint32_t K, void *stream) {
    return guard([&] {
        matmul_impl(x, false, codes, scales, tensor_scale, out, tokens, rows, K, as_stream(stream));
    });
}

int apex_nvfp4_matmul_bf16(const uint16_t *x, const uint32_t *codes, const uint8_t *scales,
                           float tensor_scale, uint16_t *out, uint32_t tokens, uint32_t rows,
                           uint32_t K, void *stream) {
    return guard([&] {
        matmul_impl(x, true, codes, scales, tensor_scale, out, tokens, rows, K, as_stream(stream));
    });
}

int apex_nvfp4_gemm_bf16(const uint16_t *A, const uint32_t *codes, const uint8_t *scales,
                         float tensor_scale, uint16_t *C, uint32_t M, uint32_t N, uint32_t K,
                         void *stream) {
    return guard([&] { gemm_impl(A, codes, scales, tensor_scale, C, M, N, K, as_stream(stream)); });
}

int apex_nvfp4_geglu_f32(const float *x, const uint32_t *gate_codes, const uint8_t *gate_scales,
                         float gate_tensor_scale, const uint32_t *up_codes,
                         const uint8_t *up_scales, float up_tensor_scale, float *out,
                         uint32_t tokens, uint32_t rows, uint32_t K, void *stream) {
    return guard([&] {
        geglu_impl(x, false, gate_codes, gate_scales, gate_tensor_scale, up_codes, up_scales,
                   up_tensor_scale, out, tokens, rows, K, as_stream(stream));
    });
}

int apex_nvfp4_geglu_rms_norm_f32(const float *x, const uint16_t *norm_w, float eps,
                                  const uint32_t *gate_codes, const uint8_t *gate_scales,
                                  float gate_tensor_scale, const uint32_t *up_codes,
                                  const uint8_t *up_scales, float up_tensor_scale, float *out,
                                  uint32_t tokens, uint32_t rows, uint32_t K, void *stream) {
    return guard([&] {
        require(norm_w != nullptr, "geglu_rms_norm: norm_w is null");
        geglu_impl(x, false, gate_codes, gate_scales, gate_tensor_scale, up_codes, up_scales,
                   up_tensor_scale, out, tokens, rows, K, as_stream(stream), norm_w, eps);
    });
}

int apex_nvfp4_geglu_bf16(const uint16_t *x, const uint32_t *gate_codes,
                          const uint8_t *gate_scales, float gate_tensor_scale,
                          const uint32_t *up_codes, const uint8_t *up_scales,
                          float up_tensor_scale, uint16_t *out, uint32_t tokens, uint32_t rows,
                          uint32_t K, void *stream) {
    return guard([&] {
        geglu_impl(x, true, gate_codes, gate_scales, gate_tensor_scale, up_codes, up_scales,
                   up_tensor_scale, out, tokens, rows, K, as_stream(stream));
    });
}

int apex_geglu_f32(const float *gate, const float *up, float *out, uint32_t count, void *stream) {
    return guard([&] {
        if (count == 0)
            return;
        require(gate && up && out, "null pointer");
        hip_check(apex_hip::geglu_f32_launch(gate, up, out, count, as_stream(stream)),
                  "geglu_f32 launch");
    });
}

int apex_rms_norm_f32(const float *x, const uint16_t *weights, float *y, uint32_t rows,
                      uint32_t hidden_dim, float eps, void *stream) {
    return guard([&] { rms_norm_impl(x, weights, y, rows, hidden_dim, eps, as_stream(stream)); });
}

int apex_head_norm_rope_f32(const float *x, const uint16_t *weights, int has_weights, float *y,
                            uint32_t tokens, uint32_t heads, uint32_t head_dim, uint32_t rope_pairs,
                            float rope_base, uint32_t abs_pos, uint32_t out_token_stride,
                            uint32_t out_head_stride, float eps, void *stream) {
    return guard([&] {
        apex_hip::HeadNormRopeArgs a{x, weights, y, tokens, heads, head_dim,
                                     has_weights ? 1u : 0u, rope_pairs, rope_base, abs_pos,
                                     out_token_stride, out_head_stride, eps};
        head_norm_rope_impl(a, as_stream(stream));
    });
}

int apex_nvfp4_dequant_f32(const uint32_t *codes, const uint8_t *scales, float tensor_scale,
                           float *out, uint32_t rows, uint32_t K, void *stream) {
    return guard([&] {
        check_nvfp4_shape(rows, K);
        require(rows == 0 || (codes && scales && out), "null pointer");
        hip_check(apex_hip::dequant_launch(codes, scales, out, rows, K, tensor_scale, false,
                                           as_stream(stream)),
                  "dequant launch");
    });
}

int apex_nvfp4_dequant_bf16(const uint32_t *codes, const uint8_t *scales, float tensor_scale,
                            uint16_t *out, uint32_t rows, uint32_t K, void *stream) {
    return guard([&] {
        check_nvfp4_shape(rows, K);
        require(rows == 0 || (codes && scales && out), "null pointer");
        hip_check(apex_hip::dequant_launch(codes, scales, out, rows, K, tensor_scale, true,
                                           as_stream(stream)),
                  "dequant launch");
    });
}

// ---- plumbing ----------------------------------------------------------------------

int apex_hip_device_count(int *out) {
    return guard([&] {
        require(out != nullptr, "out is null");
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess)
            n = 0;
        *out = n;
    });
}

int apex_hip_set_device(int device) {
    return guard([&] { hip_check(hipSetDevice(device), "hipSetDevice"); });
}

int apex_hip_malloc(size_t bytes, void **out) {
    return guard([&] {
        require(out != nullptr, "out is null");
        *out = nullptr;
        if (bytes && hipMalloc(out, bytes) != hipSuccess)
            fail(APEX_HIP_E_OOM, "hipMalloc failed for " + std::to_string(bytes) + " bytes");
    });
}

int apex_hip_free(void *ptr) {
    return guard([&] {
        if (ptr)
            hip_check(hipFree(ptr), "hipFree");
    });
}

int apex_hip_memcpy_h2d(void *dst, const void *src, size_t bytes) {
    return guard([&] { hip_check(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice), "h2d"); });
}

int apex_hip_memcpy_d2h(void *dst, const void *src, size_t bytes) {
    return guard([&] { hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost), "d2h"); });
}

int apex_hip_memcpy_d2d(void *dst, const void *src, size_t bytes) {
    return guard([&] { hip_check(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice), "d2d"); });
}

int apex_hip_memset(void *dst, int value, size_t bytes) {
    return guard([&] { hip_check(hipMemset(dst, value, bytes), "memset"); });
}

int apex_hip_mem_info(size_t *free_bytes, size_t *total_bytes) {
    return guard([&] {
        require(free_bytes && total_bytes, "mem_info: null pointer");
        hip_check(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo");
    });
}

int apex_hip_device_synchronize(void) {
    return guard([&] { hip_check(hipDeviceSynchronize(), "device sync"); });
}

int apex_hip_stream_create(void **out) {
    return guard([&] {
        require(out != nullptr, "out is null");
        hipStream_t s;
        hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream create");
        *out = s;
    });
}

int apex_hip_stream_destroy(void *stream) {
    return guard([&] { hip_check(hipStreamDestroy(as_stream(stream)), "stream destroy"); });
}

int apex_hip_stream_synchronize(void *stream) {
    return guard([&] { hip_check(hipStreamSynchronize(as_stream(stream)), "stream sync"); });
}

int apex_hip_event_create(void **out) {
    return guard([&] {
        require(out != nullptr, "out is null");
        hipEvent_t e;
        hip_check(hipEventCreate(&e), "event create");
        *out = e;
    });
}

int apex_hip_event_destroy(void *event) {
    return guard([&] { hip_check(hipEventDestroy(static_cast<hipEvent_t>(event)), "event destroy"); });
}

int apex_hip_event_record(void *event, void *stream) {
    return guard([&] {
        hip_check(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)), "event record");
    });
}

int apex_hip_event_synchronize(void *event) {
    return guard([&] {
        hip_check(hipEventSynchronize(static_cast<hipEvent_t>(event)), "event sync");
    });
}

int apex_hip_event_elapsed_ms(void *start, void *stop, float *ms) {
    return guard([&] {
        require(ms != nullptr, "ms is null");
        hip_check(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                      static_cast<hipEvent_t>(stop)),
                  "event elapsed");
    });
}

int apex_hip_read_probe(const void *ptr, size_t bytes, uint32_t *sink, void *stream) {
    return guard([&] {
        require(ptr && sink, "null pointer");
        require(bytes >= 16 && bytes < (1ull << 31), "bytes must be in [16, 2 GiB)");
        init_device_tuning();
        hip_check(apex_hip::read_probe_launch(ptr, bytes, sink, as_stream(stream)), "read probe");
    });
}

int apex_hip_read_probe_sink_words(void) { return (int)apex_hip::read_probe_blocks(); }

int apex_hip_set_gemm_min_tokens(uint32_t bf16_tokens, uint32_t f32_tokens) {
    return guard([&] {
        g_gemm_min_tokens[0].store(bf16_tokens, std::memory_order_relaxed);
        g_gemm_min_tokens[1].store(f32_tokens, std::memory_order_relaxed);
    });
}

int apex_hip_dense_dispatch_counts(uint64_t counts[4]) {
    return guard([&] {
        require(counts != nullptr, "counts is null");
        for (int i = 0; i < kDispKinds; ++i)
            counts[i] = g_dispatch[i].load(std::memory_order_relaxed);
    });
}

int apex_hip_gemm_tail_plan(uint32_t m, uint32_t n, int geglu, uint32_t ncu, uint32_t out[3]) {
    return guard([&] {
        require(out != nullptr, "out is null");
        require(m > 0 && n > 0, "empty product");
        if (ncu == 0) {
            init_device_tuning();
            ncu = (uint32_t)apex_hip::num_cus();
        }
        const apex_hip::GemmTailPlan p = apex_hip::gemm_tail_plan(m, n, geglu != 0, ncu);
        out[0] = p.nf;
        out[1] = p.nt;
        out[2] = p.ns;
    });
}

int apex_hip_set_gemv_waves_per_cu(int waves) {
    return guard([&] {
        require(waves >= 1 && waves <= 32, "waves per CU must be in [1, 32]");
        apex_hip::kTargetWavesPerCU.store(waves, std::memory_order_relaxed);
    });
}

size_t apex_moe_workspace_bytes(uint32_t tokens, uint32_t experts, uint32_t top_k, uint32_t hidden,
                                uint32_t inter) {
    return apex_hip::moe_workspace(tokens, experts, top_k, hidden, inter, true).total;
}

size_t apex_moe_workspace_plan_offset(uint32_t tokens, uint32_t experts, uint32_t top_k,
                                      uint32_t hidden, uint32_t inter) {
    return apex_hip::moe_workspace(tokens, experts, top_k, hidden, inter, true).plan;
}

int apex_moe_route_bf16(const uint16_t *logits, uint32_t tokens, uint32_t experts, uint32_t top_k,
                        int32_t *ids, float *weights, void *stream) {
    return guard([&] { moe_route_impl(logits, tokens, experts, top_k, ids, weights, as_stream(stream)); });
}

int apex_moe_ffn_bf16(const uint16_t *x, const uint16_t *logits, const apex_moe_slots *slots,
                      uint16_t *y, uint32_t tokens, uint32_t experts, uint32_t top_k,
                      uint32_t hidden, uint32_t inter, void *workspace, size_t workspace_bytes,
                      void *stream) {
    return guard([&] {
        require(workspace != nullptr || tokens == 0, "moe_ffn: workspace is null");
        moe_impl(x, logits, nullptr, nullptr, slots, y, tokens, experts, top_k, hidden, inter,
                 workspace, workspace_bytes, as_stream(stream));
    });
}

int apex_moe_ffn_bf16_noalloc(const uint16_t *x, const uint16_t *logits,
                              const apex_moe_slots *slots, uint16_t *y, uint32_t tokens,
                              uint32_t experts, uint32_t top_k, uint32_t hidden, uint32_t inter,
                              void *stream) {
    return guard([&] {
        // The fixed workspace is one array per device: a second thread enqueuing on the
        // same device while a call is in progress would race on it, so it is refused.
        constexpr int kMaxDevices = 64;
        static std::atomic<bool> busy[kMaxDevices] = {};
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        require(dev >= 0 && dev < kMaxDevices, "moe_ffn (no-allocation form): device index");
        if (busy[dev].exchange(true, std::memory_order_acquire))
            fail(APEX_HIP_E_INVALID,
                 "moe_ffn (no-allocation form): another call is in progress on this device; calls "
                 "sharing the fixed workspace must be serialised on one stream per device");
        struct Release {
            std::atomic<bool> &b;
            ~Release() { b.store(false, std::memory_order_release); }
        } release{busy[dev]};
        moe_impl(x, logits, nullptr, nullptr, slots, y, tokens, experts, top_k, hidden, inter,
                 nullptr, 0, as_stream(stream));
    });
}

int apex_moe_ffn_f32logits_bf16(const uint16_t *x, const float *logits,
                                const uint16_t *per_expert_scale, const apex_moe_slots *slots,
                                uint16_t *y, uint32_t tokens, uint32_t experts, uint32_t top_k,
                                uint32_t hidden, uint32_t inter, void *workspace,
                                size_t workspace_bytes, void *stream) {
    return guard([&] {
        require(logits != nullptr || tokens == 0, "moe_ffn: null pointer");
        require(workspace != nullptr || tokens == 0, "moe_ffn: workspace is null");
        moe_impl(x, nullptr, logits, per_expert_scale, slots, y, tokens, experts, top_k, hidden,
                 inter, workspace, workspace_bytes, as_stream(stream));
    });
}

int apex_moe_route_f32(const float *logits, const uint16_t *per_expert_scale, uint32_t tokens,
                       uint32_t experts, uint32_t top_k, int32_t *ids, float *weights,
                       void *stream) {
    return guard([&] {
        route_f32_impl(logits, per_expert_scale, tokens, experts, top_k, ids, weights,
                       as_stream(stream));
    });
}

int apex_moe_router_logits_q8(const float *h, const uint16_t *norm_weights, float eps,
                              const uint32_t *proj_weights, const uint16_t *proj_scales,
                              const uint16_t *proj_biases, uint32_t tokens, uint32_t experts,
                              uint32_t hidden, float *logits, void *stream) {
    return guard([&] {
        router_impl({h, norm_weights, eps, proj_weights, proj_scales, proj_biases, tokens, experts,
                     hidden, logits},
                    as_stream(stream));
    });
}

int apex_file_to_device(const char *path, uint64_t file_offset, uint64_t bytes, void *dst,
                        uint64_t chunk_bytes, uint32_t n_buffers, void *stream) {
    return guard([&] {
        require(path && (dst || bytes == 0), "null pointer");
        if (bytes == 0)
            return;
        const apex_hip::FileRange r{file_offset, bytes, dst};
        const apex_hip::FileCopyStatus st = apex_hip::copy_file_ranges(
            path, &r, 1, chunk_bytes ? chunk_bytes : kFileChunk, n_buffers ? n_buffers : kFileBuffers,
            as_stream(stream));
        if (!st.error.empty())
            fail(APEX_HIP_E_INVALID, "file_to_device: " + st.error);
    });
}

int apex_experts_to_device(const char *path, uint64_t stride, uint64_t slot_bytes,
                           const int32_t *experts, uint32_t n_experts, void *dst,
                           uint64_t dst_stride, uint64_t chunk_bytes, uint32_t n_buffers,
                           void *stream) {
    return guard([&] {
        require(path && (n_experts == 0 || (experts && dst)), "null pointer");
        require(slot_bytes <= stride && slot_bytes <= dst_stride,
                "experts_to_device: slot_bytes exceeds a stride");
        std::vector<apex_hip::FileRange> r(n_experts);
        for (uint32_t i = 0; i < n_experts; ++i) {
            require(experts[i] >= 0, "experts_to_device: negative expert index");
            r[i] = {(uint64_t)experts[i] * stride, slot_bytes,
                    static_cast<char *>(dst) + (uint64_t)i * dst_stride};
        }
        const apex_hip::FileCopyStatus st = apex_hip::copy_file_ranges(
            path, r.data(), r.size(), chunk_bytes ? chunk_bytes : kFileChunk,
            n_buffers ? n_buffers : kFileBuffers, as_stream(stream));
        if (!st.error.empty())
            fail(APEX_HIP_E_INVALID, "experts_to_device: " + st.error);
    });
}

int apex_hip_set_moe_path(int path) {
    return guard([&] {
        require(path >= 0 && path <= 2, "moe path must be 0 (by size), 1 (grouped GEMV) or 2 (grouped GEMM)");
        apex_hip::kMoePath.store(path, std::memory_order_relaxed);
    });
}

} // extern "C"
