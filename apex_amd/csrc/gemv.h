// Host-side interface of the NVFP4 GEMV kernels (decode regime).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

namespace apex_hip {

// Arguments of one GEMV launch.  codes/scales/tensor_scale index 0 is the plain
// matrix (or the gate of a GeGLU pair), index 1 the up matrix of a GeGLU pair.
struct GemvArgs {
    const void *x;              // [tokens, K] fp32 or bf16 bits, row stride K
    const uint32_t *codes[2];   // [rows, K/8]
    const uint8_t *scales[2];   // [rows, K/16]
    float tensor_scale[2];
    void *out;                  // [tokens, out_stride] fp32 or bf16 bits
    uint32_t rows, K, tokens, out_stride;
    uint32_t sets_per_wave;     // filled by the launcher
    // fp32 x only: when set, each x row is RMS-normalised first, x * (1 / sqrt(mean(x^2)
    // + norm_eps)) * norm_w (bf16 [K]), as the separate rms_norm_f32 would
    const uint16_t *norm_w;
    float norm_eps;
};

enum class GemvMode { PlainF32, PlainBF16, GegluBF16, GegluF32 };

// Launch sizing, process-wide: target resident GEMV waves per CU
// (apex_hip_set_gemv_waves_per_cu) and the device's CU count (read at first use).
// Atomics: a setter may run while other threads dispatch.
extern std::atomic<int> kTargetWavesPerCU;
extern std::atomic<int> kNumCUs;
inline int num_cus() { return kNumCUs.load(std::memory_order_relaxed); }

hipError_t gemv_launch(const GemvArgs &a, GemvMode mode, bool x_is_bf16, hipStream_t stream);
hipError_t geglu_f32_launch(const float *gate, const float *up, float *out, uint32_t count,
                            hipStream_t stream);
// Streaming-read probe over [p, p+bytes) (bytes < 2 GiB); sink needs read_probe_blocks()
// words, one per workgroup of the probe's grid.
hipError_t read_probe_launch(const void *p, size_t bytes, uint32_t *sink, hipStream_t stream);
uint32_t read_probe_blocks();
hipError_t dequant_launch(const uint32_t *codes, const uint8_t *scales, void *out, uint32_t rows,
                          uint32_t K, float tensor_scale, bool bf16, hipStream_t stream);

} // namespace apex_hip
