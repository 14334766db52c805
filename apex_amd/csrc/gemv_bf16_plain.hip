// Instantiation unit: NVFP4 GEMV variants with uint16_t activations, epilogue mode(s) 1.
#include "gemv_kernels.h"

namespace apex_hip {
namespace gemv_detail {
template hipError_t gemv_dispatch<uint16_t, 1>(const GemvArgs &, hipStream_t);
} // namespace gemv_detail
} // namespace apex_hip
