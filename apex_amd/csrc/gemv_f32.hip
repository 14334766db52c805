// Instantiation unit: NVFP4 GEMV variants with float activations, epilogue mode(s) 0, 3.
#include "gemv_kernels.h"

namespace apex_hip {
namespace gemv_detail {
template hipError_t gemv_dispatch<float, 0>(const GemvArgs &, hipStream_t);
template hipError_t gemv_dispatch<float, 3>(const GemvArgs &, hipStream_t);
} // namespace gemv_detail
} // namespace apex_hip
