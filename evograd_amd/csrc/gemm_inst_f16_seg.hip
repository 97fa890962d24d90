// The f16 product kernels of segmented operands (along M or N, and along K;
// definitions in gemm_kernel.hpp).
#include "gemm_kernel.hpp"

namespace eg {
namespace gk {
EG_GEMM_LAYOUTS(template, f16_t, f16_t, false, 1)
EG_GEMM_LAYOUTS(template, f16_t, f16_t, false, 2)
}  // namespace gk
}  // namespace eg
