// The f16 product kernels of plain operands (16-bit and fp32 C) and the logits
// product with the softmax epilogue (definitions in gemm_kernel.hpp).
#include "gemm_kernel.hpp"

namespace eg {
namespace gk {
EG_GEMM_LAYOUTS(template, f16_t, f16_t, false, 0)
EG_GEMM_LAYOUTS(template, f16_t, float, false, 0)
EG_GEMM_KERNEL(template, f16_t, true, true, f16_t, true, 0)
}  // namespace gk
}  // namespace eg
