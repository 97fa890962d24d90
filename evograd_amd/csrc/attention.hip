// Causal attention forward/backward for gfx950 (bf16/fp16 MFMA).
#include "eg_common.hpp"

using namespace eg;

extern "C" size_t eg_attn_workspace_bytes(int64_t batch, int64_t heads, int64_t seq,
                                          int64_t head_dim) {
  (void)head_dim;
  if (batch <= 0 || heads <= 0 || seq <= 0) return 0;
  return (size_t)(batch * heads * seq) * sizeof(float);
}

extern "C" int eg_attn_fwd(const void*, const void*, const void*, void*, float*, int64_t,
                           int64_t, int64_t, int64_t, float, int, void*) {
  set_error("eg_attn_fwd: not implemented yet");
  return 3;
}

extern "C" int eg_attn_bwd(const void*, const void*, const void*, const void*, const void*,
                           const float*, void*, void*, void*, void*, int64_t, int64_t, int64_t,
                           int64_t, float, int, void*) {
  set_error("eg_attn_bwd: not implemented yet");
  return 3;
}
