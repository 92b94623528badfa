// Entry points declared in the ABI whose kernels are not built yet fail loudly.
#include "eg_internal.hpp"

extern "C" int eg_matmul_q4_prefill(eg_context* ctx, const float*, const uint32_t*, const float*, const uint32_t*,
                                    const float*, float*, const eg_matmul_q4_dims*, int, int) {
  return eg::fail(ctx, EG_ERR_STATE, "matmul_q4_prefill: not available in this build");
}
