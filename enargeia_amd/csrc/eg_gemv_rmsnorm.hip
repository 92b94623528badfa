// GEMV kernels with the RMSNorm input stage (the q|k|v and gate|up plans, the LM head). The kernel template
// is in eg_gemv_kernel.hpp; this unit only instantiates it, in parallel with the others.
#include "eg_gemv_kernel.hpp"

namespace eg_gemv {

KernelFn pick_rmsnorm(int bits, int enc, int mode, int team, int cpl, int u) {
  return pick_fused_format<EG_INPUT_RMSNORM>(bits, enc, mode, team, cpl, u);
}

}  // namespace eg_gemv
