// GEMV kernels with the SiLU(gate) * up input stage (the down projection). The kernel template
// is in eg_gemv_kernel.hpp; this unit only instantiates it, in parallel with the others.
#include "eg_gemv_kernel.hpp"

namespace eg_gemv {

KernelFn pick_silu_mul(int bits, int enc, int mode, int team, int cpl, int u) {
  return pick_fused_format<EG_INPUT_SILU_MUL>(bits, enc, mode, team, cpl, u);
}

}  // namespace eg_gemv
