// The D = 256 dK/dV instances of flash_bwd_dkdv_kernel (16-bit, without
// extended masks), in a unit of their own: the kernel holds 256 fp32
// accumulators per lane plus the score blocks, which needs the compiler's
// default AGPR register form (the VGPR form the rest of the backward is built
// in fails to compile here).
#include "flash_bwd_kernels.h"

namespace pjx {

int launch_dkdv256(const FlashBwdArgs& a, bool f16, bool hb, hipStream_t s) {
  if (f16)
    return hb ? launch_dkdv<flash_bwd_dkdv_kernel<F16Fmt, 256, true, 0>>(a, s)
              : launch_dkdv<flash_bwd_dkdv_kernel<F16Fmt, 256, false, 0>>(a, s);
  return hb ? launch_dkdv<flash_bwd_dkdv_kernel<Bf16Fmt, 256, true, 0>>(a, s)
            : launch_dkdv<flash_bwd_dkdv_kernel<Bf16Fmt, 256, false, 0>>(a, s);
}

}  // namespace pjx
