// f16 and bf16 GEMM kernels (fp32 accumulate) for every entry of
// HXM_GEMM_CONFIG_LIST.
#include "gemm_kernel.h"

namespace hxm {

#define HXM_F16_FNS(BM, BN, BKB, ST, WM, WN)                  \
  {gemm_kernel<_Float16, BM, BN, BKB, ST, WM, WN, kEpiFloat>, \
   gemm_kernel<__bf16, BM, BN, BKB, ST, WM, WN, kEpiFloat>}

extern const gemm_fn kF16Fns[][2] = {HXM_GEMM_CONFIG_LIST(HXM_F16_FNS)};

}  // namespace hxm
