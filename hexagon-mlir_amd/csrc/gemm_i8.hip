// int8 GEMM kernels (int32 and dequant epilogues) for every entry of
// HXM_GEMM_CONFIG_LIST.
#include "gemm_kernel.h"

namespace hxm {

#define HXM_I8_FNS(BM, BN, BKB, ST, WM, WN)                \
  {gemm_kernel<int8_t, BM, BN, BKB, ST, WM, WN, kEpiI32>, \
   gemm_kernel<int8_t, BM, BN, BKB, ST, WM, WN, kEpiDequant>}

extern const gemm_fn kI8Fns[][2] = {HXM_GEMM_CONFIG_LIST(HXM_I8_FNS)};

}  // namespace hxm
