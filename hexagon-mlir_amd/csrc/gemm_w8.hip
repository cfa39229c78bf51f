// W8A16 GEMM kernels (f16 x int8 weights: per-channel scale, fused SwiGLU
// and residual-add epilogues) for every entry of HXM_W8_CONFIG_LIST.
#include "gemm_kernel.h"

namespace hxm {

// The SwiGLU image interleaves 64-channel blocks, so that epilogue exists
// only where a wave's tile is 128 columns wide.
template <int BM, int BN, int BKB, int ST, int WM, int WN>
constexpr gemm_fn swiglu_fn() {
  if constexpr (BN / WN == 128)
    return gemm_kernel<_Float16, BM, BN, BKB, ST, WM, WN, kEpiSwiglu>;
  else
    return nullptr;
}

#define HXM_W8_FNS(BM, BN, BKB, ST, WM, WN)                                    \
  {gemm_kernel<_Float16, BM, BN, BKB, ST, WM, WN, kEpiW8>,                       \
   swiglu_fn<BM, BN, BKB, ST, WM, WN>(),                                         \
   gemm_kernel<_Float16, BM, BN, BKB, ST, WM, WN, kEpiW8Res>}

extern const gemm_fn kW8Fns[][3] = {HXM_W8_CONFIG_LIST(HXM_W8_FNS)};

}  // namespace hxm
