// W8A16 GEMM kernels (f16 x int8 weights: per-channel scale, fused SwiGLU
// and residual-add epilogues) for the entries of HXM_W8_CONFIG_LIST whose
// index is HXM_PART mod kGemmParts (the Makefile compiles this file once per
// part).
#include "gemm_kernel.h"

#ifndef HXM_PART
#define HXM_PART 0
#endif
#define HXM_CAT2(a, b) a##b
#define HXM_CAT(a, b) HXM_CAT2(a, b)

namespace hxm {

// The SwiGLU image interleaves 64-channel blocks, so that epilogue exists
// only where a wave's tile is 128 columns wide.
// The stream-K forms of entry 0 are compiled in gemm_w8sk.hip.
template <int BM, int BN, int BKB, int ST, int WM, int WN, int EPI>
constexpr gemm_fn w8_fn() {
  if constexpr (config_index(kW8Keys, BM, BN, BKB, ST, WM, WN) % kGemmParts == HXM_PART &&
                (EPI != kEpiSwiglu || BN / WN == 128))
    return gemm_kernel<_Float16, BM, BN, BKB, ST, WM, WN, EPI>;
  else
    return nullptr;
}

#define HXM_W8_FNS(BM, BN, BKB, ST, WM, WN)                                     \
  {w8_fn<BM, BN, BKB, ST, WM, WN, kEpiW8>(), w8_fn<BM, BN, BKB, ST, WM, WN, kEpiSwiglu>(), \
   w8_fn<BM, BN, BKB, ST, WM, WN, kEpiW8Res>()}

extern const gemm_fn HXM_CAT(kW8Fns_p, HXM_PART)[][3] = {HXM_W8_CONFIG_LIST(HXM_W8_FNS)};

}  // namespace hxm
