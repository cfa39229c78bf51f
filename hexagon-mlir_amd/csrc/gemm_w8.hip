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
// The first entry (the FFN gate/up tile) also comes in its stream-K form
// (SK = 1, split_k = HXM_STREAM_K); the other entries have none (measured
// slower than the one-workgroup tiles at the FFN's shapes, and each form
// doubles a table entry's compile time).
template <int BM, int BN, int BKB, int ST, int WM, int WN, int EPI, int SK>
constexpr gemm_fn w8_fn() {
  constexpr int idx = config_index(kW8Keys, BM, BN, BKB, ST, WM, WN);
  if constexpr (idx % kGemmParts == HXM_PART && (EPI != kEpiSwiglu || BN / WN == 128) &&
                (SK == 0 || idx == 0))
    return gemm_kernel<_Float16, BM, BN, BKB, ST, WM, WN, EPI, SK>;
  else
    return nullptr;
}

#define HXM_W8_FNS(BM, BN, BKB, ST, WM, WN)                                       \
  {w8_fn<BM, BN, BKB, ST, WM, WN, kEpiW8, 0>(), w8_fn<BM, BN, BKB, ST, WM, WN, kEpiSwiglu, 0>(), \
   w8_fn<BM, BN, BKB, ST, WM, WN, kEpiW8Res, 0>(), w8_fn<BM, BN, BKB, ST, WM, WN, kEpiW8, 1>(), \
   w8_fn<BM, BN, BKB, ST, WM, WN, kEpiSwiglu, 1>(), w8_fn<BM, BN, BKB, ST, WM, WN, kEpiW8Res, 1>()}

extern const gemm_fn HXM_CAT(kW8Fns_p, HXM_PART)[][6] = {HXM_W8_CONFIG_LIST(HXM_W8_FNS)};

}  // namespace hxm
