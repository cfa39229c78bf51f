// int8 GEMM kernels (int32 and dequant epilogues) for the entries of
// HXM_GEMM_CONFIG_LIST whose index is HXM_PART mod kGemmParts (the Makefile
// compiles this file once per part).
#include "gemm_kernel.h"

#ifndef HXM_PART
#define HXM_PART 0
#endif
#define HXM_CAT2(a, b) a##b
#define HXM_CAT(a, b) HXM_CAT2(a, b)

namespace hxm {

template <int BM, int BN, int BKB, int ST, int WM, int WN, int EPI>
constexpr gemm_fn i8_fn() {
  if constexpr (config_index(kGemmKeys, BM, BN, BKB, ST, WM, WN) % kGemmParts == HXM_PART)
    return gemm_kernel<int8_t, BM, BN, BKB, ST, WM, WN, EPI>;
  else
    return nullptr;
}

#define HXM_I8_FNS(BM, BN, BKB, ST, WM, WN) \
  {i8_fn<BM, BN, BKB, ST, WM, WN, kEpiI32>(), i8_fn<BM, BN, BKB, ST, WM, WN, kEpiDequant>()}

extern const gemm_fn HXM_CAT(kI8Fns_p, HXM_PART)[][2] = {HXM_GEMM_CONFIG_LIST(HXM_I8_FNS)};

}  // namespace hxm
