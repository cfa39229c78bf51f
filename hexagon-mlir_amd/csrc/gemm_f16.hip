// f16 and bf16 GEMM kernels (fp32 accumulate) for the entries of
// HXM_GEMM_CONFIG_LIST whose index is HXM_PART mod kGemmParts (the Makefile
// compiles this file once per part).
#include "gemm_kernel.h"

#ifndef HXM_PART
#define HXM_PART 0
#endif
#define HXM_CAT2(a, b) a##b
#define HXM_CAT(a, b) HXM_CAT2(a, b)

namespace hxm {

template <typename T, int BM, int BN, int BKB, int ST, int WM, int WN>
constexpr gemm_fn f16_fn() {
  if constexpr (config_index(kGemmKeys, BM, BN, BKB, ST, WM, WN) % kGemmParts == HXM_PART)
    return gemm_kernel<T, BM, BN, BKB, ST, WM, WN, kEpiFloat>;
  else
    return nullptr;
}

#define HXM_F16_FNS(BM, BN, BKB, ST, WM, WN) \
  {f16_fn<_Float16, BM, BN, BKB, ST, WM, WN>(), f16_fn<__bf16, BM, BN, BKB, ST, WM, WN>()}

extern const gemm_fn HXM_CAT(kF16Fns_p, HXM_PART)[][2] = {HXM_GEMM_CONFIG_LIST(HXM_F16_FNS)};

}  // namespace hxm
