// Stream-K forms (SK = 1, split_k = HXM_STREAM_K) of the W8A16 GEMM for
// entry 0 of HXM_W8_CONFIG_LIST, the FFN gate/up tile, one epilogue per
// part (the Makefile compiles this file once per part, HXM_PART = 0, 1, 2),
// so the three build in parallel with the other kernel objects.  The other
// entries have no stream-K form: it measured slower than the one-workgroup
// tiles at the FFN's shapes, and each form doubles an entry's compile time.
#include "gemm_kernel.h"

#ifndef HXM_PART
#define HXM_PART 0
#endif
#define HXM_CAT2(a, b) a##b
#define HXM_CAT(a, b) HXM_CAT2(a, b)

namespace hxm {

template <int EPI, int PART>
constexpr gemm_fn w8sk_fn() {
  constexpr ConfigKey k = kW8Keys[0];
  if constexpr (PART == HXM_PART)
    return gemm_kernel<_Float16, k.bm, k.bn, k.bkb, k.st, k.wm, k.wn, EPI, 1>;
  else
    return nullptr;
}

// {kEpiW8, kEpiSwiglu, kEpiW8Res}: part p holds entry p.
extern const gemm_fn HXM_CAT(kW8SkFns_p, HXM_PART)[3] = {
    w8sk_fn<kEpiW8, 0>(), w8sk_fn<kEpiSwiglu, 1>(), w8sk_fn<kEpiW8Res, 2>()};

}  // namespace hxm
