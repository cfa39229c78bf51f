// The compiled GEMM configurations: X(BM, BN, WAVES_M, WAVES_N).  K is staged
// 128 bytes at a time (128 int8 or 64 f16/bf16 elements), split_k is 1.
// The tile search (search.cpp) measures exactly this list.
#pragma once

#define HXM_GEMM_CONFIG_LIST(X)                                              \
  X(256, 256, 2, 2), X(256, 128, 2, 2), X(128, 256, 2, 2), X(128, 128, 2, 2), \
      X(64, 64, 2, 2), X(32, 32, 1, 1)
