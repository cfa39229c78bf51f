// The compiled GEMM configurations: X(BM, BN, BKB, STAGES, WAVES_M, WAVES_N)
// with BKB the K bytes per LDS stage (bk = BKB int8 or BKB/2 f16/bf16
// elements).  split_k is 1.  The tile search (search.hip) measures exactly
// this list; the LDS footprint is STAGES * (BM + BN) * BKB bytes.  The two
// large tiles also come with a second wave grid (8 waves of 128x64, and 4x1
// waves of 64x128), listed after the 2x2 grid that a lookup with wildcard
// wave fields finds first.
#pragma once

// A build may predefine the list (for example to compile one configuration).
#ifndef HXM_GEMM_CONFIG_LIST
#define HXM_GEMM_CONFIG_LIST(X)                                                 \
  X(256, 256, 128, 2, 2, 2), X(256, 256, 64, 4, 2, 2),                           \
      X(256, 128, 128, 3, 2, 2), X(256, 128, 64, 4, 2, 2),                       \
      X(128, 256, 64, 4, 2, 2), X(128, 128, 128, 2, 2, 2),                       \
      X(128, 128, 64, 4, 2, 2), X(64, 64, 128, 2, 2, 2), X(32, 32, 128, 2, 1, 1), \
      X(256, 256, 128, 2, 2, 4), X(256, 128, 128, 3, 4, 1)
#endif

// W8A16 GEMM (f16 activations x int8 [N, K] weights, BKB = A bytes per
// stage; B rows hold BKB/2 int8).  The SwiGLU variant exists for the entries
// whose wave tile is 128 columns wide (BN / WAVES_N == 128).  The default
// tile is the first entry that gives every CU a workgroup, so among equal
// tile counts the entry with fewer B columns per wave (fewer int8 -> f16
// conversions per MFMA) comes first.
#ifndef HXM_W8_CONFIG_LIST
#define HXM_W8_CONFIG_LIST(X)                                                   \
  X(256, 256, 128, 3, 2, 2), X(256, 256, 128, 2, 2, 2),                          \
      X(256, 128, 128, 3, 2, 2), X(128, 256, 128, 4, 2, 2),                      \
      X(128, 128, 128, 3, 2, 2)
#endif
