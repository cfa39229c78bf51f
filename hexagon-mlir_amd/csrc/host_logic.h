// Host-only arithmetic of the library, free of HIP: the guards that keep
// 32-bit offsets and launch grids in range, the K split, and the tuning-cache
// entry format.  libhxm uses these functions; tests/sanitize compiles this
// header on its own under -fsanitize=address,undefined and drives it with
// boundary and random inputs.
#pragma once

#include <cerrno>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

#include "../../include/hxm.h"

namespace hxm {

// A launch holds at most 2^32 - 1 work-items along x (workgroups times
// threads) and, as used here, at most 65535 workgroups along y.
inline bool grid_fits(int64_t groups_x, int threads, int64_t groups_y = 1) {
  return threads > 0 && groups_x >= 0 && groups_x <= 0xffffffffLL / threads && groups_y >= 0 &&
         groups_y <= 65535;
}

// Extents of a GEMM whose kernels index rows and K bytes with 32-bit values:
// M, N and K * elem_bytes at most 2^30 (no product here can overflow).
inline bool extents_fit(int64_t M, int64_t N, int64_t K, int64_t elem_bytes) {
  constexpr int64_t kMax = INT32_MAX / 2;
  return M >= 0 && N >= 0 && K >= 0 && elem_bytes > 0 && M <= kMax && N <= kMax &&
         K <= kMax / elem_bytes;
}

// The kernels address a tile's rows of an operand with 32-bit offsets from
// the tile's first row, inside a buffer resource of at most 2 GiB: the
// kTileRowsMax rows of the tallest tile must span less than that,
// (kTileRowsMax - 1) * ld_bytes + row_bytes <= INT32_MAX.
constexpr int64_t kTileRowsMax = 256;
inline bool tile_rows_addressable(int64_t ld_bytes, int64_t row_bytes) {
  return ld_bytes >= 0 && row_bytes >= 0 && row_bytes <= INT32_MAX &&
         ld_bytes <= (INT32_MAX - row_bytes) / (kTileRowsMax - 1);
}

// Workgroup rows a K split of `split` launches: K bytes in slices of whole
// stages, ceil(stages / split) stages each; the last slice may be short and
// no slice is empty.  1 for no split or no K.
inline int64_t ceil_div(int64_t a, int64_t b) {  // a >= 0, b > 0; no overflow
  return a / b + (a % b != 0);
}
inline int32_t k_slices(int64_t k_bytes, int64_t stage_bytes, int32_t split) {
  if (split <= 1 || k_bytes <= 0 || stage_bytes <= 0) return 1;
  const int64_t stages = ceil_div(k_bytes, stage_bytes);
  const int64_t per = ceil_div(stages, split);
  return static_cast<int32_t>(ceil_div(stages, per));
}

// Whether `slices` int32 partial planes of [M, N] fit in max_bytes,
// slices * M * N * 4 <= max_bytes, decided without forming the product:
// extents_fit admits M and N up to 2^30 each, so with 16 slices the product
// would pass 2^63.  For positive integers a * b <= c exactly when
// a <= floor(c / b), and nested floor divisions equal one.
inline bool split_planes_fit(int64_t slices, int64_t M, int64_t N, int64_t max_bytes) {
  if (slices < 1 || M < 0 || N < 0 || max_bytes < 0) return false;
  if (M == 0 || N == 0) return true;
  return M <= max_bytes / 4 / slices / N;
}

// Stream-K layout of an int8-weight GEMM launch of `ntiles` tiles of KT K
// stages each on `cus` CUs (one workgroup per CU): the first dp tiles, whole
// rounds, run one per workgroup; the rest (tiles = ntiles mod cus) are cut
// into one stream of tiles * KT stages, and `groups` (= cus) workgroups take
// `iters` consecutive stages each, so every CU does the same share of the
// last round.  With xcd, each XCD's cus / 8 workgroups stream only that
// XCD's tiles/8 tiles (its own window of the tile walk, whose A and B panels
// its L2 holds); it needs ntiles, dp and cus to be multiples of 8.  maxseg:
// the most workgroups one tile's stages are spread over (partial-tile slots
// per tile).  False when nothing is left for a stream (whole rounds) or an
// argument is out of range.
struct StreamKLayout {
  int32_t dp, groups, tiles, iters, maxseg, xcd;
};
inline bool stream_k_layout(int64_t ntiles, int64_t KT, int64_t cus, StreamKLayout* out) {
  if (!out || ntiles <= 0 || KT <= 0 || cus <= 0 || ntiles > INT32_MAX / 2 ||
      KT > INT32_MAX / 2 || cus > 65536)
    return false;
  const int64_t S = ntiles % cus;
  if (S == 0) return false;
  const int64_t dp = ntiles - S;
  const bool xcd = ntiles % 8 == 0 && dp % 8 == 0 && cus % 8 == 0;
  const int64_t streams = xcd ? 8 : 1;
  const int64_t tiles = S / streams, groups = cus / streams;
  const int64_t iters = ceil_div(tiles * KT, groups);
  int64_t maxseg = 1;
  for (int64_t t = 0; t < tiles; ++t) {
    const int64_t nseg = (t * KT + KT - 1) / iters - (t * KT) / iters + 1;
    if (nseg > maxseg) maxseg = nseg;
  }
  *out = StreamKLayout{static_cast<int32_t>(dp), static_cast<int32_t>(cus),
                       static_cast<int32_t>(S), static_cast<int32_t>(iters),
                       static_cast<int32_t>(maxseg), xcd ? 1 : 0};
  return true;
}

// One entry of the tuning-cache file: "op M N K bm bn bk waves_m waves_n
// stages split_k reps".  Every field is read as 64-bit and range-checked
// before it narrows, so an out-of-range value cannot wrap onto a compiled
// configuration.  Returns false for anything else.
struct CacheEntry {
  int32_t op;
  int64_t m, n, k;
  hxm_gemm_config cfg;
  int32_t reps;
};

inline bool parse_cache_entry(const char* line, CacheEntry* out) {
  if (!line) return false;
  long long v[12];
  const char* p = line;
  for (int i = 0; i < 12; ++i) {
    while (*p == ' ' || *p == '\t') ++p;
    char* end = nullptr;
    errno = 0;
    v[i] = std::strtoll(p, &end, 10);  // saturates and sets ERANGE out of range
    if (end == p || errno == ERANGE) return false;
    p = end;
  }
  for (; *p; ++p)  // only blanks may follow
    if (*p != ' ' && *p != '\t' && *p != '\n' && *p != '\r') return false;
  bool in_range = v[0] >= 0 && v[0] <= INT32_MAX && v[11] >= 1 && v[11] <= 10000;
  for (int i = 1; i <= 3; ++i) in_range = in_range && v[i] >= 0 && v[i] <= INT32_MAX;
  for (int i = 4; i <= 10; ++i) in_range = in_range && v[i] >= 0 && v[i] <= 4096;
  if (!in_range) return false;
  out->op = static_cast<int32_t>(v[0]);
  out->m = v[1], out->n = v[2], out->k = v[3];
  out->cfg = hxm_gemm_config{static_cast<int32_t>(v[4]), static_cast<int32_t>(v[5]),
                             static_cast<int32_t>(v[6]), static_cast<int32_t>(v[7]),
                             static_cast<int32_t>(v[8]), static_cast<int32_t>(v[9]),
                             static_cast<int32_t>(v[10])};
  out->reps = static_cast<int32_t>(v[11]);
  return true;
}

}  // namespace hxm
