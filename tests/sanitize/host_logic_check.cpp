// Sanitizer check of libhxm's host-only arithmetic (hexagon-mlir_amd/csrc/
// host_logic.h): built with g++ -fsanitize=address,undefined by
// tests/test_host_sanitize.py.  Every function is driven with boundary values
// and a seeded random sweep and compared with a restatement in 128-bit
// integers; the tuning-cache entry parser is also fed malformed and random
// lines; stream-K layouts are walked segment by segment as the kernel walks
// them.  Prints "host_logic ok" and exits 0 when every check holds.
#include <algorithm>
#include <climits>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "../../hexagon-mlir_amd/csrc/host_logic.h"

using i128 = __int128;
static int failures = 0;
#define CHECK(cond, ...)                    \
  do {                                      \
    if (!(cond)) {                          \
      std::fprintf(stderr, __VA_ARGS__);    \
      std::fputc('\n', stderr);             \
      if (++failures > 20) std::exit(1);    \
    }                                       \
  } while (0)

static bool ref_grid(int64_t gx, int threads, int64_t gy) {
  return threads > 0 && gx >= 0 && static_cast<i128>(gx) * threads <= 0xffffffffLL && gy >= 0 &&
         gy <= 65535;
}
static bool ref_extents(int64_t M, int64_t N, int64_t K, int64_t eb) {
  const i128 lim = INT32_MAX / 2;
  return M >= 0 && N >= 0 && K >= 0 && eb > 0 && M <= lim && N <= lim &&
         static_cast<i128>(K) * eb <= lim;
}
static bool ref_rows(int64_t ld, int64_t row) {
  return ld >= 0 && row >= 0 && row <= INT32_MAX &&
         static_cast<i128>(hxm::kTileRowsMax - 1) * ld + row <= INT32_MAX;
}

static const int64_t kEdges[] = {0, 1, 2, 3, 15, 16, 17, 255, 256, 4095, 4096, 65535, 65536,
                                 (1LL << 20) - 1, 1LL << 20, 8421504, 8421505,
                                 1073741823, 1073741824, INT32_MAX - 1, INT32_MAX,
                                 (int64_t)INT32_MAX + 1, 0xffffffffLL, 1LL << 40,
                                 INT64_MAX / 4, INT64_MAX / 2, INT64_MAX - 1, INT64_MAX,
                                 -1, -2, INT64_MIN + 1, INT64_MIN};

int main() {
  std::mt19937_64 rng(20261202);
  auto any64 = [&]() -> int64_t {
    switch (rng() % 4) {
      case 0: return kEdges[rng() % (sizeof(kEdges) / sizeof(kEdges[0]))];
      case 1: return static_cast<int64_t>(rng() % 100000);
      case 2: return static_cast<int64_t>(rng() >> (rng() % 64));
      default: return static_cast<int64_t>(rng());
    }
  };

  // Launch grids and extents.
  for (int it = 0; it < 200000; ++it) {
    const int64_t gx = any64(), gy = any64();
    const int threads = static_cast<int>(rng() % 2 ? 64 << (rng() % 5) : rng() % 2048);
    CHECK(hxm::grid_fits(gx, threads, gy) == ref_grid(gx, threads, gy),
          "grid_fits(%lld, %d, %lld)", (long long)gx, threads, (long long)gy);
    const int64_t M = any64(), N = any64(), K = any64();
    const int64_t eb = static_cast<int64_t>(rng() % 6);
    CHECK(hxm::extents_fit(M, N, K, eb) == ref_extents(M, N, K, eb),
          "extents_fit(%lld, %lld, %lld, %lld)", (long long)M, (long long)N, (long long)K,
          (long long)eb);
    const int64_t ld = any64(), row = any64();
    CHECK(hxm::tile_rows_addressable(ld, row) == ref_rows(ld, row),
          "tile_rows_addressable(%lld, %lld)", (long long)ld, (long long)row);
  }

  // K splits: at most `split` slices, each non-empty, covering every stage.
  for (int it = 0; it < 200000; ++it) {
    const int64_t kb = rng() % 4 ? static_cast<int64_t>(rng() % (1 << 22)) : any64();
    const int64_t sb = rng() % 2 ? 64 << (rng() % 2) : any64();
    const int32_t split = static_cast<int32_t>(rng() % 2 ? 1 << (rng() % 6) : rng() % 40 - 3);
    const int32_t s = hxm::k_slices(kb, sb, split);
    if (split <= 1 || kb <= 0 || sb <= 0) {
      CHECK(s == 1, "k_slices(%lld, %lld, %d) = %d, want 1", (long long)kb, (long long)sb, split, s);
      continue;
    }
    const i128 stages = (static_cast<i128>(kb) + sb - 1) / sb;
    const i128 per = (stages + split - 1) / split;
    CHECK(s >= 1 && s <= split, "k_slices(%lld, %lld, %d) = %d out of [1, split]",
          (long long)kb, (long long)sb, split, s);
    CHECK(static_cast<i128>(s - 1) * per < stages && static_cast<i128>(s) * per >= stages,
          "k_slices(%lld, %lld, %d) = %d leaves an empty or missing slice", (long long)kb,
          (long long)sb, split, s);
  }

  // Split-K plane budgets: slices * M * N * 4 <= max_bytes without forming
  // the product, against the 128-bit product (extents up to 2^30 and beyond).
  for (int it = 0; it < 200000; ++it) {
    const int64_t sl = rng() % 2 ? 1 << (rng() % 5) : any64();
    const int64_t M = rng() % 2 ? static_cast<int64_t>(rng() % (1LL << 31)) : any64();
    const int64_t N = rng() % 2 ? static_cast<int64_t>(rng() % (1LL << 31)) : any64();
    const int64_t mx = rng() % 2 ? int64_t(256) << 20 : any64();
    // The product in steps, each checked against mx <= 2^63 before the next
    // factor, so no step passes 2^127.
    auto ref = [&]() {
      if (sl < 1 || M < 0 || N < 0 || mx < 0) return false;
      if (M == 0 || N == 0) return true;
      i128 p = static_cast<i128>(sl) * M;
      if (p > mx) return false;
      p *= N;
      if (p > mx) return false;
      return p * 4 <= mx;
    };
    const bool want = ref();
    CHECK(hxm::split_planes_fit(sl, M, N, mx) == want, "split_planes_fit(%lld, %lld, %lld, %lld)",
          (long long)sl, (long long)M, (long long)N, (long long)mx);
  }
  CHECK(hxm::split_planes_fit(16, 512, 512, int64_t(256) << 20) &&
            !hxm::split_planes_fit(8, 4096, 4096, int64_t(256) << 20) &&
            hxm::split_planes_fit(16, 1024, 4096, int64_t(256) << 20) &&
            !hxm::split_planes_fit(16, 1024, 4097, int64_t(256) << 20) &&
            !hxm::split_planes_fit(16, 1073741823, 1073741823, int64_t(256) << 20),
        "split_planes_fit known answers");

  // Tuning-cache entries: exact fields back, range checks at both edges.
  hxm::CacheEntry e;
  CHECK(hxm::parse_cache_entry("4 4096 4096 4096 256 256 128 2 2 2 1 10\n", &e) && e.op == 4 &&
            e.m == 4096 && e.k == 4096 && e.cfg.bm == 256 && e.cfg.bk == 128 &&
            e.cfg.stages == 2 && e.cfg.split_k == 1 && e.reps == 10,
        "valid entry");
  CHECK(hxm::parse_cache_entry("  17\t2147483647 0 1 4096 0 0 0 0 0 0 10000", &e) && e.op == 17 &&
            e.m == INT32_MAX && e.reps == 10000,
        "edge entry");
  const char* bad[] = {
      "", "\n", "4", "4 1 1 1 1 1 1 1 1 1 1", "4 1 1 1 1 1 1 1 1 1 1 1 1",
      "4 1 1 1 1 1 1 1 1 1 1 1 x", "-1 1 1 1 1 1 1 1 1 1 1 1", "4 -1 1 1 1 1 1 1 1 1 1 1",
      "4 2147483648 1 1 1 1 1 1 1 1 1 1", "2147483648 1 1 1 1 1 1 1 1 1 1 1",
      "4 1 1 1 4097 1 1 1 1 1 1 1", "4 1 1 1 1 1 1 1 1 1 -1 1", "4 1 1 1 1 1 1 1 1 1 1 0",
      "4 1 1 1 1 1 1 1 1 1 1 10001", "4 9223372036854775807 1 1 1 1 1 1 1 1 1 1",
      "4 9223372036854775808 1 1 1 1 1 1 1 1 1 1", "4 -9223372036854775809 1 1 1 1 1 1 1 1 1 1",
      "4 99999999999999999999999999 1 1 1 1 1 1 1 1 1 1", "4 1 1 1 256 256 128 2 2 2 1 1.5",
      "4 1 1 1 256 256 128 2 2 2 1 +", "x 1 1 1 1 1 1 1 1 1 1 1", "4,1,1,1,1,1,1,1,1,1,1,1"};
  for (const char* b : bad) CHECK(!hxm::parse_cache_entry(b, &e), "accepted \"%s\"", b);
  CHECK(!hxm::parse_cache_entry(nullptr, &e), "accepted NULL");

  // Random lines: never a crash or an out-of-range acceptance; formatted
  // valid entries come back unchanged.
  const char alphabet[] = "0123456789-+ \t\nxe.,";
  for (int it = 0; it < 200000; ++it) {
    std::string line;
    if (rng() % 3 == 0) {
      char buf[256];
      const long long f[12] = {(long long)(rng() % 20), (long long)(rng() % 100000),
                               (long long)(rng() % 100000), (long long)(rng() % 100000),
                               (long long)(rng() % 4097), (long long)(rng() % 4097),
                               (long long)(rng() % 4097), (long long)(rng() % 4097),
                               (long long)(rng() % 4097), (long long)(rng() % 4097),
                               (long long)(rng() % 4097), (long long)(1 + rng() % 10000)};
      std::snprintf(buf, sizeof(buf), "%lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld %lld\n",
                    f[0], f[1], f[2], f[3], f[4], f[5], f[6], f[7], f[8], f[9], f[10], f[11]);
      CHECK(hxm::parse_cache_entry(buf, &e) && e.op == f[0] && e.m == f[1] && e.n == f[2] &&
                e.k == f[3] && e.cfg.bm == f[4] && e.cfg.split_k == f[10] && e.reps == f[11],
            "round trip of \"%s\"", buf);
      continue;
    }
    const int fields = static_cast<int>(rng() % 15);
    for (int i = 0; i < fields; ++i) {
      const int len = static_cast<int>(rng() % 24);
      for (int j = 0; j < len; ++j) line += alphabet[rng() % (sizeof(alphabet) - 1)];
      line += ' ';
    }
    if (hxm::parse_cache_entry(line.c_str(), &e)) {
      bool ok = e.op >= 0 && e.m >= 0 && e.n >= 0 && e.k >= 0 && e.reps >= 1 && e.reps <= 10000;
      const int32_t* c = &e.cfg.bm;
      for (int i = 0; i < 7; ++i) ok = ok && c[i] >= 0 && c[i] <= 4096;
      CHECK(ok, "accepted out of range: \"%s\"", line.c_str());
    }
  }

  if (failures) {
    std::fprintf(stderr, "%d failure(s)\n", failures);
    return 1;
  }
  // Stream-K layouts: every (tile, stage) of the launch is computed by
  // exactly one workgroup, with the segment walk the kernel runs
  // (gemm_kernel.h, the SK loop), each segment's index below its tile's
  // segment count, which is at most maxseg, every partial-tile slot index in
  // range, and the data-parallel tiles the whole rounds.
  for (int it = 0; it < 3000; ++it) {
    const int64_t cus = (it % 3 == 0) ? 256 : 1 + static_cast<int64_t>(rng() % 300);
    const int64_t ntiles = 1 + static_cast<int64_t>(rng() % (it % 5 == 0 ? 2000 : 700));
    const int64_t KT = 1 + static_cast<int64_t>(rng() % (it % 7 == 0 ? 700 : 70));
    hxm::StreamKLayout L;
    const bool ok = hxm::stream_k_layout(ntiles, KT, cus, &L);
    CHECK(ok == (ntiles % cus != 0), "stream_k_layout(%lld,%lld,%lld) -> %d",
          (long long)ntiles, (long long)KT, (long long)cus, ok);
    if (!ok) continue;
    CHECK(L.dp + L.tiles == ntiles && L.dp % cus == 0 && L.tiles < cus && L.groups == cus,
          "stream-K split of %lld tiles", (long long)ntiles);
    CHECK(!L.xcd || (ntiles % 8 == 0 && L.dp % 8 == 0 && cus % 8 == 0), "xcd streams");
    const int64_t streams = L.xcd ? 8 : 1;
    const int64_t per = L.tiles / streams, gper = cus / streams;
    CHECK(L.iters >= 1 && per * streams == L.tiles && gper * L.iters >= per * KT,
          "stream coverage");
    std::vector<int> hits(static_cast<size_t>(L.tiles * KT), 0);
    std::vector<int> segs(static_cast<size_t>(L.tiles), 0);
    for (int64_t b = 0; b < cus; ++b) {             // the stream-K workgroups
      const int64_t x = L.xcd ? b & 7 : 0, w = L.xcd ? b >> 3 : b;
      int64_t i = w * L.iters;
      const int64_t end = std::min<int64_t>(per * KT, (w + 1) * L.iters);
      while (i < end) {
        const int64_t st = i / KT, k0 = i % KT, k1 = std::min<int64_t>(KT, k0 + (end - i));
        const int64_t tfirst = st * KT, seg0 = tfirst / L.iters;
        const int64_t nseg = (tfirst + KT - 1) / L.iters - seg0 + 1, seg = w - seg0;
        const int64_t slot = x * per + st;
        CHECK(seg >= 0 && seg < nseg && nseg <= L.maxseg && slot >= 0 && slot < L.tiles,
              "segment %lld of %lld (maxseg %d), slot %lld", (long long)seg, (long long)nseg,
              L.maxseg, (long long)slot);
        if (slot < 0 || slot >= L.tiles) break;
        for (int64_t k = k0; k < k1; ++k) ++hits[static_cast<size_t>(slot * KT + k)];
        ++segs[static_cast<size_t>(slot)];
        CHECK(k1 > k0, "empty segment");
        i += k1 - k0;
      }
    }
    for (size_t q = 0; q < hits.size(); ++q)
      CHECK(hits[q] == 1, "stage %zu computed %d times (ntiles %lld KT %lld cus %lld)", q, hits[q],
            (long long)ntiles, (long long)KT, (long long)cus);
    int64_t most = 0;
    for (int v : segs) most = std::max<int64_t>(most, v);
    CHECK(most == L.maxseg, "maxseg %d, most segments %lld", L.maxseg, (long long)most);
  }
  hxm::StreamKLayout L0;
  CHECK(!hxm::stream_k_layout(0, 4, 256, &L0) && !hxm::stream_k_layout(10, 0, 256, &L0) &&
            !hxm::stream_k_layout(10, 4, 0, &L0) && !hxm::stream_k_layout(512, 4, 256, &L0) &&
            !hxm::stream_k_layout(10, 4, 256, nullptr) &&
            !hxm::stream_k_layout(INT64_MAX, 4, 256, &L0),
        "stream_k_layout refusals");
  CHECK(hxm::stream_k_layout(688, 64, 256, &L0) && L0.dp == 512 && L0.tiles == 176 &&
            L0.xcd == 1 && L0.iters == 44 && L0.maxseg == 3,
        "the benchmark's gate/up layout");

  std::printf("host_logic ok\n");
  return 0;
}
