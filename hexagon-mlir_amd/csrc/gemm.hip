// Host side of the MFMA GEMMs: the compiled-config tables, kernel choice
// (tuned winner, else a default per shape), argument validation, the [K,N]
// weight pack and the extern "C" entry points.  The kernels themselves are
// in gemm_kernel.h, instantiated by gemm_i8.hip, gemm_f16.hip and
// gemm_w8.hip.
#include <algorithm>
#include <cstring>
#include <mutex>
#include <vector>

#include "gemm_kernel.h"

namespace hxm {

// Transpose [K,N] -> [N,K] (the resident weight image).  32x32 element tiles
// through LDS.
template <typename E>
__global__ __launch_bounds__(256) void transpose_kernel(const E* __restrict__ src,
                                                        int64_t lds_, E* __restrict__ dst,
                                                        int64_t ldd, int64_t K,
                                                        int64_t N) {
  __shared__ E tile[32][33];
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int64_t k = k0 + r, n = n0 + tx;
    if (k < K && n < N) tile[r][tx] = src[k * lds_ + n];
  }
  __syncthreads();
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int64_t n = n0 + r, k = k0 + tx;
    if (n < N && k < K) dst[n * ldd + k] = tile[tx][r];
  }
}

// f32 operands of a matmul enter the fp16 MFMA through these packs (the
// reference's hmx_pack_act_f32 / hmx_pack_weight_f32, HMXAPI.h:107-137,
// which quantise in the pack; its host prepack spells the conversion as
// x + 0.0f -- -0 becomes +0 -- then IEEE round to nearest even,
// hmx_weight_prepack.py:196-207).  The images are fp16 with rows of kp
// elements, kp = K rounded up to 8 (16-byte rows for the LDS-DMA); the
// padding columns hold +0, which adds nothing to any sum.
__device__ __forceinline__ _Float16 f32_operand_to_f16(float x) {
  return static_cast<_Float16>(x + 0.0f);
}

// Row-major [rows, cols] f32 (row stride ld) -> [rows, kp] f16.  Each unit
// is 8 output elements (one 16-byte store).
__global__ __launch_bounds__(256) void pack_f32_rows_kernel(const float* __restrict__ src,
                                                            int64_t ld, _Float16* __restrict__ dst,
                                                            int64_t rows, int64_t cols,
                                                            int64_t kp) {
  const int64_t units = rows * (kp / 8);
  for (int64_t u = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; u < units;
       u += static_cast<int64_t>(gridDim.x) * 256) {
    const int64_t r = u / (kp / 8), c0 = (u % (kp / 8)) * 8;
    v8f16 h;
#pragma unroll
    for (int e = 0; e < 8; ++e)
      h[e] = c0 + e < cols ? f32_operand_to_f16(src[r * ld + c0 + e]) : static_cast<_Float16>(0.0f);
    *reinterpret_cast<v8f16*>(dst + r * kp + c0) = h;
  }
}

// [K, N] f32 (row stride ld) -> the [N, kp] f16 image, 32 x 32 tiles through
// LDS; image columns k in [K, kp) are +0.
__global__ __launch_bounds__(256) void pack_f32_kn_kernel(const float* __restrict__ src,
                                                          int64_t ld, _Float16* __restrict__ dst,
                                                          int64_t K, int64_t N, int64_t kp) {
  __shared__ float tile[32][33];
  const int64_t k0 = static_cast<int64_t>(blockIdx.y) * 32;
  const int64_t n0 = static_cast<int64_t>(blockIdx.x) * 32;
  const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int64_t k = k0 + r, n = n0 + tx;
    tile[r][tx] = k < K && n < N ? src[k * ld + n] : 0.0f;
  }
  __syncthreads();
#pragma unroll
  for (int r = ty; r < 32; r += 8) {
    const int64_t n = n0 + r, k = k0 + tx;
    if (n < N && k < kp) dst[n * kp + k] = f32_operand_to_f16(tile[tx][r]);
  }
}

// ------------------------------------------------------------------------
// Host side: the compiled-config table and dispatch.
// ------------------------------------------------------------------------

struct KernelEntry {
  hxm_gemm_config cfg;  // bk in BYTES here; converted per dtype on the way out
  int threads;
};

#define HXM_ENTRY(BM, BN, BKB, ST, WM, WN) KernelEntry{{BM, BN, BKB, WM, WN, ST, 1}, WM * WN * 64}

// Row i holds the configuration of row i of the kI8Fns / kF16Fns tables.
static const KernelEntry kKernels[] = {HXM_GEMM_CONFIG_LIST(HXM_ENTRY)};
constexpr int kNumKernels = sizeof(kKernels) / sizeof(kKernels[0]);

// W8A16 kernels (row i of the kW8Fns tables): cfg.bk in A bytes (bk = BKB/2 f16
// elements on the way out).
static const KernelEntry kW8Kernels[] = {HXM_W8_CONFIG_LIST(HXM_ENTRY)};
constexpr int kNumW8Kernels = sizeof(kW8Kernels) / sizeof(kW8Kernels[0]);

// Entry e of row i of a kernel table compiled in kGemmParts parts: row i
// lives in part i mod kGemmParts, the other parts hold null there.
template <int E>
static gemm_fn part_fn(const gemm_fn (*const parts[kGemmParts])[E], int i, int e) {
  return parts[i % kGemmParts][i][e];
}
static const gemm_fn (*const kI8Parts[kGemmParts])[2] = {kI8Fns_p0, kI8Fns_p1, kI8Fns_p2};
static const gemm_fn (*const kF16Parts[kGemmParts])[2] = {kF16Fns_p0, kF16Fns_p1, kF16Fns_p2};
static const gemm_fn (*const kW8Parts[kGemmParts])[3] = {kW8Fns_p0, kW8Fns_p1, kW8Fns_p2};
static const gemm_fn* const kW8SkParts[kGemmParts] = {kW8SkFns_p0, kW8SkFns_p1, kW8SkFns_p2};

static int elem_bytes(int32_t dt) { return dt == HXM_I8 ? 1 : 2; }

int num_kernels() { return kNumKernels; }
hxm_gemm_config kernel_config(int i, int32_t dt) {
  hxm_gemm_config c = kKernels[i].cfg;
  c.bk /= elem_bytes(dt);
  return c;
}

// K splits an int8 GEMM may take (grid rows along K, exact int32 partials).
static bool valid_split(int32_t s, int32_t dt) {
  return s == 0 || s == 1 || (dt == HXM_I8 && (s == 2 || s == 4 || s == 8 || s == 16));
}

// A config matches when every non-zero field agrees (0 = any).
const KernelEntry* find_kernel(const hxm_gemm_config& c, int32_t dt) {
  for (int i = 0; i < kNumKernels; ++i) {
    const hxm_gemm_config k = kernel_config(i, dt);
    if (k.bm == c.bm && k.bn == c.bn && (c.bk == 0 || c.bk == k.bk) &&
        (c.waves_m == 0 || c.waves_m == k.waves_m) &&
        (c.waves_n == 0 || c.waves_n == k.waves_n) &&
        (c.stages == 0 || c.stages == k.stages) && valid_split(c.split_k, dt))
      return &kKernels[i];
  }
  return nullptr;
}

// Default configuration for a shape (used when no tuned winner is cached):
// the first entry of this preference list whose tile count still gives every
// CU a workgroup, else a small tile (below).
hxm_gemm_config default_config(int64_t M, int64_t N, int32_t dt) {
  // bm, bn, bk bytes, stages.  The two-stage 256x256 tile with 128-byte K
  // stages leads for every dtype (measured at 4096^3: f16 110 us against
  // 112 us for the four-stage 64-byte tile, bf16 98 against 104 us).
  static const int order_i8[][4] = {{256, 256, 128, 2}, {256, 256, 64, 4}, {128, 128, 128, 2}};
  static const int order_f16[][4] = {{256, 256, 128, 2}, {256, 256, 64, 4}, {128, 128, 128, 2}};
  for (auto& o : (dt == HXM_I8 ? order_i8 : order_f16)) {
    const int64_t tiles = ((M + o[0] - 1) / o[0]) * ((N + o[1] - 1) / o[1]);
    if (tiles >= 256) {
      hxm_gemm_config c{o[0], o[1], o[2] / elem_bytes(dt), 0, 0, o[3], 1};
      if (find_kernel(c, dt)) return kernel_config(static_cast<int>(find_kernel(c, dt) - kKernels), dt);
    }
  }
  // Small C: 64x64 tiles, or 32x32 tiles (one wave each) where 64x64 would
  // occupy fewer than a quarter of the CUs: more workgroups share the
  // latency of the K walk (f16 256^3, one box, back-to-back launches in a
  // HIP graph: 3.11 us against 3.43 us).
  const int64_t tiles64 = ((M + 63) / 64) * ((N + 63) / 64);
  hxm_gemm_config c{64, 64, 0, 0, 0, 0, 1};
  if (tiles64 < 64) c = hxm_gemm_config{32, 32, 0, 0, 0, 0, 1};
  return kernel_config(static_cast<int>(find_kernel(c, dt) - kKernels), dt);
}

// Tuned winners, filled by hxm_tune_gemm (search.cpp).
bool lookup_tuned(int32_t op, int64_t M, int64_t N, int64_t K, hxm_gemm_config* out);

hxm_status launch_gemm(const KernelEntry& e, int32_t ab_dtype, int epi,
                       const GemmArgs& g, hipStream_t stream) {
  const int bm = e.cfg.bm, bn = e.cfg.bn;
  const int64_t tiles = static_cast<int64_t>((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
  const int i = static_cast<int>(&e - kKernels);
  hxm_status st = check_grid("gemm", tiles, e.threads, g.split);
  if (st != HXM_OK) return st;
  gemm_fn fn = nullptr;
  if (ab_dtype == HXM_I8)
    fn = part_fn(kI8Parts, i, epi == kEpiDequant ? 1 : 0);
  else
    fn = part_fn(kF16Parts, i, ab_dtype == HXM_F16 ? 0 : 1);
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(tiles), static_cast<unsigned>(g.split)),
                     dim3(e.threads), 0, stream, g);
  return check_launch("gemm kernel");
}

// Split-K read-out: sums the S int32 partial planes ([S, M, N], plane order,
// exact in int32 like the unsplit accumulator) and applies the int8 GEMM's
// epilogue: int32 out (C += sum when accumulating) or the dequant
// f16(((float)sum * rs[m]) * cs[n]), each product rounded to fp32.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(
    const int32_t* __restrict__ planes, int S, int64_t plane, int N, void* C, int64_t ldc,
    int dequant, int accumulate, const float* __restrict__ rs, const float* __restrict__ cs) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= plane) return;
  const int64_t m = i / N, n = i % N;
  uint32_t s = 0;
  for (int z = 0; z < S; ++z) s += static_cast<uint32_t>(planes[z * plane + i]);
  if (dequant) {
    float p = (static_cast<float>(static_cast<int32_t>(s)) * rs[m]) * cs[n];
    asm volatile("" : "+v"(p));  // one rounding to fp32, then one to f16
    static_cast<_Float16*>(C)[m * ldc + n] = static_cast<_Float16>(p);
  } else {
    int32_t* c = static_cast<int32_t*>(C) + m * ldc + n;
    *c = static_cast<int32_t>(accumulate ? static_cast<uint32_t>(*c) + s : s);
  }
}

namespace {
// Row stride (elements) of the per-call [N, K] image of a [K, N] B: rows
// start on 128-byte lines, so each row's K chunk of a stage is whole lines,
// when 256 such rows still lie within 2 GiB (else rows of K elements).
// Measured with an int8 [N, K] image at 4000^3 + dequant (one box): row
// stride 4000 bytes 59.5 us, 4096 bytes 56.7 us.
int64_t kn_image_ld(int64_t K, int64_t eb) {
  const int64_t padded = ((K * eb + 127) / 128) * 128 / eb;
  return tile_rows_addressable(padded * eb, K * eb) ? padded : K;
}

// kTileRowsMax (host_logic.h) bounds the tallest compiled tile.
#define HXM_TILE_EDGE(BM, BN, BKB, ST, WM, WN) ((BM) > (BN) ? (BM) : (BN))
constexpr int kTileEdges[] = {HXM_GEMM_CONFIG_LIST(HXM_TILE_EDGE),
                              HXM_W8_CONFIG_LIST(HXM_TILE_EDGE)};
#undef HXM_TILE_EDGE
constexpr bool tile_edges_fit() {
  for (int e : kTileEdges)
    if (e > kTileRowsMax) return false;
  return true;
}
static_assert(tile_edges_fit(), "a compiled tile is taller than kTileRowsMax");


hxm_status validate_common(const char* op, const void* A, int64_t lda,
                           const void* B, int64_t ldb, int32_t b_layout,
                           const void* C, int64_t ldc, int64_t M, int64_t N,
                           int64_t K, int64_t eb) {
  if (M < 0 || N < 0 || K < 0)
    return fail(HXM_INVALID_ARG, "invalid-argument: %s negative extent", op);
  if (b_layout != HXM_B_KN && b_layout != HXM_B_NK)
    return fail(HXM_INVALID_ARG, "invalid-argument: %s b_layout=%d", op, b_layout);
  if (M > 0 && N > 0 && (!C || (K > 0 && (!A || !B))))
    return fail(HXM_INVALID_ARG, "invalid-argument: %s null operand", op);
  if (lda < K || ldc < N ||
      (b_layout == HXM_B_NK ? ldb < K : ldb < N))
    return fail(HXM_INVALID_ARG, "invalid-argument: %s leading dimension too small",
                op);
  if (!extents_fit(M, N, K, eb))
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: %s extent beyond 2^30", op);
  // A [K,N] B is packed into an [N,K] image (rows of kn_image_ld elements).
  const int64_t ldb_image = b_layout == HXM_B_NK ? ldb : kn_image_ld(K, eb);
  if (K > 0 && (!tile_rows_addressable(lda * eb, K * eb) ||
                !tile_rows_addressable(ldb_image * eb, K * eb)))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: %s needs %lld rows of A and of the [N,K] B image within "
                "2 GiB (lda=%lld, ldb=%lld)",
                op, (long long)kTileRowsMax, (long long)lda, (long long)ldb_image);
  // The MFMA kernels stream 16-byte K chunks of A and of the [N,K] image;
  // a [K,N] B is first packed by the library, so only its image is aligned.
  const bool b_nk = b_layout == HXM_B_NK;
  if ((K * eb) % 16 ||
      (K > 0 && ((lda * eb) % 16 || !aligned16(A) ||
                 (b_nk && ((ldb * eb) % 16 || !aligned16(B))))))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: %s needs K and lda (and ldb of a packed B) in "
                "16-byte multiples and 16-byte aligned A (and packed B) (K=%lld)",
                op, (long long)K);
  return HXM_OK;
}

// Resolves the B operand to an [N,K] image: HXM_B_NK is used as given,
// HXM_B_KN is packed into the stream's workspace first.
hxm_status resolve_b(const void* B, int64_t ldb, int32_t b_layout, int64_t K,
                     int64_t N, int64_t eb, hipStream_t stream,
                     const uint8_t** b_out, int64_t* ldb_bytes_out) {
  if (b_layout == HXM_B_NK) {
    *b_out = static_cast<const uint8_t*>(B);
    *ldb_bytes_out = ldb * eb;
    return HXM_OK;
  }
  hxm_status st = check_grid("weight pack", (N + 31) / 32, 256, (K + 31) / 32);
  if (st != HXM_OK) return st;
  void* ws = nullptr;
  const int64_t ldo = kn_image_ld(K, eb);
  if ((st = stream_workspace(stream, static_cast<size_t>(N * ldo * eb), &ws)) != HXM_OK)
    return st;
  const dim3 grid(static_cast<unsigned>((N + 31) / 32), static_cast<unsigned>((K + 31) / 32));
  if (eb == 1)
    transpose_kernel<uint8_t><<<grid, 256, 0, stream>>>(
        static_cast<const uint8_t*>(B), ldb, static_cast<uint8_t*>(ws), ldo, K, N);
  else
    transpose_kernel<uint16_t><<<grid, 256, 0, stream>>>(
        static_cast<const uint16_t*>(B), ldb, static_cast<uint16_t*>(ws), ldo, K, N);
  if ((st = check_launch("weight pack")) != HXM_OK) return st;
  *b_out = static_cast<const uint8_t*>(ws);
  *ldb_bytes_out = ldo * eb;
  return HXM_OK;
}

// LDS of one compiled kernel (its stage buffers and scale block, as
// gemm_kernel declares them).
int64_t kernel_lds_bytes(const KernelEntry& e, bool b_int8, bool dequant) {
  const int64_t bkb = e.cfg.bk;  // A bytes per stage row
  const int64_t sb = e.cfg.bm * bkb + e.cfg.bn * (b_int8 ? bkb / 2 : bkb);
  const int64_t qr = dequant ? (e.cfg.bm + 63) / 64 : 0;
  const int64_t qc = (dequant || b_int8) ? (e.cfg.bn + 63) / 64 : 0;
  const int st = e.cfg.stages;
  return 2 * sb + (st > 2 ? sb : 1024) + (st > 3 ? sb : 1024) +
         ((qr + qc) > 0 ? (qr + qc) * 64 * 4 : 16);
}

// Why a caller's config has no compiled kernel: the first rule of the
// legality lattice it breaks (wildcard fields filled the way the compiled
// configs fill them), else "no-kernel".
int32_t explain_config(hxm_gemm_config c, int64_t a_bytes, int64_t b_bytes) {
  if (!c.bk) c.bk = static_cast<int32_t>(128 / a_bytes);
  if (!c.waves_m) c.waves_m = 2;
  if (!c.waves_n) c.waves_n = 2;
  if (!c.stages) c.stages = 2;
  const int32_t r = gpu_lattice(c, a_bytes, b_bytes, 0);
  return r == HXM_REASON_OK ? HXM_REASON_NO_KERNEL : r;
}

// Records a refusal in *p and as the thread's reason.
hxm_status refuse(hxm_plan* p, hxm_status st, int32_t reason, const char* detail) {
  p->plan = HXM_PLAN_REFUSED;
  p->reason = reason;
  return fail(st, "%s: %s", hxm_reason_string(reason), detail);
}

}  // namespace

thread_local hxm_plan g_last_plan{};
thread_local bool g_has_last_plan = false;

// Chooses and explains the kernel of one matmul-family call (the manifest's
// plan/reason record): the caller's config, else the tuned winner for
// (op, M, N, K), else the shape's default; the K split it launches, its LDS,
// the library workspace it needs and its grid.  `table` is the kernel table
// dtype (HXM_I8 / HXM_F16 / HXM_BF16), `op` the tuning-cache key and the
// plan's op, `epi` the epilogue, `extra_ws` workspace the caller adds (the
// f32 operand images).  The plan is also kept as this thread's last plan.
hxm_status plan_gemm(int32_t op, int32_t table, int epi, int32_t b_layout, int64_t M,
                     int64_t N, int64_t K, const hxm_gemm_config* cfg, int64_t extra_ws,
                     hxm_plan* p, const KernelEntry** entry) {
  *p = hxm_plan{};
  p->op = op;
  p->m = M, p->n = N, p->k = K;
  p->plan = HXM_PLAN_REFUSED;
  p->k_slices = 1;
  g_last_plan = *p;
  g_has_last_plan = true;
  const int64_t eb = dtype_bytes(table);
  char why[192];
  hxm_gemm_config c;
  if (cfg && cfg->bm) {
    c = *cfg;
    p->source = HXM_SOURCE_CALLER;
  } else if (lookup_tuned(op == HXM_F32 ? HXM_F16 : op, M, N, K, &c)) {
    p->source = HXM_SOURCE_TUNED;
  } else {
    c = epi == kEpiFloat && small_gemm_fits(M, N, K, table) ? small_gemm_config()
                                                             : default_config(M, N, table);
    p->source = HXM_SOURCE_DEFAULT;
  }
  p->config = c;
  if (is_small_gemm_config(c)) {  // the direct-load small-output kernel
    hxm_status st = HXM_OK;
    if (epi != kEpiFloat || !small_gemm_fits(M, N, K, table)) {
      snprintf(why, sizeof(why),
               "the direct small-output kernel takes f16/bf16 operands, at most %lld 16x16 "
               "output tiles and 0 < K <= %lld",
               (long long)kSmallTilesMax, (long long)kSmallKMax);
      st = refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_NO_KERNEL, why);
    } else {
      p->config = small_gemm_config();
      p->threads = 64;
      p->tiles = ((M + 15) / 16) * ((N + 15) / 16);
      p->lds_bytes = 0;
      p->workspace_bytes = extra_ws + (b_layout == HXM_B_KN ? N * kn_image_ld(K, eb) * eb : 0);
      p->k_slices = 1;
      // The plan's classes use the 32-wide MFMA edge for every kernel (the
      // reference's queryContraction tile edge), also where this kernel's
      // own tiles are 16 wide.
      const bool full = M % 32 == 0 && N % 32 == 0 && K % 32 == 0;
      p->plan = full ? HXM_PLAN_MFMA_FULL : HXM_PLAN_MFMA_TAIL;
      p->reason = full ? HXM_REASON_SELECTED_ALIGNED : HXM_REASON_SELECTED_TAIL;
    }
    g_last_plan = *p;
    if (entry) *entry = nullptr;
    return st;
  }
  hxm_status st = HXM_OK;
  const KernelEntry* e = find_kernel(c, table);
  if (!e) {
    snprintf(why, sizeof(why), "no compiled GEMM for bm=%d bn=%d bk=%d waves=%dx%d stages=%d",
             c.bm, c.bn, c.bk, c.waves_m, c.waves_n, c.stages);
    st = refuse(p, HXM_UNSUPPORTED_SHAPE, explain_config(c, eb, eb), why);
  } else if (c.split_k > 1 && table != HXM_I8) {
    st = refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_NO_KERNEL,
                "split-K is compiled for int8 only");
  }
  if (st == HXM_OK) {
    const int32_t split = c.split_k > 1 ? c.split_k : 1;
    p->config = kernel_config(static_cast<int>(e - kKernels), table);
    p->config.split_k = split;
    p->threads = e->threads;
    p->tiles = ((M + e->cfg.bm - 1) / e->cfg.bm) * ((N + e->cfg.bn - 1) / e->cfg.bn);
    p->lds_bytes = kernel_lds_bytes(*e, false, epi == kEpiDequant);
    p->workspace_bytes =
        extra_ws + (b_layout == HXM_B_KN && K > 0 ? N * kn_image_ld(K, eb) * eb : 0);
    p->k_slices = k_slices(K * eb, e->cfg.bk, split);
    const bool planes_fit =
        p->k_slices <= 1 || split_planes_fit(p->k_slices, M, N, kSplitKPlaneBytesMax);
    if (p->k_slices > 1 && planes_fit) p->workspace_bytes += p->k_slices * M * N * 4;
    if (!planes_fit) {
      snprintf(why, sizeof(why),
               "split_k=%d needs %d int32 partial planes of %lld x %lld, above the %lld-byte "
               "limit",
               p->k_slices, p->k_slices, (long long)M, (long long)N,
               (long long)kSplitKPlaneBytesMax);
      st = refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_WORKSPACE_BUDGET, why);
    } else if (!grid_fits(p->tiles, e->threads, p->k_slices)) {
      snprintf(why, sizeof(why), "%lld x %d workgroups of %d threads exceed the launch limit",
               (long long)p->tiles, p->k_slices, e->threads);
      st = refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_TILE_ALIGNMENT, why);
    } else {
      const bool full = M % 32 == 0 && N % 32 == 0 && K % 32 == 0;
      p->plan = full ? HXM_PLAN_MFMA_FULL : HXM_PLAN_MFMA_TAIL;
      p->reason = full ? HXM_REASON_SELECTED_ALIGNED : HXM_REASON_SELECTED_TAIL;
    }
  }
  g_last_plan = *p;
  if (entry) *entry = st == HXM_OK ? e : nullptr;
  return st;
}

// Shared by the entry points and the tuner.  planes / planes_cap: where a
// K split keeps its int32 partial planes; nullptr takes the stream's
// library-owned workspace (grown on demand).
static hxm_status run_gemm_with(int32_t op, int32_t ab_dtype, int epi, const void* A,
                                int64_t lda, const void* B, int64_t ldb, int32_t b_layout,
                                void* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                                int32_t out_dtype, int32_t accumulate, const float* rs,
                                const float* cs, const hxm_gemm_config* cfg,
                                hipStream_t stream, void* planes, size_t planes_cap,
                                int64_t extra_ws = 0) {
  const int64_t eb = dtype_bytes(ab_dtype);
  const KernelEntry* e = nullptr;
  hxm_plan plan;
  hxm_status st = plan_gemm(op, ab_dtype, epi, b_layout, M, N, K, cfg, extra_ws, &plan, &e);
  if (st != HXM_OK) return st;
  // Caller-provided planes (the allocation-free entry's static array): the
  // call takes no library workspace, and its plan record says so.
  if (planes) g_last_plan.workspace_bytes = plan.workspace_bytes = 0;
  const int split = plan.config.split_k;
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (M == 0 || N == 0) return ok();
  const uint8_t* bk = nullptr;
  int64_t ldb_bytes = 0;
  if (K > 0 && (st = resolve_b(B, ldb, b_layout, K, N, eb, stream, &bk, &ldb_bytes)) != HXM_OK)
    return st;
  if (!e) {  // the plan chose the direct-load small-output kernel
    if ((st = launch_small_gemm(ab_dtype, A, lda, bk, ldb_bytes, C, ldc, M, N, K, out_dtype,
                                accumulate, stream)) != HXM_OK)
      return st;
    return ok();
  }
  GemmArgs g;
  g.A = static_cast<const uint8_t*>(A);
  g.B = bk;
  g.C = C;
  g.lda_bytes = lda * eb;
  g.ldb_bytes = ldb_bytes;
  g.ldc = ldc;
  g.M = static_cast<int>(M);
  g.N = static_cast<int>(N);
  g.K_bytes = static_cast<int>(K * eb);
  g.accumulate = accumulate;
  g.out_dtype = out_dtype;
  g.row_scale = rs;
  g.col_scale = cs;
  g.group_m = 4;
  g.n_out = 0;
  g.residual = nullptr;
  g.ldr = 0;
  g.res_vec8 = 0;
  {
    const int64_t ob = dtype_bytes(out_dtype);
    g.vec_store = (reinterpret_cast<uintptr_t>(C) % (4 * ob) == 0) && ((ldc * ob) % (4 * ob) == 0);
    g.vec8_store = (reinterpret_cast<uintptr_t>(C) % 16 == 0) && ((ldc * ob) % 16 == 0);
  }
  if (plan.k_slices > 1) {
    // K in S slices of whole stages (the plan's split); workgroup row z
    // writes int32 plane z of an [S, M, N] buffer, then one pass sums the
    // planes.
    const int64_t bkb = e->cfg.bk;  // stage bytes
    const int64_t kslice = ((K * eb + bkb - 1) / bkb + split - 1) / split * bkb;
    const int S = plan.k_slices;
    {
      const int64_t plane = M * N;
      void* ws = planes;
      if (planes && static_cast<size_t>(S * plane * 4) > planes_cap) {
        g_last_plan.plan = HXM_PLAN_REFUSED;
        g_last_plan.reason = HXM_REASON_WORKSPACE_BUDGET;
        return fail(HXM_UNSUPPORTED_SHAPE,
                    "workspace-budget: split_k=%d needs %lld bytes of int32 partial planes, "
                    "above the %zu-byte static scratch",
                    S, (long long)(S * plane * 4), planes_cap);
      }
      if (!planes &&
          (st = stream_workspace(stream, static_cast<size_t>(S * plane * 4), &ws, kWsSplitK)) !=
              HXM_OK)
        return st;
      GemmArgs p = g;
      p.C = ws;
      p.ldc = N;
      p.out_dtype = HXM_I32;
      p.accumulate = 0;
      p.row_scale = p.col_scale = nullptr;
      p.vec_store = (N * 4) % 16 == 0;
      p.vec8_store = (N * 4) % 16 == 0;
      p.split = S;
      p.kslice_bytes = static_cast<int>(kslice);
      p.plane_elems = plane;
      if ((st = launch_gemm(*e, ab_dtype, kEpiI32, p, stream)) != HXM_OK) return st;
      const int64_t blocks = (plane + 255) / 256;
      if ((st = check_grid("splitk_reduce", blocks, 256)) != HXM_OK) return st;
      splitk_reduce_kernel<<<static_cast<unsigned>(blocks), 256, 0, stream>>>(
          static_cast<const int32_t*>(ws), S, plane, static_cast<int>(N), C, ldc,
          epi == kEpiDequant, accumulate, rs, cs);
      return check_launch("splitk_reduce");
    }
  }
  if ((st = launch_gemm(*e, ab_dtype, epi, g, stream)) != HXM_OK) return st;
  return ok();
}

hxm_status run_gemm(int32_t op, int32_t ab_dtype, int epi, const void* A,
                    int64_t lda, const void* B, int64_t ldb, int32_t b_layout,
                    void* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                    int32_t out_dtype, int32_t accumulate, const float* rs,
                    const float* cs, const hxm_gemm_config* cfg,
                    hipStream_t stream) {
  return run_gemm_with(op, ab_dtype, epi, A, lda, B, ldb, b_layout, C, ldc, M, N, K,
                       out_dtype, accumulate, rs, cs, cfg, stream, nullptr, 0);
}

// ---- the allocation-free int8 GEMM ----
// Its K-split partial planes live in this file-scope device array, one copy
// per device for the life of the process.  In host code `scratch` names a
// host-side stand-in, not device memory: its device address is looked up once
// per device (hipGetSymbolAddress with that device current) and only that
// address is handed to kernels.
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(HXM_NOALLOC_SCRATCH_BYTES);
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
std::vector<void*> g_scratch_ptr;  // device address of `scratch`, per device

// The current device's copy of `scratch` (looked up on the first call on it).
hxm_status scratch_address(void** out) {
  int dev = 0;
  HXM_HIP_TRY(hipGetDevice(&dev));
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (static_cast<int>(g_scratch_ptr.size()) <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    HXM_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return fail(HXM_HIP_ERROR, "hip-error: no device address for the static scratch");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return HXM_OK;
}
}  // namespace

// ---- W8A16 GEMM (f16 x int8 [N, K]) ----

int num_w8_kernels() { return kNumW8Kernels; }
hxm_gemm_config w8_kernel_config(int i) {
  hxm_gemm_config c = kW8Kernels[i].cfg;
  c.bk /= 2;  // f16 elements of K per stage
  return c;
}
bool w8_kernel_has_swiglu(int i) { return part_fn(kW8Parts, i, 1) != nullptr; }
// Entry i has a stream-K form (split_k = HXM_STREAM_K): entry 0, compiled
// in gemm_w8sk.hip, part e holding epilogue e (kEpiW8, kEpiSwiglu, kEpiW8Res).
bool w8_kernel_has_stream_k(int i) { return i == 0; }
static gemm_fn w8_stream_k_fn(int e) { return kW8SkParts[e][e]; }

static const KernelEntry* find_w8_kernel(const hxm_gemm_config& c, bool swiglu) {
  for (int i = 0; i < kNumW8Kernels; ++i) {
    const hxm_gemm_config k = w8_kernel_config(i);
    if (k.bm == c.bm && k.bn == c.bn && (c.bk == 0 || c.bk == k.bk) &&
        (c.waves_m == 0 || c.waves_m == k.waves_m) &&
        (c.waves_n == 0 || c.waves_n == k.waves_n) &&
        (c.stages == 0 || c.stages == k.stages) &&
        (c.split_k == 0 || c.split_k == 1 ||
         (c.split_k == HXM_STREAM_K && w8_kernel_has_stream_k(i))) &&
        (!swiglu || w8_kernel_has_swiglu(i)))
      return &kW8Kernels[i];
  }
  return nullptr;
}

// The first table entry (largest tiles first) that still gives every CU a
// workgroup, else the entry with the most tiles.
hxm_gemm_config default_w8_config(int64_t M, int64_t N, bool swiglu) {
  int best = -1;
  int64_t best_tiles = -1;
  for (int i = 0; i < kNumW8Kernels; ++i) {
    if (swiglu && !w8_kernel_has_swiglu(i)) continue;
    const hxm_gemm_config k = w8_kernel_config(i);
    const int64_t tiles = ((M + k.bm - 1) / k.bm) * ((N + k.bn - 1) / k.bn);
    if (tiles >= 256) return k;
    if (tiles > best_tiles) best = i, best_tiles = tiles;
  }
  return w8_kernel_config(best);
}

// The SwiGLU weight image: rows [128c, 128c+64) are gate channels
// [64c, 64c+64), rows [128c+64, 128c+128) the same up channels; channels
// >= I are zero rows with zero scale.  Each weight is stored in offset
// binary (byte = w ^ 0x80, w + 128 unsigned), the form the GEMM's in-register
// f16 conversion takes without a sign flip.  One workgroup per image row.
__global__ __launch_bounds__(256) void swiglu_pack_kernel(
    const int8_t* __restrict__ wg, const int8_t* __restrict__ wu, int64_t ldw,
    const float* __restrict__ sg, const float* __restrict__ su, int64_t I, int64_t K,
    int8_t* __restrict__ out, float* __restrict__ out_scale) {
  const int64_t r = blockIdx.x;
  const int64_t ch = (r / 128) * 64 + (r % 64);
  const bool up = (r % 128) >= 64;
  const int8_t* src = up ? wu : wg;
  int8_t* dst = out + r * K;
  for (int64_t k = threadIdx.x; k < K; k += blockDim.x)
    dst[k] = static_cast<int8_t>((ch < I ? static_cast<uint8_t>(src[ch * ldw + k]) : 0) ^ 0x80);
  if (threadIdx.x == 0)
    out_scale[r] = ch < I ? (up ? su : sg)[ch] : 0.0f;
}

// Stream-K buffer of a W8A16 launch: a block of arrival counters, one per
// stream-K tile (a launch has fewer stream-K tiles than the device has CUs),
// then sk.tiles * sk.maxseg fp32 partial tiles of BM x BN.  The counter
// block has the same place and size for every shape: it is zeroed whenever
// the buffer is allocated, and every launch leaves the counters it used at
// zero, so a later shape with more stream-K tiles never finds a counter in
// bytes that an earlier shape used for partial tiles.
constexpr int64_t kStreamKCounterBytes = 4096;
static int64_t stream_k_bytes(const KernelEntry& e, const StreamKLayout& sk) {
  return kStreamKCounterBytes +
         static_cast<int64_t>(sk.tiles) * sk.maxseg * e.cfg.bm * e.cfg.bn * 4;
}

// plan_gemm for the W8A16 GEMMs (f16 A, int8 [N, K] B): N is the B rows
// (the SwiGLU image's), n_out the output columns.
hxm_status plan_gemm_w8(int32_t op, bool sw, int64_t M, int64_t N, int64_t n_out, int64_t K,
                        const hxm_gemm_config* cfg, hxm_plan* p, const KernelEntry** entry) {
  *p = hxm_plan{};
  p->op = op;
  p->m = M, p->n = n_out, p->k = K;
  p->plan = HXM_PLAN_REFUSED;
  p->k_slices = 1;
  char why[192];
  hxm_gemm_config c;
  if (cfg && cfg->bm) {
    c = *cfg;
    p->source = HXM_SOURCE_CALLER;
  } else if (lookup_tuned(op, M, sw ? n_out : N, K, &c)) {
    p->source = HXM_SOURCE_TUNED;
  } else {
    c = default_w8_config(M, N, sw);
    p->source = HXM_SOURCE_DEFAULT;
  }
  p->config = c;
  hxm_status st = HXM_OK;
  const KernelEntry* e = find_w8_kernel(c, sw);
  if (!e) {
    const bool plain = find_w8_kernel(c, false) != nullptr;
    snprintf(why, sizeof(why), "no compiled W8A16 GEMM%s for bm=%d bn=%d bk=%d waves=%dx%d",
             sw ? " with the SwiGLU epilogue (its wave tile is 128 wide)" : "", c.bm, c.bn,
             c.bk, c.waves_m, c.waves_n);
    st = refuse(p, HXM_UNSUPPORTED_SHAPE,
                plain ? HXM_REASON_NO_KERNEL : explain_config(c, 2, 1), why);
  } else {
    p->config = w8_kernel_config(static_cast<int>(e - kW8Kernels));
    p->threads = e->threads;
    p->tiles = ((M + e->cfg.bm - 1) / e->cfg.bm) * ((N + e->cfg.bn - 1) / e->cfg.bn);
    p->lds_bytes = kernel_lds_bytes(*e, true, false);
    int64_t groups = p->tiles, sk_tiles = 0;
    if (c.split_k == HXM_STREAM_K) {
      // Stream-K when the tiles leave a partial round; whole rounds run as
      // split_k = 1.  The plan records the mode, the partial-tile slots (as
      // k_slices: the most workgroups one tile is cut over) and the buffer.
      StreamKLayout sk;
      const int64_t KT = (K * 2 + e->cfg.bk - 1) / e->cfg.bk;
      if (K > 0 && stream_k_layout(p->tiles, KT, device_cu_count(), &sk)) {
        p->config.split_k = HXM_STREAM_K;
        p->k_slices = sk.maxseg;
        p->workspace_bytes = stream_k_bytes(*e, sk);
        groups = sk.dp + sk.groups;
        sk_tiles = sk.tiles;
      }
    }
    if (p->workspace_bytes > kSplitKPlaneBytesMax) {
      snprintf(why, sizeof(why),
               "stream-K needs %lld bytes of fp32 partial tiles, above the %lld-byte limit",
               (long long)p->workspace_bytes, (long long)kSplitKPlaneBytesMax);
      st = refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_WORKSPACE_BUDGET, why);
    } else if (sk_tiles > kStreamKCounterBytes / 4) {
      snprintf(why, sizeof(why), "stream-K with %lld partial-round tiles needs more than %lld "
               "arrival counters", (long long)sk_tiles, (long long)(kStreamKCounterBytes / 4));
      st = refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_WORKSPACE_BUDGET, why);
    } else if (!grid_fits(groups, e->threads)) {
      snprintf(why, sizeof(why), "%lld workgroups of %d threads exceed the launch limit",
               (long long)groups, e->threads);
      st = refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_TILE_ALIGNMENT, why);
    } else {
      const bool full = M % 32 == 0 && n_out % 32 == 0 && K % 32 == 0;
      p->plan = full ? HXM_PLAN_MFMA_FULL : HXM_PLAN_MFMA_TAIL;
      p->reason = full ? HXM_REASON_SELECTED_ALIGNED : HXM_REASON_SELECTED_TAIL;
    }
  }
  g_last_plan = *p;
  g_has_last_plan = true;
  if (entry) *entry = st == HXM_OK ? e : nullptr;
  return st;
}

hxm_status run_gemm_w8(int epi, int32_t op, const void* x, int64_t ldx, const int8_t* W,
                       int64_t ldw, const float* scale, void* C, int64_t ldc, int64_t M,
                       int64_t N, int64_t K, int64_t n_out, const hxm_gemm_config* cfg,
                       hipStream_t stream, const void* residual = nullptr, int64_t ldr = 0) {
  const bool sw = epi == kEpiSwiglu;
  const KernelEntry* e = nullptr;
  hxm_plan plan;
  hxm_status st = plan_gemm_w8(op, sw, M, N, n_out, K, cfg, &plan, &e);
  if (st != HXM_OK) return st;
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (M == 0 || N == 0) return ok();
  GemmArgs g;
  g.A = static_cast<const uint8_t*>(x);
  g.B = reinterpret_cast<const uint8_t*>(W);
  g.C = C;
  g.lda_bytes = ldx * 2;
  g.ldb_bytes = ldw;
  g.ldc = ldc;
  g.M = static_cast<int>(M);
  g.N = static_cast<int>(N);
  g.K_bytes = static_cast<int>(K * 2);
  g.accumulate = 0;
  g.out_dtype = HXM_F16;
  g.row_scale = nullptr;
  g.col_scale = scale;
  g.group_m = 4;
  g.n_out = static_cast<int>(n_out);
  g.residual = static_cast<const _Float16*>(residual);
  g.ldr = ldr;
  g.res_vec8 = residual && (reinterpret_cast<uintptr_t>(residual) % 16 == 0) && ((ldr * 2) % 16 == 0);
  g.vec_store = (reinterpret_cast<uintptr_t>(C) % 8 == 0) && ((ldc * 2) % 8 == 0);
  g.vec8_store = (reinterpret_cast<uintptr_t>(C) % 16 == 0) && ((ldc * 2) % 16 == 0);
  const int wi = static_cast<int>(e - kW8Kernels);
  int64_t groups = plan.tiles;
  if (plan.config.split_k == HXM_STREAM_K) {
    StreamKLayout sk;
    const int64_t KT = (K * 2 + e->cfg.bk - 1) / e->cfg.bk;
    if (!stream_k_layout(plan.tiles, KT, device_cu_count(), &sk))
      return fail(HXM_HIP_ERROR, "hip-error: stream-K layout changed between plan and launch");
    void* ws = nullptr;
    bool grown = false;
    if ((st = stream_workspace(stream, static_cast<size_t>(stream_k_bytes(*e, sk)), &ws,
                               kWsStreamK, &grown)) != HXM_OK)
      return st;
    // A new buffer's counter block starts at zero; every launch leaves it
    // there (the last workgroup at a tile resets its counter).  Growth is
    // refused under graph capture, so this fill is never captured.
    if (grown) HXM_HIP_TRY(hipMemsetAsync(ws, 0, static_cast<size_t>(kStreamKCounterBytes), stream));
    g.sk_first = sk.dp;
    g.sk_groups = sk.groups;
    g.sk_tiles = sk.tiles;
    g.sk_iters = sk.iters;
    g.sk_maxseg = sk.maxseg;
    g.sk_xcd = sk.xcd;
    g.sk_count = static_cast<uint32_t*>(ws);
    g.sk_part = reinterpret_cast<float*>(static_cast<char*>(ws) + kStreamKCounterBytes);
    groups = sk.dp + sk.groups;
  }
  const int fe = sw ? 1 : epi == kEpiW8Res ? 2 : 0;
  hipLaunchKernelGGL(plan.config.split_k == HXM_STREAM_K ? w8_stream_k_fn(fe)
                                                          : part_fn(kW8Parts, wi, fe),
                     dim3(static_cast<unsigned>(groups)),
                     dim3(e->threads), 0, stream, g);
  if ((st = check_launch("w8a16 gemm kernel")) != HXM_OK) return st;
  return ok();
}

// Checks shared by the W8A16 entry points.  x [M, K] f16 and W [N, K] int8
// stream 16-byte K chunks: K a multiple of 16, 16-byte aligned rows.
static hxm_status validate_w8(const char* op, const void* x, int64_t ldx, const void* W,
                              int64_t ldw, const void* scale, const void* C, int64_t ldc,
                              int64_t M, int64_t N, int64_t K, int64_t out_cols) {
  if (M < 0 || N < 0 || K < 0)
    return fail(HXM_INVALID_ARG, "invalid-argument: %s negative extent", op);
  if (M > 0 && out_cols > 0 && (!C || !scale || (K > 0 && (!x || !W))))
    return fail(HXM_INVALID_ARG, "invalid-argument: %s null operand", op);
  if (ldx < K || ldw < K || ldc < out_cols)
    return fail(HXM_INVALID_ARG, "invalid-argument: %s leading dimension too small", op);
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K > INT32_MAX / 4)
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: %s extent beyond 2^29", op);
  if (K > 0 && (!tile_rows_addressable(ldx * 2, K * 2) || !tile_rows_addressable(ldw, K)))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: %s needs %lld rows of x and of W within 2 GiB (ldx=%lld, "
                "ldw=%lld)",
                op, (long long)kTileRowsMax, (long long)ldx, (long long)ldw);
  if (K % 16 || (K > 0 && ((ldx * 2) % 16 || ldw % 16 || !aligned16(x) || !aligned16(W))))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: %s needs K, ldw in multiples of 16 and lda in multiples "
                "of 8, with 16-byte aligned x and W (K=%lld)",
                op, (long long)K);
  return HXM_OK;
}

}  // namespace hxm

using namespace hxm;

extern "C" {

hxm_status hxm_plan_matmul(int64_t M, int64_t N, int64_t K, int32_t a_dtype,
                           int32_t b_dtype, int32_t c_dtype, int32_t b_layout,
                           const hxm_gemm_config* cfg, hxm_plan* out) {
  hxm_plan local;
  hxm_plan* p = out ? out : &local;
  *p = hxm_plan{};
  p->op = a_dtype;
  p->m = M, p->n = N, p->k = K;
  p->plan = HXM_PLAN_REFUSED;
  const bool i8 = a_dtype == HXM_I8 && b_dtype == HXM_I8 &&
                  (c_dtype == HXM_I32 || c_dtype == HXM_F16);
  const bool fl = (a_dtype == HXM_F16 || a_dtype == HXM_BF16 || a_dtype == HXM_F32) &&
                  b_dtype == a_dtype &&
                  (c_dtype == HXM_F16 || c_dtype == HXM_BF16 || c_dtype == HXM_F32);
  char why[160];
  if (!i8 && !fl) {
    snprintf(why, sizeof(why), "a=%d b=%d c=%d", a_dtype, b_dtype, c_dtype);
    return refuse(p, HXM_UNSUPPORTED_DTYPE, HXM_REASON_UNSUPPORTED_DTYPE, why);
  }
  if (M <= 0 || N <= 0 || K <= 0 || (b_layout != HXM_B_KN && b_layout != HXM_B_NK))
    return refuse(p, HXM_INVALID_ARG, HXM_REASON_INVALID_ARGUMENT,
                  "extents must be positive and b_layout HXM_B_KN or HXM_B_NK");
  const int32_t table = a_dtype == HXM_F32 ? HXM_F16 : a_dtype;
  const int64_t eb = dtype_bytes(table);
  const int64_t kk = a_dtype == HXM_F32 ? (K + 7) / 8 * 8 : K;  // f32: the padded image
  if ((kk * eb) % 16) {
    snprintf(why, sizeof(why), "K*elem_bytes=%lld is not a multiple of 16", (long long)(K * eb));
    return refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_TILE_ALIGNMENT, why);
  }
  if (!extents_fit(M, N, kk, eb) || !tile_rows_addressable(kk * eb, kk * eb))
    return refuse(p, HXM_UNSUPPORTED_SHAPE, HXM_REASON_TILE_ALIGNMENT,
                  "extents beyond the 32-bit offsets of the kernels");
  const int epi = a_dtype == HXM_I8 ? (c_dtype == HXM_F16 ? kEpiDequant : kEpiI32) : kEpiFloat;
  const int64_t extra = a_dtype == HXM_F32 ? (M * kk * 2 + 255) / 256 * 256 + N * kk * 2 : 0;
  // A query is not a call: the thread's last-call plan stays as it was.
  const hxm_plan saved = g_last_plan;
  const bool had = g_has_last_plan;
  const hxm_status st = plan_gemm(a_dtype, table, epi, a_dtype == HXM_F32 ? HXM_B_NK : b_layout,
                                  M, N, kk, cfg, extra, p, nullptr);
  g_last_plan = saved;
  g_has_last_plan = had;
  p->k = K;
  if (st == HXM_OK) ok();
  return st;
}

int32_t hxm_last_plan(hxm_plan* out) {
  if (!g_has_last_plan) return 0;
  if (out) *out = g_last_plan;
  return 1;
}

hxm_status hxm_query_contraction(int64_t M, int64_t N, int64_t K,
                                 int32_t a_dtype, int32_t b_dtype,
                                 int32_t c_dtype, int32_t* plan_out) {
  hxm_plan p;
  const hxm_status st = hxm_plan_matmul(M, N, K, a_dtype, b_dtype, c_dtype, HXM_B_NK, nullptr, &p);
  if (plan_out) *plan_out = st == HXM_OK ? p.plan : -1;
  return st;
}

static hxm_status matmul_f32(const float* A, int64_t lda, const float* B, int64_t ldb,
                             int32_t b_layout, void* C, int64_t ldc, int64_t M, int64_t N,
                             int64_t K, int32_t c_dtype, int32_t accumulate,
                             const hxm_gemm_config* cfg, hipStream_t stream) {
  if (M < 0 || N < 0 || K < 0)
    return fail(HXM_INVALID_ARG, "invalid-argument: matmul negative extent");
  if (b_layout != HXM_B_KN && b_layout != HXM_B_NK)
    return fail(HXM_INVALID_ARG, "invalid-argument: matmul b_layout=%d", b_layout);
  if (M > 0 && N > 0 && (!C || (K > 0 && (!A || !B))))
    return fail(HXM_INVALID_ARG, "invalid-argument: matmul null operand");
  if (lda < K || ldc < N || (b_layout == HXM_B_NK ? ldb < K : ldb < N))
    return fail(HXM_INVALID_ARG, "invalid-argument: matmul leading dimension too small");
  if ((K > 0 && ((reinterpret_cast<uintptr_t>(A) | reinterpret_cast<uintptr_t>(B)) & 3)))
    return fail(HXM_INVALID_ARG, "invalid-argument: matmul f32 operands must be 4-byte aligned");
  const int64_t kp = (K + 7) / 8 * 8;
  if (!extents_fit(M, N, kp, 2))
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: matmul extent beyond 2^30");
  if (kp > 0 && !tile_rows_addressable(kp * 2, kp * 2))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: matmul needs %lld rows of the fp16 operand images within 2 GiB",
                (long long)kTileRowsMax);
  hxm_status st = HXM_OK;
  const int64_t a_bytes = (M * kp * 2 + 255) / 256 * 256, img_bytes = a_bytes + N * kp * 2;
  hxm_plan plan;
  if ((st = plan_gemm(HXM_F32, HXM_F16, kEpiFloat, HXM_B_NK, M, N, kp, cfg, img_bytes, &plan,
                      nullptr)) != HXM_OK)
    return st;
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (M == 0 || N == 0 || (K == 0 && accumulate)) return ok();
  void* ws = nullptr;
  _Float16 *ai = nullptr, *bi = nullptr;
  if (K > 0) {
    if ((st = stream_workspace(stream, static_cast<size_t>(img_bytes), &ws)) != HXM_OK) return st;
    ai = static_cast<_Float16*>(ws);
    bi = reinterpret_cast<_Float16*>(static_cast<char*>(ws) + a_bytes);
    auto blocks = [](int64_t units) {
      return static_cast<unsigned>(std::min<int64_t>((units + 255) / 256, 65536));
    };
    pack_f32_rows_kernel<<<blocks(M * (kp / 8)), 256, 0, stream>>>(A, lda, ai, M, K, kp);
    if ((st = check_launch("f32 operand pack")) != HXM_OK) return st;
    if (b_layout == HXM_B_NK) {
      pack_f32_rows_kernel<<<blocks(N * (kp / 8)), 256, 0, stream>>>(B, ldb, bi, N, K, kp);
    } else {
      if ((st = check_grid("f32 weight pack", (N + 31) / 32, 256, (kp + 31) / 32)) != HXM_OK)
        return st;
      const dim3 grid(static_cast<unsigned>((N + 31) / 32), static_cast<unsigned>((kp + 31) / 32));
      pack_f32_kn_kernel<<<grid, 256, 0, stream>>>(B, ldb, bi, K, N, kp);
    }
    if ((st = check_launch("f32 operand pack")) != HXM_OK) return st;
  }
  return run_gemm_with(HXM_F32, HXM_F16, kEpiFloat, ai, kp, bi, kp, HXM_B_NK, C, ldc, M, N, kp,
                       c_dtype, accumulate, nullptr, nullptr, cfg, stream, nullptr, 0,
                       img_bytes);
}

hxm_status hxm_matmul(const void* A, int64_t lda, const void* B, int64_t ldb,
                      int32_t b_layout, void* C, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, int32_t ab_dtype, int32_t c_dtype,
                      int32_t accumulate, const hxm_gemm_config* cfg,
                      void* stream) {
  if (ab_dtype != HXM_F16 && ab_dtype != HXM_BF16 && ab_dtype != HXM_F32)
    return fail(HXM_UNSUPPORTED_DTYPE, "unsupported-dtype: matmul A/B dtype %d",
                ab_dtype);
  if (c_dtype != HXM_F16 && c_dtype != HXM_BF16 && c_dtype != HXM_F32)
    return fail(HXM_UNSUPPORTED_DTYPE, "unsupported-dtype: matmul C dtype %d",
                c_dtype);
  if (ab_dtype == HXM_F32)
    return matmul_f32(static_cast<const float*>(A), lda, static_cast<const float*>(B), ldb,
                      b_layout, C, ldc, M, N, K, c_dtype, accumulate, cfg, as_stream(stream));
  hxm_status st = validate_common("matmul", A, lda, B, ldb, b_layout, C, ldc, M,
                                  N, K, 2);
  if (st != HXM_OK) return st;
  if (K == 0) {
    if ((st = require_device(nullptr)) != HXM_OK) return st;
    if (accumulate || M == 0 || N == 0) return ok();
    // C = 0: run the kernel with a zero-length K (every chunk is the zero page).
  }
  return run_gemm(ab_dtype, ab_dtype, kEpiFloat, A, lda, B, ldb, b_layout, C,
                  ldc, M, N, K, c_dtype, accumulate, nullptr, nullptr, cfg,
                  as_stream(stream));
}

hxm_status hxm_gemm_i8(const int8_t* A, int64_t lda, const int8_t* B,
                       int64_t ldb, int32_t b_layout, int32_t* C, int64_t ldc,
                       int64_t M, int64_t N, int64_t K, int32_t accumulate,
                       const hxm_gemm_config* cfg, void* stream) {
  hxm_status st = validate_common("gemm_i8", A, lda, B, ldb, b_layout, C, ldc,
                                  M, N, K, 1);
  if (st != HXM_OK) return st;
  if (K == 0 && accumulate) {
    if ((st = require_device(nullptr)) != HXM_OK) return st;
    return ok();
  }
  return run_gemm(HXM_I8, HXM_I8, kEpiI32, A, lda, B, ldb, b_layout, C, ldc, M,
                  N, K, HXM_I32, accumulate, nullptr, nullptr, cfg,
                  as_stream(stream));
}

hxm_status hxm_gemm_i8_noalloc(const int8_t* A, int64_t lda, const int8_t* B_nk,
                               int64_t ldb, int32_t* C, int64_t ldc, int64_t M, int64_t N,
                               int64_t K, int32_t accumulate, const hxm_gemm_config* cfg,
                               void* stream) {
  hxm_status st = validate_common("gemm_i8_noalloc", A, lda, B_nk, ldb, HXM_B_NK, C, ldc, M,
                                  N, K, 1);
  if (st != HXM_OK) return st;
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (K == 0 && accumulate) return ok();
  void* planes = nullptr;
  if ((st = scratch_address(&planes)) != HXM_OK) return st;
  return run_gemm_with(HXM_I8, HXM_I8, kEpiI32, A, lda, B_nk, ldb, HXM_B_NK, C, ldc, M, N, K,
                       HXM_I32, accumulate, nullptr, nullptr, cfg, as_stream(stream), planes,
                       kNoAllocScratchBytes);
}

hxm_status hxm_gemm_i8_dequant(const int8_t* A, int64_t lda, const int8_t* B,
                               int64_t ldb, int32_t b_layout,
                               const float* row_scale, const float* col_scale,
                               void* C_f16, int64_t ldc, int64_t M, int64_t N,
                               int64_t K, const hxm_gemm_config* cfg,
                               void* stream) {
  hxm_status st = validate_common("gemm_i8_dequant", A, lda, B, ldb, b_layout,
                                  C_f16, ldc, M, N, K, 1);
  if (st != HXM_OK) return st;
  if (M > 0 && N > 0 && (!row_scale || !col_scale))
    return fail(HXM_INVALID_ARG, "invalid-argument: gemm_i8_dequant null scales");
  return run_gemm(HXM_I8, HXM_I8, kEpiDequant, A, lda, B, ldb, b_layout,
                  C_f16, ldc, M, N, K, HXM_F16, 0, row_scale, col_scale, cfg,
                  as_stream(stream));
}

hxm_status hxm_prepack_weight(const void* B, int64_t ldb, void* out,
                              int64_t ldo, int64_t K, int64_t N, int32_t dtype,
                              void* stream) {
  if (dtype != HXM_I8 && dtype != HXM_F16 && dtype != HXM_BF16)
    return fail(HXM_UNSUPPORTED_DTYPE, "unsupported-dtype: prepack dtype %d", dtype);
  if (K < 0 || N < 0 || ldb < N || ldo < K)
    return fail(HXM_INVALID_ARG, "invalid-argument: prepack extents/leading dims");
  if (K > 0 && N > 0 && (!B || !out))
    return fail(HXM_INVALID_ARG, "invalid-argument: prepack null pointer");
  if (K > (int64_t(65535) * 32))
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: prepack K=%lld too large",
                (long long)K);
  hxm_status st = require_device(nullptr);
  if (st != HXM_OK) return st;
  if (K == 0 || N == 0) return ok();
  if ((st = check_grid("prepack", (N + 31) / 32, 256, (K + 31) / 32)) != HXM_OK) return st;
  hipStream_t s = as_stream(stream);
  const dim3 grid(static_cast<unsigned>((N + 31) / 32), static_cast<unsigned>((K + 31) / 32));
  if (dtype == HXM_I8)
    transpose_kernel<uint8_t><<<grid, 256, 0, s>>>(static_cast<const uint8_t*>(B), ldb,
                                                   static_cast<uint8_t*>(out), ldo, K, N);
  else
    transpose_kernel<uint16_t><<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(B), ldb,
                                                    static_cast<uint16_t*>(out), ldo, K, N);
  return check_launch("prepack");
}

hxm_status hxm_gemm_w8a16(const void* x, int64_t ldx, const int8_t* W, int64_t ldw,
                          const float* w_scale, void* y, int64_t ldy, int64_t M, int64_t N,
                          int64_t K, const hxm_gemm_config* cfg, void* stream) {
  hxm_status st = validate_w8("gemm_w8a16", x, ldx, W, ldw, w_scale, y, ldy, M, N, K, N);
  if (st != HXM_OK) return st;
  return run_gemm_w8(kEpiW8, kOpW8, x, ldx, W, ldw, w_scale, y, ldy, M, N, K, N, cfg,
                     as_stream(stream));
}

hxm_status hxm_gemm_w8a16_residual(const void* x, int64_t ldx, const int8_t* W, int64_t ldw,
                                   const float* w_scale, const void* r, int64_t ldr, void* y,
                                   int64_t ldy, int64_t M, int64_t N, int64_t K,
                                   const hxm_gemm_config* cfg, void* stream) {
  hxm_status st =
      validate_w8("gemm_w8a16_residual", x, ldx, W, ldw, w_scale, y, ldy, M, N, K, N);
  if (st != HXM_OK) return st;
  if (M > 0 && N > 0 && !r)
    return fail(HXM_INVALID_ARG, "invalid-argument: gemm_w8a16_residual null residual");
  if (ldr < N)
    return fail(HXM_INVALID_ARG, "invalid-argument: gemm_w8a16_residual ldr=%lld < N=%lld",
                (long long)ldr, (long long)N);
  // r is either y itself (an in-place update: every element is read by the
  // lane that then writes it) or disjoint from y.
  if (M > 0 && N > 0 && r != y) {
    const uintptr_t r0 = reinterpret_cast<uintptr_t>(r), y0 = reinterpret_cast<uintptr_t>(y);
    const uintptr_t r1 = r0 + static_cast<uintptr_t>(((M - 1) * ldr + N) * 2);
    const uintptr_t y1 = y0 + static_cast<uintptr_t>(((M - 1) * ldy + N) * 2);
    if (r0 < y1 && y0 < r1)
      return fail(HXM_INVALID_ARG,
                  "invalid-argument: gemm_w8a16_residual r overlaps y without being y");
  }
  if (r == y && ldr != ldy)
    return fail(HXM_INVALID_ARG,
                "invalid-argument: gemm_w8a16_residual in place needs ldr == ldy");
  return run_gemm_w8(kEpiW8Res, kOpW8, x, ldx, W, ldw, w_scale, y, ldy, M, N, K, N, cfg,
                     as_stream(stream), r, ldr);
}

int64_t hxm_swiglu_packed_rows(int64_t I) { return I < 0 ? -1 : 128 * ((I + 63) / 64); }

hxm_status hxm_swiglu_pack(const int8_t* Wg, const int8_t* Wu, int64_t ldw,
                           const float* gate_scale, const float* up_scale, int64_t I,
                           int64_t K, int8_t* Wgu, float* sgu, void* stream) {
  if (I < 0 || K < 0 || ldw < K)
    return fail(HXM_INVALID_ARG, "invalid-argument: swiglu_pack extents/leading dim");
  if (I > 0 && (!Wgu || !sgu || !gate_scale || !up_scale || (K > 0 && (!Wg || !Wu))))
    return fail(HXM_INVALID_ARG, "invalid-argument: swiglu_pack null pointer");
  if (I > INT32_MAX / 4)
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: swiglu_pack I=%lld too large",
                (long long)I);
  hxm_status st = require_device(nullptr);
  if (st != HXM_OK) return st;
  if (I == 0) return ok();
  const int64_t rows = hxm_swiglu_packed_rows(I);
  if ((st = check_grid("swiglu pack", rows, 256)) != HXM_OK) return st;
  swiglu_pack_kernel<<<static_cast<unsigned>(rows), 256, 0, as_stream(stream)>>>(
      Wg, Wu, ldw, gate_scale, up_scale, I, K, Wgu, sgu);
  return check_launch("swiglu pack");
}

hxm_status hxm_gemm_w8a16_swiglu(const void* x, int64_t ldx, const int8_t* Wgu,
                                 const float* sgu, void* h, int64_t ldh, int64_t M,
                                 int64_t I, int64_t K, const hxm_gemm_config* cfg,
                                 void* stream) {
  if (I < 0) return fail(HXM_INVALID_ARG, "invalid-argument: gemm_w8a16_swiglu I < 0");
  const int64_t N = hxm_swiglu_packed_rows(I);
  hxm_status st = validate_w8("gemm_w8a16_swiglu", x, ldx, Wgu, K, sgu, h, ldh, M, N, K, I);
  if (st != HXM_OK) return st;
  return run_gemm_w8(kEpiSwiglu, kOpSwiglu, x, ldx, Wgu, K, sgu, h, ldh, M, N, K, I, cfg,
                     as_stream(stream));
}

}  // extern "C"
