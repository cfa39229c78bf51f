// MFMA GEMMs on gfx950: int8 x int8 -> int32 (exact) and f16/bf16 -> fp32.
//
// Reference path: linalg.matmul lowered by matmul-to-hmx -> hmx-partition ->
// weight-resident (qcom_hexagon_backend/lib/Dialect/Hmx/Transforms/
// HmxPartitionPass.cpp:783-864: for m-tiles { pack A row-tile; for n-tiles
// { clear acc; K batches of mma; read-out } }, weights resident across m), and
// the leaves hmx_mma_f16 / hmx_acc_store_f16 (bin/runtime/hmx/src/HMXAPI.c:36-55).
//
// GPU form.  C[M,N] = A[M,K] . B^T where B is held as the resident [N,K]
// image (K contiguous), so both operands stream K-contiguous 16-byte chunks.
//   * workgroup tile BM x BN, K staged 128 BYTES at a time (128 int8 or 64
//     f16), two LDS stages: stage s+1 is fetched by LDS-DMA
//     (global_load_lds_dwordx4, no VGPR round trip) while stage s feeds MFMA;
//   * LDS rows are 128 B with 16-byte chunks XOR-swizzled by
//     (row % 8) ^ ((row / 8) % 2), so the 16 lanes of a ds_read_b128 phase
//     hit distinct banks for both 32- and 64-bank LDS;
//   * each wave owns a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks
//     (v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_{f16,bf16}; both consume
//     32 bytes of K per row per instruction, 16 per lane);
//   * the tile order is XCD-aware: workgroups are dispatched round-robin over
//     the 8 XCDs, so consecutive tile ids are remapped onto one XCD and walked
//     in groups of 4 tile-rows, keeping each XCD's A rows and B columns in its
//     own L2;
//   * epilogues write int32 (optionally += C), fp32->{f16,bf16,f32}
//     (optionally += C, one rounding), or the int8 dequant
//     f16(((float)acc * row_scale) * col_scale).
// Edge tiles: rows beyond M / N and K chunks beyond K are fetched from a
// zero page, so any M, N and any K that is a multiple of 16 bytes works.
#include <cstring>
#include <mutex>
#include <vector>

#include "device_util.h"
#include "gemm_configs.h"
#include "hxm_internal.h"

namespace hxm {

__device__ __attribute__((aligned(16))) uint8_t g_zero_page[64];  // never written

constexpr int kStageBytes = 128;  // K bytes per LDS stage (one LDS row)

__device__ __forceinline__ int swz(int row) { return (row & 7) ^ ((row >> 3) & 1); }

enum Epilogue {
  kEpiI32 = 0,      // int32 out (accumulate flag honoured)
  kEpiDequant = 1,  // int8: f16(((float)acc * rs[m]) * cs[n])
  kEpiFloat = 2     // f16/bf16: fp32 acc -> out dtype (accumulate honoured)
};

struct GemmArgs {
  const uint8_t* A;  // [M, K] row-major, lda_bytes
  const uint8_t* B;  // [N, K] row-major, ldb_bytes
  void* C;
  int64_t lda_bytes, ldb_bytes, ldc;  // ldc in elements
  int M, N, K_bytes;
  int accumulate;
  int out_dtype;  // HXM_I32, HXM_F16, HXM_BF16, HXM_F32
  const float* row_scale;
  const float* col_scale;
  int group_m;  // tile-rows per group in the XCD walk
};

template <typename T>
struct Mfma;

template <>
struct Mfma<int8_t> {
  typedef v16i32 acc_t;
  __device__ static __forceinline__ acc_t run(v4i32 a, v4i32 b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<_Float16> {
  typedef v16f32 acc_t;
  __device__ static __forceinline__ acc_t run(v4i32 a, v4i32 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8f16, a),
                                                  __builtin_bit_cast(v8f16, b),
                                                  c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  typedef v16f32 acc_t;
  __device__ static __forceinline__ acc_t run(v4i32 a, v4i32 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(v8bf16, a), __builtin_bit_cast(v8bf16, b), c, 0, 0, 0);
  }
};

typedef __attribute__((address_space(3))) void lds_void;

// Issues the LDS-DMA loads of one stage of `rows` x 128 bytes of a K-major
// operand.  The wave instruction q covers LDS bytes [q*1024, q*1024+1024):
// lane l fills 16 bytes at row q*8 + l/8, slot l%8, which holds source chunk
// slot ^ swz(row).
template <int ROWS, int NWAVES>
__device__ __forceinline__ void stage_load(const uint8_t* __restrict__ base,
                                           int64_t ld_bytes, int row0,
                                           int rows_valid, int kb0,
                                           int K_bytes, uint8_t* lds,
                                           int wave, int lane) {
  constexpr int kInstr = ROWS / 8;  // wave-instructions for the whole tile
  static_assert(kInstr % NWAVES == 0, "tile rows must split over waves");
#pragma unroll
  for (int i = 0; i < kInstr / NWAVES; ++i) {
    const int q = i * NWAVES + wave;
    const int row = q * 8 + (lane >> 3);
    const int chunk = (lane & 7) ^ swz(row);
    const int kb = kb0 + chunk * 16;
    const uint8_t* src = g_zero_page;
    if (row0 + row < rows_valid && kb < K_bytes)
      src = base + static_cast<int64_t>(row0 + row) * ld_bytes + kb;
    __builtin_amdgcn_global_load_lds(
        reinterpret_cast<const void*>(src),
        (lds_void*)(lds + q * 1024), 16, 0, 0);
  }
}

__device__ __forceinline__ v4i32 lds_frag(const uint8_t* lds, int row, int chunk) {
  return *reinterpret_cast<const v4i32*>(lds + row * kStageBytes +
                                         ((chunk ^ swz(row)) << 4));
}

template <typename T, int BM, int BN, int WM, int WN, int EPI>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(GemmArgs g) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;  // wave sub-tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 blocks per wave
  static_assert(FM >= 1 && FN >= 1, "wave tile must hold a 32x32 block");
  using acc_t = typename Mfma<T>::acc_t;

  __shared__ __attribute__((aligned(1024))) uint8_t lds[2][(BM + BN) * kStageBytes];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave / WN, wn = wave % WN;

  // ---- XCD-aware tile order ----
  const int tiles_m = (g.M + BM - 1) / BM;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int ntiles = tiles_m * tiles_n;
  int t = blockIdx.x;
  if ((ntiles & 7) == 0) t = (t & 7) * (ntiles >> 3) + (t >> 3);
  const int gm = g.group_m;
  const int per_group = gm * tiles_n;
  const int group = t / per_group;
  const int first_m = group * gm;
  const int gsize = min(tiles_m - first_m, gm);
  const int tm = first_m + (t % per_group) % gsize;
  const int tn = (t % per_group) / gsize;
  const int m0 = tm * BM, n0 = tn * BN;

  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = acc_t{};

  const int ksteps = (g.K_bytes + kStageBytes - 1) / kStageBytes;

  auto issue = [&](int kt, int buf) {
    uint8_t* la = lds[buf];
    uint8_t* lb = lds[buf] + BM * kStageBytes;
    stage_load<BM, NW>(g.A, g.lda_bytes, m0, g.M, kt * kStageBytes, g.K_bytes,
                       la, wave, lane);
    stage_load<BN, NW>(g.B, g.ldb_bytes, n0, g.N, kt * kStageBytes, g.K_bytes,
                       lb, wave, lane);
  };

  if (ksteps > 0) issue(0, 0);
  for (int kt = 0; kt < ksteps; ++kt) {
    const int buf = kt & 1;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's DMA landed
    __syncthreads();                     // everyone's landed; buf^1 is free
    if (kt + 1 < ksteps) issue(kt + 1, buf ^ 1);
    const uint8_t* la = lds[buf] + (wm * TM) * kStageBytes;
    const uint8_t* lb = lds[buf] + (BM + wn * TN) * kStageBytes;
#pragma unroll
    for (int ks = 0; ks < kStageBytes / 32; ++ks) {
      const int chunk = ks * 2 + (lane >> 5);
      v4i32 af[FM], bf[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) af[i] = lds_frag(la, i * 32 + (lane & 31), chunk);
#pragma unroll
      for (int j = 0; j < FN; ++j) bf[j] = lds_frag(lb, j * 32 + (lane & 31), chunk);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = Mfma<T>::run(af[i], bf[j], acc[i][j]);
    }
  }

  // ---- epilogue: lane l holds column l%32, rows 8*(v/4) + 4*(l/32) + v%4 ----
  const int col_in = lane & 31;
  const int row_in = (lane >> 5) * 4;
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn * TN + j * 32 + col_in;
    if (n >= g.N) continue;
    float cs = 0.0f;
    if constexpr (EPI == kEpiDequant) cs = g.col_scale[n];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * TM + i * 32 + (v >> 2) * 8 + row_in + (v & 3);
        if (m >= g.M) continue;
        const int64_t off = static_cast<int64_t>(m) * g.ldc + n;
        if constexpr (EPI == kEpiI32) {
          int32_t* c = static_cast<int32_t*>(g.C) + off;
          const int32_t r = acc[i][j][v];
          *c = g.accumulate ? static_cast<int32_t>(static_cast<uint32_t>(*c) +
                                                   static_cast<uint32_t>(r))
                            : r;
        } else if constexpr (EPI == kEpiDequant) {
          // fp32, left to right, each product rounded to fp32 and then once
          // to f16.  The empty asm pins d as an fp32 register value: without
          // it the backend folds the last multiply and the f16 conversion
          // into v_fma_mixlo_f16 (a single rounding), which differs from the
          // defined spelling in the last f16 bit for some inputs.
          float d = (static_cast<float>(acc[i][j][v]) * g.row_scale[m]) * cs;
          asm volatile("" : "+v"(d));
          static_cast<_Float16*>(g.C)[off] = static_cast<_Float16>(d);
        } else {
          float r = acc[i][j][v];
          if (g.out_dtype == HXM_F32) {
            float* c = static_cast<float*>(g.C) + off;
            *c = g.accumulate ? *c + r : r;
          } else if (g.out_dtype == HXM_F16) {
            _Float16* c = static_cast<_Float16*>(g.C) + off;
            if (g.accumulate) r += static_cast<float>(*c);
            *c = static_cast<_Float16>(r);
          } else {
            __bf16* c = static_cast<__bf16*>(g.C) + off;
            if (g.accumulate) r += static_cast<float>(*c);
            *c = static_cast<__bf16>(r);
          }
        }
      }
    }
  }
}

// Transpose [K,N] -> [N,K] (the resident weight image).  32x32 element tiles
// through LDS; ELEM bytes per element.
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

// ------------------------------------------------------------------------
// Host side: the compiled-config table and dispatch.
// ------------------------------------------------------------------------

typedef void (*gemm_fn)(GemmArgs);

struct KernelEntry {
  hxm_gemm_config cfg;
  int threads;
  gemm_fn i8_i32, i8_deq, f16, bf16;
};

#define HXM_ENTRY(BM, BN, WM, WN)                                              \
  KernelEntry{{BM, BN, 0, WM, WN, 1},                                          \
              WM * WN * 64,                                                    \
              gemm_kernel<int8_t, BM, BN, WM, WN, kEpiI32>,                    \
              gemm_kernel<int8_t, BM, BN, WM, WN, kEpiDequant>,                \
              gemm_kernel<_Float16, BM, BN, WM, WN, kEpiFloat>,                \
              gemm_kernel<__bf16, BM, BN, WM, WN, kEpiFloat>}

static const KernelEntry kKernels[] = {HXM_GEMM_CONFIG_LIST(HXM_ENTRY)};
constexpr int kNumKernels = sizeof(kKernels) / sizeof(kKernels[0]);

static int bk_elems(int32_t dt) { return dt == HXM_I8 ? kStageBytes : kStageBytes / 2; }

const KernelEntry* find_kernel(const hxm_gemm_config& c, int32_t dt) {
  for (const KernelEntry& e : kKernels) {
    if (e.cfg.bm == c.bm && e.cfg.bn == c.bn && e.cfg.waves_m == c.waves_m &&
        e.cfg.waves_n == c.waves_n && (c.bk == 0 || c.bk == bk_elems(dt)) &&
        (c.split_k == 0 || c.split_k == 1))
      return &e;
  }
  return nullptr;
}

int num_kernels() { return kNumKernels; }
hxm_gemm_config kernel_config(int i, int32_t dt) {
  hxm_gemm_config c = kKernels[i].cfg;
  c.bk = bk_elems(dt);
  return c;
}

// Default configuration for a shape (used when no tuned winner is cached):
// the largest tile that still yields at least one workgroup per CU, else the
// smallest tile.
hxm_gemm_config default_config(int64_t M, int64_t N, int32_t dt) {
  static const int order[][2] = {{256, 256}, {256, 128}, {128, 128}, {64, 64}};
  for (auto& o : order) {
    const int64_t tiles = ((M + o[0] - 1) / o[0]) * ((N + o[1] - 1) / o[1]);
    if (tiles >= 256) {
      for (const KernelEntry& e : kKernels)
        if (e.cfg.bm == o[0] && e.cfg.bn == o[1]) return kernel_config(&e - kKernels, dt);
    }
  }
  for (const KernelEntry& e : kKernels)
    if (e.cfg.bm == 64 && e.cfg.bn == 64) return kernel_config(&e - kKernels, dt);
  return kernel_config(0, dt);
}

// Tuned winners, filled by hxm_tune_gemm (search.cpp).
bool lookup_tuned(int32_t op, int64_t M, int64_t N, int64_t K, hxm_gemm_config* out);

hxm_status launch_gemm(const KernelEntry& e, int32_t ab_dtype, int epi,
                       const GemmArgs& g, hipStream_t stream) {
  const int bm = e.cfg.bm, bn = e.cfg.bn;
  const int64_t tiles = static_cast<int64_t>((g.M + bm - 1) / bm) * ((g.N + bn - 1) / bn);
  gemm_fn fn = nullptr;
  if (ab_dtype == HXM_I8)
    fn = (epi == kEpiDequant) ? e.i8_deq : e.i8_i32;
  else if (ab_dtype == HXM_F16)
    fn = e.f16;
  else
    fn = e.bf16;
  hipLaunchKernelGGL(fn, dim3(static_cast<unsigned>(tiles)), dim3(e.threads), 0,
                     stream, g);
  return check_launch("gemm kernel");
}

namespace {

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
  if (M > INT32_MAX / 2 || N > INT32_MAX / 2 || K * eb > INT32_MAX / 2)
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: %s extent beyond 2^30", op);
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
  void* ws = nullptr;
  hxm_status st = stream_workspace(stream, static_cast<size_t>(N * K * eb), &ws);
  if (st != HXM_OK) return st;
  const dim3 grid(static_cast<unsigned>((N + 31) / 32), static_cast<unsigned>((K + 31) / 32));
  if (eb == 1)
    transpose_kernel<uint8_t><<<grid, 256, 0, stream>>>(
        static_cast<const uint8_t*>(B), ldb, static_cast<uint8_t*>(ws), K, K, N);
  else
    transpose_kernel<uint16_t><<<grid, 256, 0, stream>>>(
        static_cast<const uint16_t*>(B), ldb, static_cast<uint16_t*>(ws), K, K, N);
  if ((st = check_launch("weight pack")) != HXM_OK) return st;
  *b_out = static_cast<const uint8_t*>(ws);
  *ldb_bytes_out = K * eb;
  return HXM_OK;
}

hxm_status pick_kernel(int32_t op, int32_t ab_dtype, int64_t M, int64_t N,
                       int64_t K, const hxm_gemm_config* cfg,
                       const KernelEntry** out) {
  hxm_gemm_config c;
  if (cfg && cfg->bm) {
    c = *cfg;
  } else if (!lookup_tuned(op, M, N, K, &c)) {
    c = default_config(M, N, ab_dtype);
  }
  const KernelEntry* e = find_kernel(c, ab_dtype);
  if (!e)
    return fail(HXM_UNSUPPORTED_SHAPE,
                "no-kernel: no compiled GEMM for bm=%d bn=%d bk=%d waves=%dx%d split_k=%d",
                c.bm, c.bn, c.bk, c.waves_m, c.waves_n, c.split_k);
  *out = e;
  return HXM_OK;
}

}  // namespace

// Shared by the entry points and the tuner.
hxm_status run_gemm(int32_t op, int32_t ab_dtype, int epi, const void* A,
                    int64_t lda, const void* B, int64_t ldb, int32_t b_layout,
                    void* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                    int32_t out_dtype, int32_t accumulate, const float* rs,
                    const float* cs, const hxm_gemm_config* cfg,
                    hipStream_t stream) {
  const int64_t eb = dtype_bytes(ab_dtype);
  const KernelEntry* e = nullptr;
  hxm_status st = pick_kernel(op, ab_dtype, M, N, K, cfg, &e);
  if (st != HXM_OK) return st;
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (M == 0 || N == 0) return ok();
  const uint8_t* bk = nullptr;
  int64_t ldb_bytes = 0;
  if (K > 0 && (st = resolve_b(B, ldb, b_layout, K, N, eb, stream, &bk, &ldb_bytes)) != HXM_OK)
    return st;
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
  if ((st = launch_gemm(*e, ab_dtype, epi, g, stream)) != HXM_OK) return st;
  return ok();
}

}  // namespace hxm

using namespace hxm;

extern "C" {

hxm_status hxm_query_contraction(int64_t M, int64_t N, int64_t K,
                                 int32_t a_dtype, int32_t b_dtype,
                                 int32_t c_dtype, int32_t* plan_out) {
  if (plan_out) *plan_out = -1;
  const bool i8 = a_dtype == HXM_I8 && b_dtype == HXM_I8 &&
                  (c_dtype == HXM_I32 || c_dtype == HXM_F16);
  const bool fl = (a_dtype == HXM_F16 || a_dtype == HXM_BF16) && b_dtype == a_dtype &&
                  (c_dtype == HXM_F16 || c_dtype == HXM_BF16 || c_dtype == HXM_F32);
  if (!i8 && !fl)
    return fail(HXM_UNSUPPORTED_DTYPE, "unsupported-dtype: a=%d b=%d c=%d",
                a_dtype, b_dtype, c_dtype);
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(HXM_INVALID_ARG, "invalid-argument: extents must be positive");
  const int64_t eb = dtype_bytes(a_dtype);
  if ((K * eb) % 16)
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: K*elem_bytes=%lld is not a multiple of 16",
                (long long)(K * eb));
  const bool full = M % 32 == 0 && N % 32 == 0 && K % 32 == 0;
  if (plan_out) *plan_out = full ? 0 : 1;
  return ok();
}

hxm_status hxm_matmul(const void* A, int64_t lda, const void* B, int64_t ldb,
                      int32_t b_layout, void* C, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, int32_t ab_dtype, int32_t c_dtype,
                      int32_t accumulate, const hxm_gemm_config* cfg,
                      void* stream) {
  if (ab_dtype != HXM_F16 && ab_dtype != HXM_BF16)
    return fail(HXM_UNSUPPORTED_DTYPE, "unsupported-dtype: matmul A/B dtype %d",
                ab_dtype);
  if (c_dtype != HXM_F16 && c_dtype != HXM_BF16 && c_dtype != HXM_F32)
    return fail(HXM_UNSUPPORTED_DTYPE, "unsupported-dtype: matmul C dtype %d",
                c_dtype);
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

}  // extern "C"
