// Small-output f16 / bf16 GEMM: the default kernel of hxm_matmul when the
// output is at most kSmallTilesMax 16x16 tiles and K at most kSmallKMax
// (an fp16 256^3 matmul is 256 such tiles).
//
// Such a call is launch-bound: the LDS-staged kernel spends most of its
// time on its staging round trips, barriers and the staged epilogue, not on
// MFMA work.  Here one wave owns one 16x16 output tile and loads its MFMA
// fragments straight from memory into registers -- every k-step's A row
// chunk and B column chunk (16 bytes per lane) issued at once, one round
// trip -- then runs its v_mfma_f32_16x16x32 chain on two accumulators and
// stores.  No LDS, no barrier.  Measured in a HIP graph of 50 launches (one
// box): 256^3 2.20 against 3.19 us for the staged kernel's 32x32 tiles,
// 128^3 2.03 against 2.77, 300x260x200 2.29 against 3.38; at 512x512x256
// (1024 tiles) 3.66 against 3.55 and beyond that the staged kernel's
// operand reuse wins by far (1024x1024x256: 9.59 against 3.93), hence the
// limits.
//
// Operand layout of v_mfma_f32_16x16x32_{f16,bf16}: lane l holds row l%16 of
// the first operand and column l%16 of the second, K [8*(l/16), +8) of the
// 32-wide k-step; the result D[i][j] sits in lane j + 16*(i/4), element i%4.
// B (the [N, K] image) goes in as the first operand and A as the second, so
// D[i][j] = C[m0 + j][n0 + i] and a lane's four results are four consecutive
// columns of one row of C.  K past the end (K is a multiple of 8) and rows
// past M or N load a valid address and are zeroed or never stored.
#include <type_traits>

#include "device_util.h"
#include "hxm_internal.h"

namespace hxm {

namespace {

struct SmallArgs {
  const uint8_t* A;  // [M, K] row-major, lda elements
  const uint8_t* B;  // [N, K] image, ldb bytes per row
  void* C;
  int64_t lda, ldb_bytes, ldc;
  int M, N, K;
  int32_t out_dtype;
  int32_t accumulate;
};

template <typename T>
__device__ __forceinline__ v4f32 mfma16(v4i32 a, v4i32 b, v4f32 c) {
  if constexpr (std::is_same<T, _Float16>::value)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8f16, a),
                                                  __builtin_bit_cast(v8f16, b), c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(v8bf16, a),
                                                   __builtin_bit_cast(v8bf16, b), c, 0, 0, 0);
}

// OUT: the output element type; ACC: C += A B instead of C = A B.  Both are
// compile-time, so the common store (f16, no accumulate) carries no branches
// (256^3: 2.20 us; 2.49 with them chosen at run time).
template <typename T, int KS, typename OUT, bool ACC>
__global__ __launch_bounds__(64) void small_gemm_kernel(SmallArgs g) {
  const int lane = threadIdx.x;
  const int r = lane & 15, kq = lane >> 4;
  const int m0 = blockIdx.y * 16, n0 = blockIdx.x * 16;
  const int m = m0 + r, n = n0 + r;
  const uint8_t* a = g.A + static_cast<int64_t>(m < g.M ? m : g.M - 1) * g.lda * 2;
  const uint8_t* b = g.B + static_cast<int64_t>(n < g.N ? n : g.N - 1) * g.ldb_bytes;
  v4i32 av[KS], bv[KS];
  const v4i32 zero = {0, 0, 0, 0};
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const int k = s * 32 + kq * 8;
    const bool in = k < g.K;
    av[s] = *reinterpret_cast<const v4i32*>(a + (in ? k : 0) * 2);
    bv[s] = *reinterpret_cast<const v4i32*>(b + (in ? k : 0) * 2);
    if (!in) av[s] = bv[s] = zero;
  }
  // Two independent chains; their sum is one more fp32 rounding per output.
  v4f32 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
#pragma unroll
  for (int s = 0; s < KS; s += 2) {
    acc0 = mfma16<T>(bv[s], av[s], acc0);
    if (s + 1 < KS) acc1 = mfma16<T>(bv[s + 1], av[s + 1], acc1);
  }
  const v4f32 acc = acc0 + acc1;
  const int mo = m0 + (lane & 15);
  if (mo >= g.M) return;
  OUT* c = static_cast<OUT*>(g.C) + static_cast<int64_t>(mo) * g.ldc + n0 + 4 * (lane >> 4);
  const int nv = g.N - (n0 + 4 * (lane >> 4));  // columns of this lane's run inside C
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    if (v >= nv) break;
    // f32: the sum as it stands; f16 / bf16: the fp32 sum, one rounding.
    const float r = ACC ? acc[v] + static_cast<float>(c[v]) : acc[v];
    c[v] = static_cast<OUT>(r);
  }
}

template <typename T, int KS>
void launch_ks(const SmallArgs& g, dim3 grid, hipStream_t s) {
  if (g.out_dtype == HXM_F32)
    g.accumulate ? small_gemm_kernel<T, KS, float, true><<<grid, 64, 0, s>>>(g)
                 : small_gemm_kernel<T, KS, float, false><<<grid, 64, 0, s>>>(g);
  else if (g.out_dtype == HXM_F16)
    g.accumulate ? small_gemm_kernel<T, KS, _Float16, true><<<grid, 64, 0, s>>>(g)
                 : small_gemm_kernel<T, KS, _Float16, false><<<grid, 64, 0, s>>>(g);
  else
    g.accumulate ? small_gemm_kernel<T, KS, __bf16, true><<<grid, 64, 0, s>>>(g)
                 : small_gemm_kernel<T, KS, __bf16, false><<<grid, 64, 0, s>>>(g);
}

template <typename T>
hxm_status launch_t(const SmallArgs& g, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((g.N + 15) / 16), static_cast<unsigned>((g.M + 15) / 16));
  const int ks = (g.K + 31) / 32;
  if (ks <= 1) launch_ks<T, 1>(g, grid, s);
  else if (ks <= 2) launch_ks<T, 2>(g, grid, s);
  else if (ks <= 4) launch_ks<T, 4>(g, grid, s);
  else launch_ks<T, 8>(g, grid, s);
  return check_launch("small gemm");
}

}  // namespace

hxm_gemm_config small_gemm_config() { return hxm_gemm_config{16, 16, 32, 1, 1, 0, 1}; }

bool is_small_gemm_config(const hxm_gemm_config& c) {
  const hxm_gemm_config s = small_gemm_config();
  return c.bm == s.bm && c.bn == s.bn && c.bk == s.bk && c.waves_m == s.waves_m &&
         c.waves_n == s.waves_n && c.stages == s.stages && c.split_k <= 1;
}

bool small_gemm_fits(int64_t M, int64_t N, int64_t K, int32_t ab_dtype) {
  return (ab_dtype == HXM_F16 || ab_dtype == HXM_BF16) && K > 0 && K <= kSmallKMax &&
         M > 0 && N > 0 && ((M + 15) / 16) * ((N + 15) / 16) <= kSmallTilesMax;
}

hxm_status launch_small_gemm(int32_t ab_dtype, const void* A, int64_t lda, const uint8_t* B,
                             int64_t ldb_bytes, void* C, int64_t ldc, int64_t M, int64_t N,
                             int64_t K, int32_t out_dtype, int32_t accumulate,
                             hipStream_t stream) {
  SmallArgs g;
  g.A = static_cast<const uint8_t*>(A);
  g.B = B;
  g.C = C;
  g.lda = lda;
  g.ldb_bytes = ldb_bytes;
  g.ldc = ldc;
  g.M = static_cast<int>(M);
  g.N = static_cast<int>(N);
  g.K = static_cast<int>(K);
  g.out_dtype = out_dtype;
  g.accumulate = accumulate;
  return ab_dtype == HXM_BF16 ? launch_t<__bf16>(g, stream) : launch_t<_Float16>(g, stream);
}

}  // namespace hxm
