// W8A16 weight-resident skinny GEMM / GEMV on gfx950 (M <= 16 per pass).
//
// Reference semantics: an int8-weight linalg.matmul, which the reference's
// engine refuses (qcom_hexagon_backend/include/hexagon/Dialect/Hmx/Transforms/
// HmxTarget.h:198-211: unsupported-dtype, and min-rows for M <= 4) and lowers
// on the HVX generic path (lib/Conversion/LinalgToLLVM/
// ScheduleMatmulForHVXPass.cpp:44-80); weight residency as in
// lib/Dialect/Hmx/Transforms/WeightResidentPass.cpp:10-53.
//   y[m,n] = f16( (sum_k f32(x[m,k]) * f32(W[n,k])) * f32(scale[n]) )
//
// GPU form.  The weight stream dominates (N*K bytes vs M*K*2 for x), so the
// kernel is built to read W exactly once with 128-bit loads:
//   * a workgroup owns 16 output channels; its KW waves split K;
//   * per 64-wide K slab, lane l loads 16 bytes of W row n0 + l%16 at K offset
//     16*(l/16): one wave instruction covers 16 rows x 64 bytes;
//   * the 16 int8 become 16 exact f16 (byte permute with an 0x64 exponent,
//     then a packed f16 subtract of 1152) and feed two
//     v_mfma_f32_16x16x32_f16 with W as the A operand (rows = channels) and x
//     as the B operand (columns = the M <= 16 activation rows, zero past M);
//     the K order inside an instruction is the same permutation for both
//     operands, so the sum is the plain dot product;
//   * the KW partial 16x16 tiles meet in LDS; wave 0 applies the per-channel
//     scale and writes f16.
#include "device_util.h"
#include "hxm_internal.h"

namespace hxm {

struct GemvArgs {
  const _Float16* x;
  int64_t ldx;
  const int8_t* W;
  int64_t ldw;
  const _Float16* scale;
  _Float16* y;
  int64_t ldy;
  int M, N, K;
};

// 8 int8 (two dwords) -> 8 exact f16.  (b ^ 0x80) | 0x6400 is the f16
// 1024 + b + 128; subtracting 1152 leaves b exactly.
__device__ __forceinline__ v8f16 i8x8_to_f16(uint32_t lo, uint32_t hi) {
  lo ^= 0x80808080u;
  hi ^= 0x80808080u;
  const uint32_t k64 = 0x64646464u;
  uint32_t w0 = __builtin_amdgcn_perm(k64, lo, 0x05010400u);
  uint32_t w1 = __builtin_amdgcn_perm(k64, lo, 0x05030402u);
  uint32_t w2 = __builtin_amdgcn_perm(k64, hi, 0x05010400u);
  uint32_t w3 = __builtin_amdgcn_perm(k64, hi, 0x05030402u);
  const v2f16 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
  v2f16 h0 = __builtin_bit_cast(v2f16, w0) - bias;
  v2f16 h1 = __builtin_bit_cast(v2f16, w1) - bias;
  v2f16 h2 = __builtin_bit_cast(v2f16, w2) - bias;
  v2f16 h3 = __builtin_bit_cast(v2f16, w3) - bias;
  v8f16 r;
  r[0] = h0[0]; r[1] = h0[1]; r[2] = h1[0]; r[3] = h1[1];
  r[4] = h2[0]; r[5] = h2[1]; r[6] = h3[0]; r[7] = h3[1];
  return r;
}

template <int KW, int UNROLL>
__global__ __launch_bounds__(KW * 64) void gemv_w8a16_kernel(GemvArgs g) {
  __shared__ v4f32 part[KW][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int m_base = blockIdx.y * 16;
  const int r16 = lane & 15;   // W row (channel) for A; x row (m) for B
  const int kq = lane >> 4;    // which 16-byte quarter of the 64-wide slab
  const int n = n0 + r16;
  const int m = m_base + r16;
  const bool n_ok = n < g.N;
  const bool m_ok = m < g.M;
  const int8_t* wrow = g.W + static_cast<int64_t>(n_ok ? n : 0) * g.ldw;
  const _Float16* xrow = g.x + static_cast<int64_t>(m_ok ? m : 0) * g.ldx;
  const int slabs = (g.K + 63) / 64;

  v4f32 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int s0 = wave; s0 < slabs; s0 += KW * UNROLL) {
    v4i32 w[UNROLL];
    v4i32 xa[UNROLL], xb[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const int s = s0 + u * KW;
      const int k = s * 64 + kq * 16;
      const bool k_ok = s < slabs && k < g.K;
      w[u] = (n_ok && k_ok) ? *reinterpret_cast<const v4i32*>(wrow + k) : v4i32{0, 0, 0, 0};
      if (m_ok && k_ok) {
        xa[u] = *reinterpret_cast<const v4i32*>(xrow + k);
        xb[u] = *reinterpret_cast<const v4i32*>(xrow + k + 8);
      } else {
        xa[u] = v4i32{0, 0, 0, 0};
        xb[u] = v4i32{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const v8f16 wa = i8x8_to_f16(static_cast<uint32_t>(w[u][0]), static_cast<uint32_t>(w[u][1]));
      const v8f16 wb = i8x8_to_f16(static_cast<uint32_t>(w[u][2]), static_cast<uint32_t>(w[u][3]));
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, __builtin_bit_cast(v8f16, xa[u]), acc, 0, 0, 0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, __builtin_bit_cast(v8f16, xb[u]), acc, 0, 0, 0);
    }
  }

  part[wave][lane] = acc;
  __syncthreads();
  if (wave != 0) return;
  v4f32 tot = part[0][lane];
#pragma unroll
  for (int w = 1; w < KW; ++w) tot += part[w][lane];
  // D[row = channel 4*(l/16)+v][col = m l%16]
  const int mo = m_base + (lane & 15);
  if (mo >= g.M) return;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int no = n0 + 4 * (lane >> 4) + v;
    if (no < g.N) {
      const float sc = static_cast<float>(g.scale[no]);
      g.y[static_cast<int64_t>(mo) * g.ldy + no] = static_cast<_Float16>(tot[v] * sc);
    }
  }
}

}  // namespace hxm

using namespace hxm;

extern "C" hxm_status hxm_gemv_w8a16(const void* x, int64_t ldx, const int8_t* W,
                                     int64_t ldw, const void* w_scale, void* y,
                                     int64_t ldy, int64_t M, int64_t N, int64_t K,
                                     void* stream) {
  if (M < 0 || N < 0 || K < 0)
    return fail(HXM_INVALID_ARG, "invalid-argument: gemv_w8a16 negative extent");
  if (M > 0 && N > 0 && (!y || !w_scale || (K > 0 && (!x || !W))))
    return fail(HXM_INVALID_ARG, "invalid-argument: gemv_w8a16 null operand");
  if (ldx < K || ldw < K || ldy < N)
    return fail(HXM_INVALID_ARG, "invalid-argument: gemv_w8a16 leading dimension too small");
  if (K % 16 || ldx % 8 || ldw % 16 || (K > 0 && (!aligned16(x) || !aligned16(W))))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: gemv_w8a16 needs K and ldw multiples of 16, ldx of 8, "
                "16-byte aligned x and W (K=%lld)",
                (long long)K);
  if (N > INT32_MAX - 16 || K > INT32_MAX - 64 || M > 65535LL * 16)
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: gemv_w8a16 extent too large");
  hxm_status st = require_device(nullptr);
  if (st != HXM_OK) return st;
  if (M == 0 || N == 0) return ok();
  GemvArgs g{static_cast<const _Float16*>(x), ldx, W, ldw,
             static_cast<const _Float16*>(w_scale), static_cast<_Float16*>(y), ldy,
             static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)};
  const dim3 grid(static_cast<unsigned>((N + 15) / 16), static_cast<unsigned>((M + 15) / 16));
  gemv_w8a16_kernel<4, 4><<<grid, 256, 0, as_stream(stream)>>>(g);
  return check_launch("gemv_w8a16");
}
