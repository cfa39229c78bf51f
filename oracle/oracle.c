/*
 * oracle.c -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference
 * semantics of the hot path, used by tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg as the checker.  Nothing in the product links
 * or calls this file.
 *
 * Each function cites what it restates (paths relative to the reference
 * root):
 *   hxo_gemm_i8        linalg.matmul on int8 -> int32 as lowered on the HVX
 *                      generic path (qcom_hexagon_backend/lib/Conversion/
 *                      LinalgToLLVM/ScheduleMatmulForHVXPass.cpp:44-80,
 *                      test/Conversion/LinalgToLLVM/matmul_linalg.mlir:1-30):
 *                      C = init + sum_k A[m,k]*B[k,n], exact integer.
 *   hxo_dequant_f16    the read-out convert (bin/runtime/hmx/src/HMXAPI.c:36-44)
 *                      with per-channel scales: f16(((float)acc*rs)*cs).
 *   hxo_matmul_f16     hmx.matmul (HmxOps.td:47) / test_matmul.py:73-88:
 *                      wide accumulate (fp32 here), one rounding to C.
 *   hxo_gemv_w8a16     int8-weight matmul, fp32 accumulate, per-channel scale.
 *   hxo_gemm_w8a16     the same with fp32 scales (the FFN projections of the
 *                      SwiGLU FFN block; int8 operands of linalg.matmul
 *                      take the HVX path, ScheduleMatmulForHVXPass.cpp:44-80).
 *   hxo_gemm_w8a16_residual  the same plus a residual (x + FFN(x)):
 *                      f16(f32(acc * scale) + f32(r)).
 *   hxo_swiglu_gateup  gate/up projections + SiLU * mul of that block:
 *                      h = f16(silu(g) * u), g = acc_g * sg, u = acc_u * su,
 *                      silu(g) = g / (1 + exp(-g)) evaluated in fp64.
 *   hxo_softmax_rows   test/python/triton/test_softmax.py:41-69 (fp32 sum).
 *   hxo_rmsnorm_rows   test/python/triton/test_rms_norm.py:34-60.
 *   hxo_layernorm_rows test/python/triton/test_layer_norm.py:39-79.
 *
 * Built with -ffp-contract=off so that a*b+c is never fused: every fp32
 * operation rounds once, as written.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- IEEE 754 binary16 / bfloat16 conversions (round to nearest even) --- */

float hxo_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  uint32_t bits;
  if (e == 0x1f) {
    bits = sign | 0x7f800000u | (m << 13);
  } else if (e == 0) {
    if (m == 0) {
      bits = sign;
    } else { /* subnormal: m * 2^-24 */
      int shift = 0;
      while (!(m & 0x400u)) {
        m <<= 1;
        ++shift;
      }
      m &= 0x3ffu;
      bits = sign | ((uint32_t)(113 - shift) << 23) | (m << 13);
    }
  } else {
    bits = sign | ((e + 112u) << 23) | (m << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t hxo_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? (0x200u | ((ax >> 13) & 0x3ffu)) : 0u));
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
  if (ax >= 0x38800000u) { /* normal f16 */
    ax += 0x0fffu + ((ax >> 13) & 1u);
    return (uint16_t)(sign | ((ax - (112u << 23)) >> 13));
  }
  /* f16 subnormal or zero: round(|f| * 2^24) */
  const uint32_t e = ax >> 23;
  if (e == 0) return sign; /* f32 zero/subnormal: far below 2^-25 */
  const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
  const uint32_t shift = 126u - e; /* >= 14 */
  if (shift > 31u) return sign;
  uint32_t r = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (r & 1u))) ++r;
  return (uint16_t)(sign | r);
}

float hxo_bf16_to_f32(uint16_t h) {
  uint32_t bits = (uint32_t)h << 16;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

uint16_t hxo_f32_to_bf16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}

void hxo_f16_to_f32_array(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = hxo_f16_to_f32(in[i]);
}
void hxo_f32_to_f16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = hxo_f32_to_f16(in[i]);
}
void hxo_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = hxo_f32_to_bf16(in[i]);
}

/* dtype codes shared with include/hxm.h */
enum { D_F16 = 1, D_BF16 = 2, D_F32 = 3 };

static float ld(const void* p, int64_t i, int dt) {
  if (dt == D_F16) return hxo_f16_to_f32(((const uint16_t*)p)[i]);
  if (dt == D_BF16) return hxo_bf16_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}
static void st(void* p, int64_t i, int dt, float v) {
  if (dt == D_F16)
    ((uint16_t*)p)[i] = hxo_f32_to_f16(v);
  else if (dt == D_BF16)
    ((uint16_t*)p)[i] = hxo_f32_to_bf16(v);
  else
    ((float*)p)[i] = v;
}

/* ---- int8 GEMM, exact ---------------------------------------------------- */

/* C[m,n] = (accumulate ? C[m,n] : 0) + sum_k A[m,k] * B(k,n), int32 with
 * wrap-around addition of the prior C.  b_nk: B is [N,K] (ldb >= K) instead
 * of [K,N] (ldb >= N).  Each product is at most 128*128 = 16384 in
 * magnitude, so an int32 running sum is exact for K <= 131071; longer K sums
 * in int64 and keeps the low 32 bits (the same wrap an int32 accumulator
 * gives).  Integer addition is associative, so any summation order agrees. */
void hxo_gemm_i8(const int8_t* A, int64_t lda, const int8_t* B, int64_t ldb,
                 int b_nk, int32_t* C, int64_t ldc, int64_t M, int64_t N,
                 int64_t K, int accumulate, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t m = 0; m < M; ++m) {
    const int8_t* a = A + m * lda;
    for (int64_t n = 0; n < N; ++n) {
      int32_t s = 0;
      if (K > 131071) {
        int64_t w = 0;
        for (int64_t k = 0; k < K; ++k)
          w += (int64_t)a[k] * (int64_t)(b_nk ? B[n * ldb + k] : B[k * ldb + n]);
        s = (int32_t)(uint32_t)(uint64_t)w;
      } else if (b_nk) {
        const int8_t* b = B + n * ldb;
        for (int64_t k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)b[k];
      } else {
        for (int64_t k = 0; k < K; ++k) s += (int32_t)a[k] * (int32_t)B[k * ldb + n];
      }
      int32_t* c = C + m * ldc + n;
      *c = accumulate ? (int32_t)((uint32_t)*c + (uint32_t)s) : s;
    }
  }
}

/* out[m,n] = f16( ((float)acc[m,n] * rs[m]) * cs[n] ), fp32, two roundings. */
void hxo_dequant_f16(const int32_t* acc, int64_t lda, const float* rs,
                     const float* cs, uint16_t* out, int64_t ldo, int64_t M,
                     int64_t N) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      const float a = (float)acc[m * lda + n];
      const float t = a * rs[m];
      const float d = t * cs[n];
      out[m * ldo + n] = hxo_f32_to_f16(d);
    }
}

/* ---- f16/bf16 matmul, fp32 accumulate ------------------------------------ */

void hxo_matmul(const uint16_t* A, int64_t lda, const uint16_t* B, int64_t ldb,
                int b_nk, int ab_dtype, void* C, int64_t ldc, int c_dtype,
                int accumulate, int64_t M, int64_t N, int64_t K, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float s = accumulate ? ld(C, m * ldc + n, c_dtype) : 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float a = ld(A, m * lda + k, ab_dtype);
        const float b = b_nk ? ld(B, n * ldb + k, ab_dtype) : ld(B, k * ldb + n, ab_dtype);
        s += a * b;
      }
      st(C, m * ldc + n, c_dtype, s);
    }
}

/* ---- W8A16 GEMV ------------------------------------------------------------ */

void hxo_gemv_w8a16(const uint16_t* x, int64_t ldx, const int8_t* W, int64_t ldw,
                    const uint16_t* scale, uint16_t* y, int64_t ldy, int64_t M,
                    int64_t N, int64_t K, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t n = 0; n < N; ++n) {
    const float sc = hxo_f16_to_f32(scale[n]);
    for (int64_t m = 0; m < M; ++m) {
      float s = 0.0f;
      for (int64_t k = 0; k < K; ++k)
        s += hxo_f16_to_f32(x[m * ldx + k]) * (float)W[n * ldw + k];
      y[m * ldy + n] = hxo_f32_to_f16(s * sc);
    }
  }
}

/* ---- row reductions --------------------------------------------------------- */

/* y = exp(x - max) / sum exp(x - max); exp in fp32, sum in fp64 (the most
 * accurate reading of "fp32 sum"), one rounding of the quotient. */
void hxo_softmax_rows(const void* x, int64_t ldx, void* y, int64_t ldy,
                      int64_t rows, int64_t cols, int dtype, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    float m = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) {
      const float v = ld(x, r * ldx + c, dtype);
      if (v > m || isnan(v)) m = v;
    }
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += (double)expf(ld(x, r * ldx + c, dtype) - m);
    for (int64_t c = 0; c < cols; ++c) {
      const float e = expf(ld(x, r * ldx + c, dtype) - m);
      st(y, r * ldy + c, dtype, (float)((double)e / s));
    }
  }
}

/* y = x * (1/sqrt(mean(x^2) + eps)) * gamma; statistics in fp64. */
/* y[m,n] = f16((sum_k f32(x[m,k]) * f32(W[n,k])) * scale[n]), the sum in
 * fp32 in increasing k. */
void hxo_gemm_w8a16(const uint16_t* x, int64_t ldx, const int8_t* W, int64_t ldw,
                    const float* scale, uint16_t* y, int64_t ldy, int64_t M, int64_t N,
                    int64_t K, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      float s = 0.0f;
      for (int64_t k = 0; k < K; ++k)
        s += hxo_f16_to_f32(x[m * ldx + k]) * (float)W[n * ldw + k];
      y[m * ldy + n] = hxo_f32_to_f16(s * scale[n]);
    }
  }
}

/* y[m,n] = f16(f32(acc * scale[n]) + f32(r[m,n])) with acc the fp32 sum of
 * hxo_gemm_w8a16: the read-out that adds a resident tensor before the store
 * (hmx_unpack_acc_f32 with residual, bin/runtime/hmx/include/HMXAPI.h
 * :245-275).  Product and sum each round to fp32 (no fma: -ffp-contract=off),
 * then one rounding to f16.  r may be y (in place). */
void hxo_gemm_w8a16_residual(const uint16_t* x, int64_t ldx, const int8_t* W, int64_t ldw,
                             const float* scale, const uint16_t* r, int64_t ldr, uint16_t* y,
                             int64_t ldy, int64_t M, int64_t N, int64_t K, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t n = 0; n < N; ++n) {
    for (int64_t m = 0; m < M; ++m) {
      float s = 0.0f;
      for (int64_t k = 0; k < K; ++k)
        s += hxo_f16_to_f32(x[m * ldx + k]) * (float)W[n * ldw + k];
      const float p = s * scale[n];
      y[m * ldy + n] = hxo_f32_to_f16(p + hxo_f16_to_f32(r[m * ldr + n]));
    }
  }
}

/* h[m,i] = f16(silu(g) * u) with g = f32(sum_k x*Wg[i,k]) * sg[i] and
 * u = f32(sum_k x*Wu[i,k]) * su[i] (fp32 sums in increasing k, fp32
 * products); silu and the product in fp64. */
void hxo_swiglu_gateup(const uint16_t* x, int64_t ldx, const int8_t* Wg, const int8_t* Wu,
                       int64_t ldw, const float* sg, const float* su, uint16_t* h,
                       int64_t ldh, int64_t M, int64_t I, int64_t K, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t i = 0; i < I; ++i) {
    for (int64_t m = 0; m < M; ++m) {
      float ag = 0.0f, au = 0.0f;
      for (int64_t k = 0; k < K; ++k) {
        const float xv = hxo_f16_to_f32(x[m * ldx + k]);
        ag += xv * (float)Wg[i * ldw + k];
        au += xv * (float)Wu[i * ldw + k];
      }
      const double g = (double)(ag * sg[i]), u = (double)(au * su[i]);
      h[m * ldh + i] = hxo_f32_to_f16((float)(g / (1.0 + exp(-g)) * u));
    }
  }
}

void hxo_rmsnorm_rows(const void* x, int64_t ldx, const void* gamma, void* y,
                      int64_t ldy, int64_t rows, int64_t cols, float eps,
                      int dtype, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    double ss = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      const double v = ld(x, r * ldx + c, dtype);
      ss += v * v;
    }
    const double rstd = 1.0 / sqrt(ss / (double)cols + (double)eps);
    for (int64_t c = 0; c < cols; ++c) {
      const double g = gamma ? ld(gamma, c, dtype) : 1.0;
      st(y, r * ldy + c, dtype, (float)(ld(x, r * ldx + c, dtype) * rstd * g));
    }
  }
}

/* y = (x - mean) * rstd * gamma + beta, biased variance, statistics in fp64;
 * mean/rstd written as fp32 when the pointers are non-NULL. */
void hxo_layernorm_rows(const void* x, int64_t ldx, const void* gamma,
                        const void* beta, void* y, int64_t ldy, float* mean_out,
                        float* rstd_out, int64_t rows, int64_t cols, float eps,
                        int dtype, int threads) {
#ifdef _OPENMP
  if (threads > 0) omp_set_num_threads(threads);
#pragma omp parallel for schedule(static)
#endif
  for (int64_t r = 0; r < rows; ++r) {
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += ld(x, r * ldx + c, dtype);
    const double mean = s / (double)cols;
    double q = 0.0;
    for (int64_t c = 0; c < cols; ++c) {
      const double d = ld(x, r * ldx + c, dtype) - mean;
      q += d * d;
    }
    const double rstd = 1.0 / sqrt(q / (double)cols + (double)eps);
    if (mean_out) mean_out[r] = (float)mean;
    if (rstd_out) rstd_out[r] = (float)rstd;
    for (int64_t c = 0; c < cols; ++c) {
      const double g = gamma ? ld(gamma, c, dtype) : 1.0;
      const double b = beta ? ld(beta, c, dtype) : 0.0;
      st(y, r * ldy + c, dtype, (float)((ld(x, r * ldx + c, dtype) - mean) * rstd * g + b));
    }
  }
}

int hxo_max_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
