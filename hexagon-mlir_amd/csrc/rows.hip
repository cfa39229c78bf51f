// Row reductions on gfx950: softmax, RMSNorm, LayerNorm.
//
// Reference semantics: test/python/triton/test_softmax.py:41-69 (max-subtract,
// exp in fp32, sum, divide), test_rms_norm.py:34-60 (x / sqrt(mean(x^2)+eps)
// * g), test_layer_norm.py:39-79 (mean, biased variance, rstd, affine, mean and
// rstd written per row), as lowered on the HVX path by
// lib/Conversion/LinalgToLLVM/VectorRowReducePass.cpp:10-31 (vector fold +
// rotate butterfly) and SplitReduceGenericPass.cpp:62-93.
//
// Design: one wave per row, four rows per 256-thread workgroup.  A row of up to
// 64 lanes x 16 vectors x 16 bytes is loaded ONCE into registers with 128-bit
// coalesced loads (consecutive lanes read consecutive 16-byte chunks), reduced
// across the wave with DPP + readlane (no LDS, no barriers) and written back
// from registers: one HBM read and one HBM write per element.  Full rows of 8
// vectors per lane (4096 f16) are split over two or four waves whose totals
// meet in LDS (see row_kernel).  Longer rows use the streaming variant
// (VPL = 0) that re-reads the row per pass.
#include <type_traits>

#include "device_util.h"
#include "hxm_internal.h"

namespace hxm {

enum RowOp { kSoftmax = 0, kRmsNorm = 1, kLayerNorm = 2 };

constexpr int kRowWaves = 4;  // rows (waves) per workgroup

template <typename T>
struct RowVec {
  static constexpr int N = 16 / sizeof(T);  // elements per 16-byte vector
};

// Loads the 16-byte vector starting at column c0 into f[], padding columns
// >= cols with `fill`.  ALIGNED means the row base is 16-byte aligned, so a
// full in-bounds vector is one dwordx4 load.
template <typename T, bool ALIGNED>
__device__ __forceinline__ void load_vec(const T* __restrict__ row, int64_t c0,
                                         int64_t cols, float fill,
                                         float (&f)[RowVec<T>::N]) {
  constexpr int N = RowVec<T>::N;
  if (ALIGNED && c0 + N <= cols) {
    typedef T vt __attribute__((ext_vector_type(N)));
    vt v = *reinterpret_cast<const vt*>(row + c0);
#pragma unroll
    for (int j = 0; j < N; ++j) f[j] = tof(v[j]);
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) f[j] = (c0 + j < cols) ? tof(row[c0 + j]) : fill;
  }
}

template <typename T, bool ALIGNED>
__device__ __forceinline__ void store_vec(T* __restrict__ row, int64_t c0,
                                          int64_t cols,
                                          const float (&f)[RowVec<T>::N]) {
  constexpr int N = RowVec<T>::N;
  if (ALIGNED && c0 + N <= cols) {
    typedef T vt __attribute__((ext_vector_type(N)));
    vt v;
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = fromf<T>(f[j]);
    *reinterpret_cast<vt*>(row + c0) = v;
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (c0 + j < cols) row[c0 + j] = fromf<T>(f[j]);
  }
}

// exp(x) for x <= 0 via the hardware exp2 (v_exp_f32): exp(x) = 2^(x*log2 e).
__device__ __forceinline__ float exp_f32(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

struct RowArgs {
  const void* x;
  int64_t ldx;
  void* y;
  int64_t ldy;
  const void* gamma;
  const void* beta;
  float* mean_out;
  float* rstd_out;
  int64_t rows;
  int64_t cols;
  float eps;
};

// One 16-byte vector of a row in its storage type.
template <typename T>
using RawVec = T __attribute__((ext_vector_type(RowVec<T>::N)));

// Loads the vector at column c0 in storage form, columns >= cols set to
// `fill`.  ALIGNED (16-byte aligned rows, cols a multiple of N): the vector
// lies wholly inside the row or wholly past it, and one dwordx4 load reads
// it.  A lane past the row loads column 0 instead (a valid address) and takes
// the fill, so no branch splits the wave's loads and all of them are in
// flight together.
//
// Row loads are plain (cacheable) and row stores nontemporal.  On a stream
// that reads and writes HBM at once this pairing ran fastest of the four
// (64 MiB copy, one box: plain loads + nontemporal stores 20.2 us,
// nontemporal both 22.2-22.6, nontemporal loads + plain stores 22.5, plain
// both 24.6); RMSNorm 22.1 -> 20.8 us and softmax 22.9 -> 20.9 us at
// 8192 x 4096 f16 with nontemporal loads replaced.  A read-only stream is the
// other way round (the GEMV's weights stay nontemporal).
template <typename T, bool ALIGNED>
__device__ __forceinline__ RawVec<T> load_raw(const T* __restrict__ row, int64_t c0,
                                              int64_t cols, T fill) {
  constexpr int N = RowVec<T>::N;
  if constexpr (ALIGNED) {
    const bool in = c0 < cols;
    const RawVec<T> v = *reinterpret_cast<const RawVec<T>*>(row + (in ? c0 : 0));
    return in ? v : RawVec<T>(fill);
  }
  RawVec<T> v;
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = (c0 + j < cols) ? row[c0 + j] : fill;
  return v;
}

template <typename T, bool ALIGNED>
__device__ __forceinline__ void store_raw(T* __restrict__ row, int64_t c0, int64_t cols,
                                          RawVec<T> v) {
  constexpr int N = RowVec<T>::N;
  if constexpr (ALIGNED) {
    if (c0 < cols) __builtin_nontemporal_store(v, reinterpret_cast<RawVec<T>*>(row + c0));
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j)
      if (c0 + j < cols) row[c0 + j] = v[j];
  }
}

// Makes the compiler treat the row registers as rewritten, so that each pass
// widens the stored values again instead of keeping fp32 copies of the
// whole row alive across passes (which would double the register count).
template <typename T, int VPL>
__device__ __forceinline__ void fresh(RawVec<T> (&v)[VPL]) {
#pragma unroll
  for (int i = 0; i < VPL; ++i) asm volatile("" : "+v"(v[i]));
}

// Register-resident kernel: each lane holds VPL vectors of the row in the
// storage type (f16/bf16 rows take half the registers of fp32 copies, so
// more waves fit per SIMD and more bytes are in flight).  Values are
// widened to fp32 as each pass reads them.
//
// FULL (chosen on the host): the rows are aligned and fill every slot,
// cols == VPL * 64 * N, so every access is a plain 16-byte vector and no
// padding logic is compiled.  The kernel that also handles partial rows
// holds more registers for that logic (LayerNorm f16 at 4096 columns: 107
// VGPRs, four waves per SIMD, against 62 and eight waves); measured 25.7
// against 25.2 us (8192 rows, one box).
//
// S > 1 (full rows only): S waves share a row, each holding every S-th
// vector, and the wave totals meet in LDS behind a barrier.  Each wave's
// chain of arithmetic after its loads is S times shorter, and that chain is
// what the last rows of the grid add after the last bytes land.  Every op
// takes it on full rows of 8 vectors per lane.  Measured (8192 x 4096 f16,
// one box, two alternating passes each): S = 1 against S = 2, RMSNorm
// 20.74 -> 20.20 us, LayerNorm 21.77 -> 20.70 us, softmax 20.86 -> 20.88 us;
// S = 2 against S = 4 (one row per workgroup), softmax 20.87 -> 19.96 us,
// RMSNorm 19.97 -> 19.84 us, LayerNorm 20.8 -> 20.94 us.  So softmax and
// RMSNorm take four waves per row and LayerNorm two.  (With nontemporal row
// loads S = 2 had gained softmax 23.1 -> 22.8 us and cost RMSNorm and
// LayerNorm 1.5 us each.)
template <typename T, int OP, int VPL, bool ALIGNED, bool FULL, int S = 1>
__global__ __launch_bounds__(256) void row_kernel(RowArgs a) {
  static_assert(!FULL || ALIGNED, "full rows are aligned rows");
  static_assert(S == 1 || (FULL && kRowWaves % S == 0), "split rows are full rows");
  constexpr int N = RowVec<T>::N;
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const int half = wv % S;  // this wave's share of the row
  // Softmax takes its row groups XCD-contiguously: workgroups are dispatched
  // round-robin over the 8 XCDs, so ordinal b (on XCD x = b % 8) takes group
  // x * (G / 8) + min(x, G % 8) + b / 8 of the G in the grid (a bijection),
  // and each XCD streams one contiguous eighth of the rows.  Measured at
  // 8192 x 4096 f16 (three alternating passes, one box): softmax 20.01-20.02
  // against 20.16-20.22 us; RMSNorm 19.90-19.97 against 19.89-19.91 and
  // LayerNorm 20.98-21.01 against 20.88-20.93, so those keep the plain order.
  int blk = blockIdx.x;
  if constexpr (OP == kSoftmax) {
    const int G = gridDim.x, x = blk & 7;
    blk = x * (G >> 3) + min(x, G & 7) + (blk >> 3);
  }
  const int64_t r = static_cast<int64_t>(blk) * (kRowWaves / S) + wv / S;
  if constexpr (S == 1) {
    if (r >= a.rows) return;  // whole wave leaves; no barriers below
  }
  // S > 1: a wave past the last row stays for the barriers, reads row 0 and
  // stores nothing.
  const bool valid = r < a.rows;
  const int64_t rv = valid ? r : 0;
  const T* __restrict__ xr = static_cast<const T*>(a.x) + rv * a.ldx;
  T* __restrict__ yr = static_cast<T*>(a.y) + rv * a.ldy;
  // Row total: the wave's, then (S > 1) the S waves' in a fixed order, so
  // every wave of the row holds the same value.  Each slot serves one
  // reduction of the kernel, so no slot is rewritten after the barrier.
  __shared__ float red[2][kRowWaves];
  auto row_reduce = [&](float x, auto op, int slot) {
    x = wave_reduce(x, op);
    if constexpr (S > 1) {
      if (lane == 0) red[slot][wv] = x;
      __syncthreads();
      const int base = (wv / S) * S;
      x = red[slot][base];
#pragma unroll
      for (int k = 1; k < S; ++k) x = op(x, red[slot][base + k]);
    }
    return x;
  };
  const int64_t cols = a.cols;
  const T* __restrict__ g = static_cast<const T*>(a.gamma);
  const T* __restrict__ b = static_cast<const T*>(a.beta);
  auto col0 = [&](int i) { return ((static_cast<int64_t>(i) * S + half) * 64 + lane) * N; };

  const T fill = static_cast<T>(OP == kSoftmax ? -__builtin_huge_valf() : 0.0f);
  // A row that fills every slot takes plain loads: with a fill select the
  // compiler puts each load in its own branch and waits for it before
  // issuing the next, so one load per wave would be in flight.
  constexpr bool full = FULL;
  auto plain = [&](const T* p, int i) {
    return *reinterpret_cast<const RawVec<T>*>(p + col0(i));
  };
  RawVec<T> v[VPL];
  if constexpr (full) {
#pragma unroll
    for (int i = 0; i < VPL; ++i)
      v[i] = *reinterpret_cast<const RawVec<T>*>(xr + col0(i));
  } else {
#pragma unroll
    for (int i = 0; i < VPL; ++i) v[i] = load_raw<T, ALIGNED>(xr, col0(i), cols, fill);
  }
  // gamma / beta vector i, read in the output pass (cache hits: every row
  // shares them), so no registers hold them while the row is in flight.
  auto gamma_at = [&](int i) {
    if (!g) return RawVec<T>(T(1));
    if constexpr (full) return plain(g, i);
    return load_raw<T, ALIGNED>(g, col0(i), cols, T(0));
  };
  auto beta_at = [&](int i) {
    if (!b) return RawVec<T>(T(0));
    if constexpr (full) return plain(b, i);
    return load_raw<T, ALIGNED>(b, col0(i), cols, T(0));
  };

  if constexpr (OP == kSoftmax) {
    // The row maximum is exact in the storage type, so f16 rows take it with
    // packed f16 max (two lanes per instruction) before widening once.
    float m;
    if constexpr (std::is_same<T, _Float16>::value) {
      RawVec<T> mv = v[0];
#pragma unroll
      for (int i = 1; i < VPL; ++i) mv = __builtin_elementwise_max(mv, v[i]);
      m = tof(mv[0]);
#pragma unroll
      for (int j = 1; j < N; ++j) m = fmaxf(m, tof(mv[j]));
    } else {
      m = -__builtin_huge_valf();
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int j = 0; j < N; ++j) m = fmaxf(m, tof(v[i][j]));
    }
    m = row_reduce(m, OpMax(), 0);
    fresh(v);
    // exp(x - m) = 2^(x*log2(e) - m*log2(e)): one (mixed-precision) fma per
    // element feeds the hardware exp2, once per element.  Each numerator is
    // rounded to the storage type in place of its input, and the fp32 sum
    // adds those rounded numerators: the reference's kernel computes
    // num = exp(z).to(x.dtype), denom = sum(num) in fp32, y = num / denom
    // (test/python/triton/test_softmax.py:64-66).  The row stays in the
    // registers it arrived in.
    // The output pass is one mixed-precision fma per element, x * inv +
    // (-0), with `nzero` hidden from the optimizer so it stays an fma (it
    // rounds exactly like the product).  Padded -inf columns give 0.
    // Measured (8192 x 4096 f16, one box): 23.2 us, against 23.4 us with
    // two exponentials per element (eight waves per SIMD either way).
    constexpr float kLog2e = 1.4426950408889634f;
    const float mb = -m * kLog2e;
    float nzero = -0.0f;
    asm volatile("" : "+v"(nzero));
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      RawVec<T> e;
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const float ej = __builtin_amdgcn_exp2f(fmaf(tof(v[i][j]), kLog2e, mb));
        e[j] = fromf<T>(ej);
        s += tof(e[j]);
      }
      // The numerators exist in the storage type here, one vector at a
      // time: otherwise the compiler sinks the roundings into the output
      // pass and keeps every fp32 exponential live (80 instead of 45 VGPRs).
      asm volatile("" : "+v"(e));
      v[i] = e;
    }
    s = row_reduce(s, OpSum(), 1);
    const float inv = 1.0f / s;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      RawVec<T> o;
#pragma unroll
      for (int j = 0; j < N; ++j) {
        // The pin keeps every element on the same two roundings (fp32, then
        // the storage type): left free, the backend fuses some of them into
        // a single-rounding v_fma_mixlo_f16 and not others.
        float p = fmaf(tof(v[i][j]), inv, nzero);
        asm volatile("" : "+v"(p));
        o[j] = fromf<T>(p);
      }
      if (valid) store_raw<T, ALIGNED>(yr, col0(i), cols, o);
    }
  } else if constexpr (OP == kRmsNorm) {
    // Every pass is written as fmas whose f16 operands gfx950 takes straight
    // into v_fma_mix_f32 (no separate widening).  `nzero` (-0) is hidden from
    // the optimizer so x*y + (-0) stays an fma: it rounds exactly like x*y,
    // the sign of zero included.  For f16 rows the backend folds the output
    // fma and the conversion into one v_fma_mix{lo,hi}_f16, which rounds
    // once to f16 instead of to fp32 and then to f16 (the two differ only
    // next to an f16 rounding midpoint, inside the tolerance; LayerNorm's
    // output is the same).  Measured (8192 x 4096 f16): 22.23 against
    // 22.30 us with widen-then-multiply, at the copy rate of its bytes.
    float nzero = -0.0f;
    asm volatile("" : "+v"(nzero));
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int j = 0; j < N; ++j) ss = fmaf(tof(v[i][j]), tof(v[i][j]), ss);
    ss = row_reduce(ss, OpSum(), 0);
    fresh(v);
    const float rstd = 1.0f / sqrtf(ss / static_cast<float>(cols) + a.eps);
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const RawVec<T> gi = gamma_at(i);
      RawVec<T> o;
#pragma unroll
      for (int j = 0; j < N; ++j)
        o[j] = fromf<T>(fmaf(fmaf(tof(v[i][j]), rstd, nzero), tof(gi[j]), nzero));
      if (valid) store_raw<T, ALIGNED>(yr, col0(i), cols, o);
    }
  } else {  // kLayerNorm
    // The row is widened into mixed-precision fmas as in RMSNorm: the sum as
    // fma(x, 1, s), the centred values as fma(x, 1, -mean) (x - mean,
    // rounded once), with `one` hidden from the optimizer so x*1 stays an
    // fma.  The output is fma((x - mean) * rstd, gamma, beta) from the same
    // centred value: it differs from separately rounded steps in the last
    // fp32 bit only.  (A form that folded the mean into one fma,
    // fma(fma(x, rstd, -mean*rstd), gamma, beta), saved an operation per
    // element but lost the cancellation: a constant row gave beta plus the
    // rounding error of mean*rstd instead of beta.)
    float one = 1.0f;
    asm volatile("" : "+v"(one));
    // A scheduling barrier closes each vector of every pass: the passes
    // then run vector by vector as written (measured 25.05 against 25.2 us).
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
#pragma unroll
      for (int j = 0; j < N; ++j) s = fmaf(tof(v[i][j]), one, s);
      __builtin_amdgcn_sched_barrier(0);
    }
    const float mean = row_reduce(s, OpSum(), 0) / static_cast<float>(cols);
    const float nmean = -mean;
    fresh(v);
    // Padding slots (columns >= cols, loaded as 0) must not add mean^2: a
    // row that fills every slot (a uniform branch) skips the per-element
    // test.  Measured (8192 x 4096 f16, one box): this form 27.2 us, a
    // per-vector test on partial sums 27.9 us (it frees registers, 65
    // instead of 108 VGPRs, but the extra waves do not help), per-element
    // test with a branch around every load 28.5-29.1 us.
    float q = 0.0f;
    if (full || cols == static_cast<int64_t>(VPL) * 64 * N) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
          const float d = fmaf(tof(v[i][j]), one, nmean);
          q = fmaf(d, d, q);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < VPL; ++i)
#pragma unroll
        for (int j = 0; j < N; ++j) {
          const float d = (col0(i) + j < cols) ? fmaf(tof(v[i][j]), one, nmean) : 0.0f;
          q = fmaf(d, d, q);
        }
    }
    const float var = row_reduce(q, OpSum(), 1) / static_cast<float>(cols);
    fresh(v);
    const float rstd = 1.0f / sqrtf(var + a.eps);
    if (lane == 0 && half == 0 && valid) {
      if (a.mean_out) a.mean_out[r] = mean;
      if (a.rstd_out) a.rstd_out[r] = rstd;
    }
#pragma unroll
    for (int i = 0; i < VPL; ++i) {
      const RawVec<T> gi = gamma_at(i), bi = beta_at(i);
      RawVec<T> o;
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const float d = fmaf(tof(v[i][j]), one, nmean);
        o[j] = fromf<T>(fmaf(d * rstd, tof(gi[j]), tof(bi[j])));
      }
      if (valid) store_raw<T, ALIGNED>(yr, col0(i), cols, o);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Streaming kernel for rows longer than the register budget: the row is
// re-read per pass (softmax 3: max, sum of rounded numerators, output;
// RMSNorm 2, LayerNorm 3).
template <typename T, int OP, bool ALIGNED>
__global__ __launch_bounds__(256) void row_kernel_stream(RowArgs a) {
  constexpr int N = RowVec<T>::N;
  const int lane = threadIdx.x & 63;
  const int64_t r = static_cast<int64_t>(blockIdx.x) * kRowWaves + (threadIdx.x >> 6);
  if (r >= a.rows) return;
  const T* __restrict__ xr = static_cast<const T*>(a.x) + r * a.ldx;
  T* __restrict__ yr = static_cast<T*>(a.y) + r * a.ldy;
  const int64_t cols = a.cols;
  const int64_t step = 64 * N;
  const T* __restrict__ g = static_cast<const T*>(a.gamma);
  const T* __restrict__ b = static_cast<const T*>(a.beta);

  float scale = 1.0f, shift = 0.0f;  // y = (x - shift) * scale [* g + b]
  float m = 0.0f;
  if constexpr (OP == kSoftmax) {
    // The row max, then the fp32 sum of the numerators rounded to the
    // storage type (the reference's arithmetic, as in row_kernel): an online
    // max/sum would rescale sums of unrounded numerators instead.
    float lm = -__builtin_huge_valf();
    for (int64_t c0 = lane * N; c0 < cols; c0 += step) {
      float f[N];
      load_vec<T, ALIGNED>(xr, c0, cols, -__builtin_huge_valf(), f);
#pragma unroll
      for (int j = 0; j < N; ++j) lm = fmaxf(lm, f[j]);
    }
    m = wave_reduce(lm, OpMax());
    float ls = 0.0f;
    for (int64_t c0 = lane * N; c0 < cols; c0 += step) {
      float f[N];
      load_vec<T, ALIGNED>(xr, c0, cols, -__builtin_huge_valf(), f);
#pragma unroll
      for (int j = 0; j < N; ++j) ls += tof(fromf<T>(exp_f32(f[j] - m)));
    }
    const float s = wave_reduce(ls, OpSum());
    scale = 1.0f / s;
  } else if constexpr (OP == kRmsNorm) {
    float ss = 0.0f;
    for (int64_t c0 = lane * N; c0 < cols; c0 += step) {
      float f[N];
      load_vec<T, ALIGNED>(xr, c0, cols, 0.0f, f);
#pragma unroll
      for (int j = 0; j < N; ++j) ss += f[j] * f[j];
    }
    ss = wave_reduce(ss, OpSum());
    scale = 1.0f / sqrtf(ss / static_cast<float>(cols) + a.eps);
  } else {
    float s = 0.0f;
    for (int64_t c0 = lane * N; c0 < cols; c0 += step) {
      float f[N];
      load_vec<T, ALIGNED>(xr, c0, cols, 0.0f, f);
#pragma unroll
      for (int j = 0; j < N; ++j) s += f[j];
    }
    const float mean = wave_reduce(s, OpSum()) / static_cast<float>(cols);
    float q = 0.0f;
    for (int64_t c0 = lane * N; c0 < cols; c0 += step) {
      float f[N];
      load_vec<T, ALIGNED>(xr, c0, cols, 0.0f, f);
#pragma unroll
      for (int j = 0; j < N; ++j) {
        const float d = (c0 + j < cols) ? f[j] - mean : 0.0f;
        q += d * d;
      }
    }
    const float var = wave_reduce(q, OpSum()) / static_cast<float>(cols);
    shift = mean;
    scale = 1.0f / sqrtf(var + a.eps);
    if (lane == 0) {
      if (a.mean_out) a.mean_out[r] = mean;
      if (a.rstd_out) a.rstd_out[r] = scale;
    }
  }

  for (int64_t c0 = lane * N; c0 < cols; c0 += step) {
    float f[N];
    load_vec<T, ALIGNED>(xr, c0, cols, 0.0f, f);
    if constexpr (OP == kSoftmax) {
#pragma unroll
      for (int j = 0; j < N; ++j) f[j] = tof(fromf<T>(exp_f32(f[j] - m))) * scale;
    } else if constexpr (OP == kRmsNorm) {
      float gv[N];
      if (g) load_vec<T, ALIGNED>(g, c0, cols, 0.0f, gv);
#pragma unroll
      for (int j = 0; j < N; ++j) f[j] = (f[j] * scale) * (g ? gv[j] : 1.0f);
    } else {
      float gv[N], bv[N];
      if (g) load_vec<T, ALIGNED>(g, c0, cols, 0.0f, gv);
      if (b) load_vec<T, ALIGNED>(b, c0, cols, 0.0f, bv);
#pragma unroll
      for (int j = 0; j < N; ++j)
        f[j] = (f[j] - shift) * scale * (g ? gv[j] : 1.0f) + (b ? bv[j] : 0.0f);
    }
    store_vec<T, ALIGNED>(yr, c0, cols, f);
  }
}

namespace {

template <typename T, int OP, bool ALIGNED>
hxm_status launch_rows_t(const RowArgs& a, hipStream_t stream) {
  constexpr int N = RowVec<T>::N;
  const int64_t vpl = (a.cols + 64 * N - 1) / (64 * N);
  // Full rows of 8 vectors per lane: SPLIT waves per row, four for softmax
  // and RMSNorm, two for LayerNorm (its two dependent reductions cross the
  // LDS twice).
  constexpr int SPLIT = OP == kLayerNorm ? 2 : 4;
  const bool split = ALIGNED && a.cols == 8 * 64 * N;
  const int64_t rows_per_group = split ? kRowWaves / SPLIT : kRowWaves;
  const int64_t groups = (a.rows + rows_per_group - 1) / rows_per_group;
  hxm_status st = check_grid("row kernel", groups, 64 * kRowWaves);
  if (st != HXM_OK) return st;
  const dim3 grid(static_cast<unsigned>(groups));
  const dim3 block(64 * kRowWaves);
  // FULL kernels for aligned rows that fill the VPL slots exactly.
  auto run = [&](auto VPLC) {
    constexpr int V = decltype(VPLC)::value;
    if constexpr (ALIGNED && V == 8) {
      if (split) {
        row_kernel<T, OP, V / SPLIT, true, true, SPLIT><<<grid, block, 0, stream>>>(a);
        return;
      }
    }
    if (ALIGNED && a.cols == static_cast<int64_t>(V) * 64 * N)
      row_kernel<T, OP, V, ALIGNED, ALIGNED><<<grid, block, 0, stream>>>(a);
    else
      row_kernel<T, OP, V, ALIGNED, false><<<grid, block, 0, stream>>>(a);
  };
  if (vpl <= 1)
    run(std::integral_constant<int, 1>{});
  else if (vpl <= 2)
    run(std::integral_constant<int, 2>{});
  else if (vpl <= 4)
    run(std::integral_constant<int, 4>{});
  else if (vpl <= 8)
    run(std::integral_constant<int, 8>{});
  else if (vpl <= 16)
    run(std::integral_constant<int, 16>{});
  else
    row_kernel_stream<T, OP, ALIGNED><<<grid, block, 0, stream>>>(a);
  return check_launch("row kernel");
}

template <int OP>
hxm_status launch_rows(const RowArgs& a, int32_t dtype, hipStream_t stream) {
  const int64_t eb = dtype_bytes(dtype);
  // ALIGNED kernels: 16-byte aligned rows whose length is a whole number of
  // 16-byte vectors.
  bool al = aligned16(a.x) && aligned16(a.y) && (a.ldx * eb) % 16 == 0 &&
            (a.ldy * eb) % 16 == 0 && (!a.gamma || aligned16(a.gamma)) &&
            (!a.beta || aligned16(a.beta)) && (a.cols * eb) % 16 == 0;
  switch (dtype) {
    case HXM_F16:
      return al ? launch_rows_t<_Float16, OP, true>(a, stream)
                : launch_rows_t<_Float16, OP, false>(a, stream);
    case HXM_BF16:
      return al ? launch_rows_t<__bf16, OP, true>(a, stream)
                : launch_rows_t<__bf16, OP, false>(a, stream);
    default:
      return al ? launch_rows_t<float, OP, true>(a, stream)
                : launch_rows_t<float, OP, false>(a, stream);
  }
}

hxm_status validate_rows(const char* op, const void* x, int64_t ldx,
                         const void* y, int64_t ldy, int64_t rows,
                         int64_t cols, int32_t dtype) {
  if (dtype != HXM_F16 && dtype != HXM_BF16 && dtype != HXM_F32)
    return fail(HXM_UNSUPPORTED_DTYPE,
                "unsupported-dtype: %s takes f16, bf16 or f32 (got %d)", op,
                dtype);
  if (rows < 0 || cols < 1)
    return fail(HXM_INVALID_ARG, "invalid-argument: %s rows=%lld cols=%lld",
                op, (long long)rows, (long long)cols);
  if (rows > 0 && (!x || !y))
    return fail(HXM_INVALID_ARG, "invalid-argument: %s null x or y", op);
  if (ldx < cols || ldy < cols)
    return fail(HXM_INVALID_ARG,
                "invalid-argument: %s ldx=%lld ldy=%lld < cols=%lld", op,
                (long long)ldx, (long long)ldy, (long long)cols);
  if (rows > (int64_t(1) << 33))
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: %s rows=%lld too many",
                op, (long long)rows);
  return HXM_OK;
}

}  // namespace
}  // namespace hxm

using namespace hxm;

extern "C" {

hxm_status hxm_softmax_rows(const void* x, int64_t ldx, void* y, int64_t ldy,
                            int64_t rows, int64_t cols, int32_t dtype,
                            void* stream) {
  hxm_status st = validate_rows("softmax", x, ldx, y, ldy, rows, cols, dtype);
  if (st != HXM_OK) return st;
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (rows == 0) return ok();
  RowArgs a{x, ldx, y, ldy, nullptr, nullptr, nullptr, nullptr, rows, cols, 0.0f};
  return launch_rows<kSoftmax>(a, dtype, as_stream(stream));
}

hxm_status hxm_rmsnorm_rows(const void* x, int64_t ldx, const void* gamma,
                            void* y, int64_t ldy, int64_t rows, int64_t cols,
                            float eps, int32_t dtype, void* stream) {
  hxm_status st = validate_rows("rmsnorm", x, ldx, y, ldy, rows, cols, dtype);
  if (st != HXM_OK) return st;
  if (!(eps >= 0.0f))
    return fail(HXM_INVALID_ARG, "invalid-argument: rmsnorm eps must be >= 0");
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (rows == 0) return ok();
  RowArgs a{x, ldx, y, ldy, gamma, nullptr, nullptr, nullptr, rows, cols, eps};
  return launch_rows<kRmsNorm>(a, dtype, as_stream(stream));
}

hxm_status hxm_layernorm_rows(const void* x, int64_t ldx, const void* gamma,
                              const void* beta, void* y, int64_t ldy,
                              float* mean_out, float* rstd_out, int64_t rows,
                              int64_t cols, float eps, int32_t dtype,
                              void* stream) {
  hxm_status st = validate_rows("layernorm", x, ldx, y, ldy, rows, cols, dtype);
  if (st != HXM_OK) return st;
  if (!(eps >= 0.0f))
    return fail(HXM_INVALID_ARG, "invalid-argument: layernorm eps must be >= 0");
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (rows == 0) return ok();
  RowArgs a{x, ldx, y, ldy, gamma, beta, mean_out, rstd_out, rows, cols, eps};
  return launch_rows<kLayerNorm>(a, dtype, as_stream(stream));
}

}  // extern "C"
