// Device-side helpers for gfx950 kernels: 16-byte vector types, element
// conversions and 64-lane wave reductions built from DPP row operations plus
// cross-row readlanes (the GPU analogue of the hvx.vror rotate-and-fold
// butterfly, qcom_hexagon_backend/lib/Conversion/LinalgToLLVM/
// VectorRowReducePass.cpp:10-31).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace hxm {

typedef int32_t v4i32 __attribute__((ext_vector_type(4)));
typedef int32_t v16i32 __attribute__((ext_vector_type(16)));
typedef float v4f32 __attribute__((ext_vector_type(4)));
typedef float v16f32 __attribute__((ext_vector_type(16)));
typedef _Float16 v8f16 __attribute__((ext_vector_type(8)));
typedef __bf16 v8bf16 __attribute__((ext_vector_type(8)));
typedef _Float16 v2f16 __attribute__((ext_vector_type(2)));
typedef _Float16 v4f16_t __attribute__((ext_vector_type(4)));
typedef __bf16 v4bf16_t __attribute__((ext_vector_type(4)));
typedef uint32_t v4u32_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float tof(_Float16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float tof(__bf16 v) { return static_cast<float>(v); }
__device__ __forceinline__ float tof(float v) { return v; }

template <typename T>
__device__ __forceinline__ T fromf(float v) { return static_cast<T>(v); }

// DPP controls (GCN/CDNA encoding).
constexpr int kDppQuadXor1 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xF, 0xF, true));
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const {
    return fmaxf(a, b);
  }
};
struct OpSum {
  __device__ __forceinline__ float operator()(float a, float b) const {
    return a + b;
  }
};

// Reduces v over all 64 lanes; the result is wave-uniform.  Inside each
// 16-lane row: xor-1, xor-2, half-mirror, mirror (every lane ends with its
// row's total); across rows: four readlanes folded pairwise.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
  v = op(v, dpp<kDppQuadXor1>(v));
  v = op(v, dpp<kDppQuadXor2>(v));
  v = op(v, dpp<kDppRowHalfMirror>(v));
  v = op(v, dpp<kDppRowMirror>(v));
  float a = op(readlane(v, 0), readlane(v, 16));
  float b = op(readlane(v, 32), readlane(v, 48));
  return op(a, b);
}

// Two int8 -> two exact f16 (one packed word).  flipped is a dword of four
// int8 with every sign bit inverted (x ^ 0x80808080); H selects bytes 0-1
// (H = 0) or 2-3 (H = 1).  (b ^ 0x80) | 0x6400 is the f16 1024 + b + 128;
// subtracting 1152 leaves b exactly.
template <int H>
__device__ __forceinline__ uint32_t i8x2_flipped_to_f16(uint32_t flipped) {
  const uint32_t w =
      __builtin_amdgcn_perm(0x64646464u, flipped, H == 0 ? 0x05010400u : 0x05030402u);
  const v2f16 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
  return __builtin_bit_cast(uint32_t, __builtin_bit_cast(v2f16, w) - bias);
}

// 8 int8 (two dwords) -> 8 exact f16.  OFFSET_BINARY: the bytes are already
// w ^ 0x80 (the packed GEMV image stores them so), and the flip is skipped.
template <bool OFFSET_BINARY>
__device__ __forceinline__ v8f16 i8x8_to_f16(uint32_t lo, uint32_t hi) {
  if constexpr (!OFFSET_BINARY) {
    lo ^= 0x80808080u;
    hi ^= 0x80808080u;
  }
  v4i32 r;
  r[0] = static_cast<int>(i8x2_flipped_to_f16<0>(lo));
  r[1] = static_cast<int>(i8x2_flipped_to_f16<1>(lo));
  r[2] = static_cast<int>(i8x2_flipped_to_f16<0>(hi));
  r[3] = static_cast<int>(i8x2_flipped_to_f16<1>(hi));
  return __builtin_bit_cast(v8f16, r);
}

}  // namespace hxm
