// Ceiling probes.  MFMA: the matrix cores alone, fed a GEMM's own operand
// bytes, with the GEMM kernels' occupancy (one wave per SIMD) and their MFMA
// shapes; it measures what the power-limited clock leaves of the dense peak
// for that data, the practical ceiling of the MFMA-bound kernels.
//
// HBM probes: a streaming copy and a streaming read with the same access
// pattern as the HBM-bound kernels of this library (16-byte accesses, eight
// in flight per lane): the copy loads plainly and stores nontemporally, as
// the row kernels do; the read loads nontemporally, as the GEMV streams its
// weights.  Each pairing is the faster one for its kind of stream (a copy
// with nontemporal loads ran 22.2-22.6 us against 20.2 us for 64 MiB; a read
// with plain loads 8.4 against 8.15 us for 45 MB).  They measure the
// practical ceiling those kernels are compared against; they have no
// counterpart in the reference.
#include <type_traits>

#include "device_util.h"
#include "hxm_internal.h"

namespace hxm {

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;  // 16-byte vectors in flight per lane
constexpr int64_t kProbeChunk = int64_t(kProbeThreads) * kProbeUnroll;  // vectors per pass

// Workgroup w owns chunks w, w + groups, ... of kProbeChunk vectors; inside a
// chunk lane t takes vectors t, t + 256, ... (every load instruction of the
// workgroup covers 4 KiB contiguous), all kProbeUnroll loads issued before
// any store -- the access pattern of the row kernels, one row per wave.
__global__ __launch_bounds__(kProbeThreads) void stream_copy_kernel(
    const v4u32_t* __restrict__ src, v4u32_t* __restrict__ dst, int64_t n16) {
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kProbeChunk; c < n16;
       c += static_cast<int64_t>(gridDim.x) * kProbeChunk) {
    const int64_t i = c + threadIdx.x;
    if (c + kProbeChunk <= n16) {
      v4u32_t v[kProbeUnroll];
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u)
        v[u] = src[i + u * kProbeThreads];
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u)
        __builtin_nontemporal_store(v[u], dst + i + u * kProbeThreads);
    } else {
      for (int u = 0; u < kProbeUnroll; ++u)
        if (i + u * kProbeThreads < n16)
          __builtin_nontemporal_store(src[i + u * kProbeThreads],
                                      dst + i + u * kProbeThreads);
    }
  }
}

// The same walk, reading only: every loaded word is folded into one value
// per lane, which is stored only when it equals `never` -- a value the
// compiler cannot rule out, so the loads stay, and almost nothing is written.
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(
    const v4u32_t* __restrict__ src, int64_t n16, uint32_t never, uint32_t* __restrict__ sink) {
  uint32_t acc = 0;
  for (int64_t c = static_cast<int64_t>(blockIdx.x) * kProbeChunk; c < n16;
       c += static_cast<int64_t>(gridDim.x) * kProbeChunk) {
    const int64_t i = c + threadIdx.x;
    v4u32_t v[kProbeUnroll];
    if (c + kProbeChunk <= n16) {
#pragma unroll
      for (int u = 0; u < kProbeUnroll; ++u)
        v[u] = __builtin_nontemporal_load(src + i + u * kProbeThreads);
    } else {
      for (int u = 0; u < kProbeUnroll; ++u)
        v[u] = i + u * kProbeThreads < n16 ? __builtin_nontemporal_load(src + i + u * kProbeThreads)
                                           : v4u32_t{};
    }
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == never) sink[blockIdx.x] = acc;
}

// MFMA probe.  Each wave takes two sets of four A and four B fragments
// (16 bytes per lane each) from the operand bytes -- wave w reads A bytes
// [8 KiB * w, +8 KiB) and the same window of B, wrapped at the buffers' ends
// -- and then runs `steps` rounds of 2 x 16 MFMAs over a 4 x 4 grid of 32x32
// accumulator blocks, the sets alternating and the blocks in the GEMM
// kernels' snake order, so every instruction shares one operand with the one
// before it and no more (the operand toggling, and so the power, of a GEMM's
// k-steps).  MODE: 0 int8 x int8 (v_mfma_i32_32x32x32_i8), 1 f16,
// 2 bf16 (v_mfma_f32_32x32x16_*), 3 f16 x int8 (B bytes converted exactly to
// f16 once, as the W8A16 kernels convert theirs).  Every accumulator is
// folded into one word per lane, stored only when it equals `never`, so the
// MFMAs stay and almost nothing is written.
template <int MODE>
__global__ __launch_bounds__(256) void mfma_probe_kernel(const uint8_t* __restrict__ a,
                                                          int64_t a16, const uint8_t* __restrict__ b,
                                                          int64_t b16, int64_t steps,
                                                          uint32_t never, uint32_t* __restrict__ sink) {
  const int lane = threadIdx.x & 63;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  v4i32 fa[2][4], fb[2][4];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int64_t off = w * 8192 + j * 1024 + lane * 16;
    fa[j / 4][j % 4] = *reinterpret_cast<const v4i32*>(a + (off % a16));
    fb[j / 4][j % 4] = *reinterpret_cast<const v4i32*>(b + (off % b16));
    if constexpr (MODE == 3) {  // 16 int8 -> the 8 f16 of the first 8 bytes
      const v8f16 h = i8x8_to_f16<false>(static_cast<uint32_t>(fb[j / 4][j % 4][0]),
                                         static_cast<uint32_t>(fb[j / 4][j % 4][1]));
      fb[j / 4][j % 4] = __builtin_bit_cast(v4i32, h);
    }
  }
  using acc_t = typename std::conditional<MODE == 0, v16i32, v16f32>::type;
  acc_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = acc_t{};
  for (int64_t it = 0; it < steps; ++it) {
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int j = (i & 1) ? 3 - jj : jj;  // the GEMM kernels' snake order
          if constexpr (MODE == 0)
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[s][j], fa[s][i], acc[i][j], 0, 0, 0);
          else if constexpr (MODE == 2)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                __builtin_bit_cast(v8bf16, fb[s][j]), __builtin_bit_cast(v8bf16, fa[s][i]),
                acc[i][j], 0, 0, 0);
          else
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                __builtin_bit_cast(v8f16, fb[s][j]), __builtin_bit_cast(v8f16, fa[s][i]),
                acc[i][j], 0, 0, 0);
        }
  }
  uint32_t fold = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const auto v = acc[i][j][e];  // copy the element out (see gemm_kernel.h)
        fold ^= __builtin_bit_cast(uint32_t, v);
      }
  if (fold == never) sink[blockIdx.x] = fold;
}

// One chunk per workgroup, at most HXM_PROBE_SINK_WORDS workgroups (32 per
// CU); larger buffers loop.
int64_t probe_groups(int64_t n16) {
  const int64_t want = (n16 + kProbeChunk - 1) / kProbeChunk;
  return want < 1 ? 1 : want > HXM_PROBE_SINK_WORDS ? HXM_PROBE_SINK_WORDS : want;
}

hxm_status check_probe(const char* op, const void* p, int64_t bytes) {
  if (bytes < 0 || bytes % 16) return fail(HXM_INVALID_ARG, "invalid-argument: %s bytes", op);
  if (bytes > 0 && (!p || !aligned16(p)))
    return fail(HXM_INVALID_ARG, "invalid-argument: %s needs 16-byte aligned buffers", op);
  return HXM_OK;
}

}  // namespace
}  // namespace hxm

using namespace hxm;

extern "C" {

hxm_status hxm_probe_copy(const void* src, void* dst, int64_t bytes, void* stream) {
  hxm_status st = check_probe("probe_copy", src, bytes);
  if (st != HXM_OK || (st = check_probe("probe_copy", dst, bytes)) != HXM_OK) return st;
  const uintptr_t s0 = reinterpret_cast<uintptr_t>(src), d0 = reinterpret_cast<uintptr_t>(dst);
  if (bytes > 0 && s0 < d0 + static_cast<uintptr_t>(bytes) &&
      d0 < s0 + static_cast<uintptr_t>(bytes))
    return fail(HXM_INVALID_ARG, "invalid-argument: probe_copy buffers overlap");
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (bytes == 0) return ok();
  const int64_t n16 = bytes / 16;
  stream_copy_kernel<<<static_cast<unsigned>(probe_groups(n16)), kProbeThreads, 0,
                       as_stream(stream)>>>(static_cast<const v4u32_t*>(src),
                                            static_cast<v4u32_t*>(dst), n16);
  return check_launch("probe_copy");
}

hxm_status hxm_probe_read(const void* src, int64_t bytes, uint32_t* sink, void* stream) {
  hxm_status st = check_probe("probe_read", src, bytes);
  if (st != HXM_OK) return st;
  if (bytes > 0 && !sink) return fail(HXM_INVALID_ARG, "invalid-argument: probe_read sink");
  if ((st = require_device(nullptr)) != HXM_OK) return st;
  if (bytes == 0) return ok();
  const int64_t n16 = bytes / 16;
  // A fold equal to all ones writes one word per workgroup (at most
  // HXM_PROBE_SINK_WORDS): rare, bounded and harmless to the measurement.
  stream_read_kernel<<<static_cast<unsigned>(probe_groups(n16)), kProbeThreads, 0,
                       as_stream(stream)>>>(static_cast<const v4u32_t*>(src), n16, 0xffffffffu,
                                            sink);
  return check_launch("probe_read");
}

hxm_status hxm_probe_mfma(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes,
                          int32_t a_dtype, int32_t b_dtype, int64_t mfma_per_wave,
                          int32_t workgroups, uint32_t* sink, void* stream) {
  int mode = -1;
  if (a_dtype == HXM_I8 && b_dtype == HXM_I8) mode = 0;
  else if (a_dtype == HXM_F16 && b_dtype == HXM_F16) mode = 1;
  else if (a_dtype == HXM_BF16 && b_dtype == HXM_BF16) mode = 2;
  else if (a_dtype == HXM_F16 && b_dtype == HXM_I8) mode = 3;
  if (mode < 0)
    return fail(HXM_UNSUPPORTED_DTYPE,
                "unsupported-dtype: probe_mfma takes int8 x int8, f16 x f16, bf16 x bf16 or "
                "f16 x int8 (got %d x %d)", a_dtype, b_dtype);
  if (a_bytes < 16 || b_bytes < 16 || a_bytes % 16 || b_bytes % 16)
    return fail(HXM_INVALID_ARG, "invalid-argument: probe_mfma operand bytes must be positive "
                                 "multiples of 16");
  if (!a || !b || !aligned16(a) || !aligned16(b) || !sink)
    return fail(HXM_INVALID_ARG, "invalid-argument: probe_mfma needs 16-byte aligned operands "
                                 "and a sink");
  // At most 2^24 MFMAs per wave (about a third of a second per launch at the
  // clock this load runs at), so one launch cannot hold the device for long.
  if (mfma_per_wave <= 0 || mfma_per_wave % 32 || mfma_per_wave > (int64_t(1) << 24))
    return fail(HXM_INVALID_ARG, "invalid-argument: probe_mfma mfma_per_wave must be a positive "
                                 "multiple of 32, at most 2^24 (got %lld)",
                (long long)mfma_per_wave);
  if (workgroups < 1 || workgroups > HXM_PROBE_SINK_WORDS)
    return fail(HXM_INVALID_ARG, "invalid-argument: probe_mfma workgroups in [1, %d]",
                HXM_PROBE_SINK_WORDS);
  hxm_status st = require_device(nullptr);
  if (st != HXM_OK) return st;
  const int64_t steps = mfma_per_wave / 32;
  const uint8_t* pa = static_cast<const uint8_t*>(a);
  const uint8_t* pb = static_cast<const uint8_t*>(b);
  hipStream_t s = as_stream(stream);
  switch (mode) {
    case 0: mfma_probe_kernel<0><<<workgroups, 256, 0, s>>>(pa, a_bytes, pb, b_bytes, steps, 0xffffffffu, sink); break;
    case 1: mfma_probe_kernel<1><<<workgroups, 256, 0, s>>>(pa, a_bytes, pb, b_bytes, steps, 0xffffffffu, sink); break;
    case 2: mfma_probe_kernel<2><<<workgroups, 256, 0, s>>>(pa, a_bytes, pb, b_bytes, steps, 0xffffffffu, sink); break;
    default: mfma_probe_kernel<3><<<workgroups, 256, 0, s>>>(pa, a_bytes, pb, b_bytes, steps, 0xffffffffu, sink); break;
  }
  return check_launch("probe_mfma");
}

}  // extern "C"
