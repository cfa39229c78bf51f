// HBM probes: a streaming copy and a streaming read with the same access
// pattern as the HBM-bound kernels of this library (16-byte nontemporal
// accesses, several in flight per lane).  They measure the practical
// ceiling those kernels are compared against; they have no counterpart in
// the reference.
#include "device_util.h"
#include "hxm_internal.h"

namespace hxm {

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 4;  // 16-byte vectors in flight per lane

// Lane `t` of `threads` handles vectors t, t + threads, ... ; each pass
// issues kProbeUnroll loads before any store.
__global__ __launch_bounds__(kProbeThreads) void stream_copy_kernel(
    const v4u32_t* __restrict__ src, v4u32_t* __restrict__ dst, int64_t n16) {
  const int64_t threads = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  for (; i + (kProbeUnroll - 1) * threads < n16; i += kProbeUnroll * threads) {
    v4u32_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * threads);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) __builtin_nontemporal_store(v[u], dst + i + u * threads);
  }
  for (; i < n16; i += threads) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Folds every loaded word into one value per lane; the value is stored only
// when it equals `never`, which the compiler cannot rule out, so the loads
// stay and almost nothing is written.
__global__ __launch_bounds__(kProbeThreads) void stream_read_kernel(
    const v4u32_t* __restrict__ src, int64_t n16, uint32_t never, uint32_t* __restrict__ sink) {
  const int64_t threads = static_cast<int64_t>(gridDim.x) * kProbeThreads;
  int64_t i = static_cast<int64_t>(blockIdx.x) * kProbeThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kProbeUnroll - 1) * threads < n16; i += kProbeUnroll * threads) {
    v4u32_t v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(src + i + u * threads);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  for (; i < n16; i += threads) {
    const v4u32_t v = __builtin_nontemporal_load(src + i);
    acc ^= v[0] ^ v[1] ^ v[2] ^ v[3];
  }
  if (acc == never) sink[blockIdx.x] = acc;
}

// One pass of kProbeUnroll vectors per lane, capped at HXM_PROBE_SINK_WORDS
// workgroups (32 per CU); larger buffers loop.
int64_t probe_groups(int64_t n16) {
  const int64_t want = (n16 + kProbeThreads * kProbeUnroll - 1) / (kProbeThreads * kProbeUnroll);
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

}  // extern "C"
