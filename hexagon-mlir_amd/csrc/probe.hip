// HBM probes: a streaming copy and a streaming read with the same access
// pattern as the HBM-bound kernels of this library (16-byte accesses, eight
// in flight per lane): the copy loads plainly and stores nontemporally, as
// the row kernels do; the read loads nontemporally, as the GEMV streams its
// weights.  Each pairing is the faster one for its kind of stream (a copy
// with nontemporal loads ran 22.2-22.6 us against 20.2 us for 64 MiB; a read
// with plain loads 8.4 against 8.15 us for 45 MB).  They measure the
// practical ceiling those kernels are compared against; they have no
// counterpart in the reference.
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

}  // extern "C"
