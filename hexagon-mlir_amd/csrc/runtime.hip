// Library runtime: status strings, the per-thread reason record, device
// admission and the per-stream workspace (the library-owned counterpart of
// the reference's VTCM pool, bin/runtime/include/HexagonCAPI.h:26-57 --
// allocated once, kept for the process until released).
#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "hxm_internal.h"

namespace hxm {

namespace {
thread_local std::string g_last_error;

struct Workspace {
  void* ptr = nullptr;
  size_t bytes = 0;
};
std::mutex g_ws_mu;
// One buffer per (device, stream handle, slot).  The handle is compared as a
// value: the null stream (0) and the special handles such as
// hipStreamLegacy (1) are keys like any other.
typedef std::tuple<int, uintptr_t, int> WsKey;
std::map<WsKey, Workspace> g_ws;

std::mutex g_dev_mu;
std::vector<int8_t> g_dev_ok;  // -1 unknown, 0 not gfx950, 1 ok
}  // namespace

hxm_status fail(hxm_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return st;
}

hxm_status ok() {
  g_last_error.clear();
  return HXM_OK;
}

hxm_status check_grid(const char* what, int64_t groups_x, int threads, int64_t groups_y) {
  if (grid_fits(groups_x, threads, groups_y)) return HXM_OK;
  return fail(HXM_UNSUPPORTED_SHAPE,
              "tile-alignment: %s needs a grid of %lld x %lld workgroups of %d threads, beyond "
              "the launch limit",
              what, (long long)groups_x, (long long)groups_y, threads);
}

hxm_status check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return fail(HXM_HIP_ERROR, "hip-error: launch of %s failed: %s", what,
                hipGetErrorString(e));
  return ok();
}

hxm_status require_device(int* device_out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(HXM_NO_DEVICE, "no-device: hipGetDevice failed: %s",
                hipGetErrorString(e));
  std::lock_guard<std::mutex> lk(g_dev_mu);
  if ((int)g_dev_ok.size() <= dev) g_dev_ok.resize(dev + 1, -1);
  if (g_dev_ok[dev] < 0) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
      return fail(HXM_NO_DEVICE, "no-device: hipGetDeviceProperties failed");
    g_dev_ok[dev] = (std::string(prop.gcnArchName).rfind("gfx950", 0) == 0) ? 1 : 0;
  }
  if (!g_dev_ok[dev])
    return fail(HXM_NO_DEVICE, "no-device: device %d is not gfx950", dev);
  if (device_out) *device_out = dev;
  return HXM_OK;
}

int device_cu_count() {
  static std::mutex mu;
  static std::vector<int> cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lk(mu);
  if (static_cast<int>(cus.size()) <= dev) cus.resize(dev + 1, -1);
  if (cus[dev] < 0) {
    int n = 0;
    cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess
                   ? n
                   : 0;
  }
  return cus[dev];
}

hxm_status stream_workspace(hipStream_t stream, size_t bytes, void** out, int slot, bool* grown) {
  int dev = 0;
  if (grown) *grown = false;
  HXM_HIP_TRY(hipGetDevice(&dev));
  if (slot != kWsMain && slot != kWsSplitK && slot != kWsStreamK)
    return fail(HXM_INVALID_ARG, "invalid-argument: workspace slot %d", slot);
  const WsKey key(dev, reinterpret_cast<uintptr_t>(stream), slot);
  std::lock_guard<std::mutex> lk(g_ws_mu);
  Workspace& w = g_ws[key];
  if (w.bytes < bytes) {
    // Growing needs hipMalloc (and a stream synchronisation to retire the old
    // buffer), neither of which a stream under graph capture allows.  A query
    // that fails counts as a capture: the null stream, for one, reports an
    // implicit-capture error while another stream captures in global mode,
    // and a synchronisation or hipMalloc then would invalidate that capture.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t qe = hipStreamIsCapturing(stream, &cap);
    if (qe != hipSuccess) (void)hipGetLastError();  // clear the sticky query error
    if (qe != hipSuccess || cap != hipStreamCaptureStatusNone)
      return fail(HXM_UNSUPPORTED_SHAPE,
                  "workspace-budget: the stream is capturing a graph (or its capture state "
                  "cannot be read: %s) and its workspace must grow from %zu to %zu bytes; "
                  "make one call of this shape on the stream before capturing (the workspace "
                  "is kept), or use hxm_gemm_i8_noalloc",
                  qe == hipSuccess ? "capturing" : hipGetErrorString(qe), w.bytes, bytes);
    if (w.ptr) {
      // The old buffer may still be read by work queued on this stream.
      HXM_HIP_TRY(hipStreamSynchronize(stream));
      HXM_HIP_TRY(hipFree(w.ptr));
      w.ptr = nullptr;
      w.bytes = 0;
    }
    size_t grow = bytes < (size_t(1) << 20) ? (size_t(1) << 20) : bytes;
    if (hipMalloc(&w.ptr, grow) != hipSuccess) {
      w.ptr = nullptr;
      return fail(HXM_OUT_OF_MEMORY, "out-of-memory: workspace of %zu bytes",
                  grow);
    }
    w.bytes = grow;
    if (grown) *grown = true;
  }
  *out = w.ptr;
  return HXM_OK;
}

}  // namespace hxm

extern "C" {

const char* hxm_status_string(int32_t status) {
  switch (status) {
    case HXM_OK: return "ok";
    case HXM_INVALID_ARG: return "invalid-argument";
    case HXM_UNSUPPORTED_DTYPE: return "unsupported-dtype";
    case HXM_UNSUPPORTED_SHAPE: return "unsupported-shape";
    case HXM_HIP_ERROR: return "hip-error";
    case HXM_OUT_OF_MEMORY: return "out-of-memory";
    case HXM_NO_DEVICE: return "no-device";
    default: return "unknown-status";
  }
}

const char* hxm_last_error(void) { return hxm::g_last_error.c_str(); }

const char* hxm_version(void) { return "hxm 0.1.0 gfx950"; }

int32_t hxm_device_count(void) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) return 0;
  int count = 0;
  for (int d = 0; d < n; ++d) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, d) == hipSuccess &&
        std::string(prop.gcnArchName).rfind("gfx950", 0) == 0)
      ++count;
  }
  return count;
}

hxm_status hxm_release_cache(void) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return hxm::ok();
  HXM_HIP_TRY(hipDeviceSynchronize());
  hxm_status st = hxm::release_images(dev);
  if (st != HXM_OK) return st;
  std::lock_guard<std::mutex> lk(hxm::g_ws_mu);
  for (auto it = hxm::g_ws.begin(); it != hxm::g_ws.end();) {
    if (std::get<0>(it->first) == dev) {
      if (it->second.ptr) HXM_HIP_TRY(hipFree(it->second.ptr));
      it = hxm::g_ws.erase(it);
    } else {
      ++it;
    }
  }
  return hxm::ok();
}

}  // extern "C"
