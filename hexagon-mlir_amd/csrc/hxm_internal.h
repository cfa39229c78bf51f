// Internal helpers shared by the HIP translation units of libhxm: status and
// reason reporting, dtype sizes, launch checks and the library-owned
// per-stream workspace.  Nothing here is part of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/hxm.h"
#include "host_logic.h"

namespace hxm {

// Records `reason` as this thread's last error and returns `st`.  Reasons
// start with the manifest vocabulary word ("tile-alignment", ...) so that a
// caller can switch on the prefix.
hxm_status fail(hxm_status st, const char* fmt, ...)
    __attribute__((format(printf, 2, 3)));
// Clears the thread's last error and returns HXM_OK.
hxm_status ok();

inline int64_t dtype_bytes(int32_t dt) {
  switch (dt) {
    case HXM_F16:
    case HXM_BF16: return 2;
    case HXM_F32:
    case HXM_I32: return 4;
    case HXM_I8: return 1;
    default: return 0;
  }
}

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}


// Refuses a launch that grid_fits rejects ("tile-alignment"); HXM_OK otherwise.
hxm_status check_grid(const char* what, int64_t groups_x, int threads, int64_t groups_y = 1);

// Checks the launch that was just enqueued.
hxm_status check_launch(const char* what);

// Current device's gfx950 check (cached per device).  Returns HXM_OK or
// HXM_NO_DEVICE with a reason.
hxm_status require_device(int* device_out);

// Library-owned scratch for one (device, stream, slot), grown on demand and
// kept until hxm_release_cache().  Calls on the same stream are ordered, so
// one buffer per stream never races with itself.  Slot 0 holds per-call
// operand packs and the tuner's reference output; slot 1 the split-K
// partial planes, so the two never overwrite or reallocate each other.
constexpr int kWsMain = 0, kWsSplitK = 1, kWsStreamK = 2;
// Largest split-K partial-plane buffer (S * M * N int32) a call may ask for;
// the buffer stays allocated until hxm_release_cache().
constexpr int64_t kSplitKPlaneBytesMax = int64_t(256) << 20;
// Slot 2 holds the W8A16 stream-K partial tiles and arrival counters.
// *grown (when given) says whether the buffer was (re)allocated by this call.
hxm_status stream_workspace(hipStream_t stream, size_t bytes, void** out, int slot = kWsMain,
                            bool* grown = nullptr);
// CUs of the current device (cached per device; 0 when it cannot be read).
int device_cu_count();

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// The legality lattice of a GEMM config (search.hip): front-end block
// limit, min-rows, MFMA edge and wave grid, LDS budget (0 = 160 KiB) for
// a_bytes / b_bytes per element of A and B; HXM_REASON_OK or the first rule
// it breaks.  Whether the config was compiled is not part of it.
int32_t gpu_lattice(const hxm_gemm_config& c, int64_t a_bytes, int64_t b_bytes,
                    int64_t lds_budget);

// Frees the resident weight images of device `dev` (resident.hip).
hxm_status release_images(int dev);

// The direct-load small-output GEMM (gemm_small.hip): f16 / bf16 A [M, K]
// and B as the [N, K] image, one wave per 16x16 output tile, no LDS.  The
// default of hxm_matmul for outputs of at most kSmallTilesMax 16x16 tiles
// and K <= kSmallKMax; a caller names it with small_gemm_config().
constexpr int64_t kSmallTilesMax = 512;
constexpr int64_t kSmallKMax = 256;
hxm_gemm_config small_gemm_config();
bool is_small_gemm_config(const hxm_gemm_config& c);
bool small_gemm_fits(int64_t M, int64_t N, int64_t K, int32_t ab_dtype);
hxm_status launch_small_gemm(int32_t ab_dtype, const void* A, int64_t lda, const uint8_t* B,
                             int64_t ldb_bytes, void* C, int64_t ldc, int64_t M, int64_t N,
                             int64_t K, int32_t out_dtype, int32_t accumulate,
                             hipStream_t stream);

}  // namespace hxm

#define HXM_HIP_TRY(expr)                                                    \
  do {                                                                       \
    hipError_t _e = (expr);                                                  \
    if (_e != hipSuccess)                                                    \
      return ::hxm::fail(HXM_HIP_ERROR, "hip-error: %s failed: %s", #expr,   \
                         hipGetErrorString(_e));                             \
  } while (0)
