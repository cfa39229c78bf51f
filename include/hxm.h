/*
 * hxm.h - C ABI of the MI355X (gfx950) hot path: MFMA matmuls with resident
 * (pre-packed) weights, W8A16 skinny GEMM/GEMV, single-pass row reductions
 * (softmax / RMSNorm / LayerNorm) and the measured tile search.
 *
 * Boundary rules (every entry point):
 *   - plain pointers, sizes and leading dimensions (in ELEMENTS); no torch or
 *     HIP types.  `stream` is a hipStream_t passed as void* (NULL = default
 *     stream).  Every compute call is asynchronous and stream-ordered.
 *   - the caller owns every tensor; the library never frees caller memory.
 *   - arguments are validated on the host BEFORE any launch.  A refusal
 *     returns a status and leaves a reason string (hxm_last_error) whose
 *     vocabulary follows the reference's manifest reasons
 *     (qcom_hexagon_backend/include/hexagon/Dialect/Hmx/Transforms/
 *      HmxManifest.h:81-100): "unsupported-dtype", "min-rows",
 *     "tile-alignment", "lds-budget" (the VTCM budget's counterpart), plus
 *     "invalid-argument" and "workspace-budget" (a library-owned scratch
 *     buffer would exceed its stated limit, or would have to grow while the
 *     stream is capturing a HIP graph).  There is no silent fallback: a
 *     refused call computes nothing.
 *   - HIP graphs: the compute entries (matmul, GEMM, GEMV, row ops) may be
 *     captured; the tuners, the resident-weight cache and hxm_release_cache
 *     allocate or synchronise and may not.  A compute entry that uses the
 *     per-stream workspace (f32 operands, a [K,N] B, a K split) needs it
 *     already large enough: one call of the shape on the stream before the
 *     capture grows it (it is kept until hxm_release_cache).
 *   - numerics: fp16/bf16 products accumulate in fp32 and are rounded once
 *     to the output dtype; int8 products accumulate exactly in int32.
 *   - host threads: entries may run at the same time on several host
 *     threads when each uses its own stream (workspaces are per stream; the
 *     device table, the tuning cache and the resident images are locked).
 *     Calls on one stream must not overlap in time: a call may launch
 *     several kernels that share that stream's workspace, and another
 *     thread's launches in between would reuse it.  hxm_release_cache must
 *     not overlap any other call on its device (it frees buffers another
 *     call may have been handed), and hxm_gemm_i8_noalloc calls share one
 *     scratch array per device.
 *
 * Reference interfaces replaced (paths relative to the reference root):
 *   the compiled Triton kernel symbol launched by
 *   qcom_hexagon_backend/backend/driver.py:150-237 with the memref-descriptor
 *   ABI of qcom_hexagon_backend/backend/hexagon_launcher_base.py:60-75 and
 *   test/utils/dsp/include/common.h:15-30 (sizes + strides -> here sizes +
 *   leading dimensions), and below it the HMX leaves of
 *   qcom_hexagon_backend/bin/runtime/hmx/include/HMXAPI.h:53-293.
 */
#ifndef HXM_H
#define HXM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum hxm_status {
  HXM_OK = 0,
  HXM_INVALID_ARG = 1,       /* null pointer, negative size, bad ld, bad enum */
  HXM_UNSUPPORTED_DTYPE = 2, /* reason "unsupported-dtype" */
  HXM_UNSUPPORTED_SHAPE = 3, /* reason "tile-alignment" / "min-rows" / "lds-budget" */
  HXM_HIP_ERROR = 4,         /* a HIP runtime call failed; reason has hipGetErrorString */
  HXM_OUT_OF_MEMORY = 5,     /* library-owned workspace could not grow */
  HXM_NO_DEVICE = 6          /* no gfx950 device visible */
} hxm_status;

typedef enum hxm_dtype {
  HXM_F16 = 1,
  HXM_BF16 = 2,
  HXM_F32 = 3,
  HXM_I8 = 4,
  HXM_I32 = 5
} hxm_dtype;

/* Layout of the B (weight) operand of a matmul.
 *   HXM_B_KN: B is [K,N] row-major with leading dimension ldb >= N -- the
 *             plain linalg.matmul operand.  The library packs it per call
 *             into a library-owned workspace (the reference's per-launch
 *             hmx.pack_weight, HmxOps.td:229).
 *   HXM_B_NK: B is already packed, [N,K] row-major (K contiguous), ldb >= K --
 *             the resident image produced once by hxm_prepack_weight (the
 *             reference's weight-resident path, WeightResidentPass.cpp:10-53,
 *             backend/hmx_weight_prepack.py:171-183). */
typedef enum hxm_b_layout { HXM_B_KN = 0, HXM_B_NK = 1 } hxm_b_layout;

/* One GEMM kernel configuration: the tile search's variables
 * (backend/hmx_search.py:295-312 searches BM,BN,BK; the GPU adds the wave
 * grid and the K-split).  A zeroed struct means "library default for the
 * shape" (the tuned winner when one is cached). */
typedef struct hxm_gemm_config {
  int32_t bm, bn, bk;       /* workgroup tile; bk = K elements per LDS stage */
  int32_t waves_m, waves_n; /* wave grid inside the workgroup */
  int32_t stages;           /* LDS stages (2 = double buffer; prefetch depth stages-1) */
  int32_t split_k;          /* workgroup rows along K (0/1 = none; int8: 2, 4, 8 or 16,
                               int32 partial planes summed exactly).  The planes,
                               S * M * N * 4 bytes, live in a library-owned
                               per-stream buffer kept until hxm_release_cache();
                               above 256 MiB the call is refused
                               ("workspace-budget").  HXM_STREAM_K: the W8A16
                               GEMMs' stream-K mode (below) */
} hxm_gemm_config;

/* split_k of a W8A16 GEMM config (hxm_gemm_w8a16, _swiglu, _residual): when
 * the tile count is not a multiple of the CU count, the whole rounds run one
 * tile per workgroup and the remaining tiles' K stages are shared evenly by
 * one persistent workgroup per CU in the same launch, so the last round
 * keeps every CU busy.  A tile cut between workgroups is summed from fp32
 * partial tiles in a fixed order (deterministic, but not bit-identical to
 * the one-workgroup tile: within the float tolerance).  Its partial tiles
 * and arrival counters live in a library-owned per-stream buffer (256 KiB
 * per partial of a 256x256 tile) kept until hxm_release_cache(); above
 * 256 MiB the call is refused ("workspace-budget").  With whole rounds the
 * call runs as split_k = 1. */
#define HXM_STREAM_K 1024

/* ---- status / library ------------------------------------------------- */

/* Human-readable name of a status code. */
const char* hxm_status_string(int32_t status);

/* Reason string of the last non-OK status returned on this host thread
 * ("" after success).  Mirrors the manifest's plan/reason record
 * (HmxManifest.h:81-110). */
const char* hxm_last_error(void);

/* Library version string. */
const char* hxm_version(void);

/* Number of gfx950 devices visible (0 when none); touches the HIP runtime. */
int32_t hxm_device_count(void);

/* Frees every library-owned buffer (per-stream pack workspaces and resident
 * weight images) on the current device, after synchronising it.  Replaces
 * the process-lifetime VTCM release of bin/runtime/include/HexagonCAPI.h
 * :38-57. */
hxm_status hxm_release_cache(void);

/* ---- admission (HmxTarget::queryContraction, HmxTarget.h:195-218) ----- */

/* Plans a matmul without launching: the answer of hxm_plan_matmul with the
 * library's own choice of kernel.  plan_out receives 0 = "mfma-full" (every
 * extent a multiple of the 32-wide MFMA edge), 1 = "mfma-tail" (handled with
 * masked edge tiles), -1 = refused (status and hxm_last_error say why).
 * Unlike the reference's engine the GPU path admits int8 and tails. */
hxm_status hxm_query_contraction(int64_t M, int64_t N, int64_t K,
                                 int32_t a_dtype, int32_t b_dtype,
                                 int32_t c_dtype, int32_t* plan_out);

/* The plan of one GEMM call, and why (the manifest's plan/reason record,
 * HmxManifest.h:78-100; HmxTarget::queryContraction, HmxTarget.h:195-218).
 *   plan: HXM_PLAN_MFMA_FULL ("full-hmx"'s counterpart), HXM_PLAN_MFMA_TAIL
 *         ("hmx-tail"), HXM_PLAN_REFUSED (the reference would fall back to
 *         "hvx"; here the call is refused, there is no CPU path);
 *   reason: HXM_REASON_SELECTED_ALIGNED / _SELECTED_TAIL for an admitted
 *         call, else the refusal: unsupported-dtype, invalid-argument,
 *         tile-alignment, min-rows, frontend-block-limit, lds-budget,
 *         workspace-budget, no-kernel (hxm_reason_string names each). */
enum { HXM_PLAN_MFMA_FULL = 0, HXM_PLAN_MFMA_TAIL = 1, HXM_PLAN_REFUSED = -1 };
/* Where the kernel config came from. */
enum { HXM_SOURCE_DEFAULT = 0, HXM_SOURCE_TUNED = 1, HXM_SOURCE_CALLER = 2 };

typedef struct hxm_plan {
  int32_t op;              /* HXM_I8 / HXM_F16 / HXM_BF16 / HXM_F32 (operand dtype of a
                              matmul) or HXM_OP_W8A16 / HXM_OP_W8A16_SWIGLU */
  int32_t plan;            /* HXM_PLAN_* */
  int32_t reason;          /* HXM_REASON_* */
  int32_t source;          /* HXM_SOURCE_* */
  hxm_gemm_config config;  /* the compiled config that runs (split_k = the K split
                              asked for, 1 for none) */
  int32_t k_slices;        /* workgroup rows along K actually launched (1 = unsplit) */
  int32_t threads;         /* threads per workgroup */
  int64_t tiles;           /* output tiles (workgroups per K slice) */
  int64_t lds_bytes;       /* LDS per workgroup */
  int64_t workspace_bytes; /* library-owned device bytes the call uses (B pack,
                              split-K planes) */
  int64_t m, n, k;         /* the shape planned */
} hxm_plan;

/* Plans C[M,N] = A[M,K] . B without launching, exactly as the matmul entry
 * points would run it: a_dtype == b_dtype in {I8, F16, BF16, F32};
 * c_dtype I32 or F16 for I8 operands (F16 = the dequant epilogue), F16 / BF16
 * / F32 otherwise; b_layout as the call's (HXM_B_KN costs a pack
 * workspace); cfg NULL or zeroed = the library's choice (tuned winner, else
 * the default), else that config.  Operands are taken densely packed
 * (lda = ldb = K).  Fills *out (also for a refusal: plan
 * HXM_PLAN_REFUSED and the reason) and returns the status the call would
 * return. */
hxm_status hxm_plan_matmul(int64_t M, int64_t N, int64_t K, int32_t a_dtype,
                           int32_t b_dtype, int32_t c_dtype, int32_t b_layout,
                           const hxm_gemm_config* cfg, hxm_plan* out);

/* The plan of the last matmul / GEMM call on this host thread that got as
 * far as choosing a kernel (hxm_matmul, hxm_gemm_i8*, hxm_gemm_w8a16*):
 * returns 1 and fills *out, or 0 when there is none. */
int32_t hxm_last_plan(hxm_plan* out);

/* ---- matmuls ------------------------------------------------------------ */

/* linalg.matmul on f16/bf16 (reference: the hmx.matmul contract,
 * HmxOps.td:47, MatmulToHmxPass.cpp:101-121 for the init semantics; leaves
 * hmx_mma_f16 / hmx_acc_store_f16, HMXAPI.c:36-55).
 *   C[M,N] = (accumulate ? C : 0) + A[M,K] . B
 * A row-major (lda >= K), dtype ab_dtype in {F16, BF16}; B of the same
 * dtype in layout b_layout; C row-major (ldc >= N), c_dtype in
 * {F16, BF16, F32}.  Products accumulate in fp32 (with the prior C added
 * in fp32 when accumulate != 0) and round once to c_dtype.
 * K*sizeof(elem) must be a multiple of 16 bytes, lda/ldb likewise, and
 * A/B 16-byte aligned ("tile-alignment" otherwise); M and N are free.
 * 256 rows of A and of the [N,K] B image must lie within 2 GiB
 * (255 * ld * sizeof(elem) + K * sizeof(elem) < 2^31; "tile-alignment"
 * otherwise): the kernels address a tile's rows with 32-bit offsets.
 * With cfg NULL and no tuned winner, an output of at most 512 16x16 tiles
 * with K <= 256 runs on the direct-load small-output kernel (config
 * {16,16,32,1,1,0,1}, one wave per 16x16 tile, no LDS); the same config
 * passed in cfg asks for it and is refused (HXM_UNSUPPORTED_SHAPE,
 * "no-kernel") outside those limits. */
hxm_status hxm_matmul(const void* A, int64_t lda, const void* B, int64_t ldb,
                      int32_t b_layout, void* C, int64_t ldc, int64_t M,
                      int64_t N, int64_t K, int32_t ab_dtype, int32_t c_dtype,
                      int32_t accumulate, const hxm_gemm_config* cfg,
                      void* stream);

/* int8 linalg.matmul with exact int32 accumulation (the reference refuses
 * int8 on the engine, HmxTarget.h:198-200, and lowers it on the HVX
 * generic path, LinalgToLLVMPass.cpp:364-365; its result is the exact
 * integer product).  C_i32[M,N] = (accumulate ? C : 0) + A . B, wrapping
 * int32 addition.  K, lda, ldb multiples of 16; A, B 16-byte aligned; the
 * same 2 GiB span of 256 rows as hxm_matmul. */
hxm_status hxm_gemm_i8(const int8_t* A, int64_t lda, const int8_t* B,
                       int64_t ldb, int32_t b_layout, int32_t* C, int64_t ldc,
                       int64_t M, int64_t N, int64_t K, int32_t accumulate,
                       const hxm_gemm_config* cfg, void* stream);

/* hxm_gemm_i8 that allocates no device memory.  It has no counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and result as hxm_gemm_i8 with B as the resident [N,K] image
 * (b_layout HXM_B_NK; the per-call pack of a [K,N] B would need a
 * workspace).  A K split (cfg->split_k, or a tuned winner that has one)
 * keeps its S*M*N int32 partial planes in a library-static device array of
 * HXM_NOALLOC_SCRATCH_BYTES per device; a split needing more is refused
 * ("workspace-budget").  The array is part of the library's code object: every
 * process that loads libhxm.so holds those 64 MiB on each device it uses,
 * until the process ends, whether or not it ever calls this entry.  Its plan
 * record (hxm_last_plan) reports no library workspace.  Every call on a
 * device shares that array: calls that overlap on one device (on different
 * streams) race, and nothing detects it; calls on one stream are ordered.
 * The call may be captured in a HIP graph (it allocates, frees and
 * synchronises nothing, and records no memset). */
#define HXM_NOALLOC_SCRATCH_BYTES (64ll << 20)
hxm_status hxm_gemm_i8_noalloc(const int8_t* A, int64_t lda, const int8_t* B_nk,
                               int64_t ldb, int32_t* C, int64_t ldc, int64_t M,
                               int64_t N, int64_t K, int32_t accumulate,
                               const hxm_gemm_config* cfg, void* stream);

/* int8 GEMM with the fused dequant epilogue (the GPU counterpart of the
 * fused read-out convert, HMXAPI.c:36-44, with per-channel scales):
 *   C_f16[i,j] = rne_f16( ((float)acc_i32[i,j] * row_scale[i]) * col_scale[j] )
 * evaluated in fp32 exactly in that order (two roundings, no FMA), so the
 * result is bit-exact against any implementation of the same spelling.
 * row_scale: fp32 [M]; col_scale: fp32 [N]. */
hxm_status hxm_gemm_i8_dequant(const int8_t* A, int64_t lda, const int8_t* B,
                               int64_t ldb, int32_t b_layout,
                               const float* row_scale, const float* col_scale,
                               void* C_f16, int64_t ldc, int64_t M, int64_t N,
                               int64_t K, const hxm_gemm_config* cfg,
                               void* stream);

/* Weight pre-pack: the host half of weight residency
 * (backend/hmx_weight_prepack.py:171-212, WeightPrepack._permute) done on
 * the device.  Transposes B [K,N] (ldb >= N) into the resident image
 * out [N,K] (ldo >= K), K contiguous -- the operand order every MFMA kernel
 * here reads.  dtype in {I8, F16, BF16}.  Run once per weight; matmuls then
 * take b_layout = HXM_B_NK.  An ldo whose rows start on 128-byte lines
 * (ldo * elem a multiple of 128) streams fastest: int8 4000^3 + dequant
 * 56.7 us against 59.5 us with ldo = K = 4000 (one box); the per-call pack
 * of a [K,N] B uses such rows. */
hxm_status hxm_prepack_weight(const void* B, int64_t ldb, void* out,
                              int64_t ldo, int64_t K, int64_t N, int32_t dtype,
                              void* stream);

/* Layout of the int8 weight of the W8A16 GEMV.
 *   HXM_W_NK:     W is [N,K] row-major (output-channel major, K contiguous),
 *                 ldw >= K.
 *   HXM_W_PACKED: W is the resident image made once by hxm_prepack_w8a16
 *                 (ldw ignored): 1 KiB blocks per (16 channels, 64 K), in the
 *                 order one wave instruction consumes them, each weight w
 *                 stored in offset binary (byte = w ^ 0x80; padding holds
 *                 zero weights, 0x80) -- the GEMV's counterpart of the
 *                 reference's weight pre-pack
 *                 (backend/hmx_weight_prepack.py:171-183). */
typedef enum hxm_w_layout { HXM_W_NK = 0, HXM_W_PACKED = 1 } hxm_w_layout;

/* W8A16 weight-resident skinny GEMM / GEMV (M in {1, 4, 16}; the
 * reference's int8 matmul on the HVX path, ScheduleMatmulForHVXPass.cpp:44-80):
 *   y[m,n] = rne_f16( (sum_k f32(x[m,k]) * f32(W[n,k])) * f32(w_scale[n]) )
 * x fp16 [M,K] (ldx >= K); W int8 in layout w_layout; w_scale fp16 [N];
 * y fp16 [M,N] (ldy >= N).  fp32 accumulation in any order (tolerance
 * rtol 1e-2 / atol 1e-3 against the fp32 restatement).  W is streamed once
 * per 16 rows of M.  K multiple of 16, ldx multiple of 8, ldw (HXM_W_NK)
 * multiple of 16, x and W 16-byte aligned; HXM_W_PACKED images up to
 * K = 134,215,680 (2^21 - 32 slabs of 64). */
hxm_status hxm_gemv_w8a16(const void* x, int64_t ldx, const int8_t* W,
                          int64_t ldw, int32_t w_layout, const void* w_scale,
                          void* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                          void* stream);

/* Bytes of the packed W8A16 image for [N,K] (-1 for negative extents). */
int64_t hxm_w8a16_packed_bytes(int64_t N, int64_t K);

/* Builds the packed W8A16 image from W [N,K] (ldw) into out (at least
 * hxm_w8a16_packed_bytes(N,K) bytes, 16-byte aligned, caller-owned).
 * Run once per weight (the weight-resident contract: WeightResidentPass.cpp
 * :10-53, HexagonCAPI.h:52-53). */
hxm_status hxm_prepack_w8a16(const int8_t* W, int64_t ldw, int64_t N,
                             int64_t K, int8_t* out, int64_t out_bytes,
                             void* stream);

/* ---- content-addressed resident weights (WeightPrepack.pack,
 *      backend/hmx_weight_prepack.py:124-212; hexagon_runtime_weight_resident_v2,
 *      bin/runtime/include/HexagonCAPI.h:52-53) ---- */

typedef enum hxm_image_kind {
  HXM_IMAGE_GEMM = 0,  /* src B [K,N] (rows = K, cols = N) -> the [N,K] image of
                          hxm_prepack_weight; I8/F16/BF16 keep their dtype, an F32
                          source becomes an F16 image (-0 -> +0, then RNE) */
  HXM_IMAGE_W8A16 = 1  /* src W [N,K] int8 (rows = N, cols = K) -> the packed
                          image of hxm_prepack_w8a16 */
} hxm_image_kind;

/* Returns (in *image) the library-owned resident image of src, packing it on
 * the first call for this content and reusing it afterwards: the cache key
 * is (kind, device, rows, cols, src_dtype, a 128-bit hash of every source
 * element and its position), so equal content at another address hits and a
 * one-element change misses.  expect_dtype >= 0 and expect_shape (rows,
 * cols) != NULL are the caller's contract: a mismatch is refused
 * ("unsupported-dtype" / "invalid-argument") before anything is packed, and
 * so are extents the image's pack would refuse ("tile-alignment"), before
 * the weight is hashed.
 * *image_dtype receives the image dtype.  Synchronises `stream` once (the
 * hash is read back), and once more when it builds a new image, so an
 * image is complete before any thread or stream can be handed it.  Images
 * stay valid until hxm_release_cache(). */
hxm_status hxm_resident_weight(const void* src, int64_t ld, int64_t rows,
                               int64_t cols, int32_t src_dtype,
                               int32_t expect_dtype, const int64_t* expect_shape,
                               int32_t kind, const void** image,
                               int32_t* image_dtype, void* stream);

/* ---- SwiGLU FFN block (RMSNorm -> int8-weight gate/up
 *      GEMMs -> SiLU*mul -> down GEMM).  The reference composes it from the
 *      linalg ops its pipeline lowers: linalg.matmul (MatmulToHmxPass.cpp
 *      :101-121 admission; int8 operands take the HVX path,
 *      ScheduleMatmulForHVXPass.cpp:44-80) and elementwise linalg.generic
 *      ops.  The int8 weights stay int8 in HBM and are converted to fp16 in
 *      registers (exactly) in front of the fp16 MFMA. ---- */

/* Tuning-cache op codes of the W8A16 GEMMs (hxm_tune_w8a16). */
enum { HXM_OP_W8A16 = 16, HXM_OP_W8A16_SWIGLU = 17 };

/* Large-M W8A16 GEMM (the gate/up/down projections of the FFN; the GEMV
 * above covers M <= 16 best):
 *   y[m,n] = rne_f16( (sum_k f32(x[m,k]) * f32(W[n,k])) * f32(w_scale[n]) )
 * x fp16 [M,K] (ldx >= K); W int8 [N,K] (ldw >= K); w_scale fp32 [N];
 * y fp16 [M,N] (ldy >= N).  fp32 accumulation in MFMA order (tolerance
 * rtol 1e-2 / atol 1e-3).  K multiple of 16, ldx multiple of 8, ldw
 * multiple of 16, x and W 16-byte aligned, and 256 rows of x and of W
 * within 2 GiB (as for hxm_matmul).  cfg: NULL = tuned winner or the
 * default tile; else one of hxm_w8a16_configs. */
hxm_status hxm_gemm_w8a16(const void* x, int64_t ldx, const int8_t* W,
                          int64_t ldw, const float* w_scale, void* y,
                          int64_t ldy, int64_t M, int64_t N, int64_t K,
                          const hxm_gemm_config* cfg, void* stream);

/* W8A16 GEMM with a fused residual add -- the read-out that adds a resident
 * tensor before the store (hmx_unpack_acc_f32 with residual,
 * bin/runtime/hmx/include/HMXAPI.h:245-275; the FFN block's x + FFN(x)):
 *   y[m,n] = rne_f16( f32( (sum_k f32(x[m,k]) * f32(W[n,k])) * f32(w_scale[n]) )
 *                     + f32(r[m,n]) )
 * the product and the sum each rounded to fp32, then one rounding to f16.
 * r fp16 [M,N] (ldr >= N) is either y itself (in place, ldr == ldy) or
 * disjoint from y ("invalid-argument" otherwise).  Everything else as
 * hxm_gemm_w8a16 (tiles from the same tuned-winner cache). */
hxm_status hxm_gemm_w8a16_residual(const void* x, int64_t ldx, const int8_t* W,
                                   int64_t ldw, const float* w_scale,
                                   const void* r, int64_t ldr, void* y,
                                   int64_t ldy, int64_t M, int64_t N, int64_t K,
                                   const hxm_gemm_config* cfg, void* stream);

/* Rows of the fused gate/up image for I intermediate channels:
 * 128 * ceil(I / 64) (-1 for I < 0). */
int64_t hxm_swiglu_packed_rows(int64_t I);

/* Builds the gate/up image once per weight pair (the weight-resident
 * contract, WeightResidentPass.cpp:10-53): Wgu int8 [hxm_swiglu_packed_rows(I),
 * K] (row stride K) whose rows [128c, 128c+64) are gate channels
 * [64c, 64c+64) and rows [128c+64, 128c+128) the same up channels, channels
 * >= I zero; sgu fp32 [rows] the matching scales (zero for padding).  Each
 * weight w is stored in offset binary, byte = w ^ 0x80 (w + 128 unsigned;
 * a zero weight is 0x80), the form the GEMM converts to f16 without a sign
 * flip; the image is this library's own and feeds only
 * hxm_gemm_w8a16_swiglu.
 * Wg, Wu int8 [I,K] (ldw >= K); gate_scale, up_scale fp32 [I]. */
hxm_status hxm_swiglu_pack(const int8_t* Wg, const int8_t* Wu, int64_t ldw,
                           const float* gate_scale, const float* up_scale,
                           int64_t I, int64_t K, int8_t* Wgu, float* sgu,
                           void* stream);

/* Fused gate/up projection + SiLU * mul:
 *   g = f32(sum_k x[m,k] * Wg[i,k]) * sg[i],  u = (same with Wu) * su[i]
 *   h[m,i] = rne_f16( g / (1 + exp(-g)) * u )
 * x fp16 [M,K] (ldx >= K); Wgu/sgu from hxm_swiglu_pack; h fp16 [M,I]
 * (ldh >= I).  exp and the reciprocal use the hardware approximations
 * (tolerance rtol 1e-2 / atol 1e-3).  Same K/alignment rules as
 * hxm_gemm_w8a16; cfg must have a 128-column wave tile (bn / waves_n). */
hxm_status hxm_gemm_w8a16_swiglu(const void* x, int64_t ldx, const int8_t* Wgu,
                                 const float* sgu, void* h, int64_t ldh,
                                 int64_t M, int64_t I, int64_t K,
                                 const hxm_gemm_config* cfg, void* stream);

/* The compiled W8A16 GEMM configurations (bk in fp16 elements of K); with
 * swiglu != 0 only those that have the fused SwiGLU kernel.  Returns the
 * count; writes up to cap entries. */
int32_t hxm_w8a16_configs(int32_t swiglu, hxm_gemm_config* out, int32_t cap);

/* hxm_tune_gemm for the W8A16 GEMMs (same protocol, report and cache):
 * op HXM_OP_W8A16 measures hxm_gemm_w8a16 (scale = w_scale, N output
 * channels); HXM_OP_W8A16_SWIGLU measures hxm_gemm_w8a16_swiglu (W = Wgu
 * with ldw == K, scale = sgu, N = I).  C is the [M,N] fp16 output. */
hxm_status hxm_tune_w8a16(int32_t op, const void* x, int64_t ldx,
                          const int8_t* W, int64_t ldw, const float* scale,
                          void* C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                          int32_t reps, hxm_gemm_config* best, char* report,
                          int64_t report_cap, void* stream);

/* ---- row reductions (test/python/triton/test_softmax.py:41-69,
 *      test_rms_norm.py:34-60, test_layer_norm.py:39-79, as lowered by
 *      VectorRowReducePass.cpp:10-31 / SplitReduceGenericPass.cpp:62-93) -- */

/* y[r,:] = exp(x[r,:] - max_r) / sum(exp(x[r,:] - max_r)), computed in fp32
 * (max-subtract, fp32 sum), rounded once to dtype.  dtype in {F16, BF16,
 * F32}; x and y may alias.  cols >= 1. */
hxm_status hxm_softmax_rows(const void* x, int64_t ldx, void* y, int64_t ldy,
                            int64_t rows, int64_t cols, int32_t dtype,
                            void* stream);

/* y[r,c] = x[r,c] * rsqrt(mean_c(x[r,:]^2) + eps) * gamma[c], fp32 inside,
 * one rounding to dtype.  gamma (same dtype, [cols]) may be NULL (= 1). */
hxm_status hxm_rmsnorm_rows(const void* x, int64_t ldx, const void* gamma,
                            void* y, int64_t ldy, int64_t rows, int64_t cols,
                            float eps, int32_t dtype, void* stream);

/* y = (x - mean) * rstd * gamma + beta with rstd = 1/sqrt(var + eps)
 * (biased variance), fp32 inside.  gamma/beta may be NULL (1 / 0).
 * mean_out / rstd_out: fp32 [rows] or NULL (the reference kernel writes
 * them for the backward pass, test_layer_norm.py:67-69). */
hxm_status hxm_layernorm_rows(const void* x, int64_t ldx, const void* gamma,
                              const void* beta, void* y, int64_t ldy,
                              float* mean_out, float* rstd_out, int64_t rows,
                              int64_t cols, float eps, int32_t dtype,
                              void* stream);

/* ---- ceiling probes (measurement helpers; no counterpart in the reference) --
 * The practical ceiling of the HBM-bound kernels above, measured with the
 * same access pattern (16-byte accesses, eight in flight per lane; the copy
 * loads plainly and stores nontemporally like the row kernels, the read
 * loads nontemporally like the GEMV).  bytes: a multiple of 16; buffers
 * 16-byte aligned. */
#define HXM_PROBE_SINK_WORDS 8192

/* dst[0, bytes) = src[0, bytes); the buffers must not overlap. */
hxm_status hxm_probe_copy(const void* src, void* dst, int64_t bytes, void* stream);

/* Reads src[0, bytes) and folds it; sink (at least HXM_PROBE_SINK_WORDS
 * uint32 of device memory) receives a word only for one rare fold value. */
hxm_status hxm_probe_read(const void* src, int64_t bytes, uint32_t* sink, void* stream);

/* MFMA probe (measurement helper; no counterpart in the reference): the
 * practical ceiling of the MFMA-bound kernels.  `workgroups` workgroups of
 * four waves (one per SIMD, the GEMM kernels' occupancy: one per CU) each run
 * mfma_per_wave 32x32 MFMAs (a positive multiple of 32, at most 2^24: about
 * a third of a second per launch) of the GEMMs' shapes
 * -- int8 x int8 (v_mfma_i32_32x32x32_i8), f16 x f16 or bf16 x bf16
 * (v_mfma_f32_32x32x16_*), or f16 x int8 (B converted to f16 as the W8A16
 * kernels do) -- on operand fragments read once from a[0, a_bytes) and
 * b[0, b_bytes) (multiples of 16, 16-byte aligned): a GEMM's own operands
 * give its data-dependent power draw, and so its clock.  Nothing else runs:
 * no staging, no epilogue.  sink: at least HXM_PROBE_SINK_WORDS uint32,
 * written only for one rare fold value of the accumulators. */
hxm_status hxm_probe_mfma(const void* a, int64_t a_bytes, const void* b, int64_t b_bytes,
                          int32_t a_dtype, int32_t b_dtype, int64_t mfma_per_wave,
                          int32_t workgroups, uint32_t* sink, void* stream);

/* ---- tile search (backend/hmx_search.py) -------------------------------- */

/* Reason codes shared by the two verdict functions below. */
enum {
  HXM_REASON_OK = 0,
  HXM_REASON_FRONTEND_BLOCK_LIMIT = 1,
  HXM_REASON_MIN_ROWS = 2,
  HXM_REASON_TILE_ALIGNMENT = 3,
  HXM_REASON_VTCM_BUDGET = 4,
  HXM_REASON_LDS_BUDGET = 5,
  HXM_REASON_UNSUPPORTED_DTYPE = 6,
  HXM_REASON_NO_KERNEL = 7,
  HXM_REASON_SELECTED_ALIGNED = 8,  /* "selected-aligned" */
  HXM_REASON_SELECTED_TAIL = 9,     /* "selected-tail" */
  HXM_REASON_WORKSPACE_BUDGET = 10, /* "workspace-budget" */
  HXM_REASON_INVALID_ARGUMENT = 11  /* "invalid-argument" */
};

/* Reason code -> the reference's vocabulary string ("ok", "min-rows", ...). */
const char* hxm_reason_string(int32_t reason);

/* hmx_search.tile_ladder (hmx_search.py:246-266): powers of two from 32 to
 * next_pow2(extent), plus extent itself when it is a power of two, sorted.
 * Writes up to cap values; returns the full count, or -1 for an extent
 * above 2^62, whose padded power of two (2^63) no int64 holds. */
int32_t hxm_tile_ladder(int64_t extent, int64_t* out, int32_t cap);

/* hmx_search.tile_verdict (hmx_search.py:269-292), the reference's engine
 * legality predicate restated exactly (VTCM budget in bytes). */
int32_t hxm_hmx_tile_verdict(int64_t bm, int64_t bn, int64_t bk,
                             int64_t vtcm_budget);

/* The same lattice on gfx950: frontend limit -> min-rows -> the 32-wide MFMA
 * edge -> LDS budget (stages x (bm+bn) x bk x elem_bytes <= lds_budget)
 * -> a compiled kernel exists for (cfg, dtype).  elem_bytes 1 (int8) or 2. */
int32_t hxm_gpu_tile_verdict(const hxm_gemm_config* cfg, int32_t ab_dtype,
                             int64_t lds_budget);

/* Every compiled GEMM configuration for ab_dtype (I8, F16 or BF16).
 * Writes up to cap entries; returns the full count. */
int32_t hxm_gemm_configs(int32_t ab_dtype, hxm_gemm_config* out, int32_t cap);

/* hmx_search.champion_gate (hmx_search.py:1280-1289): max(3*|cv|, 0.15). */
double hxm_champion_gate(double cv);

/* hmx_search.quantile_spread_cv (hmx_search.py:1254-1277). */
double hxm_quantile_spread_cv(double q20, double q50, double q80);

/* hmx_search._quantile (hmx_search.py:1095-1106): linear interpolation. */
double hxm_quantile(const double* samples, int32_t n, double q);

/* hmx_search.calibration_iters (hmx_search.py:1159-1171). */
int32_t hxm_calibration_iters(double perf_us, double target_us, int32_t lo,
                              int32_t hi);

/* The gated walk of hmx_search.judge_champion_round (hmx_search.py:1460-1478).
 * Rows are given in enumeration order with their q20/q50/q80; `start` is the
 * incumbent's index (the control arm, else the first measured row); rows
 * whose q50 is not finite are skipped.  A challenger takes the crown only when
 * (q50_inc - q50_ch)/q50_inc > max(3*max(cv_ch, cv_inc), 15%) (strict: a tie
 * keeps the incumbent).  outcome[i] (may be NULL): -1 not compared, 0 kept,
 * 1 takeover; delta_out/gate_out (may be NULL) receive the fractions.
 * Returns the champion's index, -1 when start is not a measured row, -2 for
 * n < 0 or a NULL q20/q50/q80 with n > 0. */
int32_t hxm_champion_walk(const double* q20, const double* q50,
                          const double* q80, int32_t n, int32_t start,
                          int32_t* outcome, double* delta_out,
                          double* gate_out);

/* hmx_search.canary_verdict's status (hmx_search.py:1292-1367):
 * 0 "ok", 1 "missing" (present == 0), 2 "unmeasured" (q50 not finite),
 * 3 "drift" (|q50/ref - 1| > champion_gate(cv)), 4 "reference-established"
 * (no finite positive reference).  delta_out/gate_out may be NULL. */
int32_t hxm_canary_status(int32_t present, double q20, double q50, double q80,
                          double reference_q50, double* delta_out,
                          double* gate_out);

/* One search round judged as a whole (the decision of
 * hmx_search.judge_champion_round, hmx_search.py:1370-1571, as codes; the
 * measured tuner and the Python mirror both call it).  Arms are given in
 * walk order (the caller sorts them by their config); an arm whose q50 is
 * not finite was never measured. */
typedef struct hxm_arm_quantiles {
  double q20, q50, q80;
} hxm_arm_quantiles;

/* Where the walk began. */
enum {
  HXM_START_CONTROL = 0,            /* at the measured control arm */
  HXM_START_NOMINAL = 1,            /* no control named: the first measured arm */
  HXM_START_CONTROL_UNMEASURED = 2, /* the control arm scored inf: no walk */
  HXM_START_CONTROL_ABSENT = 3,     /* the named control is not an arm: no walk */
  HXM_START_EMPTY = 4               /* nothing was measured */
};
/* What the round proves about its champion against the control arm. */
enum {
  HXM_PROOF_PROVEN = 0,       /* beat the control by more than the gate */
  HXM_PROOF_WITHIN_GATE = 1,  /* won the walk, not by the gate against the control */
  HXM_PROOF_CONTROL_HELD = 2, /* the control kept the crown */
  HXM_PROOF_NO_CONTROL = 3,   /* no measured control arm to prove against */
  HXM_PROOF_VOID = 4          /* the canary voided the round */
};

typedef struct hxm_round_verdict {
  int32_t canary;    /* hxm_canary_status code */
  int32_t valid;     /* 1 when the canary is ok or reference-established */
  int32_t start;     /* HXM_START_* */
  int32_t champion;  /* arm index of the walk's survivor, -1 for none */
  int32_t proof;     /* HXM_PROOF_* */
  int32_t measured;  /* arms with a finite q50 */
  int32_t takeovers; /* crown changes during the walk */
  int32_t reserved;
  double canary_cv, canary_delta, canary_gate;    /* NaN where not judged */
  double control_cv, control_delta, control_gate; /* champion vs control; NaN without one */
} hxm_round_verdict;

/* control: arm index of the control, -1 when none is named, any other
 * negative value when one is named but is not among the arms.  canary: the
 * canary's quantiles, NULL when no canary ran.  Per arm (each array may be
 * NULL): outcome -1 not compared, 0 the incumbent kept the crown,
 * 1 takeover; faced = the incumbent's index it was compared with (-1);
 * delta/gate as in hxm_champion_walk.  Returns the champion's index (-1 for
 * none), or -2 for invalid arguments (n < 0, or arms NULL with n > 0). */
int32_t hxm_judge_round(const hxm_arm_quantiles* arms, int32_t n, int32_t control,
                        const hxm_arm_quantiles* canary, double canary_reference_q50,
                        hxm_round_verdict* out, int32_t* outcome, int32_t* faced,
                        double* delta, double* gate);

/* Measured tile search for one GEMM shape on the caller's operands (the
 * reference's autotune sweep + hexagon_bench + judge_champion_round,
 * hmx_search.py:1109-1156,1370-1571).  op: HXM_I8 (int8 -> i32, B in
 * layout NK) or HXM_F16 / HXM_BF16 (-> C of the same dtype, B in layout
 * NK).  The control is what an untuned call runs: the default config, or
 * for f16 / bf16 shapes the small-output kernel takes (see hxm_matmul)
 * that kernel, also a candidate.  First the
 * cost model prices every legal compiled config on this device
 * (hxm_predict_tile_time) and the conservative prune (hxm_cost_prune, margin
 * 0.15, envelope 0.70 / 1.25, the control always kept) drops those whose
 * modeled lower bound is out of reach; a dropped config is not launched.
 * Every other config is launched `reps` times after one discarded warm call
 * (reps 0: calibrated per config, hxm_calibration_iters of the timed warm
 * call against a 10 ms budget, 5 to 1000 launches);
 * its output is checked against the control config's, bit-exact within a
 * kernel family and within |c - r| <= 1e-3 + 1e-2 |r| between the
 * small-output kernel and the LDS-staged tiles, whose dot products sum in
 * different orders (a config that differs scores inf); the champion is the deterministic gated walk
 * from the control config with gate max(3*CV, 15%), preceded by the
 * 32x32x32 canary.  The winner is cached for (op, M, N, K) and used by
 * later calls with cfg == NULL.  report (JSON, may be NULL) receives the
 * per-config quantiles, sample counts, modeled bounds and prune marks, and
 * the verdict.  C is overwritten. */
hxm_status hxm_tune_gemm(int32_t op, const void* A, int64_t lda, const void* B,
                         int64_t ldb, void* C, int64_t ldc, int64_t M,
                         int64_t N, int64_t K, int32_t reps,
                         hxm_gemm_config* best, char* report,
                         int64_t report_cap, void* stream);

/* Forget every cached tuning winner. */
void hxm_tune_cache_clear(void);

/* The cached tuning winner for (op, M, N, K): returns 1 and writes *out
 * (if non-NULL) when there is one, else 0.  op as in hxm_tune_gemm /
 * hxm_tune_w8a16. */
int32_t hxm_tune_cache_lookup(int32_t op, int64_t M, int64_t N, int64_t K,
                              hxm_gemm_config* out);

/* Persisted winners.  The reference keys its search results on the build
 * and the measurement protocol so that no result crosses a rebuild
 * (backend/hmx_search.py:416-442, tuning_key_int).  hxm_tune_cache_save
 * writes every cached winner to `path` (text; replaced atomically), headed by
 * a hash of this library's binary and the device's CU count, each entry with
 * the reps it was measured with.  hxm_tune_cache_load adds the winners of
 * such a file to the cache (*loaded = how many) only when both match this
 * library and device ("invalid-argument" otherwise: results of another build
 * or device are re-measured, not reused); entries naming a tile this build
 * did not compile are skipped. */
hxm_status hxm_tune_cache_save(const char* path);
hxm_status hxm_tune_cache_load(const char* path, int32_t* loaded);

/* ---- modeled cost: ordering and the conservative prune ------------------
 * hmx_search.predict_tile_pcyc (hmx_search.py:778-887), rank_tile_candidates
 * (:1030-1067) and cost_prune (:916-1027).  The reference prices a tile from
 * a table of measured Hexagon leaf costs qualified by a runtime fingerprint;
 * here a GEMM config is priced from the device's own rates (MFMA ops per
 * clock, LDS fill bytes per clock, HBM bytes per second, launch cost), and
 * the model's tier plays the fingerprint's part: only a model read from the
 * device this process runs on (HXM_TIER_CURRENT) may drive a drop. */
enum { HXM_TIER_UNKNOWN = 0, HXM_TIER_CURRENT = 1, HXM_TIER_NOMINAL = 2 };

typedef struct hxm_device_model {
  int32_t cus;               /* compute units */
  int32_t tier;              /* HXM_TIER_* */
  double sclk_mhz_peak;      /* lower bound: MFMA and LDS fill at this clock */
  double sclk_mhz_sustained; /* upper bound: the clock under sustained load */
  double hbm_gbps_peak;      /* lower bound: HBM bytes at this rate */
  double hbm_gbps_sustained; /* upper bound */
  double lds_fill_peak;      /* bytes per clock per CU into LDS, lower bound */
  double lds_fill_sustained; /* bytes per clock per CU into LDS, upper bound */
  double launch_us;          /* launch cost, charged to the upper bound only */
  int64_t lds_bytes;         /* LDS per CU */
  int64_t cache_bytes;       /* last-level (Infinity) cache */
} hxm_device_model;

/* Abstain classes, tested in this order: dtype, model missing, tail blocks,
 * heat band, heat cross-boundary, no price (hmx_search.py:844-866).
 * MANIFEST is cost_prune's own class (hmx_search.py:895-913). */
enum {
  HXM_ABSTAIN_NONE = 0,
  HXM_ABSTAIN_HEAT_BAND = 1,     /* "heat-band" */
  HXM_ABSTAIN_HEAT_CROSS = 2,    /* "heat-cross-boundary" */
  HXM_ABSTAIN_TAIL = 3,          /* "tail-blocks" */
  HXM_ABSTAIN_DTYPE = 4,         /* "dtype-no-cell" */
  HXM_ABSTAIN_MANIFEST = 5,      /* "manifest-strategy-unknown" */
  HXM_ABSTAIN_NO_CELL = 6,       /* "no-applicable-cell" */
  HXM_ABSTAIN_TABLE_MISSING = 7  /* "table-missing" */
};

typedef struct hxm_tile_prediction {
  double lb_us, ub_us, p50_us; /* NaN when abstaining; p50 = (lb + ub) / 2 */
  int64_t units[3];            /* tiles, tiles per CU, K stages per tile */
  int32_t abstain;             /* HXM_ABSTAIN_* */
  int32_t tier;                /* the model's tier */
  int32_t heat;                /* 0 cache-resident, 1 HBM, -1 not classified */
  int32_t reserved;
} hxm_tile_prediction;

/* Abstain code -> the reference's vocabulary string. */
const char* hxm_abstain_string(int32_t abstain);

/* The spec-sheet gfx950 model (tier HXM_TIER_NOMINAL): 256 CUs, 2.4 GHz peak
 * and 1.4 GHz sustained clock, 8.0 / 5.0 TB/s HBM, 128 / 48 bytes per clock
 * LDS fill, 2.5 us launch, 160 KiB LDS, 256 MiB Infinity Cache. */
void hxm_device_model_nominal(hxm_device_model* out);

/* The model of the current device: CUs, peak clock and LDS size read from
 * it, the other rates from the nominal model; tier HXM_TIER_CURRENT on a
 * gfx950 device, HXM_TIER_UNKNOWN on any other. */
hxm_status hxm_device_model_query(hxm_device_model* out);

/* Modeled time interval of one compiled config for C[M,N] = A[M,K] B[K,N]
 * (ab_dtype HXM_I8 / HXM_F16 / HXM_BF16; out_dtype HXM_I32, HXM_F16,
 * HXM_BF16 or HXM_F32 sizes the C stream).  Lower bound: the largest of the
 * MFMA floor, the LDS fill floor and (HBM heat only) the HBM floor at peak
 * rates.  Upper bound: launch + MFMA + LDS fill + HBM at sustained rates, no
 * overlap credit.  Writes *out and returns out->abstain. */
int32_t hxm_predict_tile_time(int64_t M, int64_t N, int64_t K,
                              const hxm_gemm_config* cfg, int32_t ab_dtype,
                              int32_t out_dtype, const hxm_device_model* model,
                              hxm_tile_prediction* out);

/* rank_tile_candidates: order[] receives a permutation of 0..n-1 sorted by
 * (abstains last, lower bound, span count, config fields).  Returns n, or -1
 * on a NULL array with n > 0. */
int32_t hxm_rank_tile_candidates(int64_t M, int64_t N, int64_t K,
                                 int32_t ab_dtype, int32_t out_dtype,
                                 const hxm_gemm_config* cands, int32_t n,
                                 const hxm_device_model* model, int32_t* order);

/* cost_prune over given predictions: the champion A is the priced candidate
 * with the lowest p50 (ties: config fields); candidate B is dropped only when
 * lb(B) > (1 + margin) * env_hi / env_lo * ub(A).  kept[i] receives 0
 * dropped, 1 kept inside the band, 2 kept as the control (index `control`,
 * -1 for none), 3 kept abstaining, 4 kept because vouched[i] == 0 (vouched
 * may be NULL: no manifest consulted), 5 kept because its tier is not
 * HXM_TIER_CURRENT, 6 kept because nothing is priced.  *threshold_out (may
 * be NULL) receives the factor.  Returns the champion's index, -1 when
 * nothing is priced, -2 on invalid arguments. */
int32_t hxm_cost_prune(const hxm_tile_prediction* preds,
                       const hxm_gemm_config* cands, int32_t n, int32_t control,
                       const int32_t* vouched, double margin, double env_lo,
                       double env_hi, int32_t* kept, double* threshold_out);

#ifdef __cplusplus
}
#endif

#endif /* HXM_H */
