#pragma once
// MFMA GEMMs on gfx950: int8 x int8 -> int32 (exact) and f16/bf16 -> fp32.
//
// Reference path: linalg.matmul lowered by matmul-to-hmx -> hmx-partition ->
// weight-resident (qcom_hexagon_backend/lib/Dialect/Hmx/Transforms/
// HmxPartitionPass.cpp:783-864: for m-tiles { pack A row-tile; for n-tiles
// { clear acc; K batches of mma; read-out } }, weights resident across m), the
// activation staging ring of depth 1/2 (HmxPartitionPass.cpp:253), and the
// leaves hmx_mma_f16 / hmx_acc_store_f16 (bin/runtime/hmx/src/HMXAPI.c:36-55).
//
// GPU form.  C[M,N] = A[M,K] . B^T where B is the resident [N,K] image (K
// contiguous), so both operands stream K-contiguous 16-byte chunks.
//   * workgroup tile BM x BN; K is staged BKB bytes at a time (64 or 128) in
//     STAGES LDS buffers, each its own __shared__ array.  Stage s+STAGES-1 is
//     fetched by LDS-DMA (buffer_load_dwordx4 ... lds) while stage s feeds the
//     MFMAs; an exact s_waitcnt vmcnt(N) waits for the oldest stage only.
//     Because every buffer is a distinct object, the compiler can prove the
//     DMA into one buffer does not alias the ds_reads of another and does not
//     add a full vmcnt(0) drain before them;
//   * the loads use a buffer resource per operand: each lane's 32-bit offset
//     (row * ld + chunk * 16) is computed once and the K position rides in the
//     scalar offset, so a stage costs no per-lane address arithmetic.  Rows
//     past M / N use an offset beyond the resource's range and read as zero,
//     as do K chunks past K (last stage only);
//   * LDS rows are BKB bytes, 16-byte chunks XOR-swizzled per row so the 16
//     lanes of a ds_read_b128 phase hit distinct banks;
//   * each wave owns a (BM/WM) x (BN/WN) sub-tile of 32x32 MFMA blocks
//     (v_mfma_i32_32x32x32_i8 / v_mfma_f32_32x32x16_{f16,bf16}; both take 32
//     bytes of K per row per instruction, 16 per lane).  Fragments of k-step
//     ks+1 are read while the MFMAs of ks issue.  The B tile is the MFMA's
//     first operand, so each lane ends with 4 CONSECUTIVE output columns per
//     register group: the epilogue stores 8 (f16) or 16 (int32) bytes per lane;
//   * the tile order is XCD-aware: workgroups are dispatched round-robin over
//     the 8 XCDs, so consecutive tile ids are remapped onto one XCD and walked
//     in groups of 4 tile-rows, keeping each XCD's A rows and B columns in its
//     own L2;
//   * epilogues: int32 (optionally += C, wrapping), fp32 -> {f16, bf16, f32}
//     (optionally += C, one rounding), or the int8 dequant
//     f16(((float)acc * row_scale) * col_scale).
#include <type_traits>

#include "device_util.h"
#include "gemm_configs.h"
#include "hxm_internal.h"

namespace hxm {

constexpr uint32_t kOob = 0x80000000u;  // an offset past every resource's range

template <int BKB>
__device__ __forceinline__ int swz(int row) {
  if constexpr (BKB == 128)
    return (row & 7) ^ ((row >> 3) & 1);  // 8 chunks per row
  else
    return ((row >> 1) & 3) ^ ((row >> 3) & 1);  // 4 chunks per row
}

enum Epilogue {
  kEpiI32 = 0,      // int32 out (accumulate flag honoured)
  kEpiDequant = 1,  // int8: f16(((float)acc * rs[m]) * cs[n])
  kEpiFloat = 2,    // f16/bf16: fp32 acc -> out dtype (accumulate honoured)
  kEpiW8 = 3,       // f16 A x int8 B: f16(acc * cs[n])
  kEpiSwiglu = 4,   // f16 A x int8 gate/up image: f16(silu(g * sg) * (u * su))
  kEpiW8Res = 5     // f16 A x int8 B: f16((acc * cs[n]) + r[m, n]), fp32 sum
};

// The int8-weight epilogues take B as int8 [N, K] converted to f16 in
// registers (the W8A16 GEMM of the SwiGLU FFN).
constexpr bool b_is_int8(int epi) {
  return epi == kEpiW8 || epi == kEpiSwiglu || epi == kEpiW8Res;
}
// The SwiGLU image (built by this library, never by the caller) stores each
// weight in offset binary, byte = w + 128 (w ^ 0x80 as a bit pattern): that
// byte is the low byte of the f16 1024 + byte = 1152 + w directly, so the
// conversion skips the sign flip the two's-complement B of kEpiW8 /
// kEpiW8Res needs (eight VALU operations per 8 weights instead of ten;
// gate/up of the FFN block at 2048x4096x11008 ran 302.5 -> 297.1 us).
constexpr bool b_offset_binary(int epi) { return epi == kEpiSwiglu; }
constexpr int32_t kOpW8 = HXM_OP_W8A16, kOpSwiglu = HXM_OP_W8A16_SWIGLU;  // tuning-cache keys

// 16-byte f16 output store.  The int8-weight epilogues write activations
// that the next kernel of the FFN block reads (h for the down projection,
// y for the next block's RMSNorm): plain stores keep them in the caches,
// the Infinity Cache included.  The other epilogues' outputs are streamed
// past them (nontemporal).  Measured: the FFN block 3-10 us faster with
// plain stores in its GEMMs (two boxes; the next block's RMSNorm 6.8 ->
// 5.6 us); the int8 4096^3 dequant GEMM alone 54.7 us nontemporal, 56.5 us
// plain.  The row kernels keep nontemporal stores: plain ones made them
// slower and the FFN no faster.
template <int EPI>
__device__ __forceinline__ void store_out8(v8f16 v, _Float16* p) {
  if constexpr (b_is_int8(EPI))
    *reinterpret_cast<v8f16*>(p) = v;
  else
    __builtin_nontemporal_store(v, reinterpret_cast<v8f16*>(p));
}

struct GemmArgs {
  const uint8_t* A;  // [M, K] row-major, lda_bytes
  const uint8_t* B;  // [N, K] row-major, ldb_bytes
  void* C;
  int64_t lda_bytes, ldb_bytes, ldc;  // ldc in elements
  int M, N, K_bytes;
  int accumulate;
  int out_dtype;  // HXM_I32, HXM_F16, HXM_BF16, HXM_F32
  int vec_store;  // C rows allow 4-element vector stores
  int vec8_store; // C rows allow 8-element (16-byte f16) vector stores
  const float* row_scale;
  const float* col_scale;
  int group_m;  // tile-rows per group in the XCD walk
  int n_out;    // kEpiSwiglu: output columns (gate/up channel count)
  const _Float16* residual;  // kEpiW8Res: r [M, N] f16, row stride ldr
  int64_t ldr;
  int res_vec8;  // r rows allow 16-byte loads
  // K split over blockIdx.y: workgroup row z takes A/B bytes [z * kslice_bytes,
  // +kslice_bytes) of K and writes its own C plane at z * plane_elems.
  int split = 1;
  int kslice_bytes = 0;
  int64_t plane_elems = 0;
  // Stream-K (the int8-weight kernels): workgroups [sk_first, sk_first +
  // sk_groups) of the launch each take sk_iters consecutive K stages of the
  // stream over the tiles the data-parallel workgroups [0, sk_first) leave
  // (sk_tiles of them); a tile whose stages span several workgroups is
  // finished by the last to arrive (below).  sk_groups = 0: none.
  int sk_first = 0, sk_groups = 0, sk_tiles = 0, sk_iters = 0, sk_maxseg = 0;
  int sk_xcd = 0;            // 1: each XCD's workgroups stream that XCD's own tiles
  float* sk_part = nullptr;  // fp32 partial tiles, sk_tiles * sk_maxseg slots
  uint32_t* sk_count = nullptr;  // one arrival counter per stream-K tile, left at 0
};

// Cache-policy bit of the buffer intrinsics' aux operand: sc1, coherent at
// device scope across the XCDs' separate L2s (stores write through, loads do
// not hit a line another XCD may have changed).
constexpr int kAuxSc1 = 16;

template <typename T>
struct Mfma;

template <>
struct Mfma<int8_t> {
  typedef v16i32 acc_t;
  __device__ static __forceinline__ acc_t run(v4i32 a, v4i32 b, acc_t c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mfma<_Float16> {
  typedef v16f32 acc_t;
  __device__ static __forceinline__ acc_t run(v4i32 a, v4i32 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8f16, a),
                                                  __builtin_bit_cast(v8f16, b),
                                                  c, 0, 0, 0);
  }
};
template <>
struct Mfma<__bf16> {
  typedef v16f32 acc_t;
  __device__ static __forceinline__ acc_t run(v4i32 a, v4i32 b, acc_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(v8bf16, a), __builtin_bit_cast(v8bf16, b), c, 0, 0, 0);
  }
};

typedef __attribute__((address_space(3))) void lds_void;

// Waits until at most N of this wave's LDS-DMA loads are in flight and all
// its LDS reads are done, then joins the workgroup barrier.  __syncthreads()
// would also drain every outstanding load (vmcnt(0)) and so discard the
// prefetch; the memory clobber keeps the compiler from moving LDS accesses
// across the barrier.
template <int N>
__device__ __forceinline__ void wait_and_barrier() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Buffer resource over rows [row0, rows_valid) of a K-major operand whose
// rows hold row_bytes valid bytes (gfx9 descriptor: 48-bit base, stride 0,
// num_records in bytes, data format word 0x00020000).  Offsets at or past
// num_records read as zero.  The range ends at the last valid byte of the
// last row, (rows - 1) * ld_bytes + row_bytes: the bytes between rows lie
// inside the operand's storage, the bytes after its last row need not.
__device__ __forceinline__ v4i32 operand_rsrc(const uint8_t* base, int64_t ld_bytes,
                                              int row0, int rows_valid, int64_t row_bytes) {
  const int64_t rows = rows_valid > row0 ? rows_valid - row0 : 0;
  int64_t bytes = rows > 0 ? (rows - 1) * ld_bytes + row_bytes : 0;
  if (bytes > 0x7fffffff) bytes = 0x7fffffff;
  const uint64_t a = reinterpret_cast<uint64_t>(base + static_cast<int64_t>(row0) * ld_bytes);
  v4i32 r;
  r[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a & 0xffffffffu));
  r[1] = __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes));
  r[3] = 0x00020000;
  return r;
}

// One LDS-DMA: 16 bytes per lane from rsrc at voffset + soffset into LDS at
// lds + lane*16.  Issued as inline asm so that the compiler's waitcnt pass
// does not track it: every wait on these loads is the kernel's own
// (wait_and_barrier).  Compiler-issued loads stay correct regardless, since
// vmcnt counts in issue order and extra loads in flight only make the
// compiler's own waits stricter.
// `lds` is the LDS byte address (M0).  Callers form it from the low 32 bits
// of the stage buffer's generic address (a generic address in the shared
// aperture carries the LDS address there): that folds to scalar constants,
// where a cast of the generic pointer back to the LDS address space cost a
// null check and two readfirstlanes per load in the main loop.
__device__ __forceinline__ void dma16(uint32_t lds, v4i32 rsrc, uint32_t voffset, int soffset) {
  // The LDS address (M0) and the scalar offset are wave-uniform by construction.
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds);
  soffset = __builtin_amdgcn_readfirstlane(soffset);
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dwordx4 %1, %2, %3 offen lds"
      :
      : "s"(m0), "v"(voffset), "s"(rsrc), "s"(soffset)
      : "memory", "m0");
}

// Per-lane offsets of one operand's stage loads.  Wave instruction q covers
// LDS bytes [q*1024, q*1024+1024): lane l fills the 16 bytes of LDS row
// q*RPI + l/CH, slot l%CH, which hold source chunk slot ^ swz(row).
template <int ROWS, int BKB, int NW>
struct StageLoad {
  static constexpr int CH = BKB / 16;
  static constexpr int RPI = 64 / CH;               // LDS rows per wave instruction
  static constexpr int L = ROWS / RPI / NW;         // instructions per wave per stage
  static_assert(L >= 1 && (ROWS / RPI) % NW == 0, "tile rows must split over waves");
  uint32_t off[L];

  // LDS row and source chunk (16-byte unit within the row's BKB bytes) that
  // lane fills in instruction i.
  __device__ static __forceinline__ int row_of(int i, int wave, int lane) {
    return (i * NW + wave) * RPI + lane / CH;
  }
  __device__ static __forceinline__ int chunk_of(int i, int wave, int lane) {
    return (lane % CH) ^ swz<BKB>(row_of(i, wave, lane));
  }

  __device__ __forceinline__ void init(int64_t ld_bytes, int rows_left, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < L; ++i) {
      const int row = row_of(i, wave, lane);
      off[i] = row < rows_left ? static_cast<uint32_t>(row * ld_bytes + chunk_of(i, wave, lane) * 16)
                               : kOob;
    }
  }

  // Instruction i of a stage at K byte kb0 into the stage buffer at LDS
  // address lds.  CHECK: 16-byte chunks at or past K_bytes read as zero (a
  // per-lane test).  Without it, a stage issued past the end of K reads other
  // bytes of the operand or, past the resource, zeros; the kernel runs the
  // unchecked form only when K_bytes is a multiple of the stage depth, where
  // no stage it multiplies straddles K and the stages past the end land in
  // buffers that are never multiplied.
  template <int I, bool CHECK>
  __device__ __forceinline__ void issue_one(v4i32 r, uint32_t lds, int wave, int lane, int kb0,
                                            int K_bytes) const {
    uint32_t o = off[I];
    if constexpr (CHECK) o = kb0 + chunk_of(I, wave, lane) * 16 < K_bytes ? o : kOob;
    dma16(lds + (I * NW + wave) * 1024, r, o, kb0);
  }
};

// One LDS-DMA of 4 bytes per lane: rsrc at voffset into LDS at lds + lane*4.
__device__ __forceinline__ void dma4(float* lds, v4i32 rsrc, uint32_t voffset) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)lds)));
  asm volatile(
      "s_mov_b32 m0, %0\n\t"
      "buffer_load_dword %1, %2, 0 offen lds"
      :
      : "s"(m0), "v"(voffset), "s"(rsrc)
      : "memory", "m0");
}

// Calls f(integral_constant<int, I>) for I = B .. E-1, so every index inside
// f is a compile-time constant (register arrays stay in registers).
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

template <int BKB>
__device__ __forceinline__ v4i32 lds_frag(const uint8_t* lds, int row, int chunk) {
  return *reinterpret_cast<const v4i32*>(lds + row * BKB + ((chunk ^ swz<BKB>(row)) << 4));
}

template <typename T, int BM, int BN, int BKB, int STAGES, int WM, int WN, int EPI, int SK = 0>
__global__ __launch_bounds__(WM * WN * 64) void gemm_kernel(GemmArgs g0) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;  // wave sub-tile
  constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 blocks per wave
  constexpr int KS = BKB / 32;               // MFMA k-steps per stage
  constexpr bool BQ = b_is_int8(EPI);        // B int8, converted to f16 in registers
  constexpr int BKB_B = BQ ? BKB / 2 : BKB;  // B bytes per LDS row
  constexpr int SB = BM * BKB + BN * BKB_B;  // bytes per stage
  constexpr int NF = FM * FN;                // MFMA slots per k-step
  constexpr int NR = FM + FN;                // fragment reads per k-step
  constexpr int HALF = NF / 2;               // barrier slot of the last k-step
  constexpr int PB = (KS - 1) * NF + HALF;   // slots of a stage before its barrier
  static_assert(FM >= 1 && FN >= 1, "wave tile must hold a 32x32 block");
  static_assert(STAGES >= 2 && STAGES <= 4, "2..4 stages");
  static_assert(KS % 2 == 0, "fragment double buffer assumes an even k-step count");
  using acc_t = typename Mfma<T>::acc_t;
  using LA = StageLoad<BM, BKB, NW>;
  using LB = StageLoad<BN, BKB_B, NW>;
  constexpr int LPW = LA::L + LB::L;  // DMA instructions per wave per stage
  static_assert(!BQ || std::is_same<T, _Float16>::value, "int8 B pairs with f16 A");
  // int8 B: block 0 of a stage's first k-step is read at the barrier slot
  // NF/2 of the previous stage's last k-step and converted in its slots
  // NF-2 and NF-1, which must not come before the read.
  static_assert(!BQ || NF >= 4, "int8 B needs at least 4 MFMA slots per k-step");
  static_assert(EPI != kEpiSwiglu || TN == 128, "SwiGLU image interleaves 64-channel blocks");
  static_assert(!SK || BQ, "stream-K is compiled for the int8-weight kernels");
  // Epilogue scales in LDS: rows [0, QR*64), columns [QR*64, (QR+QC)*64) floats.
  constexpr int QR = EPI == kEpiDequant ? (BM + 63) / 64 : 0;
  constexpr int QC = EPI == kEpiDequant || BQ ? (BN + 63) / 64 : 0;

  // One __shared__ object per stage (see the header comment).
  __shared__ __attribute__((aligned(1024))) uint8_t s0[SB];
  __shared__ __attribute__((aligned(1024))) uint8_t s1[SB];
  __shared__ __attribute__((aligned(1024))) uint8_t s2[STAGES > 2 ? SB : 1024];
  __shared__ __attribute__((aligned(1024))) uint8_t s3[STAGES > 3 ? SB : 1024];
  __shared__ __attribute__((aligned(16))) float ssc[QR + QC > 0 ? (QR + QC) * 64 : 4];
  auto buf = [&](int u) -> uint8_t* {
    return u == 0 ? s0 : u == 1 ? s1 : u == 2 ? s2 : s3;
  };

  if (g0.split > 1) {  // uniform: this workgroup's K slice and C plane
    const int z = blockIdx.y;
    const int kb0 = z * g0.kslice_bytes;  // a multiple of BKB (host)
    g0.A += kb0;
    g0.B += BQ ? kb0 / 2 : kb0;
    g0.K_bytes = min(g0.kslice_bytes, g0.K_bytes - kb0);
    g0.C = static_cast<char*>(g0.C) +
           static_cast<int64_t>(z) * g0.plane_elems * (g0.out_dtype == HXM_I32 || g0.out_dtype == HXM_F32 ? 4 : 2);
  }

  // ---- XCD-aware tile order ----
  // Workgroups are dispatched round-robin over the 8 XCDs, so ordinal b is
  // remapped to position b >> 3 of XCD b & 7's window of ntiles / 8 tiles,
  // and each window is walked in groups of g.group_m tile-rows.
  const int tiles_m = (g0.M + BM - 1) / BM;
  const int tiles_n = (g0.N + BN - 1) / BN;
  const int ntiles = tiles_m * tiles_n;
  auto walk = [&](int b) { return (ntiles & 7) == 0 ? (b & 7) * (ntiles >> 3) + (b >> 3) : b; };
  auto tile_origin = [&](int t, int& m0, int& n0) {
    const int gm = g0.group_m;
    const int per_group = gm * tiles_n;
    const int group = t / per_group;
    const int first_m = group * gm;
    const int gsize = min(tiles_m - first_m, gm);
    m0 = (first_m + (t % per_group) % gsize) * BM;
    n0 = ((t % per_group) / gsize) * BN;
  };

  // The tile body runs once per tile, or (stream-K) once per segment: K
  // stages [k0, k1) of one tile, with A, B and K_bytes of the arguments
  // moved to cover the segment.  After the main loop a whole tile
  // goes to the epilogue; a segment of a tile spread over several
  // workgroups goes through the partial-tile exchange, which leaves the last
  // workgroup to arrive with the whole tile.  Without stream-K the loop
  // condition is constant false: one pass, the body as straight-line code.
  __shared__ int sk_last;
  const int KT_all = (g0.K_bytes + BKB - 1) / BKB;
  // Stream-K: workgroups [0, sk_first) take one whole tile each, as the
  // plain kernel; the sk_groups after them each take sk_iters consecutive K
  // stages of the stream of the remaining tiles (per XCD, the stream of that
  // XCD's own window when sk_xcd: its tiles share A and B panels in that
  // XCD's L2), segment by segment.
  const bool whole = !SK || static_cast<int>(blockIdx.x) < g0.sk_first;
  const int sk_b = blockIdx.x - g0.sk_first;
  const int sk_x = SK && g0.sk_xcd ? sk_b & 7 : 0;
  const int sk_w = SK && g0.sk_xcd ? sk_b >> 3 : sk_b;                      // index in the stream
  const int sk_tn = SK && g0.sk_xcd ? g0.sk_tiles >> 3 : g0.sk_tiles;       // tiles in the stream
  int64_t it = whole ? 0 : static_cast<int64_t>(sk_w) * g0.sk_iters;
  const int64_t it_end =
      whole ? KT_all
            : min(static_cast<int64_t>(sk_tn) * KT_all, static_cast<int64_t>(sk_w + 1) * g0.sk_iters);
  if (SK && it >= it_end) return;  // a stream-K workgroup with no stages left
  const uint8_t* const sk_A = g0.A;
  const uint8_t* const sk_B = g0.B;
  const int sk_K = g0.K_bytes;
  do {
    int m0, n0, sk_slot = -1, sk_seg = 0, sk_nseg = 1;
    if constexpr (SK) {
      const int st = whole ? 0 : static_cast<int>(it / KT_all);
      const int k0 = static_cast<int>(it % KT_all);
      const int k1 = static_cast<int>(min<int64_t>(KT_all, k0 + (it_end - it)));
      if (!whole) {
        const int64_t tfirst = static_cast<int64_t>(st) * KT_all;
        const int seg0 = static_cast<int>(tfirst / g0.sk_iters);
        sk_nseg = static_cast<int>((tfirst + KT_all - 1) / g0.sk_iters) - seg0 + 1;
        sk_seg = sk_w - seg0;
        sk_slot = sk_x * sk_tn + st;
      }
      // The tile's walk index: the workgroup's own, or position sk_first / 8
      // + st of this XCD's window, or ordinal sk_first + st.
      tile_origin(whole       ? walk(blockIdx.x)
                  : g0.sk_xcd ? sk_x * (ntiles >> 3) + (g0.sk_first >> 3) + st
                              : walk(g0.sk_first + st),
                  m0, n0);
      g0.A = sk_A + k0 * BKB;
      g0.B = sk_B + k0 * (BKB / 2);
      g0.K_bytes = min(sk_K, k1 * BKB) - k0 * BKB;
      it += k1 - k0;
      wait_and_barrier<0>();  // the previous segment is done with the LDS
    } else {
      tile_origin(walk(blockIdx.x), m0, n0);
    }
    const GemmArgs& g = g0;
    // The lane's indices.  In the stream-K loop they come from an opaque
    // copy of the thread id made in each pass, so the compiler recomputes
    // what depends on them per tile instead of hoisting it out of the loop
    // and holding it in registers through the main loop.
    int tid = threadIdx.x;
    if constexpr (SK) asm volatile("" : "+v"(tid));
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform
    const int wm = wave / WN, wn = wave % WN;

  const v4i32 ra = operand_rsrc(g.A, g.lda_bytes, m0, g.M, g.K_bytes);
  const v4i32 rb = operand_rsrc(g.B, g.ldb_bytes, n0, g.N, BQ ? g.K_bytes / 2 : g.K_bytes);
  LA la;
  LB lb;
  la.init(g.lda_bytes, g.M - m0, wave, lane);
  lb.init(g.ldb_bytes, g.N - n0, wave, lane);

  // The tile's epilogue scales go to LDS by DMA ahead of the first stage, so
  // they arrive under the prologue and cost the epilogue one LDS read each.
  // Scales of rows / columns outside C read as zero.
  if constexpr (QR + QC > 0) {
    const v4i32 rr = QR ? operand_rsrc(reinterpret_cast<const uint8_t*>(g.row_scale), 4, m0, g.M, 4)
                        : v4i32{};
    const v4i32 rc = operand_rsrc(reinterpret_cast<const uint8_t*>(g.col_scale), 4, n0, g.N, 4);
    for (int q = wave; q < QR + QC; q += NW) {
      if (q < QR) dma4(ssc + q * 64, rr, (q * 64 + lane) * 4);
      else dma4(ssc + q * 64, rc, ((q - QR) * 64 + lane) * 4);
    }
  }

  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = acc_t{};

  const int KT = (g.K_bytes + BKB - 1) / BKB;
  const int K_bytes = g.K_bytes;                    // of A
  const int K_bytes_B = BQ ? K_bytes / 2 : K_bytes;  // of B

  // DMA instruction D (A's first, then B's) of the stage at A byte kb0.
  // CHK: std::true_type / std::false_type, the K-range test of issue_one.
  auto dma = [&](auto D, auto CHK, uint8_t* dst, int kb0) {
    constexpr int d = decltype(D)::value;
    constexpr bool chk = decltype(CHK)::value;
    const uint32_t l = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(dst));
    if constexpr (d < LA::L) {
      la.template issue_one<d, chk>(ra, l, wave, lane, kb0, K_bytes);
    } else {
      const int kb0_b = BQ ? kb0 / 2 : kb0;
      lb.template issue_one<d - LA::L, chk>(rb, l + BM * BKB, wave, lane, kb0_b, K_bytes_B);
    }
  };
  auto issue_stage = [&](int kt, uint8_t* dst) {
    static_for<0, LPW>([&](auto D) { dma(D, std::true_type{}, dst, kt * BKB); });
  };

  // Fragments of the k-step being multiplied ([ks & 1]) and of the next one.
  // Read R of a k-step: A block 0, the FN B blocks, then A blocks 1..FM-1 --
  // the order the MFMA slots (i, j) = (s / FN, s % FN) first need them.
  // With an int8 B the read brings the lane's 16 bytes of a pair of k-steps
  // (below) into braw, and the slots run column-major,
  // (i, j) = (s % FM, s / FM), so B block j is first needed at slot j*FM:
  // its conversion to f16 (cvt_word, four words) is spread over the FM slots
  // before that, block 0's over the end of the previous k-step.  A wave is
  // alone on its SIMD, so a conversion issued whole between two MFMAs that
  // the second one needs (ten dependent VALU operations, longer than one
  // MFMA) would leave the matrix core idle.  The B reads come first, then
  // the A blocks.
  //
  // int8 B is read a pair of k-steps at a time.  The K order inside a pair
  // of MFMAs is free as long as A and B follow the same one, so the pair's
  // 32 K values are split by lane half, not by k-step: lane half hi takes K
  // [32p + 16hi, +16) of pair p, the first 8 values for the pair's first
  // MFMA and the next 8 for its second.  Those 16 bytes are one 16-byte
  // chunk of the B row, so one ds_read_b128 per lane serves both k-steps,
  // and 16 consecutive rows at one chunk index fall on distinct banks under
  // the swizzle.  (Per k-step, each lane half took the matching 8 bytes of a
  // chunk, and the 32 lanes of a half met every bank twice: measured
  // SQ_LDS_BANK_CONFLICT of the FFN's GEMMs was about one conflict cycle per
  // LDS instruction.)  A's chunk for k-step ks = 2p + j is then 4p + 2hi + j.
  v4i32 af[2][FM], bf[2][FN];
  uint4 braw[2][BQ ? FN : 1];         // [pair parity]: both k-steps of a pair
  uint32_t bflip[2][BQ ? FN : 1][2];  // [k-step parity]: its words in offset binary
  const int r32 = lane & 31, hi = lane >> 5;
  static_assert(!BQ || KS % 4 == 0, "int8 B pairs: an even number of pairs per stage");
  auto read = [&](auto R, int dstb, const uint8_t* stage, auto KSC) {
    constexpr int r = decltype(R)::value;
    constexpr int ks = decltype(KSC)::value;
    constexpr bool is_b = BQ ? r < FN : r >= 1 && r <= FN;
    constexpr int idx = BQ ? (is_b ? r : r - FN) : r == 0 ? 0 : is_b ? r - 1 : r - FN;
    if constexpr (is_b && BQ) {
      if constexpr (ks % 2 == 0) {  // the pair (ks, ks + 1)
        const int row = idx * 32 + r32;
        braw[(ks >> 1) & 1][idx] = *reinterpret_cast<const uint4*>(
            stage + BM * BKB + (wn * TN + row) * BKB_B + (((ks + hi) ^ swz<BKB_B>(row)) << 4));
      }
    } else if constexpr (is_b) {
      bf[dstb][idx] = lds_frag<BKB>(stage + (BM + wn * TN) * BKB, idx * 32 + r32, ks * 2 + hi);
    } else if constexpr (BQ) {
      af[dstb][idx] = lds_frag<BKB>(stage + (wm * TM) * BKB, idx * 32 + r32,
                                    4 * (ks >> 1) + 2 * hi + (ks & 1));
    } else {
      af[dstb][idx] = lds_frag<BKB>(stage + (wm * TM) * BKB, idx * 32 + r32, ks * 2 + hi);
    }
  };
  // Word P of B block j's f16 fragment (elements 2P, 2P+1) for k-step ks of
  // a stage, from its pair's braw words 2 * (ks & 1) and 2 * (ks & 1) + 1.
  auto cvt_word = [&](auto P, auto KSC, int j) {
    constexpr int p = decltype(P)::value;
    constexpr int ks = decltype(KSC)::value;
    constexpr int b = ks & 1;
    if constexpr (BQ) {
      if constexpr (p % 2 == 0) {
        const uint4& w = braw[(ks >> 1) & 1][j];
        const uint32_t raw = b == 0 ? (p == 0 ? w.x : w.y) : (p == 0 ? w.z : w.w);
        bflip[b][j][p / 2] = raw ^ (b_offset_binary(EPI) ? 0u : 0x80808080u);
      }
      bf[b][j][p] = static_cast<int>(i8x2_flipped_to_f16<p % 2>(bflip[b][j][p / 2]));
    }
  };
  // The conversion words issued in slot sl of k-step ks (multiplying buffer
  // cb): words of blocks 1..FN-1 of this k-step in the FM slots before their
  // first use, words of block 0 of the next k-step in the last FM slots (in
  // the last k-step of a stage, whose reads of the next stage start at the
  // barrier, in its last two slots).
  auto cvt_slot = [&](auto KSI, auto SI) {
    constexpr int ks = decltype(KSI)::value, sl = decltype(SI)::value;
    if constexpr (BQ) {
      static_for<0, 4>([&](auto P) {
        constexpr int p = decltype(P)::value;
        static_for<1, FN>([&](auto J) {
          constexpr int j = decltype(J)::value;
          if constexpr ((j - 1) * FM + (p * FM) / 4 == sl) cvt_word(P, KSI, j);
        });
        constexpr int s0 = ks == KS - 1 ? NF - 2 + p / 2 : (FN - 1) * FM + (p * FM) / 4;
        if constexpr (s0 == sl) cvt_word(P, std::integral_constant<int, (ks + 1) % KS>{}, 0);
      });
    }
  };

  // Every stage slot issues its DMAs, also past the end of K: a stage at or
  // past K_bytes reads zeros (see issue_one) into a buffer no later stage
  // uses, so the number of stages in flight is the same at every wait and
  // the instruction stream has no branches for the compiler's waitcnt
  // analysis to merge.

  // DMA schedule.  Stage j goes to buffer j % STAGES, which is free from the
  // barrier of iteration j-STAGES on (every read of stage j-STAGES precedes
  // that barrier) and must have landed at the barrier of iteration j-1.
  // Instruction d of stage j issues at position dv(d) of iteration
  // j-STAGES+1, counted from its first slot; a negative position is a slot
  // after the barrier of the iteration before.  With two stages the
  // instructions are packed into the first two thirds of the window so the
  // last ones land before the wait; with more stages they are spread over
  // the whole window.
  constexpr int SLOTS = KS * NF;             // MFMA slots per stage
  constexpr int POST = SLOTS - PB;           // slots after the barrier
  constexpr int DW = STAGES == 2 ? (2 * SLOTS) / 3 : SLOTS;
  static_assert(((LPW - 1) * DW) / LPW - POST < PB, "DMA window ends before the barrier");
  constexpr int NEG = [] {                   // instructions issued a stage early
    int n = 0;
    for (int d = 0; d < LPW; ++d) n += (d * DW) / LPW - POST < 0;
    return n;
  }();
  static_assert((STAGES - 2) * LPW + NEG <= 63, "vmcnt range");

  // One stage.  Its KS*NF MFMA slots run in a fixed order (a scheduling
  // barrier closes each slot).  Spread over the slots: the DMA instructions
  // (above), and the fragment reads of k-step ks+1.  At slot HALF of the
  // last k-step the wave waits for stage kt+1 (stages kt+2 .. kt+STAGES-1 may
  // stay in flight); the barrier also tells it that every wave is done
  // reading stage kt, whose buffer the early DMAs of stage kt+STAGES then
  // refill.  It then reads stage kt+1's first fragments under the remaining
  // MFMAs.
  auto stage = [&](auto U, auto CHK, int kt) {
    constexpr int u = decltype(U)::value;
    const uint8_t* cur = buf(u);
    const uint8_t* nxt = buf((u + 1) % STAGES);
    uint8_t* dbuf = buf((u + STAGES - 1) % STAGES);  // stage kt+STAGES-1
    uint8_t* ebuf = buf(u);                          // stage kt+STAGES (early part)
    const int kbd = (kt + STAGES - 1) * BKB;
    static_for<0, KS>([&](auto KSI) {
      constexpr int ks = decltype(KSI)::value;
      constexpr int cb = ks & 1;
      static_for<0, NF>([&](auto SI) {
        constexpr int sl = decltype(SI)::value;
        constexpr int slot = ks * NF + sl;
        if constexpr (ks == KS - 1 && sl == HALF) wait_and_barrier<(STAGES - 2) * LPW>();
        static_for<0, LPW>([&](auto D) {
          constexpr int v = (decltype(D)::value * DW) / LPW - POST;
          if constexpr (v >= 0 && v == slot) dma(D, CHK, dbuf, kbd);
          if constexpr (v < 0 && SLOTS + v == slot) dma(D, CHK, ebuf, kbd + BKB);
        });
        static_for<0, NR>([&](auto R) {
          constexpr int r = decltype(R)::value;
          if constexpr (ks < KS - 1) {
            if constexpr ((r * NF) / NR == sl)
              read(R, cb ^ 1, cur, std::integral_constant<int, ks + 1>{});
          } else {
            if constexpr (HALF + (r * (NF - HALF)) / NR == sl)
              read(R, cb ^ 1, nxt, std::integral_constant<int, 0>{});
          }
        });
        // A snake over the wave's blocks: rows (columns, for an int8 B) in
        // turn, every other one walked backwards, so each MFMA shares one
        // operand with the one before it.  Operand changes cost power: an
        // MFMA-only loop on random operands ran 0.7% faster in this order
        // than in the plain row order (int8 and f16 alike).  Every fragment
        // is still first needed at the slot the plain order gives it.
        constexpr int i0 = BQ ? sl % FM : sl / FN, j0 = BQ ? sl / FM : sl % FN;
        constexpr int i = BQ && (j0 & 1) ? FM - 1 - i0 : i0;
        constexpr int j = !BQ && (i0 & 1) ? FN - 1 - j0 : j0;
        acc[i][j] = Mfma<T>::run(bf[cb][j], af[cb][i], acc[i][j]);
        cvt_slot(KSI, SI);
        __builtin_amdgcn_sched_barrier(0);
      });
    });
  };

  if (KT > 0) {
    // Prologue: stages 0 .. STAGES-2, the early part of stage STAGES-1, then
    // the first k-step's fragments.
    static_for<0, STAGES - 1>([&](auto Pi) {
      issue_stage(decltype(Pi)::value, buf(decltype(Pi)::value));
    });
    static_for<0, LPW>([&](auto D) {
      if constexpr ((decltype(D)::value * DW) / LPW - POST < 0)
        dma(D, std::true_type{}, buf(STAGES - 1), (STAGES - 1) * BKB);
    });
    wait_and_barrier<(STAGES - 2) * LPW + NEG>();
    static_for<0, NR>([&](auto R) { read(R, 0, buf(0), std::integral_constant<int, 0>{}); });
    static_for<0, 4>([&](auto P) { cvt_word(P, std::integral_constant<int, 0>{}, 0); });

    // Main loop, unrolled by STAGES so every buffer choice is static.  It is
    // compiled twice: without the per-lane K test (K_bytes a multiple of the
    // stage depth: two VALU operations fewer per LDS-DMA) and with it.
    auto main_loop = [&](auto CHK) {
      for (int kt0 = 0; kt0 < KT; kt0 += STAGES) {
        static_for<0, STAGES>([&](auto U) {
          const int kt = kt0 + decltype(U)::value;
          if (kt < KT) stage(U, CHK, kt);
        });
      }
    };
    if (K_bytes % BKB == 0)
      main_loop(std::false_type{});
    else
      main_loop(std::true_type{});
  }

  // ---- stream-K: partial tiles ----
  // Every segment of a shared tile stores its fp32 accumulators (each lane's
  // registers, 16 bytes a store, device-coherent) in its slot, then counts
  // its arrival; the workgroup that arrives last adds the slots in segment
  // order -- a fixed order, so the result does not depend on which
  // workgroup that is -- resets the counter for the next launch and runs the
  // epilogue.  Nobody waits for anybody: a workgroup that is not last is
  // done.
  if constexpr (SK) {
    if (sk_slot >= 0 && sk_nseg > 1) {
      constexpr int kWaveFloats = FM * FN * 16 * 64;
      wait_and_barrier<0>();  // the main loop's last (past-K) loads have landed
      const int64_t slot_bytes = static_cast<int64_t>(NW) * kWaveFloats * 4;
      const uint8_t* part0 = reinterpret_cast<const uint8_t*>(g.sk_part) +
                             static_cast<int64_t>(sk_slot) * g.sk_maxseg * slot_bytes;
      auto slot_rsrc = [&](int seg) {
        return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(part0 + seg * slot_bytes),
                                                 static_cast<short>(0),
                                                 static_cast<int>(slot_bytes), 0x00020000);
      };
      const uint32_t wave_off = static_cast<uint32_t>(wave) * kWaveFloats * 4 + lane * 16;
      {
        const __amdgpu_buffer_rsrc_t mine = slot_rsrc(sk_seg);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              v4f32 v;
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float a = acc[i][j][q * 4 + e];  // copy the element out first
                v[e] = a;
              }
              __builtin_amdgcn_raw_buffer_store_b128(
                  __builtin_bit_cast(v4u32_t, v), mine,
                  wave_off + static_cast<uint32_t>(((i * FN + j) * 4 + q) * 1024), 0, kAuxSc1);
              __builtin_amdgcn_sched_barrier(0);
            }
      }
      // Every wave's stores complete before the workgroup's one arrival.
      asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
      if (threadIdx.x == 0) {
        const uint32_t before = __hip_atomic_fetch_add(g.sk_count + sk_slot, 1u, __ATOMIC_RELAXED,
                                                       __HIP_MEMORY_SCOPE_AGENT);
        const int last = before == static_cast<uint32_t>(sk_nseg - 1);
        if (last)
          __hip_atomic_store(g.sk_count + sk_slot, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        sk_last = last;
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (!sk_last) continue;
      // The whole tile: every slot, this segment's own included (its stores
      // completed above), added in segment order, ((p0 + p1) + p2) ..., and
      // written over the accumulators, which are not read again.  One row
      // of FN blocks of one slot is loaded per round trip (every load of the
      // row in flight at once): a block at a time, each a device-coherent
      // round trip, cost 21 us on the FFN's gate/up GEMM.
      auto slot_row = [&](int sg, int i, acc_t (&v)[FN]) {
        const __amdgpu_buffer_rsrc_t r = slot_rsrc(sg);
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const v4f32 x = __builtin_bit_cast(
                v4f32, __builtin_amdgcn_raw_buffer_load_b128(
                           r, wave_off + static_cast<uint32_t>(((i * FN + j) * 4 + q) * 1024), 0,
                           kAuxSc1));
#pragma unroll
            for (int e = 0; e < 4; ++e) v[j][q * 4 + e] = x[e];
          }
      };
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        acc_t t[FN];
        slot_row(0, i, t);
        for (int sg = 1; sg < sk_nseg; ++sg) {
          acc_t v[FN];
          slot_row(sg, i, v);
#pragma unroll
          for (int j = 0; j < FN; ++j) t[j] += v[j];
        }
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = t[j];
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }

  // ---- epilogue ----
  // Lane l holds, for block (i, j) and register group q = v/4, row
  // m = i*32 + l%32 of the wave tile and the four consecutive columns
  // j*32 + 8q + 4*(l/32) + 0..3.  The tile is written through LDS one 32-row
  // block at a time: each lane stages its 4-element runs as 32-bit words
  // (int32, or the fp32 accumulator) in a padded [32][TN+4] array, and the
  // wave reads back row-contiguous 16-byte runs, applies the output
  // conversion (the dequant scales come from LDS) and stores whole rows.
  // Keeping the register-to-LDS copy a plain move keeps the accumulators in
  // AGPRs through the epilogue.
  constexpr int kPad = TN + 4;                 // staging row stride (words)
  constexpr int kStageWords = 32 * kPad;       // one wave's 32-row block
  constexpr int kWavesPerBuf = (NW + STAGES - 1) / STAGES;
  static_assert(kWavesPerBuf * kStageWords * 4 <= SB, "epilogue staging must fit a stage");
  const int mw = m0 + wm * TM, nw = n0 + wn * TN;

  wait_and_barrier<0>();  // stage buffers free; scales landed and visible
  float* stg = reinterpret_cast<float*>(buf(wave % STAGES)) + (wave / STAGES) * kStageWords;

  // A tile wholly inside C with 16-byte aligned rows takes a branch-free
  // path (one wave per SIMD: nothing hides a per-run LDS round trip).  A tile
  // that crosses M or N takes the same path with a predicate on each run's
  // store (and residual load) when N is a multiple of the run length, so
  // that every run lies wholly inside or wholly outside C.
  const bool full8 = g.vec8_store && m0 + BM <= g.M && n0 + BN <= g.N;

  // 1. registers -> LDS: block row i, lane row r32, 4 consecutive columns
  // per register group, as raw 32-bit words.
  auto stage_block = [&](int i) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v4f32 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if constexpr (EPI == kEpiFloat || BQ) {
            w[e] = acc[i][j][q * 4 + e];
          } else {
            // int32 bits.  Copy the element out first: clang lowers
            // __builtin_bit_cast of an ext-vector element expression as a
            // read of element 0.
            const int32_t a = acc[i][j][q * 4 + e];
            w[e] = __builtin_bit_cast(float, a);
          }
        }
        *reinterpret_cast<v4f32*>(stg + r32 * kPad + j * 32 + q * 8 + hi * 4) = w;
      }
  };

  // 8-element f16 output rows (full tiles, or edge tiles with N % 8 == 0):
  // a branch-free pipeline over half-blocks (32 rows x TN/2 columns, block
  // row i = n / 2, columns half h = n % 2) through two LDS staging buffers
  // per wave.  Half-block n+1 is
  // written to LDS while the VALU converts half-block n, and all LDS reads of
  // a half-block are issued before its arithmetic.  The buffer written for
  // n+1 was last read for n-1, earlier in program order; a wave's LDS
  // operations complete in order, so the write never overtakes that read.
  // With 8-element runs a lane's columns are the same in every pass,
  // col8 = (lane % kRprH) * 8, so its column scales are read once.
  // kEpiW8Res adds the residual run of each output run: its loads are
  // issued two half-blocks ahead (a ring of three register sets), so they
  // land under the staging and arithmetic of the half-blocks in between.
  if constexpr ((EPI == kEpiDequant || EPI == kEpiW8 || EPI == kEpiW8Res) && FN % 2 == 0) {
    const bool edge8 = !full8 && g.vec8_store && g.N % 8 == 0;
    if ((full8 || edge8) && (EPI != kEpiW8Res || g.res_vec8)) {
      auto pipeline = [&](auto EDGE) {
        constexpr bool edge = decltype(EDGE)::value;
        constexpr int TNH = TN / 2;
        constexpr int kPadH = TNH + 4;             // staging row stride (words)
        constexpr int kWordsH = 32 * kPadH;        // one half-block buffer
        constexpr int kRprH = TNH / 8;             // 8-element runs per staged row
        constexpr int kRowsItH = 64 / kRprH;       // rows one pass of the wave covers
        constexpr int kItH = 32 / kRowsItH;        // passes per half-block
        constexpr int NH = FM * 2;                 // half-blocks per wave
        static_assert(64 % kRprH == 0 && kItH >= 1, "8-element runs must tile the wave");
        static_assert(kWavesPerBuf * 2 * kWordsH * 4 <= SB, "epilogue staging must fit a stage");
        float* hb0 = reinterpret_cast<float*>(buf(wave % STAGES)) + (wave / STAGES) * 2 * kWordsH;
        float* hb1 = hb0 + kWordsH;
        const int col8 = (lane % kRprH) * 8, rsub8 = lane / kRprH;
        v4f32 csh[2][2];
  #pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float* csp = ssc + QR * 64 + wn * TN + h * TNH + col8;
          csh[h][0] = *reinterpret_cast<const v4f32*>(csp);
          csh[h][1] = *reinterpret_cast<const v4f32*>(csp + 4);
        }
        // Registers -> LDS: block columns [h*FN/2, (h+1)*FN/2) of block row i.
        auto stage_half = [&](int n, float* dst) {
          const int i = n / 2, h = n % 2;
  #pragma unroll
          for (int jj = 0; jj < FN / 2; ++jj)
  #pragma unroll
            for (int q = 0; q < 4; ++q) {
              v4f32 w;
  #pragma unroll
              for (int e = 0; e < 4; ++e) {
                if constexpr (EPI != kEpiDequant) {
                  w[e] = acc[i][h * (FN / 2) + jj][q * 4 + e];
                } else {
                  // Copy the element out first (see stage_block).
                  const int32_t a = acc[i][h * (FN / 2) + jj][q * 4 + e];
                  w[e] = __builtin_bit_cast(float, a);
                }
              }
              *reinterpret_cast<v4f32*>(dst + r32 * kPadH + jj * 32 + q * 8 + hi * 4) = w;
            }
        };
        v4f32 w0[2][kItH], w1[2][kItH];
        float rsv[2][kItH];
        auto read_half = [&](int n, const float* src, int set) {
  #pragma unroll
          for (int it = 0; it < kItH; ++it) {
            const int row = it * kRowsItH + rsub8;
            w0[set][it] = *reinterpret_cast<const v4f32*>(src + row * kPadH + col8);
            w1[set][it] = *reinterpret_cast<const v4f32*>(src + row * kPadH + col8 + 4);
            rsv[set][it] = EPI == kEpiDequant ? ssc[wm * TM + (n / 2) * 32 + row] : 1.0f;
          }
        };
        const int64_t step = static_cast<int64_t>(kRowsItH) * g.ldc;
        constexpr int kRes = EPI == kEpiW8Res ? kItH : 1;
        v8f16 rres[3][kRes];
        const _Float16* rbase =
            EPI == kEpiW8Res ? g.residual + static_cast<int64_t>(mw + rsub8) * g.ldr + nw + col8
                             : nullptr;
        auto load_res = [&](int n) {
          if constexpr (EPI == kEpiW8Res) {
  #pragma unroll
            for (int it = 0; it < kItH; ++it) {
              const int row = (n / 2) * 32 + it * kRowsItH, col = (n % 2) * TNH;
              if (!edge || (mw + row + rsub8 < g.M && nw + col + col8 < g.N))
                rres[n % 3][it] = *reinterpret_cast<const v8f16*>(
                    rbase + static_cast<int64_t>(row) * g.ldr + col);
              else
                rres[n % 3][it] = v8f16{};
            }
          }
        };
        load_res(0);
        if (NH > 1) load_res(1);
        stage_half(0, hb0);
        read_half(0, hb0, 0);
  #pragma unroll
        for (int n = 0; n < NH; ++n) {
          const int cur = n & 1;
          if (n + 2 < NH) load_res(n + 2);
          if (n + 1 < NH) stage_half(n + 1, cur ? hb0 : hb1);
          const int i = n / 2, h = n % 2;
          _Float16* c = static_cast<_Float16*>(g.C) +
                        static_cast<int64_t>(mw + i * 32 + rsub8) * g.ldc + nw + h * TNH + col8;
  #pragma unroll
          for (int it = 0; it < kItH; ++it) {
            v8f16 hv;
  #pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float we = e < 4 ? w0[cur][it][e] : w1[cur][it][e - 4];
              const float ce = csh[h][e / 4][e % 4];
              // Same spellings as the general path below.
              float p;
              if constexpr (EPI == kEpiDequant)
                p = (static_cast<float>(__builtin_bit_cast(int32_t, we)) * rsv[cur][it]) * ce;
              else
                p = we * ce;
              asm volatile("" : "+v"(p));
              if constexpr (EPI == kEpiW8Res) {
                // fp32 sum, then one rounding to f16: the pin keeps the
                // backend from fusing the add into a mixed-precision fma.
                p = p + static_cast<float>(rres[n % 3][it][e]);
                asm volatile("" : "+v"(p));
              }
              hv[e] = static_cast<_Float16>(p);
            }
            if (!edge || (mw + i * 32 + it * kRowsItH + rsub8 < g.M && nw + h * TNH + col8 < g.N))
              store_out8<EPI>(hv, c + it * step);
          }
          if (n + 1 < NH) read_half(n + 1, cur ? hb0 : hb1, cur ^ 1);
        }
      };
      if (full8)
        pipeline(std::false_type{});
      else
        pipeline(std::true_type{});
      continue;
    }
  }
  // SwiGLU (full tiles, or edge tiles with n_out % 8 == 0): the same
  // two-buffer half-block pipeline.  The wave's 128 image columns are 64
  // gate channels then the same 64 up channels, so half-block h (h = 0, 1)
  // stages gate block h next to up block h + 2: each staged row holds 32
  // gate and the matching 32 up values, output channels nw/2 + 32h + 0..31.
  if constexpr (EPI == kEpiSwiglu) {
    const bool full_sw = g.vec8_store && m0 + BM <= g.M && n0 + BN <= g.N &&
                         (n0 + BN) / 2 <= g.n_out;
    if (full_sw || (g.vec8_store && g.n_out % 8 == 0)) {
      auto pipeline = [&](auto EDGE) {
        constexpr bool edge = decltype(EDGE)::value;
        constexpr int kPadS = 64 + 4;              // staging row stride (words)
        constexpr int kWordsS = 32 * kPadS;        // one half-block buffer
        constexpr int kRprS = 32 / 8;              // 8-channel runs per staged row
        constexpr int kRowsItS = 64 / kRprS;       // rows one pass covers
        constexpr int kItS = 32 / kRowsItS;        // passes per half-block
        constexpr int NH = FM * 2;
        static_assert(FN == 4, "SwiGLU wave tile is 128 columns");
        static_assert(kWavesPerBuf * 2 * kWordsS * 4 <= SB, "epilogue staging must fit a stage");
        float* hb0 = reinterpret_cast<float*>(buf(wave % STAGES)) + (wave / STAGES) * 2 * kWordsS;
        float* hb1 = hb0 + kWordsS;
        const int ch = (lane % kRprS) * 8, rsub = lane / kRprS;
        v4f32 sgv[2][2], suv[2][2];
  #pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float* sp = ssc + QR * 64 + wn * TN + h * 32 + ch;
          sgv[h][0] = *reinterpret_cast<const v4f32*>(sp);
          sgv[h][1] = *reinterpret_cast<const v4f32*>(sp + 4);
          suv[h][0] = *reinterpret_cast<const v4f32*>(sp + 64);
          suv[h][1] = *reinterpret_cast<const v4f32*>(sp + 68);
        }
        auto stage_sw = [&](int n, float* dst) {
          const int i = n / 2, h = n % 2;
  #pragma unroll
          for (int part = 0; part < 2; ++part)
  #pragma unroll
            for (int q = 0; q < 4; ++q) {
              v4f32 w;
  #pragma unroll
              for (int e = 0; e < 4; ++e) w[e] = acc[i][h + 2 * part][q * 4 + e];
              *reinterpret_cast<v4f32*>(dst + r32 * kPadS + part * 32 + q * 8 + hi * 4) = w;
            }
        };
        v4f32 gv[2][kItS][2], uv[2][kItS][2];
        auto read_sw = [&](const float* src, int set) {
  #pragma unroll
          for (int it = 0; it < kItS; ++it) {
            const float* sp = src + (it * kRowsItS + rsub) * kPadS + ch;
            gv[set][it][0] = *reinterpret_cast<const v4f32*>(sp);
            gv[set][it][1] = *reinterpret_cast<const v4f32*>(sp + 4);
            uv[set][it][0] = *reinterpret_cast<const v4f32*>(sp + 32);
            uv[set][it][1] = *reinterpret_cast<const v4f32*>(sp + 36);
          }
        };
        const int64_t step = static_cast<int64_t>(kRowsItS) * g.ldc;
        stage_sw(0, hb0);
        read_sw(hb0, 0);
  #pragma unroll
        for (int n = 0; n < NH; ++n) {
          const int cur = n & 1;
          if (n + 1 < NH) stage_sw(n + 1, cur ? hb0 : hb1);
          const int i = n / 2, h = n % 2;
          _Float16* c = static_cast<_Float16*>(g.C) +
                        static_cast<int64_t>(mw + i * 32 + rsub) * g.ldc + nw / 2 + h * 32 + ch;
  #pragma unroll
          for (int it = 0; it < kItS; ++it) {
            v8f16 hv;
  #pragma unroll
            for (int e = 0; e < 8; ++e) {
              // Same arithmetic as the general path below.
              const float gval = gv[cur][it][e / 4][e % 4] * sgv[h][e / 4][e % 4];
              const float uval = uv[cur][it][e / 4][e % 4] * suv[h][e / 4][e % 4];
              const float ex = __builtin_amdgcn_exp2f(-gval * 1.4426950408889634f);
              hv[e] = static_cast<_Float16>(gval * __builtin_amdgcn_rcpf(1.0f + ex) * uval);
            }
            if (!edge || (mw + i * 32 + it * kRowsItS + rsub < g.M && nw / 2 + h * 32 + ch < g.n_out))
              store_out8<EPI>(hv, c + it * step);
          }
          if (n + 1 < NH) read_sw(cur ? hb0 : hb1, cur ^ 1);
        }
      };
      if (full_sw)
        pipeline(std::false_type{});
      else
        pipeline(std::true_type{});
      continue;
    }
  }
  if constexpr (EPI == kEpiI32 || EPI == kEpiFloat) {
    // Plain overwrite (full tiles, or edge tiles with N % 4 == 0):
    // 4-element runs, one row address per block, a per-run check only on
    // edge tiles.
    const bool full4 = g.vec_store && !g.accumulate && m0 + BM <= g.M && n0 + BN <= g.N;
    if (full4 || (g.vec_store && !g.accumulate && g.N % 4 == 0)) {
      auto plain = [&](auto EDGE) {
        constexpr bool edge = decltype(EDGE)::value;
        constexpr int kRunsPerRow = TN / 4;
        constexpr int kIt4 = 32 * TN / 4 / 64;
        constexpr int kRowsIt4 = 64 / kRunsPerRow;
        static_assert(64 % kRunsPerRow == 0, "4-element runs must tile the wave");
        const int col = (lane % kRunsPerRow) * 4, rsub = lane / kRunsPerRow;
        const int64_t step = static_cast<int64_t>(kRowsIt4) * g.ldc;
        // The run of pass it of block row i lies inside C (tiles crossing M or N).
        auto in_c = [&](int i, int it) {
          return mw + i * 32 + it * kRowsIt4 + rsub < g.M && nw + col < g.N;
        };
  #pragma unroll
        for (int i = 0; i < FM; ++i) {
          stage_block(i);
          v4f32 wv[kIt4];
  #pragma unroll
          for (int it = 0; it < kIt4; ++it)
            wv[it] = *reinterpret_cast<const v4f32*>(stg + (it * kRowsIt4 + rsub) * kPad + col);
          const int64_t off0 = static_cast<int64_t>(mw + i * 32 + rsub) * g.ldc + nw + col;
          if constexpr (EPI == kEpiI32) {
            int32_t* c = static_cast<int32_t*>(g.C) + off0;
  #pragma unroll
            for (int it = 0; it < kIt4; ++it)
              if (!edge || in_c(i, it))
                __builtin_nontemporal_store(__builtin_bit_cast(v4u32_t, wv[it]),
                                            reinterpret_cast<v4u32_t*>(c + it * step));
          } else if (g.out_dtype == HXM_F32) {
            float* c = static_cast<float*>(g.C) + off0;
  #pragma unroll
            for (int it = 0; it < kIt4; ++it)
              if (!edge || in_c(i, it)) *reinterpret_cast<v4f32*>(c + it * step) = wv[it];
          } else if (g.out_dtype == HXM_F16) {
            _Float16* c = static_cast<_Float16*>(g.C) + off0;
  #pragma unroll
            for (int it = 0; it < kIt4; ++it) {
              v4f16_t h;
  #pragma unroll
              for (int e = 0; e < 4; ++e) h[e] = static_cast<_Float16>(wv[it][e]);
              if (!edge || in_c(i, it)) *reinterpret_cast<v4f16_t*>(c + it * step) = h;
            }
          } else {
            __bf16* c = static_cast<__bf16*>(g.C) + off0;
  #pragma unroll
            for (int it = 0; it < kIt4; ++it) {
              v4bf16_t h;
  #pragma unroll
              for (int e = 0; e < 4; ++e) h[e] = static_cast<__bf16>(wv[it][e]);
              if (!edge || in_c(i, it)) *reinterpret_cast<v4bf16_t*>(c + it * step) = h;
            }
          }
        }
      };
      if (full4)
        plain(std::false_type{});
      else
        plain(std::true_type{});
      continue;
    }
  }

  // General path: accumulate, unaligned rows, edge tiles whose runs may
  // straddle N.
#pragma unroll
  for (int i = 0; i < FM; ++i) {
    stage_block(i);
    // 2. LDS -> global.  The dequant output takes 8 consecutive f16 of one
    // row per lane (16-byte stores); the other outputs 4 elements per lane.
    if constexpr (EPI == kEpiDequant) {
      constexpr int kRuns8 = 32 * TN / 8, kRunsPerRow8 = TN / 8;
      static_assert(kRuns8 % 64 == 0, "8-element runs must fill the wave");
#pragma unroll
      for (int it = 0; it < kRuns8 / 64; ++it) {
        const int run = it * 64 + lane;
        const int row = run / kRunsPerRow8, col = (run % kRunsPerRow8) * 8;
        const v4f32 w0 = *reinterpret_cast<const v4f32*>(stg + row * kPad + col);
        const v4f32 w1 = *reinterpret_cast<const v4f32*>(stg + row * kPad + col + 4);
        const int m = mw + i * 32 + row, n = nw + col;
        if (m >= g.M || n >= g.N) continue;
        // fp32, left to right, each product rounded to fp32, then one
        // rounding to f16.  The empty asm pins the fp32 product in a
        // register so the backend cannot fuse the last multiply and the
        // conversion into a single-rounding v_fma_mixlo_f16.
        const float rs = ssc[wm * TM + i * 32 + row];
        const float* csp = ssc + QR * 64 + wn * TN + col;
        const v4f32 c0 = *reinterpret_cast<const v4f32*>(csp);
        const v4f32 c1 = *reinterpret_cast<const v4f32*>(csp + 4);
        v8f16 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float we = e < 4 ? w0[e] : w1[e - 4];
          const float ce = e < 4 ? c0[e] : c1[e - 4];
          float p = (static_cast<float>(__builtin_bit_cast(int32_t, we)) * rs) * ce;
          asm volatile("" : "+v"(p));
          h[e] = static_cast<_Float16>(p);
        }
        _Float16* c = static_cast<_Float16*>(g.C) + static_cast<int64_t>(m) * g.ldc + n;
        if (g.vec8_store && n + 8 <= g.N) {
          __builtin_nontemporal_store(h, reinterpret_cast<v8f16*>(c));  // C is not re-read here
        } else {
          for (int e = 0; e < 8 && n + e < g.N; ++e) c[e] = h[e];
        }
      }
      continue;
    }
    if constexpr (EPI == kEpiW8 || EPI == kEpiW8Res) {
      // f16(acc * cs[n]) (+ r[m, n] in fp32 for kEpiW8Res): the fp32
      // product, the fp32 sum, then one rounding to f16.
      constexpr int kRuns8 = 32 * TN / 8, kRunsPerRow8 = TN / 8;
#pragma unroll
      for (int it = 0; it < kRuns8 / 64; ++it) {
        const int run = it * 64 + lane;
        const int row = run / kRunsPerRow8, col = (run % kRunsPerRow8) * 8;
        const v4f32 w0 = *reinterpret_cast<const v4f32*>(stg + row * kPad + col);
        const v4f32 w1 = *reinterpret_cast<const v4f32*>(stg + row * kPad + col + 4);
        const int m = mw + i * 32 + row, n = nw + col;
        if (m >= g.M || n >= g.N) continue;
        const float* csp = ssc + QR * 64 + wn * TN + col;
        const v4f32 c0 = *reinterpret_cast<const v4f32*>(csp);
        const v4f32 c1 = *reinterpret_cast<const v4f32*>(csp + 4);
        v8f16 rv = {};
        if constexpr (EPI == kEpiW8Res) {
          const _Float16* r = g.residual + static_cast<int64_t>(m) * g.ldr + n;
          if (g.res_vec8 && n + 8 <= g.N)
            rv = *reinterpret_cast<const v8f16*>(r);
          else
            for (int e = 0; e < 8 && n + e < g.N; ++e) rv[e] = r[e];
        }
        v8f16 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float p = (e < 4 ? w0[e] : w1[e - 4]) * (e < 4 ? c0[e] : c1[e - 4]);
          asm volatile("" : "+v"(p));
          if constexpr (EPI == kEpiW8Res) {
            p = p + static_cast<float>(rv[e]);
            asm volatile("" : "+v"(p));
          }
          h[e] = static_cast<_Float16>(p);
        }
        _Float16* c = static_cast<_Float16*>(g.C) + static_cast<int64_t>(m) * g.ldc + n;
        if (g.vec8_store && n + 8 <= g.N) {
          store_out8<EPI>(h, c);
        } else {
          for (int e = 0; e < 8 && n + e < g.N; ++e) c[e] = h[e];
        }
      }
      continue;
    }
    if constexpr (EPI == kEpiSwiglu) {
      // The wave's 128 image rows are 64 gate channels then the same 64 up
      // channels: output column o = (n0 + wn*128)/2 + col takes the gate
      // value from staged column col and the up value from column 64 + col.
      // h = f16(silu(g) * u) with g = acc_g * sg, u = acc_u * su in fp32 and
      // silu(g) = g / (1 + exp(-g)).
      constexpr int kRunsS = 32 * 64 / 8, kRunsPerRowS = 64 / 8;
#pragma unroll
      for (int it = 0; it < kRunsS / 64; ++it) {
        const int run = it * 64 + lane;
        const int row = run / kRunsPerRowS, col = (run % kRunsPerRowS) * 8;
        const float* sp = stg + row * kPad + col;
        const v4f32 g0 = *reinterpret_cast<const v4f32*>(sp);
        const v4f32 g1 = *reinterpret_cast<const v4f32*>(sp + 4);
        const v4f32 u0 = *reinterpret_cast<const v4f32*>(sp + 64);
        const v4f32 u1 = *reinterpret_cast<const v4f32*>(sp + 68);
        const int m = mw + i * 32 + row, o = nw / 2 + col;
        if (m >= g.M || o >= g.n_out) continue;
        const float* csp = ssc + QR * 64 + wn * TN + col;
        const v4f32 sg0 = *reinterpret_cast<const v4f32*>(csp);
        const v4f32 sg1 = *reinterpret_cast<const v4f32*>(csp + 4);
        const v4f32 su0 = *reinterpret_cast<const v4f32*>(csp + 64);
        const v4f32 su1 = *reinterpret_cast<const v4f32*>(csp + 68);
        v8f16 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float gv = (e < 4 ? g0[e] : g1[e - 4]) * (e < 4 ? sg0[e] : sg1[e - 4]);
          const float uv = (e < 4 ? u0[e] : u1[e - 4]) * (e < 4 ? su0[e] : su1[e - 4]);
          const float ex = __builtin_amdgcn_exp2f(-gv * 1.4426950408889634f);
          h[e] = static_cast<_Float16>(gv * __builtin_amdgcn_rcpf(1.0f + ex) * uv);
        }
        _Float16* c = static_cast<_Float16*>(g.C) + static_cast<int64_t>(m) * g.ldc + o;
        if (g.vec8_store && o + 8 <= g.n_out) {
          store_out8<EPI>(h, c);
        } else {
          for (int e = 0; e < 8 && o + e < g.n_out; ++e) c[e] = h[e];
        }
      }
      continue;
    }
    constexpr int kRuns = 32 * TN / 4;          // 4-element runs in the block
    constexpr int kRunsPerRow = TN / 4;
    constexpr int kIt4 = kRuns / 64;
    static_assert(64 % kRunsPerRow == 0, "4-element runs must tile the wave");
    // Every run of the block is read from LDS before any is converted.
    v4f32 wv[kIt4];
#pragma unroll
    for (int it = 0; it < kIt4; ++it) {
      const int run = it * 64 + lane;
      wv[it] = *reinterpret_cast<const v4f32*>(stg + (run / kRunsPerRow) * kPad +
                                               (run % kRunsPerRow) * 4);
    }
#pragma unroll
    for (int it = 0; it < kIt4; ++it) {
      const int run = it * 64 + lane;
      const int row = run / kRunsPerRow, col = (run % kRunsPerRow) * 4;
      const v4f32 w = wv[it];
      const int m = mw + i * 32 + row, n = nw + col;
      if (m >= g.M || n >= g.N) continue;
      const int64_t off = static_cast<int64_t>(m) * g.ldc + n;
      const bool full = g.vec_store && n + 4 <= g.N;
      if constexpr (EPI == kEpiI32) {
        int32_t* c = static_cast<int32_t*>(g.C) + off;
        v4u32_t r = __builtin_bit_cast(v4u32_t, w);
        if (full) {
          if (g.accumulate) {
            r += *reinterpret_cast<const v4u32_t*>(c);
            *reinterpret_cast<v4u32_t*>(c) = r;
          } else {
            __builtin_nontemporal_store(r, reinterpret_cast<v4u32_t*>(c));
          }
        } else {
          for (int e = 0; e < 4 && n + e < g.N; ++e)
            c[e] = static_cast<int32_t>(g.accumulate ? static_cast<uint32_t>(c[e]) + r[e] : r[e]);
        }
      } else {
        v4f32 r = w;
        if (g.out_dtype == HXM_F32) {
          float* c = static_cast<float*>(g.C) + off;
          if (full) {
            if (g.accumulate) r += *reinterpret_cast<const v4f32*>(c);
            *reinterpret_cast<v4f32*>(c) = r;
          } else {
            for (int e = 0; e < 4 && n + e < g.N; ++e) c[e] = g.accumulate ? c[e] + r[e] : r[e];
          }
        } else if (g.out_dtype == HXM_F16) {
          _Float16* c = static_cast<_Float16*>(g.C) + off;
          if (full) {
            if (g.accumulate) {
              const v4f16_t o = *reinterpret_cast<const v4f16_t*>(c);
              for (int e = 0; e < 4; ++e) r[e] += static_cast<float>(o[e]);
            }
            v4f16_t h;
            for (int e = 0; e < 4; ++e) h[e] = static_cast<_Float16>(r[e]);
            *reinterpret_cast<v4f16_t*>(c) = h;
          } else {
            for (int e = 0; e < 4 && n + e < g.N; ++e)
              c[e] = static_cast<_Float16>(g.accumulate ? r[e] + static_cast<float>(c[e]) : r[e]);
          }
        } else {
          __bf16* c = static_cast<__bf16*>(g.C) + off;
          if (full) {
            if (g.accumulate) {
              const v4bf16_t o = *reinterpret_cast<const v4bf16_t*>(c);
              for (int e = 0; e < 4; ++e) r[e] += static_cast<float>(o[e]);
            }
            v4bf16_t h;
            for (int e = 0; e < 4; ++e) h[e] = static_cast<__bf16>(r[e]);
            *reinterpret_cast<v4bf16_t*>(c) = h;
          } else {
            for (int e = 0; e < 4 && n + e < g.N; ++e)
              c[e] = static_cast<__bf16>(g.accumulate ? r[e] + static_cast<float>(c[e]) : r[e]);
          }
        }
      }
    }
  }
  } while (SK && it < it_end);
}

typedef void (*gemm_fn)(GemmArgs);

// The compiled kernels.  Each kernel source (gemm_i8.hip, gemm_f16.hip,
// gemm_w8.hip) is compiled kGemmParts times with HXM_PART = 0 .. kGemmParts-1
// so the objects build in parallel: part p instantiates the configurations
// whose list index is p mod kGemmParts and leaves null entries for the rest.
// Row i of kI8Fns_p* / kF16Fns_p* is entry i of HXM_GEMM_CONFIG_LIST; row i
// of kW8Fns_p* is entry i of HXM_W8_CONFIG_LIST.  The host side takes the
// non-null entry (gemm.hip).
constexpr int kGemmParts = 3;

struct ConfigKey {
  int bm, bn, bkb, st, wm, wn;
};
#define HXM_CONFIG_KEY(BM, BN, BKB, ST, WM, WN) ConfigKey{BM, BN, BKB, ST, WM, WN}
constexpr ConfigKey kGemmKeys[] = {HXM_GEMM_CONFIG_LIST(HXM_CONFIG_KEY)};
constexpr ConfigKey kW8Keys[] = {HXM_W8_CONFIG_LIST(HXM_CONFIG_KEY)};

// Position of configuration (BM, BN, BKB, ST, WM, WN) in `keys`.
template <int N>
constexpr int config_index(const ConfigKey (&keys)[N], int bm, int bn, int bkb, int st, int wm,
                           int wn) {
  for (int i = 0; i < N; ++i)
    if (keys[i].bm == bm && keys[i].bn == bn && keys[i].bkb == bkb && keys[i].st == st &&
        keys[i].wm == wm && keys[i].wn == wn)
      return i;
  return -1;
}

#define HXM_DECLARE_PART_TABLES(P)            \
  extern const gemm_fn kI8Fns_p##P[][2];  /* {kEpiI32, kEpiDequant} */ \
  extern const gemm_fn kF16Fns_p##P[][2]; /* {f16, bf16} operands, kEpiFloat */ \
  extern const gemm_fn kW8Fns_p##P[][3];  /* {kEpiW8, kEpiSwiglu (null unless TN == 128), kEpiW8Res} */ \
  extern const gemm_fn kW8SkFns_p##P[3];  /* stream-K form of entry 0: part p holds epilogue p */
HXM_DECLARE_PART_TABLES(0)
HXM_DECLARE_PART_TABLES(1)
HXM_DECLARE_PART_TABLES(2)
static_assert(kGemmParts == 3, "one HXM_DECLARE_PART_TABLES line per part");

}  // namespace hxm
