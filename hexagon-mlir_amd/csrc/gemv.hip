// W8A16 weight-resident skinny GEMM / GEMV on gfx950 (M <= 16 per pass).
//
// Reference semantics: an int8-weight linalg.matmul, which the reference's
// engine refuses (qcom_hexagon_backend/include/hexagon/Dialect/Hmx/Transforms/
// HmxTarget.h:198-211: unsupported-dtype, and min-rows for M <= 4) and lowers
// on the HVX generic path (lib/Conversion/LinalgToLLVM/
// ScheduleMatmulForHVXPass.cpp:44-80); weight residency as in
// lib/Dialect/Hmx/Transforms/WeightResidentPass.cpp:10-53.
//   y[m,n] = f16( (sum_k f32(x[m,k]) * f32(W[n,k])) * f32(scale[n]) )
//
// GPU form.  The weight stream dominates (N*K bytes vs M*K*2 for x), so the
// kernel is built to read W exactly once with 128-bit loads:
//   * a workgroup owns 16 output channels; its KW waves split K;
//   * per 64-wide K slab, lane l loads 16 bytes of W row n0 + l%16 at K offset
//     16*(l/16): one wave instruction covers 16 rows x 64 bytes;
//   * the 16 int8 become 16 exact f16 (byte permute with an 0x64 exponent,
//     then a packed f16 subtract of 1152) and feed two
//     v_mfma_f32_16x16x32_f16 with W as the A operand (rows = channels) and x
//     as the B operand (columns = the M <= 16 activation rows, zero past M);
//     the K order inside an instruction is the same permutation for both
//     operands, so the sum is the plain dot product;
//   * the KW partial 16x16 tiles meet in LDS; wave 0 applies the per-channel
//     scale and writes f16;
//   * at M = 1 and with three channel groups per workgroup, the groups go to
//     workgroups XCD-contiguously (gemv_block), so each XCD streams one
//     contiguous eighth of the weight image.
#include "device_util.h"
#include "hxm_internal.h"

namespace hxm {

struct GemvArgs {
  const _Float16* x;
  int64_t ldx;
  const int8_t* W;
  int64_t ldw;
  const _Float16* scale;
  _Float16* y;
  int64_t ldy;
  int M, N, K;
};


// Largest slab count (K / 64) of a packed image the GEMV accepts: every
// buffer offset of the pipelined kernel, (slabs + 15) * 1024 + 1008, stays
// below 2^31.
constexpr int64_t kMaxPackedSlabs = (int64_t(1) << 21) - 32;

// Three channel groups per workgroup at M > 4 from this many 16-channel
// groups up.  Measured at M=16, K=4096 (packed image, one box), one group
// against three per workgroup: N=1376 6.19 / 8.44 us, 2752 6.34 / 8.59,
// 4096 6.60 / 8.75, 5504 8.99 / 8.91, 11008 13.0 / 10.0.
constexpr int64_t kGemvCb3MinGroups = 320;

// The pipelined kernel at 1 < M <= 4 from this many 16-channel groups up;
// below it, with about one workgroup per CU or fewer, the one-chunk kernel's
// single round trip wins.  Measured at M=4, K=4096 (packed image, HIP graph
// of 480 launches, one box), one-chunk against pipelined: N=1376 4.50 /
// 5.78 us, 4096 5.61 / 6.18, 11008 10.39 / 9.46.
constexpr int64_t kGemvPipeMinGroups = 320;

// Bytes of the packed (resident) weight image for [N, K]: one 1 KiB block
// per (16-channel group, 64-wide K slab), zero-padded at the edges.
inline int64_t packed_bytes(int64_t N, int64_t K) {
  return ((N + 15) / 16) * ((K + 63) / 64) * 1024;
}

// Packs W [N, K] (ldw) into the image: block (g, s), lane l holds the 16
// bytes W[16g + l%16][64s + 16*(l/16) ... +16] at byte 16*l of the block, the
// exact order in which one wave instruction of the GEMV consumes them.
__global__ __launch_bounds__(256) void pack_w8a16_kernel(const int8_t* __restrict__ W,
                                                         int64_t ldw, int N, int K,
                                                         int8_t* __restrict__ out,
                                                         int64_t nblocks) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;  // one lane-chunk
  const int64_t blk = t >> 6;
  if (blk >= nblocks) return;
  const int lane = static_cast<int>(t & 63);
  const int slabs = (K + 63) / 64;
  const int64_t g = blk / slabs;
  const int s = static_cast<int>(blk % slabs);
  const int64_t n = g * 16 + (lane & 15);
  const int k = s * 64 + (lane >> 4) * 16;
  v4i32 v = {0, 0, 0, 0};
  if (n < N && k < K) v = *reinterpret_cast<const v4i32*>(W + n * ldw + k);
  v ^= static_cast<int>(0x80808080u);
  *reinterpret_cast<v4i32*>(out + blk * 1024 + lane * 16) = v;
}

// The channel-group block a workgroup takes.  XCD_MAP: workgroups are
// dispatched round-robin over the 8 XCDs, so ordinal b runs on XCD b % 8;
// block x * (G / 8) + min(x, G % 8) + b / 8 (x = b % 8, G = gridDim.x, a
// bijection for any G) gives each XCD one contiguous run of blocks, so the
// XCD's resident workgroups read one contiguous eighth of the weight image.
// A 45 MB read in 64 KiB pieces (one 16-channel group of K = 4096) took
// 8.61 us with piece b on ordinal b (each XCD's pieces 512 KiB apart) and
// 7.86 us with this order (one box, six passes).  The GEMV at N=11008,
// K=4096 (three alternating passes, one box): M=1 8.95-9.05 against
// 9.20-9.30 us in a stream, 8.84-8.97 against 8.99-9.05 us in a HIP graph;
// M=16 (three groups per workgroup) 10.09-10.10 against 10.12-10.18 us;
// M=4 (the pipelined kernel, one group) 9.75-9.78 against 9.63-9.68 us,
// so that kernel keeps the plain order.
template <bool XCD_MAP>
__device__ __forceinline__ int gemv_block() {
  const int b = blockIdx.x;
  if constexpr (!XCD_MAP) return b;
  const int G = gridDim.x, x = b & 7;
  return x * (G >> 3) + min(x, G & 7) + (b >> 3);
}

// Wave 0, after every wave has written its partial 16x16 tiles to part:
// the sum over the KW waves, the per-channel scale, one rounding to f16, the
// store.  Lane l holds D[channel 4*(l/16) + v][m = l%16] of each group.
template <int KW, int CB>
__device__ __forceinline__ void gemv_finish(const GemvArgs& g, const v4f32 (*part)[CB][64],
                                            const float (&sc)[CB][4], int n0, int m_base,
                                            int lane) {
  const int mo = m_base + (lane & 15);
  if (mo >= g.M) return;
#pragma unroll
  for (int b = 0; b < CB; ++b) {
    v4f32 tot = part[0][b][lane];
#pragma unroll
    for (int w = 1; w < KW; ++w) tot += part[w][b][lane];
    // The lane's 4 consecutive channels: the fp32 product, then one
    // rounding to f16 (the pin keeps the backend from fusing the multiply
    // and the conversion into a single-rounding v_fma_mixlo_f16).  One
    // 8-byte store where the run lies inside y and is aligned: measured
    // (N=11008, K=4096, one box) M=1 9.51 -> 9.31 us, M=16 11.75 -> 11.40 us
    // against four 2-byte stores.
    const int no0 = n0 + 16 * b + 4 * (lane >> 4);
    v4f16_t hv;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float p = tot[v] * sc[b][v];
      asm volatile("" : "+v"(p));
      hv[v] = static_cast<_Float16>(p);
    }
    _Float16* yp = g.y + static_cast<int64_t>(mo) * g.ldy + no0;
    if (no0 + 4 <= g.N && (reinterpret_cast<uintptr_t>(yp) & 7) == 0) {
      *reinterpret_cast<v4f16_t*>(yp) = hv;
    } else {
#pragma unroll
      for (int v = 0; v < 4; ++v)
        if (no0 + v < g.N) yp[v] = hv[v];
    }
  }
}

// K == 0: every dot product is the empty sum, so y[m, n] = f16(0.0f *
// scale[n]) (+0, -0 for a negative scale, NaN for an infinite or NaN one),
// the same product the GEMV kernels round.  A kernel of its own keeps the
// K loop's structure out of this case: the M <= 4 kernels load the scales
// inside their first K chunk, which K == 0 does not have.
__global__ __launch_bounds__(256) void gemv_empty_k_kernel(GemvArgs g) {
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (t >= static_cast<int64_t>(g.M) * g.N) return;
  const int m = static_cast<int>(t / g.N), n = static_cast<int>(t % g.N);
  float p = 0.0f * static_cast<float>(g.scale[n]);
  asm volatile("" : "+v"(p));
  g.y[static_cast<int64_t>(m) * g.ldy + n] = static_cast<_Float16>(p);
}

// One workgroup = CB groups of 16 output channels x all of K; its KW waves
// split each K chunk of KW*SPW slabs, wave w taking slabs w, w + KW, ... (so
// each round of loads covers KW consecutive slabs, and every wave sums its
// slabs in the order the pipelined kernel's wave does: the two kernels
// agree bit for bit; measured at M=1, N=11008, K=4096, one box, three
// alternating passes: 9.21-9.23 against 9.32-9.38 us for contiguous runs of
// SPW slabs per wave, equal in a HIP graph), and every wave applies the
// same x fragment to the CB channel groups (more
// channels per workgroup divide the x staging over more weight bytes).  Per
// chunk the wave first loads its share of the x rows, then issues every
// weight load of the chunk (SPW x CB x 16 bytes per lane), all
// unconditionally (addresses are clamped, so the compiler's waits stay
// exact).  The x rows go to LDS (row stride padded by 16 bytes so the 16 rows
// a ds_read_b128 touches land on distinct banks) behind a barrier that does
// not wait for the weight loads, and the MFMAs then consume each slab as its
// load lands.  PACKED reads the resident image (1 KiB contiguous per wave
// instruction); otherwise W is the plain [N, K] matrix (16 rows x 64 bytes
// per instruction).
template <int KW, int SPW, bool PACKED, int MR, int CB, bool LATE_SCALES, bool XCD_MAP>
__global__ __launch_bounds__(KW * 64) void gemv_w8a16_kernel(GemvArgs g) {
  constexpr int kChunkSlabs = KW * SPW;
  constexpr int kChunkK = kChunkSlabs * 64;
  constexpr int kRowBytes = kChunkK * 2 + 16;   // padded x row in LDS
  constexpr int kXVecs = MR * kChunkK / 8;      // 16-byte x vectors per chunk
  constexpr int kXPerThread = (kXVecs + KW * 64 - 1) / (KW * 64);
  __shared__ __attribute__((aligned(16))) uint8_t xs[MR * kRowBytes];  // MR >= rows
  __shared__ v4f32 part[KW][CB][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int blk = gemv_block<XCD_MAP>();
  const int n0 = blk * 16 * CB;
  const int m_base = blockIdx.y * 16;
  const int rows = min(MR, g.M - m_base);       // x rows of this M tile (host: <= MR)
  const int r16 = lane & 15;                    // W row (channel) for A; x row for B
  const int kq = lane >> 4;                     // 16-byte quarter of the 64-wide slab
  const int slabs = (g.K + 63) / 64;
  // The per-channel scales wave 0 applies at the end.  No dependent memory
  // round trip may sit in the kernel's tail, so they are loaded early, in one
  // of two places.  LATE_SCALES (M <= 4): right after wave 0's weight loads
  // of the first K chunk; loads complete in order, so by the time wave 0 has
  // its weights the scales are there too, and nothing waits for them before
  // the weight stream starts.  Otherwise: before the weight stream, converted
  // at once (wave 0 waits one small round trip before issuing its weight
  // loads).  Measured at N=11008, K=4096 (one box, 5 runs each): M=1 9.38 us
  // late against 9.67 early, M=4 9.93 against 10.08, M=16 11.83 against
  // 11.55; a load in the tail was slower still (M=4: 11.2 us).
  float sc[CB][4];
  _Float16 sc_raw[CB][4];
  if (!LATE_SCALES && wave == 0) {
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int no = n0 + 16 * b + 4 * kq + v;
        sc[b][v] = static_cast<float>(g.scale[no < g.N ? no : g.N - 1]);
      }
  }
  const int8_t* wsrc[CB];                       // per channel group
#pragma unroll
  for (int b = 0; b < CB; ++b) {
    if constexpr (PACKED) {
      const int grp = min(blk * CB + b, (g.N + 15) / 16 - 1);
      wsrc[b] = g.W + static_cast<int64_t>(grp) * slabs * 1024 + lane * 16;
    } else {
      const int n = n0 + 16 * b + r16;
      wsrc[b] = g.W + static_cast<int64_t>(n < g.N ? n : 0) * g.ldw;
    }
  }
  const v4i32 zero = {0, 0, 0, 0};

  v4f32 acc[CB];
#pragma unroll
  for (int b = 0; b < CB; ++b) acc[b] = v4f32{0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < slabs; c0 += kChunkSlabs) {
    const int kc0 = c0 * 64;
    // x[m_base .. m_base+rows, kc0 .. kc0+kChunkK), zero past K / rows.
    v4i32 xv[kXPerThread];
#pragma unroll
    for (int q = 0; q < kXPerThread; ++q) {
      const int idx = threadIdx.x + q * KW * 64;
      const int r = idx / (kChunkK / 8), k8 = (idx % (kChunkK / 8)) * 8;
      const bool ok = idx < kXVecs && r < rows && kc0 + k8 < g.K;
      const v4i32 v = *reinterpret_cast<const v4i32*>(
          g.x + (ok ? static_cast<int64_t>(m_base + r) * g.ldx + kc0 + k8 : 0));
      xv[q] = ok ? v : zero;
    }
    v4i32 w[SPW][CB];
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
      const int s = c0 + u * KW + wave;
      // Weights are streamed exactly once: nontemporal loads keep them from
      // displacing x and other reusable lines in the caches.  Out-of-range
      // slabs, K chunks and channel groups load a valid in-range address
      // instead and need no mask: their x is zero (staged below), and
      // channels past N are never stored.  Keeping the loaded data unmasked
      // lets each MFMA wait for its own loads only.
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        if constexpr (PACKED) {
          w[u][b] = __builtin_nontemporal_load(reinterpret_cast<const v4i32*>(
              wsrc[b] + static_cast<int64_t>(s < slabs ? s : 0) * 1024));
        } else {
          const int k = s * 64 + kq * 16;
          w[u][b] = __builtin_nontemporal_load(
              reinterpret_cast<const v4i32*>(wsrc[b] + (k < g.K ? k : 0)));
        }
      }
    }
    if (LATE_SCALES && c0 == 0 && wave == 0) {
#pragma unroll
      for (int b = 0; b < CB; ++b)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int no = n0 + 16 * b + 4 * kq + v;
          sc_raw[b][v] = g.scale[no < g.N ? no : g.N - 1];
        }
    }
    // The previous chunk's LDS reads are done; then x goes to LDS.  These
    // barriers wait for LDS operations only, never for the weight loads.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int q = 0; q < kXPerThread; ++q) {
      const int idx = threadIdx.x + q * KW * 64;
      if (idx < kXVecs) {
        const int r = idx / (kChunkK / 8), k8 = (idx % (kChunkK / 8)) * 8;
        *reinterpret_cast<v4i32*>(xs + r * kRowBytes + k8 * 2) = xv[q];
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int u = 0; u < SPW; ++u) {
      const int kl = (u * KW + wave) * 64 + kq * 16;   // K offset inside the chunk
      const uint8_t* px = xs + (r16 < MR ? r16 : 0) * kRowBytes + kl * 2;
      v4i32 xa = *reinterpret_cast<const v4i32*>(px);
      v4i32 xb = *reinterpret_cast<const v4i32*>(px + 16);
      if (r16 >= rows) xa = xb = zero;
#pragma unroll
      for (int b = 0; b < CB; ++b) {
        const v8f16 wa = i8x8_to_f16<PACKED>(static_cast<uint32_t>(w[u][b][0]),
                                     static_cast<uint32_t>(w[u][b][1]));
        const v8f16 wb = i8x8_to_f16<PACKED>(static_cast<uint32_t>(w[u][b][2]),
                                     static_cast<uint32_t>(w[u][b][3]));
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, __builtin_bit_cast(v8f16, xa),
                                                        acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, __builtin_bit_cast(v8f16, xb),
                                                        acc[b], 0, 0, 0);
      }
    }
  }

#pragma unroll
  for (int b = 0; b < CB; ++b) part[wave][b][lane] = acc[b];
  __syncthreads();
  if (wave != 0) return;
  if (LATE_SCALES) {
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) sc[b][v] = static_cast<float>(sc_raw[b][v]);
  }
  gemv_finish<KW, CB>(g, part, sc, n0, m_base, lane);
}

// Pipelined form for the packed image at M > 1.  A K chunk is KW slabs,
// one per wave, and the next chunk's x and weight loads are issued before
// this chunk's x staging and MFMAs, so every wave keeps two chunks of loads
// in flight and the weight stream does not pause at chunk boundaries.  The
// weight loads are buffer loads whose range is the channel group's image
// (num_records = slabs * 1 KiB): a slab past K lies past the range and
// returns zeros without a memory access, so every load is unconditional and
// the waits the compiler places stay exact (a load under a branch makes the
// merged wait count conservative, down to waiting for the prefetch itself).
// Measured at N=11008, K=4096 (one box, 5 runs of 240 launches each): M=4
// 9.6 us against 9.85 us for the one-chunk kernel, M=16 10.1 against
// 11.4 us.  Two or four slabs per wave per chunk, all of K in one chunk, 2
// or 4 channel groups per workgroup, 4 or 16 waves per workgroup: each
// slower (10.5 to 14.6 us at M=16).
template <int KW, int MR, int CB, bool LATE_SCALES, bool XCD_MAP>
__global__ __launch_bounds__(KW * 64) void gemv_w8a16_pipe_kernel(GemvArgs g) {
  constexpr int kChunkK = KW * 64;
  constexpr int kRowBytes = kChunkK * 2 + 16;   // padded x row in LDS
  constexpr int kXVecs = MR * kChunkK / 8;      // 16-byte x vectors per chunk
  constexpr int kXPerThread = (kXVecs + KW * 64 - 1) / (KW * 64);
  __shared__ __attribute__((aligned(16))) uint8_t xs[MR * kRowBytes];
  __shared__ v4f32 part[KW][CB][64];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int blk = gemv_block<XCD_MAP>();
  const int n0 = blk * 16 * CB;
  const int m_base = blockIdx.y * 16;
  const int rows = min(MR, g.M - m_base);
  const int r16 = lane & 15;
  const int kq = lane >> 4;
  const int slabs = (g.K + 63) / 64;
  const int groups = (g.N + 15) / 16;
  float sc[CB][4];
  _Float16 sc_raw[CB][4];
  auto scale_of = [&](int b, int v) {
    const int no = n0 + 16 * b + 4 * kq + v;
    return g.scale[no < g.N ? no : g.N - 1];
  };
  if (!LATE_SCALES && wave == 0) {
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) sc[b][v] = static_cast<float>(scale_of(b, v));
  }
  __amdgpu_buffer_rsrc_t wr[CB];
#pragma unroll
  for (int b = 0; b < CB; ++b) {
    const int grp = min(blk * CB + b, groups - 1);
    wr[b] = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t*>(g.W) + static_cast<int64_t>(grp) * slabs * 1024,
        static_cast<short>(0), slabs * 1024, 0x00020000);
  }
  const v4i32 zero = {0, 0, 0, 0};
  v4f32 acc[CB];
#pragma unroll
  for (int b = 0; b < CB; ++b) acc[b] = v4f32{0.0f, 0.0f, 0.0f, 0.0f};

  // x[m_base .. m_base+rows, chunk c's K range), zero past K and rows (the
  // address is clamped to x itself, an L2 hit).
  auto load_x = [&](int c, v4i32 (&xv)[kXPerThread]) {
    const int kc0 = c * 64;
#pragma unroll
    for (int q = 0; q < kXPerThread; ++q) {
      const int idx = threadIdx.x + q * KW * 64;
      const int r = idx / (kChunkK / 8), k8 = (idx % (kChunkK / 8)) * 8;
      const bool ok = idx < kXVecs && r < rows && kc0 + k8 < g.K;
      const v4i32 v = *reinterpret_cast<const v4i32*>(
          g.x + (ok ? static_cast<int64_t>(m_base + r) * g.ldx + kc0 + k8 : 0));
      xv[q] = ok ? v : zero;
    }
  };
  // This wave's slab of chunk c, every channel group; nontemporal (aux bit 1):
  // the weights are streamed once.
  auto load_w = [&](int c, v4i32 (&w)[CB]) {
    const int s = c + wave;
#pragma unroll
    for (int b = 0; b < CB; ++b)
      w[b] = __builtin_bit_cast(
          v4i32, __builtin_amdgcn_raw_buffer_load_b128(wr[b], lane * 16 + s * 1024, 0, 2));
  };
  auto consume = [&](const v4i32 (&xv)[kXPerThread], const v4i32 (&w)[CB]) {
    // The previous chunk's LDS reads are done; then x goes to LDS.  These
    // barriers wait for LDS operations only, never for the weight loads.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int q = 0; q < kXPerThread; ++q) {
      const int idx = threadIdx.x + q * KW * 64;
      if (idx < kXVecs) {
        const int r = idx / (kChunkK / 8), k8 = (idx % (kChunkK / 8)) * 8;
        *reinterpret_cast<v4i32*>(xs + r * kRowBytes + k8 * 2) = xv[q];
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const uint8_t* px = xs + (r16 < MR ? r16 : 0) * kRowBytes + (wave * 64 + kq * 16) * 2;
    v4i32 xa = *reinterpret_cast<const v4i32*>(px);
    v4i32 xb = *reinterpret_cast<const v4i32*>(px + 16);
    if (r16 >= rows) xa = xb = zero;
#pragma unroll
    for (int b = 0; b < CB; ++b) {
      const v8f16 wa = i8x8_to_f16<true>(static_cast<uint32_t>(w[b][0]), static_cast<uint32_t>(w[b][1]));
      const v8f16 wb = i8x8_to_f16<true>(static_cast<uint32_t>(w[b][2]), static_cast<uint32_t>(w[b][3]));
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wa, __builtin_bit_cast(v8f16, xa), acc[b],
                                                      0, 0, 0);
      acc[b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(wb, __builtin_bit_cast(v8f16, xb), acc[b],
                                                      0, 0, 0);
    }
  };

  v4i32 xv0[kXPerThread], xv1[kXPerThread];
  v4i32 w0[CB], w1[CB];
  load_x(0, xv0);
  load_w(0, w0);
  if (LATE_SCALES && wave == 0) {
    // After the first weight loads: loads complete in order, so the scales
    // are in by the time this wave has its first slab.
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) sc_raw[b][v] = scale_of(b, v);
  }
  // Two chunks per trip, the buffers alternating; the loads past K fetch
  // nothing, so only the second chunk's compute needs a (uniform) test.
  for (int c0 = 0; c0 < slabs; c0 += 2 * KW) {
    const int c1 = c0 + KW;
    load_x(c1, xv1);
    load_w(c1, w1);
    consume(xv0, w0);
    load_x(c1 + KW, xv0);
    load_w(c1 + KW, w0);
    if (c1 < slabs) consume(xv1, w1);
  }

#pragma unroll
  for (int b = 0; b < CB; ++b) part[wave][b][lane] = acc[b];
  __syncthreads();
  if (wave != 0) return;
  if (LATE_SCALES) {
#pragma unroll
    for (int b = 0; b < CB; ++b)
#pragma unroll
      for (int v = 0; v < 4; ++v) sc[b][v] = static_cast<float>(sc_raw[b][v]);
  }
  gemv_finish<KW, CB>(g, part, sc, n0, m_base, lane);
}

}  // namespace hxm

using namespace hxm;

extern "C" {

int64_t hxm_w8a16_packed_bytes(int64_t N, int64_t K) {
  if (N < 0 || K < 0) return -1;
  return packed_bytes(N, K);
}

hxm_status hxm_prepack_w8a16(const int8_t* W, int64_t ldw, int64_t N, int64_t K,
                             int8_t* out, int64_t out_bytes, void* stream) {
  if (N < 0 || K < 0 || ldw < K)
    return fail(HXM_INVALID_ARG, "invalid-argument: prepack_w8a16 extents/ldw");
  if (out_bytes < packed_bytes(N, K))
    return fail(HXM_INVALID_ARG, "invalid-argument: prepack_w8a16 needs %lld output bytes",
                (long long)packed_bytes(N, K));
  if (N > 0 && K > 0 && (!W || !out))
    return fail(HXM_INVALID_ARG, "invalid-argument: prepack_w8a16 null pointer");
  if (K % 16 || ldw % 16 || (K > 0 && (!aligned16(W) || !aligned16(out))))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: prepack_w8a16 needs K and ldw multiples of 16 and 16-byte "
                "aligned buffers");
  if (N > INT32_MAX - 16 || K > INT32_MAX - 64)
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: prepack_w8a16 extent too large");
  hxm_status st = require_device(nullptr);
  if (st != HXM_OK) return st;
  if (N == 0 || K == 0) return ok();
  const int64_t nblocks = packed_bytes(N, K) / 1024;
  const int64_t threads = nblocks * 64;
  if ((st = check_grid("prepack_w8a16", (threads + 255) / 256, 256)) != HXM_OK) return st;
  pack_w8a16_kernel<<<static_cast<unsigned>((threads + 255) / 256), 256, 0, as_stream(stream)>>>(
      W, ldw, static_cast<int>(N), static_cast<int>(K), out, nblocks);
  return check_launch("prepack_w8a16");
}

hxm_status hxm_gemv_w8a16(const void* x, int64_t ldx, const int8_t* W, int64_t ldw,
                          int32_t w_layout, const void* w_scale, void* y, int64_t ldy,
                          int64_t M, int64_t N, int64_t K, void* stream) {
  if (M < 0 || N < 0 || K < 0)
    return fail(HXM_INVALID_ARG, "invalid-argument: gemv_w8a16 negative extent");
  if (w_layout != HXM_W_NK && w_layout != HXM_W_PACKED)
    return fail(HXM_INVALID_ARG, "invalid-argument: gemv_w8a16 w_layout=%d", w_layout);
  if (M > 0 && N > 0 && (!y || !w_scale || (K > 0 && (!x || !W))))
    return fail(HXM_INVALID_ARG, "invalid-argument: gemv_w8a16 null operand");
  if (ldx < K || ldy < N || (w_layout == HXM_W_NK && ldw < K))
    return fail(HXM_INVALID_ARG, "invalid-argument: gemv_w8a16 leading dimension too small");
  if (K % 16 || ldx % 8 || (w_layout == HXM_W_NK && ldw % 16) ||
      (K > 0 && (!aligned16(x) || !aligned16(W))))
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: gemv_w8a16 needs K (and ldw) multiples of 16, ldx of 8, "
                "16-byte aligned x and W (K=%lld)",
                (long long)K);
  if (N > INT32_MAX - 16 || K > INT32_MAX - 64 || M > 65535LL * 16)
    return fail(HXM_UNSUPPORTED_SHAPE, "tile-alignment: gemv_w8a16 extent too large");
  // The pipelined kernel addresses a channel group's image with 32-bit
  // buffer offsets, up to two chunks of 8 slabs past its last slab.
  if (w_layout == HXM_W_PACKED && (K + 63) / 64 > kMaxPackedSlabs)
    return fail(HXM_UNSUPPORTED_SHAPE,
                "tile-alignment: gemv_w8a16 packed image needs K <= %lld (K=%lld)",
                (long long)kMaxPackedSlabs * 64, (long long)K);
  hxm_status st = require_device(nullptr);
  if (st != HXM_OK) return st;
  if (M == 0 || N == 0) return ok();
  GemvArgs g{static_cast<const _Float16*>(x), ldx, W, ldw,
             static_cast<const _Float16*>(w_scale), static_cast<_Float16*>(y), ldy,
             static_cast<int>(M), static_cast<int>(N), static_cast<int>(K)};
  auto grid = [&](int cb) {
    return dim3(static_cast<unsigned>((N + 16 * cb - 1) / (16 * cb)),
                static_cast<unsigned>((M + 15) / 16));
  };
  // x rows staged per workgroup: a single small M tile needs less LDS, which
  // keeps more workgroups resident per CU.
  hipStream_t s = as_stream(stream);
  if (K == 0) {
    const int64_t blocks = (M * N + 255) / 256;
    if ((st = check_grid("gemv_w8a16", blocks, 256)) != HXM_OK) return st;
    gemv_empty_k_kernel<<<static_cast<unsigned>(blocks), 256, 0, s>>>(g);
    return check_launch("gemv_w8a16");
  }
  const bool pk = w_layout == HXM_W_PACKED;
  // Channel groups per workgroup at M > 4: three share each staged x chunk,
  // which pays while a workgroup per 16 channels would more than fill the
  // chip; below that (fewer than kGemvCb3MinGroups groups, a column shard
  // for example) the three-fold grid leaves CUs idle.
  const int cb = M <= 4 || (N + 15) / 16 < kGemvCb3MinGroups ? 1 : 3;
  if ((st = check_grid("gemv_w8a16", (N + 16 * cb - 1) / (16 * cb), 512, (M + 15) / 16)) != HXM_OK)
    return st;
  // M = 1 (and the plain [N, K] layout at every M, and the packed image at
  // M <= 4 below kGemvPipeMinGroups): a 4096-wide K chunk (x rows fit LDS),
  // so at K <= 4096 each wave issues all its weight loads at once and makes
  // one memory round trip.  Otherwise the packed image at M > 1 takes the
  // pipelined kernel, 512-wide chunks with the next chunk in flight.  The
  // last template argument (XCD-contiguous channel groups, gemv_block) is
  // on at M = 1 and with three groups per workgroup, where it measured
  // faster, and off elsewhere.
  if (M <= 1) {
    if (pk) gemv_w8a16_kernel<8, 8, true, 1, 1, true, true><<<grid(1), 512, 0, s>>>(g);
    else gemv_w8a16_kernel<8, 8, false, 1, 1, true, true><<<grid(1), 512, 0, s>>>(g);
  } else if (M <= 4) {
    if (pk && (N + 15) / 16 >= kGemvPipeMinGroups)
      gemv_w8a16_pipe_kernel<8, 4, 1, true, false><<<grid(1), 512, 0, s>>>(g);
    else if (pk)
      gemv_w8a16_kernel<8, 8, true, 4, 1, true, false><<<grid(1), 512, 0, s>>>(g);
    else
      gemv_w8a16_kernel<8, 8, false, 4, 1, true, false><<<grid(1), 512, 0, s>>>(g);
  } else {
    // 16 x rows: three channel groups per workgroup share each staged x
    // chunk (measured with the one-chunk kernel: 13.1 vs 14.7 us at
    // N=11008, K=4096), one group below kGemvCb3MinGroups.
    if (pk && cb == 3) gemv_w8a16_pipe_kernel<8, 16, 3, false, true><<<grid(3), 512, 0, s>>>(g);
    else if (pk) gemv_w8a16_pipe_kernel<8, 16, 1, false, false><<<grid(1), 512, 0, s>>>(g);
    else if (cb == 3) gemv_w8a16_kernel<8, 4, false, 16, 3, false, true><<<grid(3), 512, 0, s>>>(g);
    else gemv_w8a16_kernel<8, 4, false, 16, 1, false, false><<<grid(1), 512, 0, s>>>(g);
  }
  return check_launch("gemv_w8a16");
}

}  // extern "C"
