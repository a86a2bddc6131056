// Dense GEMM on the matrix cores (tensor rows' GEMM mode and the benchmark's
// 8192^3 / 4096^3 / 16384^3 GEMM configurations).
//
// C[M][N] = A[M][K] . B[K][N] with A row-major and B column-major, so both
// operands are K-contiguous in memory ("NT"); the accumulator type is the
// instruction's (fp32, int32 for INT8, fp64 for FP64). MXFP4 operands carry
// one E8M0 scale per 32 K elements in K-step blocks: SA[ceil(K/256)][M][8],
// SB[ceil(K/256)][N][8], where [b][r][g] scales row r over K elements
// 256b + 32g .. 256b + 32g + 31, so the scales of one 256-element K step of a
// tile are one contiguous run of 8 bytes per row.
// Replaces the reference's _gemm_kernel (bench_tensor.py:172-209), whose B is
// row-major; the MI355X kernel takes K-contiguous B (layout prepared outside
// timing by the caller).
//
// Two kernels:
//   * gemm_dma_kernel (BF16, FP16, INT8, FP8 on 16x16 MFMAs) and
//     gemm_staged_kernel (MXFP4): 256x256 tiles when the shape divides the
//     tile. Four waves, one per SIMD, each owning 128x128 outputs in AGPRs:
//     64 accumulators of 16x16 (the 16x16 instructions sustain a higher clock
//     under the power limit) or, for MXFP4, 16 of 32x32. In the staged kernel
//     operands flow global -> VGPR -> LDS -> VGPR -> MFMA: each K step (128
//     bytes of every row) is loaded two steps ahead into one of two register
//     sets, written to one of two LDS stages a step ahead, and read back as
//     fragments ahead of the MFMAs that use them. Loads, stage writes and
//     fragment reads are spread across the step's MFMAs, so no burst of
//     memory instructions stalls the in-order MFMA issue; one barrier per
//     step. The DMA kernel moves A straight into LDS with LDS-DMA loads
//     instead.
//   * gemm_kernel: every other tile and every ragged shape (CHECKED
//     instantiations bound each load and store), operands staged through a
//     padded, double-buffered LDS tile with 16-byte loads.
// Both number workgroups XCD-first: the hardware deals consecutive ids
// round-robin over the 8 XCDs, so id i is remapped to the i/8-th tile of XCD
// i%8's contiguous share, walked in GROUP_M-row bands that keep A and B panels
// hot in that XCD's L2.
#include "mb_internal.h"
#include "mb_mfma.h"

#include <cstring>
#include <type_traits>

namespace mb {
namespace {

constexpr int kXcds = 8;

template <class Op, int BM, int BN, int BK, int WAVES_M, int WAVES_N>
struct GemmTile {
  static constexpr int THREADS = 64 * WAVES_M * WAVES_N;
  static constexpr int BK_BYTES = BK * Op::ELEM_BITS / 8;
  static constexpr int STRIDE = BK_BYTES + 16;  // padded LDS row, keeps 16-byte alignment
  static constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
  static constexpr int TM = WM / Op::M, TN = WN / Op::N;
  static constexpr int KSTEPS = BK_BYTES / MfmaGeometry<Op>::K_BYTES;
  static constexpr int ROW_CHUNKS = BK_BYTES / 16;
  static constexpr int A_CHUNKS = BM * ROW_CHUNKS / THREADS;  // 16-byte loads per thread per step
  static constexpr int B_CHUNKS = BN * ROW_CHUNKS / THREADS;
  static constexpr int BUFFER = (BM + BN) * STRIDE;
  static constexpr int GROUPS = Op::SCALED ? BK / 32 : 0;
  static_assert(BM * ROW_CHUNKS % THREADS == 0 && BN * ROW_CHUNKS % THREADS == 0, "whole loads per thread");
  static_assert(BK_BYTES % MfmaGeometry<Op>::K_BYTES == 0, "BK must hold whole instructions");
  static_assert(WM % Op::M == 0 && WN % Op::N == 0, "wave tile must hold whole instructions");
};

// Stage one K step of A and B into registers (global loads in flight).
template <class T, bool CHECKED>
__device__ __forceinline__ void load_step(i32x4 (&ra)[T::A_CHUNKS], i32x4 (&rb)[T::B_CHUNKS],
                                          const uint8_t* a_tile, const uint8_t* b_tile, uint64_t row_bytes,
                                          int rows_a, int rows_b, int64_t k_bytes_left) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < T::A_CHUNKS; ++i) {
    const int c = i * T::THREADS + t;
    const int row = c / T::ROW_CHUNKS, chunk = c % T::ROW_CHUNKS;
    if (!CHECKED || (row < rows_a && chunk * 16 < k_bytes_left))
      ra[i] = *reinterpret_cast<const i32x4*>(a_tile + row * row_bytes + chunk * 16);
    else
      ra[i] = i32x4{0, 0, 0, 0};
  }
#pragma unroll
  for (int i = 0; i < T::B_CHUNKS; ++i) {
    const int c = i * T::THREADS + t;
    const int row = c / T::ROW_CHUNKS, chunk = c % T::ROW_CHUNKS;
    if (!CHECKED || (row < rows_b && chunk * 16 < k_bytes_left))
      rb[i] = *reinterpret_cast<const i32x4*>(b_tile + row * row_bytes + chunk * 16);
    else
      rb[i] = i32x4{0, 0, 0, 0};
  }
}

template <class T>
__device__ __forceinline__ void store_step(uint8_t* buffer, const i32x4 (&ra)[T::A_CHUNKS],
                                           const i32x4 (&rb)[T::B_CHUNKS], int bm) {
  const int t = threadIdx.x;
#pragma unroll
  for (int i = 0; i < T::A_CHUNKS; ++i) {
    const int c = i * T::THREADS + t;
    *reinterpret_cast<i32x4*>(buffer + (c / T::ROW_CHUNKS) * T::STRIDE + (c % T::ROW_CHUNKS) * 16) = ra[i];
  }
  uint8_t* b_buffer = buffer + bm * T::STRIDE;
#pragma unroll
  for (int i = 0; i < T::B_CHUNKS; ++i) {
    const int c = i * T::THREADS + t;
    *reinterpret_cast<i32x4*>(b_buffer + (c / T::ROW_CHUNKS) * T::STRIDE + (c % T::ROW_CHUNKS) * 16) = rb[i];
  }
}

template <class Op, int BM, int BN, int BK, int WAVES_M, int WAVES_N, bool CHECKED>
__global__ void __launch_bounds__(64 * WAVES_M * WAVES_N)
    gemm_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, const uint8_t* __restrict__ SA,
                const uint8_t* __restrict__ SB, typename Op::Out* __restrict__ C, int M, int N, int K,
                int group_m) {
  using T = GemmTile<Op, BM, BN, BK, WAVES_M, WAVES_N>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[2 * T::BUFFER];

  // XCD-first workgroup numbering, then GROUP_M bands of tiles.
  const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
  const int count = gridDim.x;
  int pid = blockIdx.x;
  if (count % kXcds == 0) pid = (pid % kXcds) * (count / kXcds) + pid / kXcds;
  const int band = group_m * tiles_n;
  const int first_m = (pid / band) * group_m;
  const int rows_in_band = min(tiles_m - first_m, group_m);
  const int tile_m = first_m + (pid % band) % rows_in_band;
  const int tile_n = (pid % band) / rows_in_band;
  const int m0 = tile_m * BM, n0 = tile_n * BN;

  const uint64_t row_bytes = static_cast<uint64_t>(K) * Op::ELEM_BITS / 8;
  const uint8_t* a_tile = A + m0 * row_bytes;
  const uint8_t* b_tile = B + n0 * row_bytes;
  const int rows_a = M - m0, rows_b = N - n0;
  const int k_steps = (K + BK - 1) / BK;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int lrow = lane % Op::M, lgroup = lane / Op::M;
  constexpr int KB = MfmaGeometry<Op>::K_BYTES;
  const int scale_cols = Op::SCALED ? K / 32 : 0;
  // Block layout: group col of row r at ((col / 8) * rows + r) * 8 + col % 8.
  auto scale_at = [](const uint8_t* S, int rows, int r, int col) {
    return static_cast<int>(S[(static_cast<int64_t>(col >> 3) * rows + r) * 8 + (col & 7)]);
  };

  typename Op::Acc acc[T::TM][T::TN];
#pragma unroll
  for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn) acc[tm][tn] = typename Op::Acc{};

  i32x4 ra[T::A_CHUNKS], rb[T::B_CHUNKS];
  load_step<T, CHECKED>(ra, rb, a_tile, b_tile, row_bytes, rows_a, rows_b, static_cast<int64_t>(row_bytes));
  store_step<T>(lds, ra, rb, BM);
  __syncthreads();

  for (int kt = 0; kt < k_steps; ++kt) {
    uint8_t* current = lds + (kt & 1) * T::BUFFER;
    const bool more = kt + 1 < k_steps;
    if (more)
      load_step<T, CHECKED>(ra, rb, a_tile + (kt + 1) * T::BK_BYTES, b_tile + (kt + 1) * T::BK_BYTES, row_bytes,
                            rows_a, rows_b, static_cast<int64_t>(row_bytes) - (kt + 1) * T::BK_BYTES);
    // E8M0 scales of this step: column kt*BK/32 + ks*LANE_GROUPS + group.
    int sa[T::TM][T::KSTEPS], sb[T::TN][T::KSTEPS];
    if constexpr (Op::SCALED) {
#pragma unroll
      for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
        for (int ks = 0; ks < T::KSTEPS; ++ks) {
          const int row = m0 + wm * T::WM + tm * Op::M + lrow;
          const int col = kt * T::GROUPS + ks * MfmaGeometry<Op>::LANE_GROUPS + lgroup;
          sa[tm][ks] = (!CHECKED || (row < M && col < scale_cols)) ? scale_at(SA, M, row, col) : 127;
        }
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
        for (int ks = 0; ks < T::KSTEPS; ++ks) {
          const int col_n = n0 + wn * T::WN + tn * Op::N + lrow;
          const int col = kt * T::GROUPS + ks * MfmaGeometry<Op>::LANE_GROUPS + lgroup;
          sb[tn][ks] = (!CHECKED || (col_n < N && col < scale_cols)) ? scale_at(SB, N, col_n, col) : 127;
        }
    } else {
#pragma unroll
      for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
        for (int ks = 0; ks < T::KSTEPS; ++ks) sa[tm][ks] = 0;
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
        for (int ks = 0; ks < T::KSTEPS; ++ks) sb[tn][ks] = 0;
    }
    const uint8_t* a_lds = current + (wm * T::WM + lrow) * T::STRIDE + lgroup * Op::LANE_BYTES;
    const uint8_t* b_lds = current + (BM + wn * T::WN + lrow) * T::STRIDE + lgroup * Op::LANE_BYTES;
#pragma unroll
    for (int ks = 0; ks < T::KSTEPS; ++ks) {
      typename Op::Frag a[T::TM], b[T::TN];
#pragma unroll
      for (int tm = 0; tm < T::TM; ++tm) a[tm] = load_frag<typename Op::Frag>(a_lds + tm * Op::M * T::STRIDE + ks * KB);
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn) b[tn] = load_frag<typename Op::Frag>(b_lds + tn * Op::N * T::STRIDE + ks * KB);
#pragma unroll
      for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
          acc[tm][tn] = Op::mma(a[tm], b[tn], acc[tm][tn], sa[tm][ks], sb[tn][ks]);
    }
    if (more) store_step<T>(lds + ((kt + 1) & 1) * T::BUFFER, ra, rb, BM);
    __syncthreads();
  }

#pragma unroll
  for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
      for (int r = 0; r < Op::ACC_REGS; ++r) {
        const int row = m0 + wm * T::WM + tm * Op::M + Op::out_row(lane, r);
        const int col = n0 + wn * T::WN + tn * Op::N + (lane % Op::N);
        if (!CHECKED || (row < M && col < N)) C[static_cast<int64_t>(row) * N + col] = acc[tm][tn][r];
      }
}

// ---- shared pieces of the 256x256 kernels ---------------------------------

// One 16-byte-per-lane LDS DMA: lane l's 16 bytes land at lds_addr + 16 * l.
// Issued as inline assembly so the compiler's wait-count pass does not force a
// full vmcnt(0) before every LDS read; the staged kernel issues it ahead of
// compiler-visible loads, whose in-order vmcnt waits then cover it.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, uint32_t lds_addr) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voffset), "s"(rsrc), "s"(soffset),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

// Word 3 of a gfx9 buffer resource: 32-bit data format, no swizzle, raw offsets.
constexpr int kBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const uint8_t* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, bytes, kBufferWord3);
}

// Tile (tile_m, tile_n) of workgroup blockIdx.x: XCD-first numbering, then
// GROUP_M-row bands (see the file comment).
__device__ __forceinline__ void band_tile(int tiles_m, int tiles_n, int group_m, int& tile_m, int& tile_n) {
  const int count = gridDim.x;
  int pid = blockIdx.x;
  if (count % kXcds == 0) pid = (pid % kXcds) * (count / kXcds) + pid / kXcds;
  const int band = group_m * tiles_n;
  const int first_m = (pid / band) * group_m;
  const int rows_in_band = min(tiles_m - first_m, group_m);
  tile_m = first_m + (pid % band) % rows_in_band;
  tile_n = (pid % band) / rows_in_band;
}

// s_waitcnt's immediate for vmcnt(n) alone (n < 64): vmcnt's low four bits
// at 3:0 and high two at 15:14, expcnt (6:4) and lgkmcnt (11:8) at their
// maxima, which wait for nothing.
constexpr int vmcnt_only(int n) { return (n & 15) | ((n >> 4) << 14) | (7 << 4) | (15 << 8); }

// Barrier that orders LDS only: global loads in flight stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// f(integral_constant<I>) for I = I0 .. N-1, so counts derived from I are constants.
template <int I, int N, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// ---- VGPR-staged 256x256 kernel (MXFP4) ------------------------------------

// C = A . B^T for MXFP4 operands with M, N multiples of 256, K a multiple of
// 256 (128-byte K steps) with an even number of at least 4 steps; A, B byte
// offsets and the scale blocks must fit in 31 bits. Four waves in a 2x2 grid
// own 128x128 outputs each.
//
// LDS: regions [A stage 0][A stage 1][B stage 0][B stage 1] of 256 rows x 128
// bytes (every stage and fragment offset is a ds_* immediate), then a ring of
// four 4 KiB scale stages [256 A rows][256 B rows] x 8 bytes. Row r
// of a region holds its 16-byte chunk c at r*128 + ((c ^ ((r >> 1) & 7)) << 4),
// so the 16 rows a ds_read_b128 quarter-wave touches hit 16 bank groups.
//
// Per K step kt (stage s = kt & 1): the MFMAs of substep ks use fragments read
// during substep ks-1 (the first from stage s during step kt-1's last
// substep); register set V[kt & 1 ^ 1] holds step kt+1 (loaded at step kt-2),
// which is written to stage s^1 over substeps 0..KS-2 and reloaded with step
// kt+3 right behind each write; the barrier after substep KS-2 publishes
// stage s^1 and ends every read of stage s^1's previous step. Past the last
// step the loads repeat it and the extra writes and reads go unused, so all
// steps run one branch-free body.
template <class Op>
__global__ void __launch_bounds__(256)
    gemm_staged_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                       const uint8_t* __restrict__ SA, const uint8_t* __restrict__ SB,
                       typename Op::Out* __restrict__ C, int M, int N, int K, int group_m) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 256, ROWB = 128, REGION = 256 * ROWB, NL = 16;
  constexpr int KB = MfmaGeometry<Op>::K_BYTES, KS = ROWB / KB, PIECES = Op::LANE_BYTES / 16;
  constexpr int SCALE_STAGE = 512 * 8, SCALE_RING = 4;
  static_assert(Op::SCALED && Op::M == 32 && PIECES == 1 && KS == 4,
                "scaled 32x32 instructions with 16-byte fragments in four substeps");
  constexpr int TILES = 4;  // 32x32 fragments per wave side
  __shared__ __attribute__((aligned(1024))) uint8_t lds[4 * REGION + SCALE_RING * SCALE_STAGE];
  if (K < 0) lds[threadIdx.x] = 0;  // keeps DMA-written (scale) reads live; never executed

  int tile_m, tile_n;
  band_tile(M / BM, N / BM, group_m, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BM;
  const int row_bytes = K * Op::ELEM_BITS / 8;
  const int k_steps = row_bytes / ROWB, last = k_steps - 1;

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A + static_cast<int64_t>(m0) * row_bytes, BM * row_bytes);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(B + static_cast<int64_t>(n0) * row_bytes, BM * row_bytes);
  // Load j of a step covers rows 32j .. 32j+31 of the A|B stage (j < 8: A);
  // thread t moves row 32j + t/8, chunk t%8.
  const int voff = (t >> 3) * row_bytes + (t & 7) * 16;
  uint8_t* const wa = lds + (t >> 3) * ROWB + (((t & 7) ^ ((t >> 4) & 7)) << 4);
  uint8_t* const wb = wa + 2 * REGION;
  auto load = [&](i32x4 (&v)[NL], int kt, int j0, int j1) __attribute__((always_inline)) {
#pragma unroll
    for (int j = j0; j < j1; ++j)
      v[j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                           j < 8 ? ra : rb, voff, kt * ROWB + (j & 7) * 32 * row_bytes, 0));
  };
  auto store = [&](const i32x4 (&v)[NL], int s, int j0, int j1) __attribute__((always_inline)) {
#pragma unroll
    for (int j = j0; j < j1; ++j)
      *reinterpret_cast<i32x4*>((j < 8 ? wa : wb) + s * REGION + (j & 7) * 32 * ROWB) = v[j];
  };

  // Scales: wave w DMAs 1 KiB of a step's scale stage, rows 128(w&1) .. +127
  // of A (w < 2) or B, from block kt of SA or SB (256 E2M1 elements, one
  // 128-byte step, per block).
  const __amdgpu_buffer_rsrc_t rs = wave < 2 ? buffer_rsrc(SA, k_steps * M * 8) : buffer_rsrc(SB, k_steps * N * 8);
  const int s_rows = wave < 2 ? M : N;
  const int s_row0 = (wave < 2 ? m0 : n0) + (wave & 1) * 128;
  const uint32_t scale_lds = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(
                                 (__attribute__((address_space(3))) uint8_t*)(lds + 4 * REGION))) + wave * 1024;
  // Block `block` into ring slot (slot & 3); past the last step the block is
  // clamped but the slot is not, so a slot still being read is never written.
  auto scale_dma = [&](int slot, int block) __attribute__((always_inline)) {
    dma16(rs, lane * 16, (block * s_rows + s_row0) * 8, scale_lds + (slot & 3) * SCALE_STAGE);
  };

  const int wm = wave & 1, wn = wave >> 1;
  const int lrow = lane & 31, lgroup = lane >> 5;
  // Piece p of a lane's fragment of substep ks is its row's logical chunk
  // ks*KB/16 + lgroup*PIECES + p, i.e. the lane base XOR ((ks*KB/16 + p) << 4):
  // only address bits 4..6 change, so region, stage and fragment offsets still
  // add as immediates.
  const int sw = ((lrow >> 1) & 7) ^ (lgroup * PIECES);
  const uint32_t ra_off = (wm * 128 + lrow) * ROWB + (sw << 4);
  const uint32_t rb_off = 2 * REGION + (wn * 128 + lrow) * ROWB + (sw << 4);
  using Frag8 = i32x4[8];
  auto read = [&](Frag8& fr, int s, int ks) __attribute__((always_inline)) {
    const uint32_t x = static_cast<uint32_t>(ks) << 5;
    const uint8_t* pa = lds + (ra_off ^ x) + s * REGION;
    const uint8_t* pb = lds + (rb_off ^ x) + s * REGION;
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      fr[f] = *reinterpret_cast<const i32x4*>(pa + f * 32 * ROWB);
      fr[4 + f] = *reinterpret_cast<const i32x4*>(pb + f * 32 * ROWB);
    }
  };
  // One dword per fragment row holding the scales of its lane's four
  // 32-element groups of a step (groups lgroup, 2+lgroup, 4+lgroup, 6+lgroup:
  // substep ks uses byte ks), picked out of the row's 8 bytes by v_perm_b32.
  const uint32_t pick = 0x06040200u + 0x01010101u * static_cast<uint32_t>(lgroup);
  using Scales8 = uint32_t[8];
  auto read_scales = [&](Scales8& sc, int kt) __attribute__((always_inline)) {
    const uint8_t* st = lds + 4 * REGION + (kt & 3) * SCALE_STAGE;
#pragma unroll
    for (int f = 0; f < 8; ++f) {
      const int row = f < 4 ? wm * 128 + f * 32 + lrow : 256 + wn * 128 + (f - 4) * 32 + lrow;
      const i32x2 r = *reinterpret_cast<const i32x2*>(st + row * 8);
      sc[f] = __builtin_amdgcn_perm(static_cast<uint32_t>(r[1]), static_cast<uint32_t>(r[0]), pick);
    }
  };

  typename Op::Acc acc[TILES][TILES];
#pragma unroll
  for (int i = 0; i < TILES; ++i)
#pragma unroll
    for (int j = 0; j < TILES; ++j) acc[i][j] = typename Op::Acc{};

  i32x4 v0[NL], v1[NL];
  // Prologue: steps 0 and 1 in flight, step 0 into stage 0, step 2 into v0.
  // The wait for v0 before its stage write also covers the older scale DMAs.
  scale_dma(0, 0);
  scale_dma(1, min(1, last));
  scale_dma(2, min(2, last));
  load(v0, 0, 0, NL);
  load(v1, 1, 0, NL);
  store(v0, 0, 0, NL);
  load(v0, 2, 0, NL);
  lds_barrier();

  {
    // 16-byte fragments: A and B fragments of a substep double-buffered (fa/fb).
    Frag8 fa, fb;
    Scales8 sa0, sa1;
    read(fa, 0, 0);
    read_scales(sa0, 0);
    auto step = [&](int kt, int s, i32x4 (&vnext)[NL], Scales8& sc, Scales8& sc_next) __attribute__((always_inline)) {
      auto substep = [&](auto ks_c) __attribute__((always_inline)) {
        constexpr int ks = decltype(ks_c)::value;
        Frag8& cur = (ks & 1) ? fb : fa;
        Frag8& nxt = (ks & 1) ? fa : fb;
        if constexpr (ks + 1 < KS) {
          read(nxt, s, ks + 1);
        } else {
          read(nxt, s ^ 1, 0);
          read_scales(sc_next, kt + 1);
        }
        // This substep's share of step kt+1's stage writes (all before the
        // barrier) and of step kt+3's loads, each behind the write that frees
        // its registers.
        constexpr int W0 = ks * NL / (KS - 1) < NL ? ks * NL / (KS - 1) : NL;
        constexpr int W1 = (ks + 1) * NL / (KS - 1) < NL ? (ks + 1) * NL / (KS - 1) : NL;
        constexpr int L0 = ks * NL / KS, L1 = (ks + 1) * NL / KS;
        store(vnext, s ^ 1, W0, W1);
        load(vnext, min(kt + 3, last), L0, L1);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = Op::template mma_byte<ks>(cur[i], cur[4 + j], acc[i][j], sc[i], sc[4 + j]);
        // Interleave: after each MFMA, one of the next substep's fragment reads
        // (front-loaded; in the last substep also the next step's scale rows)
        // and this substep's writes and loads, evenly spaced.
        constexpr int WR = W1 - W0, LD = L1 - L0, RD = ks == KS - 1 ? 16 : 8;
#pragma unroll
        for (int q = 0; q < 16; ++q) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);                                    // MFMA
          if (q < RD) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                        // DS read
          if ((q + 1) * WR / 16 != q * WR / 16) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);  // DS write
          if ((q + 1) * LD / 16 != q * LD / 16) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
        }
        // The scale DMA of step kt+3 (an inline-asm scheduling boundary) goes
        // after this substep's work; its data is covered by the in-order waits
        // for step kt+3's loads issued later, which the stage writes of step
        // kt+2 wait for before the barrier that publishes those scales.
        if constexpr (ks == 0) scale_dma(kt + 3, min(kt + 3, last));
        if constexpr (ks == KS - 2) lds_barrier();
        __builtin_amdgcn_sched_barrier(0);
      };
      substep(std::integral_constant<int, 0>{});
      substep(std::integral_constant<int, 1>{});
      substep(std::integral_constant<int, 2>{});
      substep(std::integral_constant<int, 3>{});
    };
    for (int kt = 0; kt < k_steps; kt += 2) {
      step(kt, 0, v1, sa0, sa1);
      step(kt + 1, 1, v0, sa1, sa0);
    }
  }

#pragma unroll
  for (int i = 0; i < TILES; ++i)
#pragma unroll
    for (int j = 0; j < TILES; ++j)
#pragma unroll
      for (int r = 0; r < Op::ACC_REGS; ++r) {
        const int row = m0 + wm * 128 + i * Op::M + Op::out_row(lane, r);
        const int col = n0 + wn * 128 + j * Op::N + lane % Op::N;
        C[static_cast<int64_t>(row) * N + col] = acc[i][j][r];
      }
#endif
}

// ---- 256x256 kernel, A and B by LDS DMA (BF16, FP16, INT8, FP8, FP32 on 16x16)

// The staged kernel's shape rules with both operands moved from global memory
// into LDS by LDS-DMA loads (buffer_load_dwordx4 ... lds) instead of through
// registers and ds_write, for the unscaled 16x16 instructions: 8x8 output
// blocks of 16x16 per wave.
//
// LDS: a ring of three A slots, then a ring of two B slots, each 256 rows x
// 128 bytes (160 KiB in all), with the staged kernel's XOR swizzle. A DMA
// writes 1 KiB per instruction, lane l at +16*l, i.e. 8 rows; lane l therefore
// loads the logical chunk that belongs at its physical position in that row.
// Instruction i of wave w moves rows 64w + 8i .. +7 of its operand's tile, so
// a wave issues 8 DMAs per operand per step.
//
// Fragments: a lane's fragment is 32 bytes of its row's 128-byte step, lane
// group g (lanes 16g .. 16g+15) holding logical chunks g and g + 4. BF16,
// FP16 and INT8 (16-byte operands, 64-byte K slices) take it in two
// instructions, chunks 0..3 and then 4..7, so each block accumulates K in
// chunk order. FP8 (16x16x128) takes it in one: the instruction's K order is
// then a permutation of the step's, the same for A and B. Chunks 2g and 2g+1
// would keep FP8's K order but measured LDS bank conflicts and 1% less. FP32
// (16x16x4) takes it in eight, instruction p taking float p of every lane's
// 32 bytes (again the same K permutation for A and B). One
// set of 8 A and 8 B fragments (128 VGPRs) is all the wave holds: every
// fragment register is refilled in place after its last use.
//
// Per K step kt (A slot kt % 3, B slot s = kt & 1): 64 block updates, and
// one wait and barrier that split them in halves:
//   first half:  blocks (i, 4 + j), i = 0..7, j = 0..3, row by row; reads of
//                B fragments 0..3 of this step (their previous contents were
//                last used at the end of the previous step); A of step kt+2
//                DMAed into slot (kt+2) % 3, whose last reads (step kt-1's)
//                ended before the previous barrier;
//   wait         vmcnt(8): the wave's DMAs in flight are then at most the
//                last eight it issued, step kt+2's A, so step kt+1's A (issued
//                in step kt-1's first half) and B (in its second half) are in
//                LDS;
//   barrier      (publishes step kt+1 from every wave, and ends every read of
//                B slot s);
//   second half: blocks (i, j), i = 0..7, j = 0..3; at its start the reads
//                of B fragments 4..7 of step kt+1, then A fragment i of step
//                kt+1 right after block (i, 3), its last use; B of step kt+2
//                DMAed into slot s.
// Each half issues its eight DMAs one every fourth block update: spread over
// the whole step, they stall the load path less than in bursts (BF16 runs
// 6-7% faster than with all sixteen in the second half). The next step's
// first use of each fragment is at least 28 block updates after its read.
// The compiler does not count the DMAs (they are inline assembly), so the one
// explicit wait is what orders them before their reads.
//
// The MFMAs are issued in their in-place form (Op::mma_tied): the compiler
// does not tie the 16-byte 16x16 instructions' accumulator input to their
// output, and at 256 accumulator registers the copies it makes instead (for
// the FP8 form as well, at this register pressure) spill. The kernel keeps
// the hazard distances the compiler cannot see: operands come straight from
// LDS reads (whose waits the compiler inserts for any reader), the two MFMAs
// of one block update accumulate into exactly the same registers (which the
// hardware orders), and ordered fences (acc_hazard_fence) separate the
// accumulators' zeroing from the first MFMA and the last MFMA from the
// epilogue's reads. Every block update is its own scheduling region, so
// program order is the issue order.
template <class Op>
__global__ void __launch_bounds__(256)
    gemm_dma_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, const uint8_t* __restrict__,
                    const uint8_t* __restrict__, typename Op::Out* __restrict__ C, int M, int N, int K,
                    int group_m) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 256, ROWB = 128, REGION = 256 * ROWB, TILES = 8;
  constexpr int PER_STEP = ROWB / MfmaGeometry<Op>::K_BYTES;  // instructions per block per step
  static_assert(Op::M == 16 && !Op::SCALED &&
                    ((PER_STEP == 1 && Op::LANE_BYTES == 32) || (PER_STEP == 2 && Op::LANE_BYTES == 16) ||
                     (PER_STEP == 8 && Op::LANE_BYTES == 4)),
                "unscaled 16x16 instructions: one with 32-byte, two with 16-byte or eight with 4-byte operands "
                "per 128-byte step");
  using Frag = i32x8;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[5 * REGION];
  if (K < 0) lds[threadIdx.x] = 0;  // keeps DMA-written reads live; never executed

  int tile_m, tile_n;
  band_tile(M / BM, N / BM, group_m, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BM;
  const int row_bytes = K * Op::ELEM_BITS / 8;
  const int k_steps = row_bytes / ROWB, last = k_steps - 1;

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A + static_cast<int64_t>(m0) * row_bytes, BM * row_bytes);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(B + static_cast<int64_t>(n0) * row_bytes, BM * row_bytes);
  // Both operands: instruction i of wave w moves rows 64w+8i .. +7 (lane l row l/8, the chunk stored at
  // physical chunk l%8 of its row) into LDS region `region`: A slots are regions 0..2, B slots 3 and 4.
  const int drow = lane >> 3;
  const int dvoff0 = drow * row_bytes + (((lane & 7) ^ (drow >> 1)) << 4);
  const int dvoff1 = drow * row_bytes + (((lane & 7) ^ ((drow >> 1) | 4)) << 4);
  const uint32_t lds_base =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)lds));
  auto dma = [&](__amdgpu_buffer_rsrc_t r, int region, int kt, int i) __attribute__((always_inline)) {
    const int row = 64 * wave + 8 * i;
    dma16(r, (i & 1) ? dvoff1 : dvoff0, kt * ROWB + row * row_bytes, lds_base + region * REGION + row * ROWB);
  };

  const int wm = wave & 1, wn = wave >> 1;
  const int lrow = lane % 16, lgroup = lane / 16;
  // Lane group g's two pieces are logical chunks g and g + 4: the swizzled
  // chunk of the first, then XOR 64 (chunk g has bit 2 clear, so the XOR
  // lands on the swizzled chunk). Fragments are 16 rows apart, which leaves
  // the swizzle unchanged.
  const int sw = ((lrow >> 1) & 7) ^ lgroup;
  const uint32_t ra0 = (wm * 128 + lrow) * ROWB + (sw << 4);
  const uint32_t rb0 = 3 * REGION + (wn * 128 + lrow) * ROWB + (sw << 4);
  auto frag = [&](uint32_t base, int region, int f) __attribute__((always_inline)) {
    const uint8_t* p = lds + base + region + f * 16 * ROWB;
    const uint8_t* q = lds + (base ^ 64u) + region + f * 16 * ROWB;
    return __builtin_shufflevector(*reinterpret_cast<const i32x4*>(p), *reinterpret_cast<const i32x4*>(q), 0, 1, 2,
                                   3, 4, 5, 6, 7);
  };
  auto mma = [&](const Frag& a, const Frag& b, typename Op::Acc& c) __attribute__((always_inline)) {
    if constexpr (PER_STEP == 1) {
      Op::mma_tied(__builtin_bit_cast(typename Op::Frag, a), __builtin_bit_cast(typename Op::Frag, b), c);
    } else if constexpr (PER_STEP == 2) {
      Op::mma_tied(__builtin_shufflevector(a, a, 0, 1, 2, 3), __builtin_shufflevector(b, b, 0, 1, 2, 3), c);
      Op::mma_tied(__builtin_shufflevector(a, a, 4, 5, 6, 7), __builtin_shufflevector(b, b, 4, 5, 6, 7), c);
    } else {
      const f32x8 af = __builtin_bit_cast(f32x8, a), bf = __builtin_bit_cast(f32x8, b);
#pragma unroll
      for (int p = 0; p < 8; ++p) Op::mma_tied(af[p], bf[p], c);
    }
  };
  auto frag_a = [&](int slot, int f) __attribute__((always_inline)) { return frag(ra0, slot * REGION, f); };
  auto frag_b = [&](int s, int f) __attribute__((always_inline)) { return frag(rb0, s * REGION, f); };

  typename Op::Acc acc[TILES][TILES];
#pragma unroll
  for (int i = 0; i < TILES; ++i)
#pragma unroll
    for (int j = 0; j < TILES; ++j) acc[i][j] = typename Op::Acc{};

  // Prologue: A and B of steps 0 and 1 into A slots 0, 1 and B slots 0, 1,
  // all of it in LDS before the barrier.
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) dma(ra, p, min(p, last), i);
#pragma unroll
  for (int p = 0; p < 2; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) dma(rb, 3 + p, min(p, last), i);
  __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
  lds_barrier();

  // Step 0's A fragments and B fragments 4..7; its B 0..3 are read by the first half.
  Frag fa[TILES], fb[TILES];
#pragma unroll
  for (int f = 0; f < TILES; ++f) fa[f] = frag_a(0, f);
#pragma unroll
  for (int f = 4; f < TILES; ++f) fb[f] = frag_b(0, f);
#pragma unroll
  for (int i = 0; i < TILES; ++i)
#pragma unroll
    for (int j = 0; j < TILES; ++j) acc_hazard_fence(acc[i][j]);

  // Slots (one block update each, its own scheduling region):
  //   First half (32 slots): B fragment reads in slots 0, 2, 4, 6; A DMA i
  //     in slot 4i + 1.
  //   Second half (32 slots): B fragment reads in slots 0, 2, 4, 6; B DMA i in
  //     slot 4i + 1; A fragment i after slot 4i + 3.
  int slot = 0;  // A slot of the current step: kt % 3
  auto step = [&](int kt, int s) __attribute__((always_inline)) {
    const int next_slot = slot == 2 ? 0 : slot + 1, prev_slot = slot == 0 ? 2 : slot - 1;
    static_for<0, 32>([&](auto q_c) __attribute__((always_inline)) {
      constexpr int q = decltype(q_c)::value, i = q / 4, j = 4 + q % 4;
      constexpr int rd = q < 8 && q % 2 == 0 ? q / 2 : -1;
      if constexpr (rd >= 0) fb[rd] = frag_b(s, rd);
      constexpr int da = q % 4 == 1 ? q / 4 : -1;
      if constexpr (da >= 0) dma(ra, prev_slot, min(kt + 2, last), da);
      mma(fa[i], fb[j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    });
    __builtin_amdgcn_s_waitcnt(vmcnt_only(8));
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, 32>([&](auto q_c) __attribute__((always_inline)) {
      constexpr int q = decltype(q_c)::value, i = q / 4, j = q % 4;
      constexpr int rd = q < 8 && q % 2 == 0 ? 4 + q / 2 : -1;
      if constexpr (rd >= 0) fb[rd] = frag_b(s ^ 1, rd);
      constexpr int db = q % 4 == 1 ? q / 4 : -1;
      if constexpr (db >= 0) dma(rb, 3 + s, min(kt + 2, last), db);
      mma(fa[i], fb[j], acc[i][j]);
      if constexpr (j == 3) fa[i] = frag_a(next_slot, i);
      __builtin_amdgcn_sched_barrier(0);
    });
    slot = next_slot;
  };
  for (int kt = 0; kt < k_steps; kt += 2) {
    step(kt, 0);
    step(kt + 1, 1);
  }
#pragma unroll
  for (int i = 0; i < TILES; ++i)
#pragma unroll
    for (int j = 0; j < TILES; ++j) acc_hazard_fence(acc[i][j]);

#pragma unroll
  for (int i = 0; i < TILES; ++i)
#pragma unroll
    for (int j = 0; j < TILES; ++j)
#pragma unroll
      for (int r = 0; r < Op::ACC_REGS; ++r) {
        const int row = m0 + wm * 128 + i * Op::M + Op::out_row(lane, r);
        const int col = n0 + wn * 128 + j * Op::N + lrow;
        C[static_cast<int64_t>(row) * N + col] = acc[i][j][r];
      }
#endif
}

// ---- 256x128 kernel, A by LDS DMA (FP64 on 16x16x4) -------------------------

// The 256x256 DMA kernel's A ring, swizzle, pipeline and rolled fragments,
// with B through registers into two LDS stages, for FP64 on a 256x128 tile: 256 accumulator registers hold 128x64 fp64
// outputs per wave (8x4 blocks of 16x16, four v_mfma_f64_16x16x4_f64 per
// block per 128-byte step of 16 doubles). M a multiple of 256, N of 128, K an
// even number of at least 4 steps.
//
// LDS (128 KiB): three A slots of 256 rows and two B stages of 128 rows, 128
// bytes each. B moves global -> VGPR (two sets of four 16-byte loads per
// thread, two steps ahead) -> stage.
//
// Fragments: lane group g holds logical chunks g and g + 4 of its row, doubles
// 2g, 2g+1, 8+2g and 9+2g; instruction p of a block takes double p of every
// lane, the same K permutation for A and B. One set of 8 A and 4 B fragments.
//
// Per K step kt (A slot kt % 3, B stage s = kt & 1), 32 block updates and one
// barrier:
//   first half:  blocks (i, 2 + j), i = 0..7, j = 0..1, row by row; reads of
//                B fragments 0..1 of this step; B registers holding step kt+1
//                written to stage s^1, and two of step kt+3's four B loads;
//   barrier      (publishes step kt+1, ends every read of A slot kt % 3);
//   second half: blocks (i, j), j = 0..1; at its start the reads of B
//                fragments 2..3 of step kt+1, then A fragment i of step kt+1
//                after block (i, 1); the A DMAs of step kt+3 into slot kt % 3
//                in the odd slots, then the last two B loads, which the stage
//                writes of step kt+2 wait for before the barrier that
//                publishes step kt+3 (so those waits also cover the DMAs).
template <class Op>
__global__ void __launch_bounds__(256)
    gemm_dma_f64_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, const uint8_t* __restrict__,
                        const uint8_t* __restrict__, typename Op::Out* __restrict__ C, int M, int N, int K,
                        int group_m) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 256, BN = 128, ROWB = 128, AREG = BM * ROWB, BREG = BN * ROWB, NB = 4, TM = 8, TN = 4;
  static_assert(Op::M == 16 && Op::ELEM_BITS == 64 && Op::LANE_BYTES == 8 && MfmaGeometry<Op>::K_BYTES == 32,
                "the FP64 16x16x4 instruction: four per block per 128-byte step");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[3 * AREG + 2 * BREG];
  if (K < 0) lds[threadIdx.x] = 0;  // keeps DMA-written reads live; never executed

  int tile_m, tile_n;
  band_tile(M / BM, N / BN, group_m, tile_m, tile_n);
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int row_bytes = K * Op::ELEM_BITS / 8;
  const int k_steps = row_bytes / ROWB, last = k_steps - 1;

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A + static_cast<int64_t>(m0) * row_bytes, BM * row_bytes);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(B + static_cast<int64_t>(n0) * row_bytes, BN * row_bytes);
  // B: load j of a step covers rows 32j .. 32j+31; thread t moves row 32j + t/8, chunk t%8.
  const int voff = (t >> 3) * row_bytes + (t & 7) * 16;
  uint8_t* const wb = lds + 3 * AREG + (t >> 3) * ROWB + (((t & 7) ^ ((t >> 4) & 7)) << 4);
  auto load = [&](i32x4 (&v)[NB], int kt, int j) __attribute__((always_inline)) {
    v[j] = __builtin_bit_cast(i32x4,
                              __builtin_amdgcn_raw_buffer_load_b128(rb, voff, kt * ROWB + j * 32 * row_bytes, 0));
  };
  auto store = [&](const i32x4 (&v)[NB], int s, int j) __attribute__((always_inline)) {
    *reinterpret_cast<i32x4*>(wb + s * BREG + j * 32 * ROWB) = v[j];
  };
  // A: the DMA kernel's mapping (instruction i of wave w moves rows 64w+8i .. +7).
  const int arow = lane >> 3;
  const int avoff0 = arow * row_bytes + (((lane & 7) ^ (arow >> 1)) << 4);
  const int avoff1 = arow * row_bytes + (((lane & 7) ^ ((arow >> 1) | 4)) << 4);
  const uint32_t lds_base =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)lds));
  auto dma_a = [&](int slot, int kt, int i) __attribute__((always_inline)) {
    const int row = 64 * wave + 8 * i;
    dma16(ra, (i & 1) ? avoff1 : avoff0, kt * ROWB + row * row_bytes, lds_base + slot * AREG + row * ROWB);
  };

  const int wm = wave & 1, wn = wave >> 1;
  const int lrow = lane % 16, lgroup = lane / 16;
  const int sw = ((lrow >> 1) & 7) ^ lgroup;
  const uint32_t ra0 = (wm * 128 + lrow) * ROWB + (sw << 4);
  const uint32_t rb0 = 3 * AREG + (wn * 64 + lrow) * ROWB + (sw << 4);
  auto frag = [&](uint32_t base, int region, int f) __attribute__((always_inline)) {
    const uint8_t* p = lds + base + region + f * 16 * ROWB;
    const uint8_t* q = lds + (base ^ 64u) + region + f * 16 * ROWB;
    return __builtin_shufflevector(*reinterpret_cast<const i32x4*>(p), *reinterpret_cast<const i32x4*>(q), 0, 1, 2,
                                   3, 4, 5, 6, 7);
  };
  auto frag_a = [&](int slot, int f) __attribute__((always_inline)) { return frag(ra0, slot * AREG, f); };
  auto frag_b = [&](int s, int f) __attribute__((always_inline)) { return frag(rb0, s * BREG, f); };
  auto mma = [&](const i32x8& a, const i32x8& b, typename Op::Acc& c) __attribute__((always_inline)) {
    const f64x4 ad = __builtin_bit_cast(f64x4, a), bd = __builtin_bit_cast(f64x4, b);
#pragma unroll
    for (int p = 0; p < 4; ++p) Op::mma_tied(ad[p], bd[p], c);
  };

  typename Op::Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = typename Op::Acc{};

  // Prologue (the DMA kernel's): A of steps 0..2 into slots 0..2, B of steps
  // 0 and 1 in flight, step 0 written to B stage 0, step 2's B into v0.
  i32x4 v0[NB], v1[NB];
#pragma unroll
  for (int p = 0; p < 3; ++p)
#pragma unroll
    for (int i = 0; i < 8; ++i) dma_a(p, min(p, last), i);
#pragma unroll
  for (int j = 0; j < NB; ++j) load(v0, 0, j);
#pragma unroll
  for (int j = 0; j < NB; ++j) load(v1, min(1, last), j);
#pragma unroll
  for (int j = 0; j < NB; ++j) store(v0, 0, j);
#pragma unroll
  for (int j = 0; j < NB; ++j) load(v0, min(2, last), j);
  lds_barrier();

  i32x8 fa[TM], fb[TN];
#pragma unroll
  for (int f = 0; f < TM; ++f) fa[f] = frag_a(0, f);
#pragma unroll
  for (int f = 2; f < TN; ++f) fb[f] = frag_b(0, f);
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc_hazard_fence(acc[i][j]);

  // Slots (one block update each, its own scheduling region):
  //   First half (16 slots): B fragment reads in slots 0 and 2; stage writes
  //     in slots 1, 4, 7, 10; B loads 0 and 1 in slots 2 and 8.
  //   Second half: B fragment reads in slots 0 and 2; A DMAs in the odd slots;
  //     B loads 2 and 3 after the last DMA; A fragment i after slot 2i + 1.
  int slot = 0;  // A slot of the current step: kt % 3
  auto step = [&](int kt, int s, i32x4 (&vnext)[NB]) __attribute__((always_inline)) {
    const int next_slot = slot == 2 ? 0 : slot + 1;
    static_for<0, 16>([&](auto q_c) __attribute__((always_inline)) {
      constexpr int q = decltype(q_c)::value, i = q / 2, j = 2 + q % 2;
      constexpr int rd = q < 4 && q % 2 == 0 ? q / 2 : -1;
      if constexpr (rd >= 0) fb[rd] = frag_b(s, rd);
      constexpr int wr = q < 12 && q % 3 == 1 ? q / 3 : -1;
      if constexpr (wr >= 0) store(vnext, s ^ 1, wr);
      constexpr int ld = q < 12 && q % 6 == 2 ? q / 6 : -1;
      if constexpr (ld >= 0) load(vnext, min(kt + 3, last), ld);
      mma(fa[i], fb[j], acc[i][j]);
      __builtin_amdgcn_sched_barrier(0);
    });
    lds_barrier();
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, 16>([&](auto q_c) __attribute__((always_inline)) {
      constexpr int q = decltype(q_c)::value, i = q / 2, j = q % 2;
      constexpr int rd = q < 4 && q % 2 == 0 ? 2 + q / 2 : -1;
      if constexpr (rd >= 0) fb[rd] = frag_b(s ^ 1, rd);
      constexpr int dm = q % 2 == 1 ? q / 2 : -1;
      if constexpr (dm >= 0) dma_a(slot, min(kt + 3, last), dm);
      mma(fa[i], fb[j], acc[i][j]);
      if constexpr (j == 1) fa[i] = frag_a(next_slot, i);
      if constexpr (q == 15) {
        load(vnext, min(kt + 3, last), 2);
        load(vnext, min(kt + 3, last), 3);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    slot = next_slot;
  };
  for (int kt = 0; kt < k_steps; kt += 2) {
    step(kt, 0, v1);
    step(kt + 1, 1, v0);
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc_hazard_fence(acc[i][j]);

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < Op::ACC_REGS; ++r) {
        const int row = m0 + wm * 128 + i * Op::M + Op::out_row(lane, r);
        const int col = n0 + wn * 64 + j * Op::N + lrow;
        C[static_cast<int64_t>(row) * N + col] = acc[i][j][r];
      }
#endif
}

// Launchers size their own grid: one workgroup per output tile of their kernel.
using GemmLauncher = void (*)(const uint8_t*, const uint8_t*, const uint8_t*, const uint8_t*, void*, int, int, int,
                              int, hipStream_t);

inline uint32_t tile_count(int m, int n, int bm, int bn) {
  return static_cast<uint32_t>(((m + bm - 1) / bm) * static_cast<int64_t>((n + bn - 1) / bn));
}

template <class Op, int BM, int BN, int BK, int WM, int WN, bool CHECKED>
void launch_gemm(const uint8_t* a, const uint8_t* b, const uint8_t* sa, const uint8_t* sb, void* c, int m, int n,
                 int k, int group_m, hipStream_t stream) {
  gemm_kernel<Op, BM, BN, BK, WM, WN, CHECKED><<<dim3(tile_count(m, n, BM, BN)), dim3(64 * WM * WN), 0, stream>>>(
      a, b, sa, sb, static_cast<typename Op::Out*>(c), m, n, k, group_m);
}

// The fast-path kernel of an instruction: the all-DMA kernel for the unscaled
// ones (256x256; its 256x128 FP64 form), the register-staged kernel (with its
// scale ring) for MXFP4.
template <class Op>
constexpr auto fast_kernel_fn() {
  if constexpr (Op::SCALED)
    return gemm_staged_kernel<Op>;
  else if constexpr (Op::ELEM_BITS == 64)
    return gemm_dma_f64_kernel<Op>;
  else
    return gemm_dma_kernel<Op>;
}

// Tile width of the fast-path kernel (its height is 256).
template <class Op>
constexpr int fast_tile_n() {
  return Op::ELEM_BITS == 64 ? 128 : 256;
}

template <class Op>
const void* fast_kernel() {
  return reinterpret_cast<const void*>(fast_kernel_fn<Op>());
}

template <class Op>
void launch_gemm_staged(const uint8_t* a, const uint8_t* b, const uint8_t* sa, const uint8_t* sb, void* c, int m,
                        int n, int k, int group_m, hipStream_t stream) {
  fast_kernel_fn<Op>()<<<dim3(tile_count(m, n, 256, fast_tile_n<Op>())), dim3(256), 0, stream>>>(
      a, b, sa, sb, static_cast<typename Op::Out*>(c), m, n, k, group_m);
}

// What a variant's fast launcher needs beyond a shape that divides its tile.
enum GemmPath { kLdsPath = 0, kStagedPath = 1 };

// launch: shapes that divide the tile and satisfy the path's rule (see
// exact_shape); launch_checked: any shape.
struct GemmVariant {
  int format;
  mb_gemm_config config;
  const char* name;
  const void* kernel;
  GemmLauncher launch;
  GemmLauncher launch_checked;
  int out_bytes;
  int elem_bits;
  int path;
  const char* checked_name;
  const void* checked_kernel;
  int default_group;  // band height in tile rows when the caller passes 0 (measured per kernel)
};

#define MB_GEMM(FMT, OP, BM, BN, BK, WM, WN, NAME)                                                           \
  GemmVariant{FMT,                                                                                           \
              mb_gemm_config{BM, BN, BK, 64 * WM * WN},                                                      \
              NAME,                                                                                          \
              reinterpret_cast<const void*>(gemm_kernel<OP, BM, BN, BK, WM, WN, false>),                     \
              launch_gemm<OP, BM, BN, BK, WM, WN, false>,                                                    \
              launch_gemm<OP, BM, BN, BK, WM, WN, true>,                                                     \
              static_cast<int>(sizeof(typename OP::Out)),                                                    \
              OP::ELEM_BITS,                                                                                 \
              kLdsPath,                                                                                      \
              NAME "_checked",                                                                               \
              reinterpret_cast<const void*>(gemm_kernel<OP, BM, BN, BK, WM, WN, true>),                      \
              8}

// 256x256 tiles (256x128 for FP64): the fast-path kernel (BK = 128 bytes of K;
// instruction SOP) for exact shapes, a checked LDS-staged kernel (tile CM x CN,
// instruction OP) for the rest.
#define MB_GEMM_STAGED(FMT, SOP, OP, BK, CM, CN, GROUP, NAME, CNAME)                                              \
  GemmVariant{FMT,                                                                                           \
              mb_gemm_config{256, fast_tile_n<SOP>(), BK, 256},                                              \
              NAME,                                                                                          \
              fast_kernel<SOP>(),                                                                            \
              launch_gemm_staged<SOP>,                                                                       \
              launch_gemm<OP, CM, CN, BK, 2, 2, true>,                                                       \
              static_cast<int>(sizeof(typename OP::Out)),                                                    \
              OP::ELEM_BITS,                                                                                 \
              kStagedPath,                                                                                   \
              CNAME,                                                                                         \
              reinterpret_cast<const void*>(gemm_kernel<OP, CM, CN, BK, 2, 2, true>),                        \
              GROUP}
// GROUP: the band height the sweeps at the benchmark sizes measured best per
// fast-path kernel (BF16 and FP16 4, FP8 6, INT8 7, MXFP4 8; FP64 flat, 8).
const GemmVariant kGemmVariants[] = {
    MB_GEMM_STAGED(MB_MATRIX_BF16, MfmaBf16x16, MfmaBf16, 64, 256, 256, 4, "gemm_bf16_256x256x64",
                   "gemm_bf16_256x256x64_checked"),
    MB_GEMM(MB_MATRIX_BF16, MfmaBf16, 256, 128, 64, 2, 2, "gemm_bf16_256x128x64"),
    MB_GEMM(MB_MATRIX_BF16, MfmaBf16, 128, 128, 64, 2, 2, "gemm_bf16_128x128x64"),
    MB_GEMM_STAGED(MB_MATRIX_F16, MfmaF16x16, MfmaF16, 64, 256, 256, 4, "gemm_f16_256x256x64",
                   "gemm_f16_256x256x64_checked"),
    MB_GEMM(MB_MATRIX_F16, MfmaF16, 256, 128, 64, 2, 2, "gemm_f16_256x128x64"),
    MB_GEMM(MB_MATRIX_F16, MfmaF16, 128, 128, 64, 2, 2, "gemm_f16_128x128x64"),
    MB_GEMM_STAGED(MB_MATRIX_FP8_E4M3, MfmaFp8x16, MfmaFp8, 128, 256, 256, 6, "gemm_fp8_256x256x128",
                   "gemm_fp8_256x256x128_checked"),
    MB_GEMM(MB_MATRIX_FP8_E4M3, MfmaFp8, 256, 128, 128, 2, 2, "gemm_fp8_256x128x128"),
    MB_GEMM(MB_MATRIX_FP8_E4M3, MfmaFp8, 128, 128, 128, 2, 2, "gemm_fp8_128x128x128"),
    MB_GEMM_STAGED(MB_MATRIX_I8, MfmaI8x16, MfmaI8, 128, 256, 256, 7, "gemm_i8_256x256x128",
                   "gemm_i8_256x256x128_checked"),
    MB_GEMM(MB_MATRIX_I8, MfmaI8, 256, 128, 128, 2, 2, "gemm_i8_256x128x128"),
    MB_GEMM(MB_MATRIX_I8, MfmaI8, 128, 128, 128, 2, 2, "gemm_i8_128x128x128"),
    MB_GEMM_STAGED(MB_MATRIX_MXFP4, MfmaMxfp4, MfmaMxfp4, 256, 128, 128, 8, "gemm_mxfp4_256x256x256",
                   "gemm_mxfp4_128x128x256_checked"),
    MB_GEMM(MB_MATRIX_MXFP4, MfmaMxfp4, 256, 128, 256, 2, 2, "gemm_mxfp4_256x128x256"),
    MB_GEMM(MB_MATRIX_MXFP4, MfmaMxfp4, 128, 128, 256, 2, 2, "gemm_mxfp4_128x128x256"),
    MB_GEMM_STAGED(MB_MATRIX_F64, MfmaF64, MfmaF64, 16, 128, 128, 8, "gemm_f64_256x128x16",
                   "gemm_f64_128x128x16_checked"),
    MB_GEMM(MB_MATRIX_F64, MfmaF64, 128, 128, 16, 2, 2, "gemm_f64_128x128x16"),
    MB_GEMM(MB_MATRIX_F64, MfmaF64, 64, 64, 16, 2, 2, "gemm_f64_64x64x16"),
    MB_GEMM_STAGED(MB_MATRIX_F32, MfmaF32x16, MfmaF32, 32, 128, 128, 8, "gemm_f32_256x256x32",
                   "gemm_f32_128x128x32_checked"),
    MB_GEMM(MB_MATRIX_F32, MfmaF32, 128, 128, 32, 2, 2, "gemm_f32_128x128x32"),
};

struct GemmRegistrar {
  GemmRegistrar() {
    for (const auto& variant : kGemmVariants) {
      register_kernel(variant.name, variant.kernel);
      // A fallback can be another variant's checked kernel: register each name once.
      bool seen = false;
      for (const auto* other = kGemmVariants; other != &variant; ++other)
        seen = seen || std::strcmp(other->checked_name, variant.checked_name) == 0;
      if (!seen) register_kernel(variant.checked_name, variant.checked_kernel);
    }
  }
};
const GemmRegistrar kGemmRegistrar;

const GemmVariant* find_gemm(int format, const mb_gemm_config* config) {
  for (const auto& variant : kGemmVariants) {
    const mb_gemm_config& v = variant.config;
    if (variant.format == format && v.tile_m == config->tile_m && v.tile_n == config->tile_n &&
        v.tile_k == config->tile_k)
      return &variant;
  }
  return nullptr;
}

// The launcher (and its registered name) a call will use: the variant's fast
// kernel when the shape divides its tile and meets the path's rule, else its
// checked kernel.
struct GemmChoice {
  const GemmVariant* variant;
  GemmLauncher launch;
  const char* name;
};

int choose_gemm(int format, const mb_gemm_config* config, uint32_t m, uint32_t n, uint32_t k, const void* scale_a,
                const void* scale_b, const char* entry, GemmChoice* out) {
  if (int rc = matrix_format_check(format, entry)) return rc;
  if (config == nullptr) return fail(MB_ERR_INVALID, "%s: config is NULL", entry);
  const GemmVariant* variant = find_gemm(format, config);
  if (variant == nullptr)
    return fail(MB_ERR_INVALID, "%s: no kernel for format %d with tile %ux%ux%u (see mb_gemm_configs)", entry, format,
                config->tile_m, config->tile_n, config->tile_k);
  if (m == 0 || n == 0 || k == 0) return fail(MB_ERR_INVALID, "%s: empty problem %ux%ux%u", entry, m, n, k);
  if (m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu)
    return fail(MB_ERR_INVALID, "%s: dimensions exceed 2^31-1", entry);
  if (format == MB_MATRIX_MXFP4 && k % 32)
    return fail(MB_ERR_INVALID, "%s: MXFP4 needs K to be a multiple of the 32-element scale group", entry);
  const uint64_t row_bits = static_cast<uint64_t>(k) * variant->elem_bits;
  if (row_bits % 128)
    return fail(MB_ERR_INVALID, "%s: K*element size must be a multiple of 16 bytes (rows are 16-byte loads)", entry);
  // The tile count of the smallest tile any launcher uses bounds the grid.
  const uint64_t max_tiles = static_cast<uint64_t>((m + 63) / 64) * ((n + 63) / 64);
  if (max_tiles > 0x7fffffffull) return fail(MB_ERR_INVALID, "%s: too many tiles", entry);
  const uint64_t row_bytes = row_bits / 8, steps = row_bytes / 128;
  const mb_gemm_config& v = variant->config;
  bool fast = m % v.tile_m == 0 && n % v.tile_n == 0 && k % v.tile_k == 0;
  // The staged kernel addresses each tile's operand rows (and the MXFP4 scale
  // blocks) with 32-bit offsets in 128-byte K steps, runs an even number of
  // at least four steps and moves scale rows with 16-byte DMAs.
  if (variant->path == kStagedPath) {
    fast = fast && row_bytes % 128 == 0 && 256 * row_bytes <= 0x7fffffffull && steps >= 4 && steps % 2 == 0;
    if (format == MB_MATRIX_MXFP4)
      fast = fast && aligned(scale_a, 16) && aligned(scale_b, 16) &&
             steps * (m > n ? m : n) * 8 <= 0x7fffffffull;
  }
  out->variant = variant;
  out->launch = fast ? variant->launch : variant->launch_checked;
  out->name = fast ? variant->name : variant->checked_name;
  return MB_OK;
}

}  // namespace
}  // namespace mb

extern "C" {

int mb_gemm_configs(int format, mb_gemm_config* out, int capacity) {
  using namespace mb;
  if (int rc = matrix_format_check(format, "mb_gemm_configs")) return rc;
  int count = 0;
  for (const auto& variant : kGemmVariants) {
    if (variant.format != format) continue;
    if (out != nullptr && count < capacity) out[count] = variant.config;
    ++count;
  }
  return count;
}

const char* mb_gemm_kernel_name(int format, const mb_gemm_config* config) {
  if (config == nullptr) return nullptr;
  const mb::GemmVariant* variant = mb::find_gemm(format, config);
  return variant ? variant->name : nullptr;
}

int mb_gemm(int format, const mb_gemm_config* config, const void* a, uint64_t a_bytes, const void* b,
            uint64_t b_bytes, const void* scale_a, uint64_t scale_a_bytes, const void* scale_b,
            uint64_t scale_b_bytes, void* c, uint64_t c_bytes, uint32_t m, uint32_t n, uint32_t k,
            uint32_t group_m, void* stream) {
  using namespace mb;
  GemmChoice choice;
  if (int rc = choose_gemm(format, config, m, n, k, scale_a, scale_b, "mb_gemm", &choice)) return rc;
  const GemmVariant* variant = choice.variant;
  const uint64_t row_bytes = static_cast<uint64_t>(k) * variant->elem_bits / 8;
  if (a == nullptr || b == nullptr || c == nullptr) return fail(MB_ERR_INVALID, "mb_gemm: NULL operand");
  if (a_bytes < m * row_bytes || b_bytes < n * row_bytes ||
      c_bytes < static_cast<uint64_t>(m) * n * variant->out_bytes)
    return fail(MB_ERR_INVALID, "mb_gemm: buffers too small for %ux%ux%u", m, n, k);
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16))
    return fail(MB_ERR_ALIGNMENT, "mb_gemm: A, B and C must be 16-byte aligned");
  if (format == MB_MATRIX_MXFP4) {
    if (scale_a == nullptr || scale_b == nullptr)
      return fail(MB_ERR_INVALID, "mb_gemm: MXFP4 needs E8M0 scales for A and B");
    const uint64_t blocks = (k + 255) / 256;
    if (scale_a_bytes < blocks * m * 8 || scale_b_bytes < blocks * n * 8)
      return fail(MB_ERR_INVALID, "mb_gemm: scale buffers too small ([ceil(K/256)][M|N][8] bytes needed)");
  }
  // A band taller than the tile rows acts as the full height, so group_m is
  // clamped to the row count of the smallest tile a launcher uses: the band's
  // tile count (group x tile columns) then stays within the int grid.
  const uint32_t max_group = (m + 63) / 64;
  const int group = static_cast<int>(group_m ? (group_m < max_group ? group_m : max_group)
                                             : static_cast<uint32_t>(variant->default_group));
  choice.launch(static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(b), static_cast<const uint8_t*>(scale_a),
                static_cast<const uint8_t*>(scale_b), c, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k),
                group, static_cast<hipStream_t>(stream));
  return launch_status(choice.name);
}

const char* mb_gemm_launched_kernel(int format, const mb_gemm_config* config, uint32_t m, uint32_t n, uint32_t k,
                                    const void* scale_a, const void* scale_b) {
  mb::GemmChoice choice;
  if (mb::choose_gemm(format, config, m, n, k, scale_a, scale_b, "mb_gemm_launched_kernel", &choice)) return nullptr;
  return choice.name;
}

}  // extern "C"
