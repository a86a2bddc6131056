// Dense GEMM on the matrix cores (tensor rows' GEMM mode and the benchmark's
// 8192^3 / 4096^3 / 16384^3 GEMM configurations).
//
// C[M][N] = A[M][K] . B[K][N] with A row-major and B column-major, so both
// operands are K-contiguous in memory ("NT"); the accumulator type is the
// instruction's (fp32, int32 for INT8, fp64 for FP64). MXFP4 operands carry
// one E8M0 scale per 32 K elements: SA[M][K/32], SB[N][K/32].
// Replaces the reference's _gemm_kernel (bench_tensor.py:172-209), whose B is
// row-major; the MI355X kernel takes K-contiguous B (layout prepared outside
// timing by the caller).
//
// Design:
//   * a workgroup of WAVES_M x WAVES_N waves owns a BM x BN tile; each wave a
//     (BM/WAVES_M) x (BN/WAVES_N) block of 32x32 (16x16 for FP64) MFMA tiles;
//   * each K step stages BM x BK and BN x BK operand tiles from HBM into a
//     padded, double-buffered LDS tile with 16-byte coalesced loads; the loads
//     of step k+1 are in flight while the MFMAs of step k run, and one barrier
//     per step separates the buffers;
//   * workgroups are numbered XCD-first: the hardware deals consecutive
//     workgroup ids round-robin over the 8 XCDs, so id i is remapped to the
//     i/8-th tile of XCD i%8's contiguous share, and within that share tiles
//     are walked in GROUP_M-row bands, keeping A and B panels hot in the XCD's L2;
//   * CHECKED instantiations bound every load and store for ragged shapes.
//
// 256x256 tiles of the 8- and 16-bit formats use gemm_dma_kernel instead when
// the shape divides the tile: 8 waves (2 per SIMD), operands fed straight from
// L2 into LDS by buffer_load_dwordx4 ... lds (no VGPR staging, no ds_write),
// XOR-swizzled LDS rows (conflict-free ds_read_b128 without padding), and
// fragment reads of substep s+1 issued ahead of the MFMAs of substep s.
#include "mb_internal.h"
#include "mb_mfma.h"

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
          sa[tm][ks] = (!CHECKED || (row < M && col < scale_cols)) ? SA[static_cast<int64_t>(row) * scale_cols + col]
                                                                    : 127;
        }
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
        for (int ks = 0; ks < T::KSTEPS; ++ks) {
          const int col_n = n0 + wn * T::WN + tn * Op::N + lrow;
          const int col = kt * T::GROUPS + ks * MfmaGeometry<Op>::LANE_GROUPS + lgroup;
          sb[tn][ks] = (!CHECKED || (col_n < N && col < scale_cols))
                           ? SB[static_cast<int64_t>(col_n) * scale_cols + col]
                           : 127;
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

// ---- DMA-fed 256x256 kernel ------------------------------------------------

// One 16-byte-per-lane LDS DMA: lane l's 16 bytes land at lds_addr + 16 * l.
// Issued as inline assembly so the compiler's wait-count pass does not force a
// full vmcnt(0) before every LDS read; the kernel waits explicitly instead.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, uint32_t lds_addr) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voffset), "s"(rsrc), "s"(soffset),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

// One 4-byte-per-lane LDS DMA (E8M0 scale rows): lane l's 4 bytes land at lds_addr + 4 * l.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rsrc, int voffset, int soffset, uint32_t lds_addr) {
  asm volatile("buffer_load_dword %0, %1, %2 offen lds" ::"v"(voffset), "s"(rsrc), "s"(soffset),
               "{m0}"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory");
}

__device__ __forceinline__ void wait_all_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Word 3 of a gfx9 buffer resource: 32-bit data format, no swizzle, raw offsets.
constexpr int kBufferWord3 = 0x00020000;

// C = A . B^T for M, N multiples of 256 and K * bits multiples of ROWB * 8;
// A, B byte offsets must fit in 31 bits. Each K step stages a 256 x ROWB-byte
// slice of A and of B (one LDS stage, double-buffered); for MXFP4 the stage
// also holds the step's E8M0 scales, 256 rows x ROWB/16 bytes for A and for B. LDS row r holds its
// 16-byte chunk c at position c ^ ((r / (256 / ROWB)) % (ROWB / 16)): any 16
// consecutive rows read at one logical chunk hit 16 distinct bank groups.
template <class Op, int ROWB, int WAVES_M, int WAVES_N>
__global__ void __launch_bounds__(64 * WAVES_M * WAVES_N)
    gemm_dma_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B, const uint8_t* __restrict__ SA,
                    const uint8_t* __restrict__ SB, typename Op::Out* __restrict__ C, int M, int N, int K,
                    int group_m) {
#if defined(__HIP_DEVICE_COMPILE__)
  constexpr int BM = 256, BN = 256;
  constexpr int NW = WAVES_M * WAVES_N;
  constexpr int CPR = ROWB / 16;      // 16-byte chunks per LDS row
  constexpr int RPI = 1024 / ROWB;    // rows one DMA instruction fills (64 lanes x 16 bytes)
  constexpr int RPB = 256 / ROWB;     // rows per 256 bytes: the swizzle period
  constexpr int DATA = (BM + BN) * ROWB;
  // MXFP4: ROWB bytes hold 2*ROWB E2M1 codes, i.e. ROWB/16 scale bytes per row.
  constexpr int SCALE_ROW = Op::SCALED ? ROWB / 16 : 0;
  constexpr int STAGE = DATA + (BM + BN) * SCALE_ROW;
  constexpr int INSTR = (BM + BN) / RPI / NW;  // DMA instructions per wave per K step
  constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N, TM = WM / Op::M, TN = WN / Op::N;
  constexpr int KB = MfmaGeometry<Op>::K_BYTES, KSTEPS = ROWB / KB, PIECES = Op::LANE_BYTES / 16;
  static_assert((BM / RPI) % NW == 0, "an instruction's rows are all A or all B, whatever the wave");
  static_assert(ROWB % KB == 0 && Op::LANE_BYTES % 16 == 0 && Op::M == 32, "whole 32x32 instructions per step");
  static_assert(!Op::SCALED || (SCALE_ROW == 8 && (BM + BN) * SCALE_ROW / 256 == 2 * NW),
                "scale DMA: one 4-byte-lane instruction of A rows and one of B rows per wave");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[2 * STAGE];
  // The array is otherwise written only by DMA, which the optimizer does not
  // see as a store; one plain (never executed) store keeps its reads live.
  if (K < 0) lds[threadIdx.x] = 0;

  const int tiles_m = M / BM, tiles_n = N / BN;
  const int count = gridDim.x;
  int pid = blockIdx.x;
  if (count % kXcds == 0) pid = (pid % kXcds) * (count / kXcds) + pid / kXcds;
  const int band = group_m * tiles_n;
  const int first_m = (pid / band) * group_m;
  const int rows_in_band = min(tiles_m - first_m, group_m);
  const int tile_m = first_m + (pid % band) % rows_in_band;
  const int tile_n = (pid % band) / rows_in_band;
  const int m0 = tile_m * BM, n0 = tile_n * BN;
  const int row_bytes = K * Op::ELEM_BITS / 8;
  const int k_steps = row_bytes / ROWB;

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  // Each resource covers exactly this tile's 256 rows of its operand.
  const __amdgpu_buffer_rsrc_t rsrc_a = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(A + static_cast<int64_t>(m0) * row_bytes), (short)0, BM * row_bytes, kBufferWord3);
  const __amdgpu_buffer_rsrc_t rsrc_b = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t*>(B + static_cast<int64_t>(n0) * row_bytes), (short)0, BN * row_bytes, kBufferWord3);
  const uint32_t lds_base =
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint8_t*)(lds)));
  // DMA instruction j of this wave fills LDS rows rb*RPI .. rb*RPI+RPI-1 of the
  // A|B stage, rb = j*NW + wave; lane l supplies row rb*RPI + l/CPR, physical
  // chunk l%CPR, i.e. the global chunk that swizzles there.
  int voff[INSTR];
#pragma unroll
  for (int j = 0; j < INSTR; ++j) {
    const int row = (j * NW + wave) * RPI + lane / CPR;
    const int chunk = (lane % CPR) ^ ((row / RPB) % CPR);
    voff[j] = (row < BM ? row : row - BM) * row_bytes + chunk * 16;
  }
  // MXFP4 scales: wave w moves A scale rows 32w .. 32w+31 and the same B
  // rows; lane l carries half l%2 of row 32w + l/2's SCALE_ROW bytes.
  const int scale_cols = Op::SCALED ? K / 32 : 0;
  __amdgpu_buffer_rsrc_t rsrc_sa = rsrc_a, rsrc_sb = rsrc_b;
  int scale_voff = 0;
  if constexpr (Op::SCALED) {
    rsrc_sa = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SA + static_cast<int64_t>(m0) * scale_cols),
                                                (short)0, BM * scale_cols, kBufferWord3);
    rsrc_sb = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(SB + static_cast<int64_t>(n0) * scale_cols),
                                                (short)0, BN * scale_cols, kBufferWord3);
    scale_voff = (wave * 32 + lane / 2) * scale_cols + (lane % 2) * 4;
  }
  auto issue = [&](int kt) {
    const uint32_t stage = lds_base + (kt & 1) * STAGE;
#pragma unroll
    for (int j = 0; j < INSTR; ++j) {
      const uint32_t dst = stage + (j * NW + wave) * 1024;
      if (j * NW < BM / RPI) dma16(rsrc_a, voff[j], kt * ROWB, dst);
      else dma16(rsrc_b, voff[j], kt * ROWB, dst);
    }
    if constexpr (Op::SCALED) {
      dma4(rsrc_sa, scale_voff, kt * SCALE_ROW, stage + DATA + wave * 256);
      dma4(rsrc_sb, scale_voff, kt * SCALE_ROW, stage + DATA + BM * SCALE_ROW + wave * 256);
    }
  };

  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int lrow = lane & 31, lgroup = lane >> 5;
  typename Op::Acc acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = typename Op::Acc{};

  // Fragment of LDS row `row` for substep ks: LANE_BYTES from logical chunks
  // ks*KB/16 + lgroup*PIECES + p.
  auto read = [&](const uint8_t* stage, int row, int ks) {
    i32x4 parts[PIECES];
#pragma unroll
    for (int p = 0; p < PIECES; ++p) {
      const int c = ks * (KB / 16) + lgroup * PIECES + p;
      parts[p] = *reinterpret_cast<const i32x4*>(stage + row * ROWB + ((c ^ ((row / RPB) % CPR)) * 16));
    }
    if constexpr (PIECES == 1) {
      return __builtin_bit_cast(typename Op::Frag, parts[0]);
    } else {
      return typename Op::Frag{parts[0][0], parts[0][1], parts[0][2], parts[0][3],
                               parts[1][0], parts[1][1], parts[1][2], parts[1][3]};
    }
  };

  issue(0);
  for (int kt = 0; kt < k_steps; ++kt) {
    // Step kt's DMA is complete for this wave; the barrier makes every wave's
    // part visible and ends all reads of the other stage, which the next DMA
    // then overwrites.
    wait_all_dma();
    __syncthreads();
    if (kt + 1 < k_steps) issue(kt + 1);
    const uint8_t* stage = lds + (kt & 1) * STAGE;
    // MXFP4: a lane's scale for substep ks is group 2*ks + lgroup of its row;
    // after shifting the row's 8 bytes by 8*lgroup, it is byte 2*ks, i.e. byte
    // 0 of the value shifted by 16*ks (the instruction reads byte 0).
    uint64_t srow_a[TM], srow_b[TN];
    if constexpr (Op::SCALED) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
        srow_a[i] = *reinterpret_cast<const uint64_t*>(stage + DATA + (wm * WM + i * 32 + lrow) * SCALE_ROW) >>
                    (8 * lgroup);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        srow_b[j] = *reinterpret_cast<const uint64_t*>(stage + DATA + (BM + wn * WN + j * 32 + lrow) * SCALE_ROW) >>
                    (8 * lgroup);
    }
    typename Op::Frag fa[2][TM], fb[2][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) fa[0][i] = read(stage, wm * WM + i * 32 + lrow, 0);
#pragma unroll
    for (int j = 0; j < TN; ++j) fb[0][j] = read(stage, BM + wn * WN + j * 32 + lrow, 0);
#pragma unroll
    for (int ks = 0; ks < KSTEPS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KSTEPS) {
#pragma unroll
        for (int i = 0; i < TM; ++i) fa[cur ^ 1][i] = read(stage, wm * WM + i * 32 + lrow, ks + 1);
#pragma unroll
        for (int j = 0; j < TN; ++j) fb[cur ^ 1][j] = read(stage, BM + wn * WN + j * 32 + lrow, ks + 1);
      }
      // Keep the next substep's reads ahead of this substep's MFMAs.
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          int scale_a = 0, scale_b = 0;
          if constexpr (Op::SCALED) {
            scale_a = static_cast<int>(srow_a[i] >> (16 * ks));
            scale_b = static_cast<int>(srow_b[j] >> (16 * ks));
          }
          acc[i][j] = Op::mma(fa[cur][i], fb[cur][j], acc[i][j], scale_a, scale_b);
        }
      __builtin_amdgcn_sched_barrier(0);
    }
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < Op::ACC_REGS; ++r) {
        const int row = m0 + wm * WM + i * 32 + Op::out_row(lane, r);
        const int col = n0 + wn * WN + j * 32 + lrow;
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

template <class Op, int ROWB, int WM, int WN>
void launch_gemm_dma(const uint8_t* a, const uint8_t* b, const uint8_t* sa, const uint8_t* sb, void* c, int m, int n,
                     int k, int group_m, hipStream_t stream) {
  gemm_dma_kernel<Op, ROWB, WM, WN><<<dim3(tile_count(m, n, 256, 256)), dim3(64 * WM * WN), 0, stream>>>(
      a, b, sa, sb, static_cast<typename Op::Out*>(c), m, n, k, group_m);
}

// launch: shapes that divide the tile (nullptr: none, use launch_checked);
// launch_checked: any shape. dma_row_bytes > 0 marks a DMA kernel, whose K
// step is that many bytes and whose operand offsets must fit in 31 bits.
struct GemmVariant {
  int format;
  mb_gemm_config config;
  const char* name;
  const void* kernel;
  GemmLauncher launch;
  GemmLauncher launch_checked;
  int out_bytes;
  int elem_bits;
  int dma_row_bytes;
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
              0}

// 256x256 tile: the DMA kernel (8 waves, 128-byte K steps) for exact shapes,
// a checked LDS-staged kernel (tile CM x CN) for ragged ones.
#define MB_GEMM_DMA(FMT, OP, BK, CM, CN, NAME)                                                               \
  GemmVariant{FMT,                                                                                           \
              mb_gemm_config{256, 256, BK, 512},                                                             \
              NAME,                                                                                          \
              reinterpret_cast<const void*>(gemm_dma_kernel<OP, 128, 2, 4>),                                 \
              launch_gemm_dma<OP, 128, 2, 4>,                                                                \
              launch_gemm<OP, CM, CN, BK, 2, 2, true>,                                                       \
              static_cast<int>(sizeof(typename OP::Out)),                                                    \
              OP::ELEM_BITS,                                                                                 \
              128}

const GemmVariant kGemmVariants[] = {
    MB_GEMM_DMA(MB_MATRIX_BF16, MfmaBf16, 64, 256, 256, "gemm_bf16_256x256x64"),
    MB_GEMM(MB_MATRIX_BF16, MfmaBf16, 256, 128, 64, 2, 2, "gemm_bf16_256x128x64"),
    MB_GEMM(MB_MATRIX_BF16, MfmaBf16, 128, 128, 64, 2, 2, "gemm_bf16_128x128x64"),
    MB_GEMM_DMA(MB_MATRIX_F16, MfmaF16, 64, 256, 256, "gemm_f16_256x256x64"),
    MB_GEMM(MB_MATRIX_F16, MfmaF16, 256, 128, 64, 2, 2, "gemm_f16_256x128x64"),
    MB_GEMM(MB_MATRIX_F16, MfmaF16, 128, 128, 64, 2, 2, "gemm_f16_128x128x64"),
    MB_GEMM_DMA(MB_MATRIX_FP8_E4M3, MfmaFp8, 128, 256, 256, "gemm_fp8_256x256x128"),
    MB_GEMM(MB_MATRIX_FP8_E4M3, MfmaFp8, 256, 128, 128, 2, 2, "gemm_fp8_256x128x128"),
    MB_GEMM(MB_MATRIX_FP8_E4M3, MfmaFp8, 128, 128, 128, 2, 2, "gemm_fp8_128x128x128"),
    MB_GEMM_DMA(MB_MATRIX_I8, MfmaI8, 128, 256, 256, "gemm_i8_256x256x128"),
    MB_GEMM(MB_MATRIX_I8, MfmaI8, 256, 128, 128, 2, 2, "gemm_i8_256x128x128"),
    MB_GEMM(MB_MATRIX_I8, MfmaI8, 128, 128, 128, 2, 2, "gemm_i8_128x128x128"),
    MB_GEMM_DMA(MB_MATRIX_MXFP4, MfmaMxfp4, 256, 128, 128, "gemm_mxfp4_256x256x256"),
    MB_GEMM(MB_MATRIX_MXFP4, MfmaMxfp4, 256, 128, 256, 2, 2, "gemm_mxfp4_256x128x256"),
    MB_GEMM(MB_MATRIX_MXFP4, MfmaMxfp4, 128, 128, 256, 2, 2, "gemm_mxfp4_128x128x256"),
    MB_GEMM(MB_MATRIX_F64, MfmaF64, 128, 128, 16, 2, 2, "gemm_f64_128x128x16"),
    MB_GEMM(MB_MATRIX_F64, MfmaF64, 64, 64, 16, 2, 2, "gemm_f64_64x64x16"),
    MB_GEMM(MB_MATRIX_F32, MfmaF32, 128, 128, 32, 2, 2, "gemm_f32_128x128x32"),
};

struct GemmRegistrar {
  GemmRegistrar() {
    for (const auto& variant : kGemmVariants) register_kernel(variant.name, variant.kernel);
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
  if (int rc = matrix_format_check(format, "mb_gemm")) return rc;
  if (config == nullptr) return fail(MB_ERR_INVALID, "mb_gemm: config is NULL");
  const GemmVariant* variant = find_gemm(format, config);
  if (variant == nullptr)
    return fail(MB_ERR_INVALID, "mb_gemm: no kernel for format %d with tile %ux%ux%u (see mb_gemm_configs)", format,
                config->tile_m, config->tile_n, config->tile_k);
  if (m == 0 || n == 0 || k == 0) return fail(MB_ERR_INVALID, "mb_gemm: empty problem %ux%ux%u", m, n, k);
  if (m > 0x7fffffffu || n > 0x7fffffffu || k > 0x7fffffffu)
    return fail(MB_ERR_INVALID, "mb_gemm: dimensions exceed 2^31-1");
  if (format == MB_MATRIX_MXFP4 && k % 32)
    return fail(MB_ERR_INVALID, "mb_gemm: MXFP4 needs K to be a multiple of the 32-element scale group");
  const uint64_t row_bits = static_cast<uint64_t>(k) * variant->elem_bits;
  if (row_bits % 128)
    return fail(MB_ERR_INVALID, "mb_gemm: K*element size must be a multiple of 16 bytes (rows are 16-byte loads)");
  const uint64_t row_bytes = row_bits / 8;
  if (a == nullptr || b == nullptr || c == nullptr) return fail(MB_ERR_INVALID, "mb_gemm: NULL operand");
  if (a_bytes < m * row_bytes || b_bytes < n * row_bytes ||
      c_bytes < static_cast<uint64_t>(m) * n * variant->out_bytes)
    return fail(MB_ERR_INVALID, "mb_gemm: buffers too small for %ux%ux%u", m, n, k);
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16))
    return fail(MB_ERR_ALIGNMENT, "mb_gemm: A, B and C must be 16-byte aligned");
  if (format == MB_MATRIX_MXFP4) {
    if (scale_a == nullptr || scale_b == nullptr)
      return fail(MB_ERR_INVALID, "mb_gemm: MXFP4 needs E8M0 scales for A and B");
    if (scale_a_bytes < static_cast<uint64_t>(m) * (k / 32) || scale_b_bytes < static_cast<uint64_t>(n) * (k / 32))
      return fail(MB_ERR_INVALID, "mb_gemm: scale buffers too small ([M|N][K/32] bytes needed)");
  }
  const mb_gemm_config& v = variant->config;
  const bool exact = m % v.tile_m == 0 && n % v.tile_n == 0 && k % v.tile_k == 0;
  // The DMA kernel addresses each tile's 256 operand rows with 32-bit offsets.
  // Its scale rows are moved 4 bytes per lane, so they must be 4-byte aligned.
  const bool offsets_fit =
      variant->dma_row_bytes == 0 ||
      (row_bytes % variant->dma_row_bytes == 0 && 256 * row_bytes <= 0x7fffffffull &&
       (format != MB_MATRIX_MXFP4 || (aligned(scale_a, 4) && aligned(scale_b, 4))));
  // The tile count of the smallest tile any launcher uses bounds the grid.
  const uint64_t max_tiles = static_cast<uint64_t>((m + 63) / 64) * ((n + 63) / 64);
  if (max_tiles > 0x7fffffffull) return fail(MB_ERR_INVALID, "mb_gemm: too many tiles");
  const int group = group_m ? static_cast<int>(group_m) : 8;
  GemmLauncher launch = exact && offsets_fit ? variant->launch : variant->launch_checked;
  launch(static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(b), static_cast<const uint8_t*>(scale_a),
         static_cast<const uint8_t*>(scale_b), c, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), group,
         static_cast<hipStream_t>(stream));
  return launch_status(variant->name);
}

}  // extern "C"
