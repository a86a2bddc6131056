// Resident-operand matrix peak (tensor_* rows).
//
// Semantics follow the reference's _tensor_peak_kernel / _tensor_peak_scaled_kernel
// (bench_tensor.py:406-488): workgroup `block` owns A[block] (BM x BK), one
// B[c][block] (BK x BN) per independent accumulator chain c, and writes
// C[c][block] = iterations * (A . B_c) accumulated in the instruction's
// accumulator type. Operands are read from HBM once per workgroup.
//
// MI355X design: the workgroup stages its tiles into LDS with 16-byte
// coalesced loads, every wave then gathers its MFMA operand fragments from LDS
// into registers, and the timed loop issues nothing but v_mfma instructions
// over CHAINS x TM x TN independent accumulators, enough to cover the MFMA
// dependency latency. Tiles are sized so that fragments plus accumulators fit
// the 512-register budget of one wave per SIMD without spilling.
//
// This header holds the kernel template and the variant record; the variant
// tables live in mb_tensor_peak.hip and mb_tensor_peak_vgpr.hip, which are
// compiled with different register-allocation options.
#pragma once

#include "mb_internal.h"
#include "mb_mfma.h"

namespace mb {

using PeakLauncher = void (*)(const uint8_t*, const uint8_t*, const uint8_t*, const uint8_t*, void*, uint32_t,
                              uint32_t, hipStream_t);

struct PeakVariant {
  int format;
  mb_peak_config config;
  const char* name;
  const void* kernel;
  PeakLauncher launch;
  int out_bytes;
  int elem_bits;
};

// Variants compiled in mb_tensor_peak_vgpr.hip (tiles whose fragments and
// accumulators fit the 256 architectural VGPRs, built with the VGPR form of
// v_mfma so no accumulator is copied between register files in the loop).
const PeakVariant* vgpr_form_peak_variants(int* count);

namespace {


template <class Op, int BM, int BN, int BK, int WAVES_M, int WAVES_N, int CHAINS, bool B_NK>
struct PeakTile {
  static constexpr int THREADS = 64 * WAVES_M * WAVES_N;
  static constexpr int BK_BYTES = BK * Op::ELEM_BITS / 8;
  static constexpr int A_BYTES = BM * BK_BYTES;
  static constexpr int B_BYTES = BK_BYTES * BN;
  static constexpr int WM = BM / WAVES_M;
  static constexpr int WN = BN / WAVES_N;
  static constexpr int TM = WM / Op::M;
  static constexpr int TN = WN / Op::N;
  static constexpr int KSTEPS = BK_BYTES / MfmaGeometry<Op>::K_BYTES;
  static constexpr int ELEM_BYTES = Op::ELEM_BITS >= 8 ? Op::ELEM_BITS / 8 : 1;
  static constexpr int GROUPS = Op::SCALED ? BK / 32 : 0;  // E8M0 scales per row
  static_assert(WM % Op::M == 0 && WN % Op::N == 0, "wave tile must hold whole instructions");
  static_assert(BK_BYTES % MfmaGeometry<Op>::K_BYTES == 0, "BK must hold whole instructions");
  static_assert(A_BYTES % 16 == 0 && B_BYTES % 16 == 0, "tiles are staged in 16-byte vectors");
};

// Gather one B fragment for column `col` when B is stored K-major ([BK][BN],
// N contiguous): LANE_BYTES bytes of K, ELEM_BYTES at a time.
template <class Op, int ELEM_BYTES, int BN>
__device__ __forceinline__ typename Op::Frag gather_b(const uint8_t* tile, int col, int kbyte) {
  union {
    typename Op::Frag frag;
    uint8_t bytes[Op::LANE_BYTES];
  } out;
#pragma unroll
  for (int i = 0; i < Op::LANE_BYTES; i += ELEM_BYTES) {
    const int row = (kbyte + i) / ELEM_BYTES;
#pragma unroll
    for (int e = 0; e < ELEM_BYTES; ++e) out.bytes[i + e] = tile[(row * BN + col) * ELEM_BYTES + e];
  }
  return out.frag;
}

template <class Op, int BM, int BN, int BK, int WAVES_M, int WAVES_N, int CHAINS, bool B_NK>
__global__ void __launch_bounds__(64 * WAVES_M * WAVES_N)
    tensor_peak_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                       const uint8_t* __restrict__ SA, const uint8_t* __restrict__ SB,
                       typename Op::Out* __restrict__ C, uint32_t blocks, uint32_t iterations) {
  using T = PeakTile<Op, BM, BN, BK, WAVES_M, WAVES_N, CHAINS, B_NK>;
  __shared__ __attribute__((aligned(16))) uint8_t lds[T::A_BYTES + CHAINS * T::B_BYTES];
  const uint64_t block = blockIdx.x;

  // Stage A[block] and every B[c][block] into LDS with 16-byte loads.
  const uint8_t* a_src = A + block * T::A_BYTES;
  for (int i = threadIdx.x * 16; i < T::A_BYTES; i += T::THREADS * 16)
    *reinterpret_cast<i32x4*>(lds + i) = *reinterpret_cast<const i32x4*>(a_src + i);
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) {
    const uint8_t* b_src = B + (static_cast<uint64_t>(c) * blocks + block) * T::B_BYTES;
    uint8_t* b_dst = lds + T::A_BYTES + c * T::B_BYTES;
    for (int i = threadIdx.x * 16; i < T::B_BYTES; i += T::THREADS * 16)
      *reinterpret_cast<i32x4*>(b_dst + i) = *reinterpret_cast<const i32x4*>(b_src + i);
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int lrow = lane % Op::M, lgroup = lane / Op::M;
  constexpr int KB = MfmaGeometry<Op>::K_BYTES;

  typename Op::Frag a[T::TM][T::KSTEPS];
  typename Op::Frag b[CHAINS][T::TN][T::KSTEPS];
#pragma unroll
  for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
    for (int ks = 0; ks < T::KSTEPS; ++ks) {
      const int row = wm * T::WM + tm * Op::M + lrow;
      a[tm][ks] = load_frag<typename Op::Frag>(lds + row * T::BK_BYTES + ks * KB + lgroup * Op::LANE_BYTES);
    }
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
      for (int ks = 0; ks < T::KSTEPS; ++ks) {
        const int col = wn * T::WN + tn * Op::N + lrow;
        const int kbyte = ks * KB + lgroup * Op::LANE_BYTES;
        const uint8_t* tile = lds + T::A_BYTES + c * T::B_BYTES;
        if constexpr (B_NK) {
          b[c][tn][ks] = load_frag<typename Op::Frag>(tile + col * T::BK_BYTES + kbyte);
        } else {
          b[c][tn][ks] = gather_b<Op, T::ELEM_BYTES, BN>(tile, col, kbyte);
        }
      }

  // E8M0 scales: every lane group covers 32 K elements, so lane (row, group) of
  // k-step ks uses scale column ks * LANE_GROUPS + group.
  int sa[T::TM][T::KSTEPS > 0 ? T::KSTEPS : 1] = {};
  int sb[T::TN][T::KSTEPS > 0 ? T::KSTEPS : 1] = {};
  if constexpr (Op::SCALED) {
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
      for (int ks = 0; ks < T::KSTEPS; ++ks) {
        const int row = wm * T::WM + tm * Op::M + lrow;
        sa[tm][ks] = SA[(block * BM + row) * T::GROUPS + ks * MfmaGeometry<Op>::LANE_GROUPS + lgroup];
      }
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
      for (int ks = 0; ks < T::KSTEPS; ++ks) {
        const int col = wn * T::WN + tn * Op::N + lrow;
        sb[tn][ks] = SB[(block * BN + col) * T::GROUPS + ks * MfmaGeometry<Op>::LANE_GROUPS + lgroup];
      }
  }

  typename Op::Acc acc[CHAINS][T::TM][T::TN];
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn) acc[c][tm][tn] = typename Op::Acc{};

  for (uint32_t it = 0; it < iterations; ++it) {
#pragma unroll
    for (int ks = 0; ks < T::KSTEPS; ++ks)
#pragma unroll
      for (int c = 0; c < CHAINS; ++c)
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < T::TN; ++tn)
            acc[c][tm][tn] = Op::mma(a[tm][ks], b[c][tn][ks], acc[c][tm][tn], sa[tm][ks], sb[tn][ks]);
  }

#pragma unroll
  for (int c = 0; c < CHAINS; ++c) {
    typename Op::Out* out = C + (static_cast<uint64_t>(c) * blocks + block) * BM * BN;
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
        for (int r = 0; r < Op::ACC_REGS; ++r) {
          const int row = wm * T::WM + tm * Op::M + Op::out_row(lane, r);
          const int col = wn * T::WN + tn * Op::N + (lane % Op::N);
          out[row * BN + col] = acc[c][tm][tn][r];
        }
  }
}

// The same computation with the 16x16 instructions issued in place
// (Op::mma_tied) on AGPR accumulators, for tiles whose 16x16 accumulators
// fill the AGPR file (256x256 per four waves: 256 registers per lane). The
// builtin forms of these instructions get accumulator copies (and spills) at
// that size, so the compiler cannot be left to allocate them.
//
// The compiler does not see the inline-assembly MFMAs, so the kernel keeps
// their hazard distances itself:
//   * every operand fragment is a plain LDS read (ds_read_b128), whose waits
//     the compiler inserts for any reader; B is therefore stored transposed
//     in LDS ([BN][BK] bytes) whatever its layout in HBM;
//   * consecutive updates of one accumulator are MFMAs writing exactly the
//     same registers, which the hardware orders;
//   * ordered fences on every accumulator (acc_hazard_fence) separate the
//     zeroing from the first MFMA and the last MFMA from the stores.
// Unscaled formats only (the scaled MXFP4 instruction takes its scales in
// VGPRs, which this kernel does not stage).
template <class Op, int BM, int BN, int BK, int WAVES_M, int WAVES_N, int CHAINS, bool B_NK>
__global__ void __launch_bounds__(64 * WAVES_M * WAVES_N)
    tensor_peak_tied_kernel(const uint8_t* __restrict__ A, const uint8_t* __restrict__ B,
                            const uint8_t* __restrict__, const uint8_t* __restrict__,
                            typename Op::Out* __restrict__ C, uint32_t blocks, uint32_t iterations) {
  using T = PeakTile<Op, BM, BN, BK, WAVES_M, WAVES_N, CHAINS, B_NK>;
  static_assert(Op::M == 16 && !Op::SCALED, "in-place tiles use the unscaled 16x16 instructions");
  static_assert(T::ELEM_BYTES == 1 || T::ELEM_BYTES == 2, "B is transposed in LDS element by element");
  __shared__ __attribute__((aligned(16))) uint8_t lds[T::A_BYTES + CHAINS * T::B_BYTES];
  const uint64_t block = blockIdx.x;

  typename Op::Acc acc[CHAINS][T::TM][T::TN];
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn) acc[c][tm][tn] = typename Op::Acc{};

  // Stage A[block] as it is, and every B[c][block] as [BN][BK] bytes.
  const uint8_t* a_src = A + block * T::A_BYTES;
  for (int i = threadIdx.x * 16; i < T::A_BYTES; i += T::THREADS * 16)
    *reinterpret_cast<i32x4*>(lds + i) = *reinterpret_cast<const i32x4*>(a_src + i);
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) {
    const uint8_t* b_src = B + (static_cast<uint64_t>(c) * blocks + block) * T::B_BYTES;
    uint8_t* b_dst = lds + T::A_BYTES + c * T::B_BYTES;
    for (int i = threadIdx.x * 16; i < T::B_BYTES; i += T::THREADS * 16) {
      const i32x4 v = *reinterpret_cast<const i32x4*>(b_src + i);
      if constexpr (B_NK) {
        *reinterpret_cast<i32x4*>(b_dst + i) = v;
      } else {
        // Byte offset i of [BK][BN] holds element (k, n) = (i / row, (i % row) / ELEM_BYTES)
        // with row = BN * ELEM_BYTES; it goes to (n * BK + k) * ELEM_BYTES.
        constexpr int E = T::ELEM_BYTES, ROW = BN * E, PER = 16 / E;
        const int k = i / ROW, n0 = (i % ROW) / E;
        if constexpr (E == 2) {
          const auto h = __builtin_bit_cast(uint16_t __attribute__((ext_vector_type(8))), v);
#pragma unroll
          for (int e = 0; e < PER; ++e) *reinterpret_cast<uint16_t*>(b_dst + ((n0 + e) * BK + k) * E) = h[e];
        } else {
          const auto h = __builtin_bit_cast(uint8_t __attribute__((ext_vector_type(16))), v);
#pragma unroll
          for (int e = 0; e < PER; ++e) b_dst[(n0 + e) * BK + k] = h[e];
        }
      }
    }
  }
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave % WAVES_M, wn = wave / WAVES_M;
  const int lrow = lane % Op::M, lgroup = lane / Op::M;
  constexpr int KB = MfmaGeometry<Op>::K_BYTES;

  typename Op::Frag a[T::TM][T::KSTEPS];
  typename Op::Frag b[CHAINS][T::TN][T::KSTEPS];
#pragma unroll
  for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
    for (int ks = 0; ks < T::KSTEPS; ++ks) {
      const int row = wm * T::WM + tm * Op::M + lrow;
      a[tm][ks] = load_frag<typename Op::Frag>(lds + row * T::BK_BYTES + ks * KB + lgroup * Op::LANE_BYTES);
    }
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
      for (int ks = 0; ks < T::KSTEPS; ++ks) {
        const int col = wn * T::WN + tn * Op::N + lrow;
        b[c][tn][ks] = load_frag<typename Op::Frag>(lds + T::A_BYTES + c * T::B_BYTES + col * T::BK_BYTES +
                                                    ks * KB + lgroup * Op::LANE_BYTES);
      }
  // lgkmcnt(0) (vmcnt and expcnt fields at their maxima): every fragment is in
  // its registers before the loop, so no wait is left inside it.
  __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn) acc_hazard_fence(acc[c][tm][tn]);

  for (uint32_t it = 0; it < iterations; ++it) {
#pragma unroll
    for (int ks = 0; ks < T::KSTEPS; ++ks)
#pragma unroll
      for (int c = 0; c < CHAINS; ++c)
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
          for (int tn = 0; tn < T::TN; ++tn) Op::mma_tied(a[tm][ks], b[c][tn][ks], acc[c][tm][tn]);
  }
#pragma unroll
  for (int c = 0; c < CHAINS; ++c)
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn) acc_hazard_fence(acc[c][tm][tn]);

#pragma unroll
  for (int c = 0; c < CHAINS; ++c) {
    typename Op::Out* out = C + (static_cast<uint64_t>(c) * blocks + block) * BM * BN;
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
      for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
        for (int r = 0; r < Op::ACC_REGS; ++r) {
          const int row = wm * T::WM + tm * Op::M + Op::out_row(lane, r);
          const int col = wn * T::WN + tn * Op::N + (lane % Op::N);
          out[row * BN + col] = acc[c][tm][tn][r];
        }
  }
}

template <class Op, int BM, int BN, int BK, int WAVES_M, int WAVES_N, int CHAINS, bool B_NK>
void launch_peak(const uint8_t* a, const uint8_t* b, const uint8_t* sa, const uint8_t* sb, void* c,
                 uint32_t blocks, uint32_t iterations, hipStream_t stream) {
  tensor_peak_kernel<Op, BM, BN, BK, WAVES_M, WAVES_N, CHAINS, B_NK>
      <<<dim3(blocks), dim3(64 * WAVES_M * WAVES_N), 0, stream>>>(
          a, b, sa, sb, static_cast<typename Op::Out*>(c), blocks, iterations);
}

template <class Op, int BM, int BN, int BK, int WAVES_M, int WAVES_N, int CHAINS, bool B_NK>
void launch_peak_tied(const uint8_t* a, const uint8_t* b, const uint8_t* sa, const uint8_t* sb, void* c,
                      uint32_t blocks, uint32_t iterations, hipStream_t stream) {
  tensor_peak_tied_kernel<Op, BM, BN, BK, WAVES_M, WAVES_N, CHAINS, B_NK>
      <<<dim3(blocks), dim3(64 * WAVES_M * WAVES_N), 0, stream>>>(
          a, b, sa, sb, static_cast<typename Op::Out*>(c), blocks, iterations);
}

}  // namespace
}  // namespace mb

#define MB_PEAK(FMT, OP, BM, BN, BK, WM, WN, CH, NK, NAME)                                                   \
  PeakVariant{FMT,                                                                                           \
              mb_peak_config{BM, BN, BK, CH, NK, OP::M, 64 * WM * WN},                                           \
              NAME,                                                                                          \
              reinterpret_cast<const void*>(tensor_peak_kernel<OP, BM, BN, BK, WM, WN, CH, NK>),             \
              launch_peak<OP, BM, BN, BK, WM, WN, CH, NK>,                                                   \
              static_cast<int>(sizeof(typename OP::Out)),                                                    \
              OP::ELEM_BITS}

// Both B layouts of every tile: [BK][BN] (the reference's default) and
// [BN][BK] (its b_transposed variant, bench_tensor.py:421-424).
#define MB_PEAK_BOTH(FMT, OP, BM, BN, BK, WM, WN, CH, NAME)             \
  MB_PEAK(FMT, OP, BM, BN, BK, WM, WN, CH, false, NAME "_kn"),          \
      MB_PEAK(FMT, OP, BM, BN, BK, WM, WN, CH, true, NAME "_nk")

// In-place (tensor_peak_tied_kernel) variants, both B layouts.
#define MB_PEAK_TIED(FMT, OP, BM, BN, BK, WM, WN, CH, NK, NAME)                                              \
  PeakVariant{FMT,                                                                                           \
              mb_peak_config{BM, BN, BK, CH, NK, OP::M, 64 * WM * WN},                                       \
              NAME,                                                                                          \
              reinterpret_cast<const void*>(tensor_peak_tied_kernel<OP, BM, BN, BK, WM, WN, CH, NK>),        \
              launch_peak_tied<OP, BM, BN, BK, WM, WN, CH, NK>,                                              \
              static_cast<int>(sizeof(typename OP::Out)),                                                    \
              OP::ELEM_BITS}
#define MB_PEAK_TIED_BOTH(FMT, OP, BM, BN, BK, WM, WN, CH, NAME)        \
  MB_PEAK_TIED(FMT, OP, BM, BN, BK, WM, WN, CH, false, NAME "_kn"),     \
      MB_PEAK_TIED(FMT, OP, BM, BN, BK, WM, WN, CH, true, NAME "_nk")

