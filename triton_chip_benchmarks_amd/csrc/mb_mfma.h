// gfx950 matrix-core (MFMA) instruction traits shared by the resident-peak and
// GEMM kernels.
//
// Every trait describes one v_mfma instruction as a wave64 operation on an
// M x N output tile with K reduction elements:
//   * operand fragments: lane l holds LANE_BYTES contiguous bytes of K for
//     row/column (l % M) of A/B, at K byte offset (l / M) * LANE_BYTES within
//     the instruction's K_BYTES = (64 / M) * LANE_BYTES;
//   * accumulator: ACC_REGS values per lane; out_row/out_col give the output
//     element each accumulator register of each lane holds.
// Storage sizes are in bytes so packed formats (two E2M1 codes per byte) use
// the same tile arithmetic as byte-sized ones.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mb {

typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x8 __attribute__((ext_vector_type(8)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef double f64x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Output position of accumulator register r in lane l for a 32x32 tile
// (four row quads per register group of four) and a 16x16 tile.
__device__ __forceinline__ int out_row_32(int lane, int r) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }
__device__ __forceinline__ int out_row_16(int lane, int r) { return 4 * (lane >> 4) + r; }

// v_mfma_f32_32x32x16_bf16: 8 bf16 per lane, fp32 accumulate.
struct MfmaBf16 {
  static constexpr int M = 32, N = 32, K = 16, ELEM_BITS = 16, LANE_BYTES = 16, ACC_REGS = 16;
  static constexpr bool SCALED = false;
  using Frag = i32x4;
  using Acc = f32x16;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_32(lane, r); }
};

// v_mfma_f32_32x32x16_f16: 8 fp16 per lane, fp32 accumulate.
struct MfmaF16 {
  static constexpr int M = 32, N = 32, K = 16, ELEM_BITS = 16, LANE_BYTES = 16, ACC_REGS = 16;
  static constexpr bool SCALED = false;
  using Frag = i32x4;
  using Acc = f32x16;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_32(lane, r); }
};

// v_mfma_i32_32x32x32_i8: 16 int8 per lane, int32 accumulate.
struct MfmaI8 {
  static constexpr int M = 32, N = 32, K = 32, ELEM_BITS = 8, LANE_BYTES = 16, ACC_REGS = 16;
  static constexpr bool SCALED = false;
  using Frag = i32x4;
  using Acc = i32x16;
  using Out = int32_t;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_32(lane, r); }
};

// v_mfma_f32_32x32x64_f8f6f4 with both formats FP8 E4M3 (cbsz = blgp = 0):
// 32 fp8 per lane, fp32 accumulate, no block scales. The scaled builtin with
// zero scale operands selects the unscaled instruction.
struct MfmaFp8 {
  static constexpr int M = 32, N = 32, K = 64, ELEM_BITS = 8, LANE_BYTES = 32, ACC_REGS = 16;
  static constexpr bool SCALED = false;
  using Frag = i32x8;
  using Acc = f32x16;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_32(lane, r); }
};

// v_mfma_scale_f32_32x32x64_f8f6f4 with both formats FP4 E2M1 (cbsz = blgp =
// 4): 32 E2M1 codes (16 bytes, low nibble first) per lane; each lane also
// supplies the E8M0 scale of its 32-element K group (byte 0 of a VGPR).
struct MfmaMxfp4 {
  static constexpr int M = 32, N = 32, K = 64, ELEM_BITS = 4, LANE_BYTES = 16, ACC_REGS = 16;
  static constexpr bool SCALED = true;
  using Frag = i32x4;
  using Acc = f32x16;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int scale_a, int scale_b) {
    const i32x8 wa = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
    const i32x8 wb = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, wb, c, 4, 4, 0, scale_a, 0, scale_b);
  }
  // Scales from byte SEL of two dwords that hold one E8M0 scale per byte: the
  // instruction's op_sel picks the byte, so no shift is issued.
  template <int SEL>
  __device__ static __forceinline__ Acc mma_byte(Frag a, Frag b, Acc c, uint32_t scales_a, uint32_t scales_b) {
    const i32x8 wa = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
    const i32x8 wb = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wa, wb, c, 4, 4, SEL, static_cast<int>(scales_a), SEL,
                                                           static_cast<int>(scales_b));
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_32(lane, r); }
};

// 16x16 forms of the same instructions. Per flop they move a quarter of the
// accumulator bytes of the 32x32 forms and twice the operand bytes; the
// resident-peak tables carry both so the sweep measures which one the power
// limit favours. Lane groups are 64 / 16 = 4, so a lane's K slice is a quarter
// of the instruction's K.
//
// mma_tied accumulates in place in AGPRs through inline assembly: for the
// 16x16 forms with 16-byte operands (BF16, FP16, INT8, and FP4 as well)
// the compiler does not tie the accumulator input to the output, so a loop of
// them copies every accumulator per instruction (and at 256 accumulator
// registers spills). The compiler does not see these as MFMAs, so callers keep
// the hazard distances themselves: operands come straight from LDS loads
// (whose waits the compiler inserts for any reader), and acc_hazard_fence()
// separates the accumulators' VALU initialisation from the first MFMA and the
// last MFMA from the reads that follow.
struct MfmaBf16x16 {
  static constexpr int M = 16, N = 16, K = 32, ELEM_BITS = 16, LANE_BYTES = 16, ACC_REGS = 4;
  static constexpr bool SCALED = false;
  using Frag = i32x4;
  using Acc = f32x4;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                   c, 0, 0, 0);
  }
  __device__ static __forceinline__ void mma_tied(Frag a, Frag b, Acc& c) {
    asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_16(lane, r); }
};

struct MfmaF16x16 {
  static constexpr int M = 16, N = 16, K = 32, ELEM_BITS = 16, LANE_BYTES = 16, ACC_REGS = 4;
  static constexpr bool SCALED = false;
  using Frag = i32x4;
  using Acc = f32x4;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                  0, 0, 0);
  }
  __device__ static __forceinline__ void mma_tied(Frag a, Frag b, Acc& c) {
    asm("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_16(lane, r); }
};

struct MfmaI8x16 {
  static constexpr int M = 16, N = 16, K = 64, ELEM_BITS = 8, LANE_BYTES = 16, ACC_REGS = 4;
  static constexpr bool SCALED = false;
  using Frag = i32x4;
  using Acc = i32x4;
  using Out = int32_t;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ void mma_tied(Frag a, Frag b, Acc& c) {
    asm("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_16(lane, r); }
};

// The FP8 form's builtin is tied by the compiler, but the GEMM's rolled
// kernel (256 accumulators, every fragment refilled in place) still gets
// accumulator copies and spills from it; mma_tied keeps the accumulator in
// place there, under the same hazard rules as above.
struct MfmaFp8x16 {
  static constexpr int M = 16, N = 16, K = 128, ELEM_BITS = 8, LANE_BYTES = 32, ACC_REGS = 4;
  static constexpr bool SCALED = false;
  using Frag = i32x8;
  using Acc = f32x4;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
  __device__ static __forceinline__ void mma_tied(Frag a, Frag b, Acc& c) {
    asm("v_mfma_f32_16x16x128_f8f6f4 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_16(lane, r); }
};

struct MfmaMxfp4x16 {
  static constexpr int M = 16, N = 16, K = 128, ELEM_BITS = 4, LANE_BYTES = 16, ACC_REGS = 4;
  static constexpr bool SCALED = true;
  using Frag = i32x4;
  using Acc = f32x4;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int scale_a, int scale_b) {
    const i32x8 wa = {a[0], a[1], a[2], a[3], 0, 0, 0, 0};
    const i32x8 wb = {b[0], b[1], b[2], b[3], 0, 0, 0, 0};
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(wa, wb, c, 4, 4, 0, scale_a, 0, scale_b);
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_16(lane, r); }
};

// v_mfma_f32_32x32x2_f32: one fp32 per lane, IEEE fp32 multiply-accumulate.
struct MfmaF32 {
  static constexpr int M = 32, N = 32, K = 2, ELEM_BITS = 32, LANE_BYTES = 4, ACC_REGS = 16;
  static constexpr bool SCALED = false;
  using Frag = float;
  using Acc = f32x16;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_32(lane, r); }
};

// v_mfma_f32_16x16x4_f32: one fp32 per lane, IEEE fp32 multiply-accumulate
// (16x16 tile), for the GEMM's DMA kernel; in place like the 16x16 forms
// above (mma_tied).
struct MfmaF32x16 {
  static constexpr int M = 16, N = 16, K = 4, ELEM_BITS = 32, LANE_BYTES = 4, ACC_REGS = 4;
  static constexpr bool SCALED = false;
  using Frag = float;
  using Acc = f32x4;
  using Out = float;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
  __device__ static __forceinline__ void mma_tied(Frag a, Frag b, Acc& c) {
    asm("v_mfma_f32_16x16x4_f32 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  __device__ static __forceinline__ int out_row(int lane, int r) { return out_row_16(lane, r); }
};

// v_mfma_f64_16x16x4_f64: one fp64 per lane, fp64 accumulate (16x16 tile).
struct MfmaF64 {
  static constexpr int M = 16, N = 16, K = 4, ELEM_BITS = 64, LANE_BYTES = 8, ACC_REGS = 4;
  static constexpr bool SCALED = false;
  using Frag = double;
  using Acc = f64x4;
  using Out = double;
  __device__ static __forceinline__ Acc mma(Frag a, Frag b, Acc c, int, int) {
    return __builtin_amdgcn_mfma_f64_16x16x4f64(a, b, c, 0, 0, 0);
  }
  // In-place form for the GEMM's DMA kernel (256 accumulator registers), under
  // the hazard rules of the 16x16 forms' mma_tied.
  __device__ static __forceinline__ void mma_tied(Frag a, Frag b, Acc& c) {
    asm("v_mfma_f64_16x16x4_f64 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
  // The four fp64 results of a lane are strided by 4 rows (measured on gfx950
  // with a row/column-marked product), unlike the 16x16 fp32 forms.
  __device__ static __forceinline__ int out_row(int lane, int r) { return (lane >> 4) + 4 * r; }
};

// An ordered (volatile) no-op that takes acc as an in-place AGPR operand:
// called once per accumulator, in the order of their last writes, after the
// accumulator loop (and after initialisation), so that every accumulator is
// read only behind at least (number of fences issued before its own) wait
// states since the loop's last MFMA.
template <class Acc>
__device__ __forceinline__ void acc_hazard_fence(Acc& c) {
  asm volatile("s_nop 1" : "+a"(c));
}

template <class Op>
struct MfmaGeometry {
  static constexpr int LANE_GROUPS = 64 / Op::M;                     // lanes sharing a row, split over K
  static constexpr int K_BYTES = LANE_GROUPS * Op::LANE_BYTES;       // K bytes per instruction
  static constexpr int FLOPS = 2 * Op::M * Op::N * Op::K;            // multiply + add per instruction
};

// Load a fragment of Frag's size from 4-byte-aligned memory (LDS or global).
template <class Frag>
__device__ __forceinline__ Frag load_frag(const uint8_t* ptr) {
  return *reinterpret_cast<const Frag*>(ptr);
}

}  // namespace mb
