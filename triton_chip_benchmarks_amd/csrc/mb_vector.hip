// Register-resident vector arithmetic chains (vector_* rows).
//
// Semantics follow the reference's vector_fma_kernel (bench_vector.py:182-319):
// every lane (element i) loads eight independent states x_c = Input[c][i],
// applies the per-dtype update ITERATIONS times with loop-invariant
// coefficients read from memory (a = Coefficients[0], b_c = Coefficients[1+c]),
// and stores all eight states to Output[c][i], so no chain is dead code.
//
//   f32  x <- fma(x, a, b_c)                     v_fma_f32 (one rounding)
//   f64  x <- fma(x, a, b_c)                     v_fma_f64
//   f16  (x_2c, x_2c+1) <- pk_fma(x, a, b)       v_pk_fma_f16, two chains per VGPR
//   bf16 x <- bf16(a*x + b_c)                    v_dot2_f32_bf16 (bf16 products,
//        two chains per VGPR, one fp32 result    fp32 sum; the other product is
//        per chain rounded to bf16 in pairs       x_other * 0) + v_cvt_pk_bf16_f32
//   bf16 (promoted) x <- bf16(fma(f32(x), a, b_c))  v_fma_f32 + v_cvt_pk_bf16_f32
//   i8   x <- dot4(bytes(x), W) + b_c            v_dot4_i32_i8: the int32 state's
//        four signed bytes times the packed weights, plus an int32 bias
//        (the reference's DP4A feedback form, bench_vector.py:134-145).
//   fp8 / fp4 widened (not native arithmetic: gfx950 has no FP8/FP4 VALU math)
//        x <- narrow(fma(f32(x), a, b_c)) with the state kept in FP8 E4M3 or
//        FP4 E2M1, two chains per conversion: v_cvt_pk_f32_fp8 or
//        v_cvt_scalef32_pk_f32_fp4 (scale 1), two v_fma_f32, then
//        v_cvt_pk_fp8_f32 or v_cvt_scalef32_pk_fp4_f32 (the reference's Ascend C
//        "converted" rows, ascendc/src/bench_vector.asc:335-572).
// The dot instructions are written as inline assembly so the VOP3P form with a
// separate addend is issued (the compiler otherwise picks the accumulating
// VOP2 form and spends moves to set up its destination). One asm block holds a
// whole update of all chains in a fixed order, because a DOT result needs three
// wait states before a different VALU instruction, or the same DOT as source A/B,
// may read it, and the compiler cannot insert those waits inside inline asm:
//   dot4 block: chain c is rewritten 7 instructions after its previous write;
//   dot2 block: eight v_dot2 first, then four v_cvt_pk, so each conversion reads
//   results written at least 3 instructions earlier, and the next block's v_dot2
//   reads a converted state at least 3 instructions after its v_cvt_pk.
#include "mb_internal.h"

namespace mb {
namespace {

constexpr int CHAINS = 8;

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

// x_c <- dot4(bytes(x_c), W) + b_c for the eight chains.
__device__ __forceinline__ void dot4_update(int (&x)[CHAINS], int w, const int (&b)[CHAINS]) {
  asm("v_dot4_i32_i8 %0, %0, %8, %9\n\t"
      "v_dot4_i32_i8 %1, %1, %8, %10\n\t"
      "v_dot4_i32_i8 %2, %2, %8, %11\n\t"
      "v_dot4_i32_i8 %3, %3, %8, %12\n\t"
      "v_dot4_i32_i8 %4, %4, %8, %13\n\t"
      "v_dot4_i32_i8 %5, %5, %8, %14\n\t"
      "v_dot4_i32_i8 %6, %6, %8, %15\n\t"
      "v_dot4_i32_i8 %7, %7, %8, %16"
      : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]), "+v"(x[4]), "+v"(x[5]), "+v"(x[6]), "+v"(x[7])
      : "v"(w), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(b[4]), "v"(b[5]), "v"(b[6]), "v"(b[7]));
}

// Four bf16 pairs: lo <- bf16(a*lo + b_2p), hi <- bf16(a*hi + b_2p+1), with
// w_lo = (a, 0) and w_hi = (0, a) selecting one product of each v_dot2.
__device__ __forceinline__ void dot2_update(uint32_t (&x)[CHAINS / 2], uint32_t w_lo, uint32_t w_hi,
                                            const float (&b)[CHAINS]) {
  float t0, t1, t2, t3, t4, t5, t6, t7;
  asm("v_dot2_f32_bf16 %0, %8, %12, %14\n\t"
      "v_dot2_f32_bf16 %1, %8, %13, %15\n\t"
      "v_dot2_f32_bf16 %2, %9, %12, %16\n\t"
      "v_dot2_f32_bf16 %3, %9, %13, %17\n\t"
      "v_dot2_f32_bf16 %4, %10, %12, %18\n\t"
      "v_dot2_f32_bf16 %5, %10, %13, %19\n\t"
      "v_dot2_f32_bf16 %6, %11, %12, %20\n\t"
      "v_dot2_f32_bf16 %7, %11, %13, %21\n\t"
      "v_cvt_pk_bf16_f32 %8, %0, %1\n\t"
      "v_cvt_pk_bf16_f32 %9, %2, %3\n\t"
      "v_cvt_pk_bf16_f32 %10, %4, %5\n\t"
      "v_cvt_pk_bf16_f32 %11, %6, %7"
      : "=&v"(t0), "=&v"(t1), "=&v"(t2), "=&v"(t3), "=&v"(t4), "=&v"(t5), "=&v"(t6), "=&v"(t7),
        "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3])
      : "v"(w_lo), "v"(w_hi), "v"(b[0]), "v"(b[1]), "v"(b[2]), "v"(b[3]), "v"(b[4]), "v"(b[5]), "v"(b[6]),
        "v"(b[7]));
}

// Three wait states between the last asm DOT/VALU writes and the stores that read them.
__device__ __forceinline__ void drain_valu_results() { asm volatile("s_nop 3"); }

__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  uint32_t out;
  asm("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(out) : "v"(lo), "v"(hi));
  return out;
}

__device__ __forceinline__ float bf16_lo(uint32_t packed) { return __uint_as_float(packed << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t packed) { return __uint_as_float(packed & 0xffff0000u); }

// One element per thread; UNROLL updates of all chains per loop trip.
template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_f32_kernel(const float* __restrict__ in, float* __restrict__ out,
                                                           const float* __restrict__ coeff, uint64_t elements,
                                                           uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  float x[CHAINS], b[CHAINS];
  const float a = coeff[0];
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) {
    x[c] = in[c * elements + i];
    b[c] = coeff[1 + c];
  }
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int c = 0; c < CHAINS; ++c) x[c] = __builtin_fmaf(x[c], a, b[c]);
  }
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) out[c * elements + i] = x[c];
}

template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_f64_kernel(const double* __restrict__ in, double* __restrict__ out,
                                                           const double* __restrict__ coeff, uint64_t elements,
                                                           uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  double x[CHAINS], b[CHAINS];
  const double a = coeff[0];
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) {
    x[c] = in[c * elements + i];
    b[c] = coeff[1 + c];
  }
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int c = 0; c < CHAINS; ++c) x[c] = __builtin_fma(x[c], a, b[c]);
  }
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) out[c * elements + i] = x[c];
}

template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_f16_kernel(const _Float16* __restrict__ in, _Float16* __restrict__ out,
                                                           const _Float16* __restrict__ coeff, uint64_t elements,
                                                           uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  f16x2 x[CHAINS / 2], b[CHAINS / 2];
  const f16x2 a = {coeff[0], coeff[0]};
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    x[p] = f16x2{in[(2 * p) * elements + i], in[(2 * p + 1) * elements + i]};
    b[p] = f16x2{coeff[1 + 2 * p], coeff[2 + 2 * p]};
  }
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int p = 0; p < CHAINS / 2; ++p) x[p] = __builtin_elementwise_fma(x[p], a, b[p]);
  }
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    out[(2 * p) * elements + i] = x[p][0];
    out[(2 * p + 1) * elements + i] = x[p][1];
  }
}

// bf16 bit patterns travel as uint16_t.
template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_bf16dot_kernel(const uint16_t* __restrict__ in,
                                                               uint16_t* __restrict__ out,
                                                               const uint16_t* __restrict__ coeff,
                                                               uint64_t elements, uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const uint32_t a = coeff[0];
  const uint32_t w_lo = a;         // (a, 0): a * x_lo + 0 * x_hi
  const uint32_t w_hi = a << 16;   // (0, a): 0 * x_lo + a * x_hi
  uint32_t x[CHAINS / 2];
  float b[CHAINS];
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p)
    x[p] = static_cast<uint32_t>(in[(2 * p) * elements + i]) |
           (static_cast<uint32_t>(in[(2 * p + 1) * elements + i]) << 16);
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) b[c] = __uint_as_float(static_cast<uint32_t>(coeff[1 + c]) << 16);
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) dot2_update(x, w_lo, w_hi, b);
  }
  drain_valu_results();
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    out[(2 * p) * elements + i] = static_cast<uint16_t>(x[p]);
    out[(2 * p + 1) * elements + i] = static_cast<uint16_t>(x[p] >> 16);
  }
}

template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_bf16fma_kernel(const uint16_t* __restrict__ in,
                                                               uint16_t* __restrict__ out,
                                                               const uint16_t* __restrict__ coeff,
                                                               uint64_t elements, uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const float a = __uint_as_float(static_cast<uint32_t>(coeff[0]) << 16);
  uint32_t x[CHAINS / 2];
  float b[CHAINS];
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p)
    x[p] = static_cast<uint32_t>(in[(2 * p) * elements + i]) |
           (static_cast<uint32_t>(in[(2 * p + 1) * elements + i]) << 16);
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) b[c] = __uint_as_float(static_cast<uint32_t>(coeff[1 + c]) << 16);
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int p = 0; p < CHAINS / 2; ++p)
        x[p] = cvt_pk_bf16(__builtin_fmaf(bf16_lo(x[p]), a, b[2 * p]), __builtin_fmaf(bf16_hi(x[p]), a, b[2 * p + 1]));
  }
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    out[(2 * p) * elements + i] = static_cast<uint16_t>(x[p]);
    out[(2 * p + 1) * elements + i] = static_cast<uint16_t>(x[p] >> 16);
  }
}

template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_dot4_kernel(const int32_t* __restrict__ in, int32_t* __restrict__ out,
                                                            const int32_t* __restrict__ coeff, uint64_t elements,
                                                            uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  int x[CHAINS], b[CHAINS];
  const int w = coeff[0];
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) {
    x[c] = in[c * elements + i];
    b[c] = coeff[1 + c];
  }
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) dot4_update(x, w, b);
  }
  drain_valu_results();
#pragma unroll
  for (int c = 0; c < CHAINS; ++c) out[c * elements + i] = x[c];
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// FP8 E4M3 state, one code per byte in memory; chains (2p, 2p+1) share the low
// 16 bits of one VGPR.
template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_fp8w_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                           const uint8_t* __restrict__ coeff, uint64_t elements,
                                                           uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t x[CHAINS / 2];
  float b[CHAINS];
  const float a = __builtin_amdgcn_cvt_pk_f32_fp8(coeff[0], false)[0];
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    x[p] = in[(2 * p) * elements + i] | (static_cast<uint32_t>(in[(2 * p + 1) * elements + i]) << 8);
    const f32x2 bp = __builtin_amdgcn_cvt_pk_f32_fp8(coeff[1 + 2 * p] | (coeff[2 + 2 * p] << 8), false);
    b[2 * p] = bp[0];
    b[2 * p + 1] = bp[1];
  }
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int p = 0; p < CHAINS / 2; ++p) {
        const f32x2 v = __builtin_amdgcn_cvt_pk_f32_fp8(x[p], false);
        x[p] = __builtin_amdgcn_cvt_pk_fp8_f32(__builtin_fmaf(v[0], a, b[2 * p]),
                                               __builtin_fmaf(v[1], a, b[2 * p + 1]), x[p], false);
      }
  }
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    out[(2 * p) * elements + i] = static_cast<uint8_t>(x[p]);
    out[(2 * p + 1) * elements + i] = static_cast<uint8_t>(x[p] >> 8);
  }
}

// FP4 E2M1 state, one code per byte (low nibble) in memory; chains (2p, 2p+1)
// share one byte (low nibble = chain 2p) of one VGPR.
template <int UNROLL>
__global__ void __launch_bounds__(1024) vector_fp4w_kernel(const uint8_t* __restrict__ in, uint8_t* __restrict__ out,
                                                           const uint8_t* __restrict__ coeff, uint64_t elements,
                                                           uint32_t trips) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t x[CHAINS / 2];
  float b[CHAINS];
  const float a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(coeff[0] & 15u, 1.0f, 0)[0];
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    x[p] = (in[(2 * p) * elements + i] & 15u) | ((in[(2 * p + 1) * elements + i] & 15u) << 4);
    const f32x2 bp =
        __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((coeff[1 + 2 * p] & 15u) | ((coeff[2 + 2 * p] & 15u) << 4), 1.0f, 0);
    b[2 * p] = bp[0];
    b[2 * p + 1] = bp[1];
  }
  for (uint32_t t = 0; t < trips; ++t) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u)
#pragma unroll
      for (int p = 0; p < CHAINS / 2; ++p) {
        const f32x2 v = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(x[p], 1.0f, 0);
        x[p] = __builtin_amdgcn_cvt_scalef32_pk_fp4_f32(x[p], __builtin_fmaf(v[0], a, b[2 * p]),
                                                        __builtin_fmaf(v[1], a, b[2 * p + 1]), 1.0f, 0);
      }
  }
#pragma unroll
  for (int p = 0; p < CHAINS / 2; ++p) {
    out[(2 * p) * elements + i] = static_cast<uint8_t>(x[p] & 15u);
    out[(2 * p + 1) * elements + i] = static_cast<uint8_t>((x[p] >> 4) & 15u);
  }
}

using VectorLauncher = void (*)(const void*, void*, const void*, uint64_t, uint32_t, uint32_t, uint32_t,
                                hipStream_t);

#define MB_VECTOR_LAUNCHER(KERNEL, T)                                                                       \
  template <int UNROLL>                                                                                     \
  void launch_##KERNEL(const void* in, void* out, const void* coeff, uint64_t elements, uint32_t threads,   \
                       uint32_t blocks, uint32_t trips, hipStream_t stream) {                               \
    KERNEL<UNROLL><<<dim3(blocks), dim3(threads), 0, stream>>>(                                             \
        static_cast<const T*>(in), static_cast<T*>(out), static_cast<const T*>(coeff), elements, trips);   \
  }

MB_VECTOR_LAUNCHER(vector_f32_kernel, float)
MB_VECTOR_LAUNCHER(vector_f64_kernel, double)
MB_VECTOR_LAUNCHER(vector_f16_kernel, _Float16)
MB_VECTOR_LAUNCHER(vector_bf16dot_kernel, uint16_t)
MB_VECTOR_LAUNCHER(vector_bf16fma_kernel, uint16_t)
MB_VECTOR_LAUNCHER(vector_dot4_kernel, int32_t)
MB_VECTOR_LAUNCHER(vector_fp8w_kernel, uint8_t)
MB_VECTOR_LAUNCHER(vector_fp4w_kernel, uint8_t)

struct VectorVariant {
  int kind;
  int unroll;
  const char* name;
  const void* kernel;
  VectorLauncher launch;
  int elem_bytes;
};

#define MB_VECTOR_UNROLLS(KIND, KERNEL, T, NAME)                                                             \
  VectorVariant{KIND, 1, NAME "_u1", reinterpret_cast<const void*>(KERNEL<1>), launch_##KERNEL<1>, sizeof(T)},     \
      VectorVariant{KIND, 4, NAME "_u4", reinterpret_cast<const void*>(KERNEL<4>), launch_##KERNEL<4>, sizeof(T)}, \
      VectorVariant{KIND, 8, NAME "_u8", reinterpret_cast<const void*>(KERNEL<8>), launch_##KERNEL<8>, sizeof(T)}, \
      VectorVariant{KIND, 16, NAME "_u16", reinterpret_cast<const void*>(KERNEL<16>), launch_##KERNEL<16>, sizeof(T)}

const VectorVariant kVectorVariants[] = {
    MB_VECTOR_UNROLLS(MB_VECTOR_F32, vector_f32_kernel, float, "vector_f32"),
    MB_VECTOR_UNROLLS(MB_VECTOR_F64, vector_f64_kernel, double, "vector_f64"),
    MB_VECTOR_UNROLLS(MB_VECTOR_F16, vector_f16_kernel, _Float16, "vector_f16"),
    MB_VECTOR_UNROLLS(MB_VECTOR_BF16_DOT2, vector_bf16dot_kernel, uint16_t, "vector_bf16dot"),
    MB_VECTOR_UNROLLS(MB_VECTOR_BF16_FMA, vector_bf16fma_kernel, uint16_t, "vector_bf16fma"),
    MB_VECTOR_UNROLLS(MB_VECTOR_I8_DOT4, vector_dot4_kernel, int32_t, "vector_dot4"),
    MB_VECTOR_UNROLLS(MB_VECTOR_FP8_WIDENED, vector_fp8w_kernel, uint8_t, "vector_fp8w"),
    MB_VECTOR_UNROLLS(MB_VECTOR_FP4_WIDENED, vector_fp4w_kernel, uint8_t, "vector_fp4w"),
};

struct VectorRegistrar {
  VectorRegistrar() {
    for (const auto& variant : kVectorVariants) register_kernel(variant.name, variant.kernel);
  }
};
const VectorRegistrar kVectorRegistrar;

const VectorVariant* find_vector(int kind, uint32_t unroll) {
  for (const auto& variant : kVectorVariants)
    if (variant.kind == kind && variant.unroll == static_cast<int>(unroll)) return &variant;
  return nullptr;
}

}  // namespace
}  // namespace mb

extern "C" {

const char* mb_vector_kernel_name(int kind, uint32_t unroll) {
  const mb::VectorVariant* variant = mb::find_vector(kind, unroll);
  return variant ? variant->name : nullptr;
}

int mb_vector_chains(int kind, const void* input, void* output, const void* coefficients, uint64_t elements,
                     uint32_t iterations, uint32_t unroll, uint32_t block_threads, uint64_t input_bytes,
                     uint64_t output_bytes, uint64_t coefficient_bytes, void* stream) {
  using namespace mb;
  if (kind == MB_VECTOR_FP8 || kind == MB_VECTOR_FP4)
    return fail(MB_ERR_UNSUPPORTED,
                "mb_vector_chains: gfx950 has no %s vector arithmetic; FP8/FP4 only exist as MFMA operands and "
                "conversions",
                kind == MB_VECTOR_FP8 ? "FP8" : "FP4");
  const VectorVariant* variant = find_vector(kind, unroll);
  if (variant == nullptr)
    return fail(MB_ERR_INVALID, "mb_vector_chains: no kernel for kind %d with unroll %u (unroll is 1, 4, 8 or 16)",
                kind, unroll);
  if (input == nullptr || output == nullptr || coefficients == nullptr)
    return fail(MB_ERR_INVALID, "mb_vector_chains: NULL buffer");
  if (block_threads == 0 || block_threads % 64 || block_threads > 1024)
    return fail(MB_ERR_INVALID, "mb_vector_chains: block_threads %u must be a multiple of 64 up to 1024",
                block_threads);
  if (elements == 0 || elements % block_threads)
    return fail(MB_ERR_INVALID, "mb_vector_chains: elements %llu must be a positive multiple of block_threads %u",
                (unsigned long long)elements, block_threads);
  if (iterations == 0 || iterations % unroll)
    return fail(MB_ERR_INVALID, "mb_vector_chains: iterations %u must be a positive multiple of unroll %u",
                iterations, unroll);
  const uint64_t need = static_cast<uint64_t>(CHAINS) * elements * variant->elem_bytes;
  if (input_bytes < need || output_bytes < need || coefficient_bytes < (CHAINS + 1ull) * variant->elem_bytes)
    return fail(MB_ERR_INVALID,
                "mb_vector_chains: buffers too small (need %llu bytes of input and output and %llu of coefficients)",
                (unsigned long long)need, (unsigned long long)((CHAINS + 1ull) * variant->elem_bytes));
  const uint64_t blocks = elements / block_threads;
  if (blocks > 0x7fffffffull) return fail(MB_ERR_INVALID, "mb_vector_chains: too many workgroups");
  variant->launch(input, output, coefficients, elements, block_threads, static_cast<uint32_t>(blocks),
                  iterations / unroll, static_cast<hipStream_t>(stream));
  return launch_status(variant->name);
}

}  // extern "C"
