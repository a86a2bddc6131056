// Resident-operand matrix peak: variant table and C entry points (the kernel
// template is in mb_tensor_peak.h).
#include "mb_tensor_peak.h"

namespace mb {
namespace {

const PeakVariant kPeakVariants[] = {
    MB_PEAK_BOTH(MB_MATRIX_BF16, MfmaBf16, 64, 64, 32, 2, 2, 2, "tensor_peak_bf16_64x64x32_c2"),
    MB_PEAK_BOTH(MB_MATRIX_BF16, MfmaBf16, 128, 128, 64, 2, 2, 2, "tensor_peak_bf16_128x128x64_c2"),
    MB_PEAK_BOTH(MB_MATRIX_BF16, MfmaBf16, 256, 256, 64, 2, 2, 1, "tensor_peak_bf16_256x256x64_c1"),
    MB_PEAK_BOTH(MB_MATRIX_F16, MfmaF16, 64, 64, 32, 2, 2, 2, "tensor_peak_f16_64x64x32_c2"),
    MB_PEAK_BOTH(MB_MATRIX_F16, MfmaF16, 128, 128, 64, 2, 2, 2, "tensor_peak_f16_128x128x64_c2"),
    MB_PEAK_BOTH(MB_MATRIX_F16, MfmaF16, 256, 256, 64, 2, 2, 1, "tensor_peak_f16_256x256x64_c1"),
    MB_PEAK_BOTH(MB_MATRIX_I8, MfmaI8, 64, 64, 64, 2, 2, 2, "tensor_peak_i8_64x64x64_c2"),
    MB_PEAK_BOTH(MB_MATRIX_I8, MfmaI8, 128, 128, 64, 2, 2, 2, "tensor_peak_i8_128x128x64_c2"),
    MB_PEAK_BOTH(MB_MATRIX_I8, MfmaI8, 256, 256, 64, 2, 2, 1, "tensor_peak_i8_256x256x64_c1"),
    MB_PEAK_BOTH(MB_MATRIX_FP8_E4M3, MfmaFp8, 64, 64, 64, 2, 2, 2, "tensor_peak_fp8_64x64x64_c2"),
    MB_PEAK_BOTH(MB_MATRIX_FP8_E4M3, MfmaFp8, 128, 128, 128, 2, 2, 2, "tensor_peak_fp8_128x128x128_c2"),
    MB_PEAK_BOTH(MB_MATRIX_FP8_E4M3, MfmaFp8, 256, 256, 128, 2, 2, 1, "tensor_peak_fp8_256x256x128_c1"),
    MB_PEAK_BOTH(MB_MATRIX_MXFP4, MfmaMxfp4, 64, 64, 128, 2, 2, 2, "tensor_peak_mxfp4_64x64x128_c2"),
    MB_PEAK_BOTH(MB_MATRIX_MXFP4, MfmaMxfp4, 128, 128, 256, 2, 2, 2, "tensor_peak_mxfp4_128x128x256_c2"),
    MB_PEAK_BOTH(MB_MATRIX_MXFP4, MfmaMxfp4, 256, 256, 256, 2, 2, 1, "tensor_peak_mxfp4_256x256x256_c1"),
    // 16x16-instruction forms (suffix _mfma16) of the 256x256 tiles: FP8's
    // builtin keeps its accumulators in place; BF16, FP16 and INT8 issue the
    // in-place form (tensor_peak_tied_kernel). The 128x128 ones are in
    // mb_tensor_peak_vgpr.hip; MXFP4's 256x256 16x16 form is not built.
    MB_PEAK_BOTH(MB_MATRIX_FP8_E4M3, MfmaFp8x16, 256, 256, 128, 2, 2, 1, "tensor_peak_fp8_256x256x128_c1_mfma16"),
    MB_PEAK_TIED_BOTH(MB_MATRIX_BF16, MfmaBf16x16, 256, 256, 64, 2, 2, 1, "tensor_peak_bf16_256x256x64_c1_mfma16"),
    MB_PEAK_TIED_BOTH(MB_MATRIX_F16, MfmaF16x16, 256, 256, 64, 2, 2, 1, "tensor_peak_f16_256x256x64_c1_mfma16"),
    MB_PEAK_TIED_BOTH(MB_MATRIX_I8, MfmaI8x16, 256, 256, 64, 2, 2, 1, "tensor_peak_i8_256x256x64_c1_mfma16"),
    MB_PEAK_BOTH(MB_MATRIX_F32, MfmaF32, 64, 64, 32, 2, 2, 2, "tensor_peak_f32_64x64x32_c2"),
    MB_PEAK_BOTH(MB_MATRIX_F32, MfmaF32, 128, 128, 32, 2, 2, 2, "tensor_peak_f32_128x128x32_c2"),
    MB_PEAK_BOTH(MB_MATRIX_F64, MfmaF64, 32, 32, 16, 2, 2, 2, "tensor_peak_f64_32x32x16_c2"),
    MB_PEAK_BOTH(MB_MATRIX_F64, MfmaF64, 64, 64, 16, 2, 2, 2, "tensor_peak_f64_64x64x16_c2"),
    MB_PEAK_BOTH(MB_MATRIX_F64, MfmaF64, 128, 128, 16, 2, 2, 2, "tensor_peak_f64_128x128x16_c2"),
};

struct PeakRegistrar {
  PeakRegistrar() {
    for (const auto& variant : kPeakVariants) register_kernel(variant.name, variant.kernel);
  }
};
const PeakRegistrar kPeakRegistrar;

// Calls f on every compiled variant: this file's table, then the VGPR-form one.
template <class F>
void for_each_peak_variant(F&& f) {
  for (const auto& variant : kPeakVariants) f(variant);
  int count = 0;
  const PeakVariant* vgpr = vgpr_form_peak_variants(&count);
  for (int i = 0; i < count; ++i) f(vgpr[i]);
}

const PeakVariant* find_peak_variant(int format, const mb_peak_config* config) {
  const PeakVariant* found = nullptr;
  for_each_peak_variant([&](const PeakVariant& variant) {
    const mb_peak_config& v = variant.config;
    if (found == nullptr && variant.format == format && v.tile_m == config->tile_m &&
        v.tile_n == config->tile_n && v.tile_k == config->tile_k && v.chains == config->chains &&
        v.b_nk == config->b_nk && (config->mfma_m == 0 || v.mfma_m == config->mfma_m))
      found = &variant;
  });
  return found;
}

const char* format_name(int format) {
  switch (format) {
    case MB_MATRIX_BF16: return "bf16";
    case MB_MATRIX_F16: return "fp16";
    case MB_MATRIX_F32: return "fp32";
    case MB_MATRIX_TF32: return "tf32";
    case MB_MATRIX_I8: return "int8";
    case MB_MATRIX_F64: return "fp64";
    case MB_MATRIX_FP8_E4M3: return "fp8_e4m3";
    case MB_MATRIX_MXFP4: return "mxfp4_e2m1";
    default: return "unknown";
  }
}

}  // namespace

int matrix_format_check(int format, const char* entry) {
  if (format == MB_MATRIX_TF32)
    return fail(MB_ERR_UNSUPPORTED,
                "%s: gfx950 (CDNA4) has no xf32/TF32 matrix instruction; v_mfma_f32_32x32x4_xf32 was removed "
                "after gfx942",
                entry);
  if (format < MB_MATRIX_BF16 || format > MB_MATRIX_MXFP4)
    return fail(MB_ERR_INVALID, "%s: unknown matrix format %d", entry, format);
  return MB_OK;
}

}  // namespace mb

extern "C" {

int mb_tensor_peak_configs(int format, mb_peak_config* out, int capacity) {
  using namespace mb;
  if (int rc = matrix_format_check(format, "mb_tensor_peak_configs")) return rc;
  int count = 0;
  for_each_peak_variant([&](const PeakVariant& variant) {
    if (variant.format != format) return;
    if (out != nullptr && count < capacity) out[count] = variant.config;
    ++count;
  });
  return count;
}

const char* mb_tensor_peak_kernel_name(int format, const mb_peak_config* config) {
  using namespace mb;
  if (config == nullptr) return nullptr;
  const PeakVariant* found = find_peak_variant(format, config);
  return found != nullptr ? found->name : nullptr;
}

int mb_tensor_peak(int format, const mb_peak_config* config, const void* a, uint64_t a_bytes, const void* b,
                   uint64_t b_bytes, const void* scale_a, uint64_t scale_a_bytes, const void* scale_b,
                   uint64_t scale_b_bytes, void* c, uint64_t c_bytes, uint32_t blocks, uint32_t iterations,
                   void* stream) {
  using namespace mb;
  if (int rc = matrix_format_check(format, "mb_tensor_peak")) return rc;
  if (config == nullptr) return fail(MB_ERR_INVALID, "mb_tensor_peak: config is NULL");
  const PeakVariant* found = find_peak_variant(format, config);
  if (found == nullptr)
    return fail(MB_ERR_INVALID, "mb_tensor_peak: no %s kernel for tile %ux%ux%u, %u chains, b_nk=%u "
                "(list them with mb_tensor_peak_configs)",
                format_name(format), config->tile_m, config->tile_n, config->tile_k, config->chains,
                config->b_nk);
  if (blocks == 0 || blocks > 0x7fffffffu) return fail(MB_ERR_INVALID, "mb_tensor_peak: blocks %u", blocks);
  if (iterations == 0) return fail(MB_ERR_INVALID, "mb_tensor_peak: iterations must be positive");
  const mb_peak_config& v = found->config;
  const uint64_t k_bytes = static_cast<uint64_t>(v.tile_k) * found->elem_bits / 8;
  const uint64_t need_a = static_cast<uint64_t>(blocks) * v.tile_m * k_bytes;
  const uint64_t need_b = static_cast<uint64_t>(v.chains) * blocks * k_bytes * v.tile_n;
  const uint64_t need_c = static_cast<uint64_t>(v.chains) * blocks * v.tile_m * v.tile_n * found->out_bytes;
  if (a == nullptr || b == nullptr || c == nullptr) return fail(MB_ERR_INVALID, "mb_tensor_peak: NULL operand");
  if (a_bytes < need_a || b_bytes < need_b || c_bytes < need_c)
    return fail(MB_ERR_INVALID,
                "mb_tensor_peak: buffers too small (A %llu < %llu, B %llu < %llu or C %llu < %llu bytes)",
                (unsigned long long)a_bytes, (unsigned long long)need_a, (unsigned long long)b_bytes,
                (unsigned long long)need_b, (unsigned long long)c_bytes, (unsigned long long)need_c);
  if (!aligned(a, 16) || !aligned(b, 16) || !aligned(c, 16))
    return fail(MB_ERR_ALIGNMENT, "mb_tensor_peak: A, B and C must be 16-byte aligned");
  if (format == MB_MATRIX_MXFP4) {
    const uint64_t groups = v.tile_k / 32;
    if (scale_a == nullptr || scale_b == nullptr)
      return fail(MB_ERR_INVALID, "mb_tensor_peak: MXFP4 needs E8M0 scales for A and B");
    if (scale_a_bytes < static_cast<uint64_t>(blocks) * v.tile_m * groups ||
        scale_b_bytes < static_cast<uint64_t>(blocks) * v.tile_n * groups)
      return fail(MB_ERR_INVALID, "mb_tensor_peak: scale buffers too small ([blocks, M|N, K/32] bytes needed)");
  }
  found->launch(static_cast<const uint8_t*>(a), static_cast<const uint8_t*>(b),
                static_cast<const uint8_t*>(scale_a), static_cast<const uint8_t*>(scale_b), c, blocks, iterations,
                static_cast<hipStream_t>(stream));
  return launch_status(found->name);
}

}  // extern "C"
