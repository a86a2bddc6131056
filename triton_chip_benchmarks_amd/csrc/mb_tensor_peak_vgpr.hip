// Resident-operand matrix peak, 16x16-instruction tiles whose fragments and
// accumulators fit the 256 architectural VGPRs. This file is compiled with the
// VGPR form of v_mfma (-amdgpu-mfma-vgpr-form): with the default allocation the
// compiler splits these accumulators between AGPRs and VGPRs and copies them
// (v_accvgpr_read/write/mov) inside the timed loop.
#include "mb_tensor_peak.h"

namespace mb {
namespace {

const PeakVariant kVgprFormVariants[] = {
    MB_PEAK_BOTH(MB_MATRIX_BF16, MfmaBf16x16, 128, 128, 64, 2, 2, 2, "tensor_peak_bf16_128x128x64_c2_mfma16"),
    MB_PEAK_BOTH(MB_MATRIX_F16, MfmaF16x16, 128, 128, 64, 2, 2, 2, "tensor_peak_f16_128x128x64_c2_mfma16"),
    MB_PEAK_BOTH(MB_MATRIX_I8, MfmaI8x16, 128, 128, 64, 2, 2, 2, "tensor_peak_i8_128x128x64_c2_mfma16"),
    MB_PEAK_BOTH(MB_MATRIX_FP8_E4M3, MfmaFp8x16, 128, 128, 128, 2, 2, 2, "tensor_peak_fp8_128x128x128_c2_mfma16"),
    MB_PEAK_BOTH(MB_MATRIX_MXFP4, MfmaMxfp4x16, 128, 128, 256, 2, 2, 2, "tensor_peak_mxfp4_128x128x256_c2_mfma16"),
};

struct VgprFormRegistrar {
  VgprFormRegistrar() {
    for (const auto& variant : kVgprFormVariants) register_kernel(variant.name, variant.kernel);
  }
};
const VgprFormRegistrar kVgprFormRegistrar;

}  // namespace

const PeakVariant* vgpr_form_peak_variants(int* count) {
  *count = static_cast<int>(sizeof(kVgprFormVariants) / sizeof(kVgprFormVariants[0]));
  return kVgprFormVariants;
}

}  // namespace mb
