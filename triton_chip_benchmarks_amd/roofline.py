"""MI355X (gfx950) roofline denominators for the 17 report rows.

Datasheet figures are AMD's published MI355X peaks (256 CUs, 2400 MHz peak
engine clock, 8 TB/s HBM3E, dense matrix rates without sparsity). Rows the
datasheet does not list are derived from the ISA issue rate and say so in
their `basis`. ceiling = CUs * clock * work per clock per CU.
"""

from __future__ import annotations

COMPUTE_UNITS = 256
PEAK_CLOCK_MHZ = 2400
HBM_PEAK_GBPS = 8000.0
HBM_CAPACITY_BYTES = 288 * 10**9
# MI355X last-level cache (AMD Infinity Cache / MALL). HIP reports only one
# XCD's 4 MiB L2, so the HBM-sized-buffer rule uses this capacity instead.
INFINITY_CACHE_BYTES = 256 * 2**20


def _tera(per_clock_per_cu: int) -> float:
    return COMPUTE_UNITS * PEAK_CLOCK_MHZ * 1e6 * per_clock_per_cu / 1e12


# metric key -> (peak value, unit, basis)
PEAKS: dict[str, tuple[float, str, str]] = {
    "memory_bandwidth": (HBM_PEAK_GBPS, "GB/s", "datasheet HBM3E 8 TB/s"),
    "tensor_bf16": (_tera(4096), "TFLOP/s", "datasheet dense BF16 MFMA (4096 flop/clk/CU)"),
    "tensor_fp16": (_tera(4096), "TFLOP/s", "datasheet dense FP16 MFMA (4096 flop/clk/CU)"),
    "tensor_fp32": (_tera(256), "TFLOP/s", "datasheet FP32 matrix (256 flop/clk/CU)"),
    "tensor_int8": (_tera(8192), "TOP/s", "datasheet dense INT8 MFMA (8192 op/clk/CU)"),
    "tensor_fp64": (_tera(128), "TFLOP/s", "datasheet FP64 matrix (128 flop/clk/CU)"),
    "tensor_fp8": (_tera(8192), "TFLOP/s", "datasheet dense FP8 MFMA (8192 flop/clk/CU)"),
    "tensor_fp4": (_tera(16384), "TFLOP/s", "datasheet dense MXFP4 MFMA (16384 flop/clk/CU)"),
    "vector_fp32": (_tera(256), "TFLOP/s", "datasheet FP32 vector, which needs packed v_pk_fma_f32 "
                                           "(256 flop/clk/CU); this build issues v_fma_f32 only, "
                                           "whose ceiling is half of it"),
    "vector_fp64": (_tera(128), "TFLOP/s", "datasheet FP64 vector (v_fma_f64, 128 flop/clk/CU)"),
    "vector_fp16": (_tera(256), "TFLOP/s", "ISA-derived: v_pk_fma_f16, 64 lanes x 2 x 2 flop/clk/CU "
                                           "(not a datasheet figure)"),
    "vector_bf16": (_tera(256), "TFLOP/s", "ISA-derived: v_dot2_f32_bf16, 64 lanes x 4 flop/clk/CU "
                                           "(not a datasheet figure)"),
    "vector_int8": (_tera(512), "TOP/s", "ISA-derived: v_dot4_i32_i8, 64 lanes x 8 op/clk/CU "
                                         "(not a datasheet figure)"),
}

# Issue-rate ceilings of the instruction this build actually uses, where it
# differs from the datasheet row above.
ISSUED_CEILINGS: dict[str, tuple[float, str]] = {
    "vector_fp32": (_tera(128), "v_fma_f32: 64 lanes x 2 flop/clk/CU"),
    # Eight v_dot2_f32_bf16 and four v_cvt_pk_bf16_f32 per eight 2-flop updates:
    # 1.5 wave64 VALU instructions per update, 256 / 3 flop/clk/CU.
    "vector_bf16": (_tera(256) / 3, "v_dot2_f32_bf16 + v_cvt_pk_bf16_f32: 1.5 VALU instructions per "
                                    "2-flop update"),
}


def fraction(metric: str, value: float | None) -> float | None:
    if value is None or metric not in PEAKS:
        return None
    return value / PEAKS[metric][0]


def describe(metric: str, value: float | None) -> dict | None:
    """Roofline block attached to a row: achieved value against the peak."""
    if metric not in PEAKS:
        return None
    peak, unit, basis = PEAKS[metric]
    block = {"peak": peak, "unit": unit, "basis": basis, "achieved": value,
             "frac": None if value is None else value / peak}
    if metric in ISSUED_CEILINGS:
        ceiling, ceiling_basis = ISSUED_CEILINGS[metric]
        block.update(issued_instruction_ceiling=ceiling, issued_instruction_basis=ceiling_basis,
                     frac_of_issued_ceiling=None if value is None else value / ceiling)
    return block
