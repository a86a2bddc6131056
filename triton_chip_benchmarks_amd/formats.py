"""Operand formats of the matrix rows: OCP MX FP4 (E2M1 + E8M0) and FP8 E4M3.

Host-side data preparation only: building packed operands for the kernels.
The constants are fixed by the OCP Microscaling Formats v1.0 specification,
as the reference states (bench_tensor.py:55-69).
"""

from __future__ import annotations

FP4_PACKING_FACTOR = 2   # E2M1 elements per uint8 container
MX_GROUP_SIZE = 32       # elements along K sharing one E8M0 scale
E8M0_UNIT_SCALE = 127    # biased exponent of 2**0
E8M0_BIAS = 127

# The sixteen E2M1 values in code order: sign, two exponent bits, one mantissa bit.
E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
E2M1_VALUES = E2M1_MAGNITUDES + tuple(-value for value in E2M1_MAGNITUDES)


def pack_e2m1_pairs(codes):
    """Pack E2M1 codes two per byte along the last axis; even k in the low nibble."""
    import torch

    if codes.shape[-1] % 2:
        raise ValueError("E2M1 packing needs an even number of elements along the packed axis")
    low = codes[..., 0::2].to(torch.int16)
    high = codes[..., 1::2].to(torch.int16)
    return ((high << 4) | (low & 15)).to(torch.uint8)


def mx_scale_blocks(scales, fill=E8M0_UNIT_SCALE):
    """Row-major E8M0 scales [rows][K/32] -> the GEMM's K-step blocks [ceil(K/256)][rows][8].

    Block b, row r, group g holds the scale of row r for K elements
    256b + 32g .. 256b + 32g + 31; groups past K are `fill`.
    """
    import torch

    rows, groups = scales.shape
    blocks = -(-groups // 8)
    padded = torch.full((rows, blocks * 8), fill, dtype=torch.uint8, device=scales.device)
    padded[:, :groups] = scales
    return padded.view(rows, blocks, 8).permute(1, 0, 2).contiguous()


def e2m1_decode(codes):
    """Float64 values of E2M1 codes (any integer tensor of 0..15)."""
    import torch

    table = torch.tensor(E2M1_VALUES, dtype=torch.float64, device=codes.device)
    return table[codes.long()]


def e8m0_decode(codes):
    """2**(code - 127) for E8M0 scale codes (255 is NaN in OCP MX)."""
    import torch

    values = torch.pow(2.0, codes.double() - E8M0_BIAS)
    return torch.where(codes == 255, torch.full_like(values, float("nan")), values)


def e2m1_encode(values):
    """E2M1 codes of values on the E2M1 lattice (raises for any other value)."""
    import torch

    magnitudes = torch.tensor(E2M1_MAGNITUDES, dtype=torch.float64, device=values.device)
    v = values.double()
    index = torch.bucketize(v.abs(), magnitudes)
    if bool((index > 7).any()) or not torch.equal(magnitudes[index.clamp(max=7)], v.abs()):
        raise ValueError("values are not all on the E2M1 lattice")
    return (index | (torch.signbit(v).to(torch.int64) << 3)).to(torch.uint8)
