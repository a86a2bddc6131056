"""Instruction and resource audit of the library's own gfx950 code object.

The reference audits the assembly text Triton returns for each compiled kernel
(bench_tensor.py:984-1146, bench_vector.py:623-799). Here the audited text is
the llvm-objdump disassembly of the code object embedded in
libmi355x_bench.so, written by build.py, so the audited instructions are the
ones the launches execute. Resource figures (VGPR/AGPR/SGPR, spills, LDS,
scratch) come from the AMDHSA metadata of the same build.

The per-dtype rules are the reference's AMDGCN rules re-targeted to gfx950
mnemonics: FP8 runs on v_mfma_f32_32x32x64_f8f6f4 with the default E4M3
formats (no cbsz/blgp modifier), MXFP4 on v_mfma_scale_f32_32x32x64_f8f6f4
with cbsz:4 blgp:4 (E2M1), and the vector INT8/BF16 rows on v_dot4 / v_dot2.
"""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path
import re

from . import build as native_build

MATRIX_MNEMONICS = ("v_mfma_", "v_wmma_", "v_mmac_")

# Registered kernel name <- mangled symbol. Each kernel family's template
# arguments are recovered from its Itanium-mangled name.
_MFMA_FORMAT = {"MfmaBf16": "bf16", "MfmaF16": "f16", "MfmaI8": "i8", "MfmaFp8": "fp8",
                "MfmaMxfp4": "mxfp4", "MfmaF32": "f32", "MfmaF64": "f64"}
_PEAK_RE = re.compile(r"tensor_peak_(?:tied_)?kernelINS_\d+(Mfma\w+?)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb([01])E")
_GEMM_RE = re.compile(r"gemm_kernelINS_\d+(Mfma\w+?)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELi(\d+)ELb([01])E")
_GEMM_STAGED_RE = re.compile(r"gemm_(?:staged|dma)_kernelINS_\d+(Mfma\w+?)EE")
_ELEM_BITS = {"bf16": 16, "f16": 16, "i8": 8, "fp8": 8, "mxfp4": 4, "f32": 32, "f64": 64}
_COPY_RE = re.compile(r"copy_kernelI(Dv4_j|j|h)Li(\d+)ELi([012])E")
_READ_RE = re.compile(r"read_sum_kernelI(f|DF16_|t)Li(\d+)E")
_VECTOR_RE = re.compile(r"vector_(\w+?)_kernelILi(\d+)E")
_COPY_UNIT = {"Dv4_j": "dwordx4", "j": "dword", "h": "byte"}
_READ_TYPE = {"f": "f32", "DF16_": "f16", "t": "bf16"}


def registered_name(symbol: str) -> str | None:
    """The registry name the library uses for a mangled kernel symbol."""
    match = _PEAK_RE.search(symbol)
    if match:
        op, bm, bn, bk, _wm, _wn, chains, nk = match.groups()
        shape = "_mfma16" if op.endswith("x16") else ""
        return (f"tensor_peak_{_MFMA_FORMAT[op.removesuffix('x16')]}_{bm}x{bn}x{bk}_c{chains}{shape}_"
                f"{'nk' if nk == '1' else 'kn'}")
    match = _GEMM_RE.search(symbol)
    if match:
        op, bm, bn, bk, _wm, _wn, checked = match.groups()
        return f"gemm_{_MFMA_FORMAT[op]}_{bm}x{bn}x{bk}{'_checked' if checked == '1' else ''}"
    match = _GEMM_STAGED_RE.search(symbol)
    if match:
        fmt = _MFMA_FORMAT[match.group(1).removesuffix("x16")]
        return f"gemm_{fmt}_256x256x{128 * 8 // _ELEM_BITS[fmt]}"
    if "gemm_dma_f64_kernelI" in symbol:
        return "gemm_f64_256x128x16"
    match = _COPY_RE.search(symbol)
    if match:
        unit, vpt, policy = match.groups()
        return f"copy_{_COPY_UNIT[unit]}_vpt{vpt}{('', '_nt', '_stream')[int(policy)]}"
    match = _READ_RE.search(symbol)
    if match:
        dtype, vec = match.groups()
        return f"read_sum_{_READ_TYPE[dtype]}{'_vec' if vec != '1' else ''}"
    match = _VECTOR_RE.search(symbol)
    if match:
        kind, unroll = match.groups()
        return f"vector_{kind}_u{unroll}"
    if "clock_witness_kernel" in symbol:
        return "clock_witness"
    if "copy_tail_kernel" in symbol:
        return "copy_tail"
    match = re.search(r"fill_kernelILi([0-2])EEEv", symbol)
    if match:
        return "fill_dwordx4" + ("", "_nt", "_stream")[int(match.group(1))]
    if "fill_tail_kernel" in symbol:
        return "fill_tail"
    return None


@lru_cache(maxsize=4)
def _disassembly(path: str) -> dict[str, list[str]]:
    """symbol -> instruction lines, from an llvm-objdump -d listing."""
    listing: dict[str, list[str]] = {}
    current = None
    for line in Path(path).read_text().splitlines():
        header = re.match(r"^[0-9a-f]+ <(\S+)>:$", line)
        if header:
            current = header.group(1)
            listing[current] = []
        elif current is not None and line.strip():
            listing[current].append(line.split("//")[0].strip())
    return listing


@lru_cache(maxsize=4)
def _metadata(build_dir: str) -> dict[str, dict]:
    """mangled symbol -> AMDHSA metadata fields, from the device assembly."""
    result: dict[str, dict] = {}
    for asm in sorted(Path(build_dir).glob("*.gfx950.s")):
        text = asm.read_text()
        if "amdhsa.kernels:" not in text:
            continue
        for entry in re.split(r"\n  - \.", text.split("amdhsa.kernels:", 1)[1]):
            name = re.search(r"\.name:\s+(\S+)", entry)
            if not name:
                continue
            fields = {}
            for key in ("vgpr_count", "agpr_count", "sgpr_count", "vgpr_spill_count", "sgpr_spill_count",
                        "group_segment_fixed_size", "private_segment_fixed_size", "wavefront_size",
                        "max_flat_workgroup_size"):
                found = re.search(r"\." + key + r":\s+(\d+)", entry)
                if found:
                    fields[key] = int(found.group(1))
            result[name.group(1)] = fields
        # Architectural VGPRs and AGPRs are split in the symbol resource sets.
        for symbol, kind, value in re.findall(r"\.set (\S+)\.num_(vgpr|agpr), (\d+)", text):
            result.setdefault(symbol, {})[f"num_{kind}"] = int(value)
    return result


def symbols(disassembly: Path | None = None) -> dict[str, str]:
    """Registered kernel name -> mangled symbol in the built code object."""
    listing = _disassembly(str(disassembly or native_build.DISASSEMBLY))
    mapping = {}
    for symbol in listing:
        name = registered_name(symbol)
        if name is not None:
            mapping[name] = symbol
    return mapping


def instructions(name: str, disassembly: Path | None = None) -> list[str]:
    path = disassembly or native_build.DISASSEMBLY
    if not Path(path).exists():
        raise FileNotFoundError(f"{path} is missing; rebuild the library to produce the audit listing")
    mapping = symbols(path)
    if name not in mapping:
        raise KeyError(f"kernel {name!r} is not in the code object disassembly")
    return _disassembly(str(path))[mapping[name]]


_ADDRESS_RE = re.compile(r"//\s*([0-9A-Fa-f]+):")
_TARGET_RE = re.compile(r"<(\S+)\+0x([0-9a-f]+)>")


@lru_cache(maxsize=4)
def _addressed(path: str) -> dict[str, list[tuple[int, str, int | None]]]:
    """symbol -> [(address, instruction, branch target address or None)]."""
    listing: dict[str, list[tuple[int, str, int | None]]] = {}
    current, start = None, 0
    for line in Path(path).read_text().splitlines():
        header = re.match(r"^([0-9a-f]+) <(\S+)>:$", line)
        if header:
            start, current = int(header.group(1), 16), header.group(2)
            listing[current] = []
            continue
        address = _ADDRESS_RE.search(line)
        if current is None or not address:
            continue
        target = _TARGET_RE.search(line)
        target_address = start + int(target.group(2), 16) if target and target.group(1) == current else None
        listing[current].append((int(address.group(1), 16), line.split("//")[0].strip(), target_address))
    return listing


def loops(name: str, disassembly: Path | None = None) -> list[list[str]]:
    """Instruction bodies of every backward branch of a kernel (target .. branch),
    in listing order. The body with the most matrix instructions of a peak
    kernel is its timed loop."""
    path = disassembly or native_build.DISASSEMBLY
    symbol = symbols(path)[name]
    code = _addressed(str(path))[symbol]
    bodies = []
    for address, _text, target in code:
        if target is not None and target <= address:
            bodies.append([text for a, text, _ in code if target <= a <= address])
    return bodies


def hot_loop(name: str, disassembly: Path | None = None) -> list[str]:
    """The loop body holding the most MFMA instructions (empty if none)."""
    candidates = loops(name, disassembly)
    best = max(candidates, key=lambda body: sum(mnemonic(l).startswith("v_mfma") for l in body), default=[])
    return best if any(mnemonic(l).startswith("v_mfma") for l in best) else []


def loop_summary(name: str, disassembly: Path | None = None) -> dict:
    """What the timed loop issues: MFMA count and every other mnemonic with its count."""
    body = hot_loop(name, disassembly)
    counts: dict[str, int] = {}
    for line in body:
        counts[mnemonic(line)] = counts.get(mnemonic(line), 0) + 1
    matrix = {k: v for k, v in counts.items() if k.startswith("v_mfma")}
    other = {k: v for k, v in counts.items() if not k.startswith("v_mfma")}
    vector_other = {k: v for k, v in other.items() if not k.startswith("s_")}
    return {"timed_loop_matrix_instructions": sum(matrix.values()),
            "timed_loop_matrix_types": sorted(matrix),
            "timed_loop_other_instructions": other,
            "timed_loop_vector_memory_or_alu": vector_other}


def resources(name: str, build_dir: Path | None = None, disassembly: Path | None = None) -> dict:
    mapping = symbols(disassembly)
    metadata = _metadata(str(build_dir or native_build.BUILD)).get(mapping.get(name, ""), {})
    vgprs = metadata.get("vgpr_count")
    return {"registers_per_thread": vgprs, "arch_vgpr_count": metadata.get("num_vgpr"),
            "agpr_count": metadata.get("num_agpr"),
            "sgpr_count": metadata.get("sgpr_count"),
            "register_spills": metadata.get("vgpr_spill_count", 0) + metadata.get("sgpr_spill_count", 0)
            if metadata else None,
            "shared_memory_bytes": metadata.get("group_segment_fixed_size"),
            "scratch_bytes": metadata.get("private_segment_fixed_size")}


def mnemonic(line: str) -> str:
    return line.split()[0] if line.split() else ""


class TensorAuditError(RuntimeError):
    """The compiled kernel does not run the requested matrix format."""


def _matrix_format_ok(dtype: str, line: str) -> bool:
    name = mnemonic(line)
    if dtype == "bf16":
        return re.fullmatch(r"v_mfma_f32_\d+x\d+x\d+_?bf16", name) is not None
    if dtype == "fp16":
        return re.fullmatch(r"v_mfma_f32_\d+x\d+x\d+_?f16", name) is not None
    if dtype == "int8":
        return re.fullmatch(r"v_mfma_i32_\d+x\d+x\d+_?i8", name) is not None
    if dtype == "fp64":
        return re.fullmatch(r"v_mfma_f64_\d+x\d+x\d+_?f64", name) is not None
    if dtype == "fp32":
        return re.fullmatch(r"v_mfma_f32_\d+x\d+x\d+_?f32", name) is not None
    if dtype == "fp8":
        # f8f6f4 selects formats with cbsz (A) / blgp (B); absent = 0 = FP8 E4M3.
        return (re.fullmatch(r"v_mfma(?:_scale)?_f32_\d+x\d+x\d+_f8f6f4", name) is not None
                and "cbsz:" not in line and "blgp:" not in line) or "fp8_fp8" in name
    if dtype == "fp4":
        return (re.fullmatch(r"v_mfma_scale_f32_\d+x\d+x\d+_f8f6f4", name) is not None
                and "cbsz:4" in line and "blgp:4" in line)
    return False


def audit_tensor(lines: list[str], dtype: str, input_precision: str | None = None) -> dict:
    """gfx950 matrix audit of one kernel listing (bench_tensor.py:984-1146 rules)."""
    tensor_lines = [line for line in lines if any(line.startswith(m) for m in MATRIX_MNEMONICS)]
    scalar_fp32 = [line for line in lines if mnemonic(line) in ("v_fma_f32", "v_fmac_f32", "v_mac_f32",
                                                                "v_pk_fma_f32", "v_fmac_f32_e32")]
    scalar_fp64 = [line for line in lines if mnemonic(line).startswith("v_fma_f64")]
    if dtype == "tf32" or input_precision == "tf32":
        reduced = [line for line in tensor_lines if "xf32" in line or "tf32" in line]
        if not tensor_lines or len(reduced) != len(tensor_lines):
            raise TensorAuditError("Cannot verify native TF32 matrix instructions for gfx950; compiled tensor "
                                   f"instructions: {sorted({mnemonic(l) for l in tensor_lines}) or 'none'}")
    if dtype == "fp32":
        reduced = [line for line in tensor_lines if "xf32" in line or "tf32" in line]
        if reduced:
            raise TensorAuditError("Requested IEEE FP32 but found reduced-precision instructions: "
                                   f"{sorted({mnemonic(l) for l in reduced})}")
    if dtype in ("fp32", "fp64") and not tensor_lines:
        if not (scalar_fp64 if dtype == "fp64" else scalar_fp32):
            raise TensorAuditError(f"No {dtype.upper()} matrix or scalar FMA instructions in the kernel")
        execution_kind, native = "simt", False
    else:
        if not tensor_lines:
            raise TensorAuditError("No v_mfma instructions in the compiled kernel")
        wrong = [line for line in tensor_lines if not _matrix_format_ok(dtype, line)]
        if wrong:
            raise TensorAuditError(f"Cannot verify native {dtype} MFMA on gfx950; compiled instructions: "
                                   f"{sorted({mnemonic(l) for l in wrong})}")
        execution_kind, native = "tensor", True
    note = (f"{dtype.upper()} execution verified as scalar/vector FMA; no native tensor MMA"
            if execution_kind == "simt" else None)
    return {"assembly_audit": "verified", "execution_kind": execution_kind,
            "instruction_precision_verified": True, "native_tensor_verified": native,
            "assembly_audit_note": note,
            "tensor_instruction_types": sorted({mnemonic(l) for l in tensor_lines}),
            "tensor_instruction_modifiers": sorted({" ".join(t for t in l.split()
                                                             if re.match(r"(?:cbsz|blgp|abid|op_sel\w*|neg\w*):", t))
                                                    for l in tensor_lines} - {""}),
            "static_tensor_instruction_count": len(tensor_lines),
            "fp32_fma_instruction_types": sorted({mnemonic(l) for l in scalar_fp32}),
            "fp64_fma_instruction_types": sorted({mnemonic(l) for l in scalar_fp64}),
            "static_fp32_fma_instruction_count": len(scalar_fp32)}


class VectorAuditError(RuntimeError):
    """The compiled vector kernel does not run the requested arithmetic."""


_VECTOR_RULES = {
    # dtype -> (regex of native instructions, description)
    "fp32": (r"v_(?:pk_)?(?:fma|fmac|mac|mad)_f32(?:_e(?:32|64))?", "FP32 FMA"),
    "fp64": (r"v_(?:fma|fmac)_f64(?:_e(?:32|64))?", "FP64 FMA"),
    "fp16": (r"v_(?:pk_)?(?:fma|fmac|mac|mad)_f16(?:_e(?:32|64))?", "FP16 FMA"),
    "bf16": (r"v_dot2c?_f32_bf16(?:_e(?:32|64))?", "BF16 dot2 (bf16 products, fp32 sum)"),
    "int8": (r"v_dot4c?_i32_i8(?:_e(?:32|64))?", "signed INT8 dot4 with INT32 output"),
}


_WIDENED_CONVERSIONS = {
    "fp8": (r"v_cvt_pk_f32_fp8(?:_e32|_e64|_sdwa)?", r"v_cvt_pk_fp8_f32(?:_e64)?"),
    "fp4": (r"v_cvt_scalef32_pk_f32_fp4", r"v_cvt_scalef32_pk_fp4_f32"),
}


def audit_widened(lines: list[str], dtype: str) -> dict:
    """Converted FP8/FP4 chains: the kernel must widen, FMA in FP32 and narrow.

    The rows are never native (gfx950's VALU has no FP8/FP4 arithmetic): the
    check is that each update is the stated v_fma_f32 between a widening and
    a narrowing conversion of the format, with no matrix instruction.
    """
    if any(line.startswith(m) for line in lines for m in MATRIX_MNEMONICS):
        raise VectorAuditError("Generated AMDGCN contains matrix instructions in a vector benchmark")
    names = [mnemonic(line) for line in lines]
    fma = [n for n in names if re.fullmatch(r"v_fmac?_f32(?:_e(?:32|64))?", n)]
    widen_pattern, narrow_pattern = _WIDENED_CONVERSIONS[dtype]
    widen = [n for n in names if re.fullmatch(widen_pattern, n)]
    narrow = [n for n in names if re.fullmatch(narrow_pattern, n)]
    if not (fma and widen and narrow):
        raise VectorAuditError(f"Widened {dtype.upper()} kernel lacks v_fma_f32 or a {dtype.upper()} conversion")
    return {"amdgcn_contains_matrix_instructions": False, "native_arithmetic_verified": False,
            "amdgcn_fp32_fma_instruction_sites": len(fma),
            "amdgcn_widen_instruction_sites": len(widen), "amdgcn_narrow_instruction_sites": len(narrow),
            "amdgcn_instruction_types": sorted(set(fma + widen + narrow)),
            "assembly_check": (f"converted, not native: {dtype.upper()} state widened to FP32, one v_fma_f32 "
                               "per update, narrowed back")}


def audit_vector(lines: list[str], dtype: str, operation: str) -> dict:
    """gfx950 vector audit (bench_vector.py:679-770 rules, gfx950 mnemonics).

    `operation` "fma" for bf16 is the promoted path (bf16 state, v_fma_f32 and
    a bf16 rounding per update): it is measured but never marked native.
    """
    if any(line.startswith(m) for line in lines for m in MATRIX_MNEMONICS):
        raise VectorAuditError("Generated AMDGCN contains matrix instructions in a vector benchmark")
    names = [mnemonic(line) for line in lines]
    result = {"amdgcn_contains_matrix_instructions": False, "native_arithmetic_verified": False}
    if dtype == "bf16" and operation == "fma":
        widened = sorted({n for n in names if re.fullmatch(r"v_(?:pk_)?(?:fma|fmac)_f32(?:_e(?:32|64))?", n)})
        count = sum(n in widened for n in names)
        if not count:
            raise VectorAuditError("Promoted BF16 kernel contains no v_fma_f32")
        result.update(amdgcn_arithmetic_instruction_sites=count, amdgcn_arithmetic_promoted=True,
                      amdgcn_promoted_instructions=widened,
                      assembly_check=("unverified: gfx950 has no BF16 FMA; the kernel keeps BF16 state and "
                                      f"rounds a {', '.join(widened)} result per update, so this is not a "
                                      "native BF16 vector rate"))
        return result
    pattern, description = _VECTOR_RULES[dtype]
    sites = [n for n in names if re.fullmatch(pattern, n)]
    if not sites:
        raise VectorAuditError(f"Generated AMDGCN does not contain native {description}")
    packed = sorted({n for n in sites if "_pk_" in n})
    result.update(amdgcn_arithmetic_instruction_sites=len(sites), native_arithmetic_verified=True,
                  amdgcn_instruction_types=sorted(set(sites)), amdgcn_packed_instruction_types=packed,
                  assembly_check=f"passed ({description}; no matrix instructions)")
    if dtype == "fp32":
        result["amdgcn_fp32_fma_instruction_sites"] = len(sites)
    return result

