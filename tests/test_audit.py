"""CPU tests of the gfx950 instruction audit, on synthetic listings and on the built library.

The reference refuses to call a rate native unless the compiled kernel issues
the format's own instruction (bench_tensor.py:984-1146,
bench_vector.py:623-799). Here the audited text is the disassembly of the
code objects inside libmi355x_bench.so, so these tests check the kernels the
GPU actually runs: each resident-peak kernel's timed loop issues only its
format's MFMA plus scalar loop control, each vector kernel issues its native
VALU instruction, nothing spills, and no packed-FP32 VALU form is emitted.
"""

from __future__ import annotations

import re

import pytest

from triton_chip_benchmarks_amd import _native, audit
from triton_chip_benchmarks_amd import build as native_build

FORMAT_OF = {"bf16": "bf16", "f16": "fp16", "i8": "int8", "fp8": "fp8", "mxfp4": "fp4", "f32": "fp32",
             "f64": "fp64"}
PEAK_INSTRUCTION = {"bf16": "v_mfma_f32_32x32x16_bf16", "fp16": "v_mfma_f32_32x32x16_f16",
                    "int8": "v_mfma_i32_32x32x32_i8", "fp8": "v_mfma_f32_32x32x64_f8f6f4",
                    "fp4": "v_mfma_scale_f32_32x32x64_f8f6f4", "fp32": "v_mfma_f32_32x32x2_f32",
                    "fp64": "v_mfma_f64_16x16x4_f64"}
# The _mfma16 peak tiles issue the 16x16 form of the same instruction.
PEAK_INSTRUCTION_16 = {"bf16": "v_mfma_f32_16x16x32_bf16", "fp16": "v_mfma_f32_16x16x32_f16",
                       "int8": "v_mfma_i32_16x16x64_i8", "fp8": "v_mfma_f32_16x16x128_f8f6f4",
                       "fp4": "v_mfma_scale_f32_16x16x128_f8f6f4", "fp32": "v_mfma_f32_16x16x4_f32"}
VECTOR_INSTRUCTION = {"f32": ("fp32", "v_fma_f32"), "f64": ("fp64", "v_fma_f64"), "f16": ("fp16", "v_pk_fma_f16"),
                      "bf16dot": ("bf16", "v_dot2_f32_bf16"), "dot4": ("int8", "v_dot4_i32_i8")}


@pytest.fixture(scope="module")
def listing():
    if not native_build.DISASSEMBLY.exists():
        pytest.fail(f"{native_build.DISASSEMBLY} is missing: run __graft_entry__.build() first")
    return audit.symbols()


def _peak_format(name):
    return FORMAT_OF[name.split("_")[2]]


# ---- synthetic listings -----------------------------------------------------------

def test_tensor_rules_accept_each_native_format_and_reject_the_others():
    lines = {fmt: [f"{inst} a[0:15], v[0:1], v[2:3], a[0:15]"] for fmt, inst in PEAK_INSTRUCTION.items()}
    lines["fp4"] = ["v_mfma_scale_f32_32x32x64_f8f6f4 a[0:15], v[0:7], v[8:15], a[0:15], v16, v17 "
                    "op_sel_hi:[0,0,0] cbsz:4 blgp:4"]
    for fmt in PEAK_INSTRUCTION:
        result = audit.audit_tensor(lines[fmt], fmt)
        assert result["native_tensor_verified"] and result["execution_kind"] == "tensor"
        for other in PEAK_INSTRUCTION:
            if other != fmt:
                with pytest.raises(audit.TensorAuditError):
                    audit.audit_tensor(lines[fmt], other)


def test_fp8_rule_rejects_a_non_default_operand_format():
    for modifier in ("cbsz:1", "blgp:2", "cbsz:4 blgp:4"):
        with pytest.raises(audit.TensorAuditError):
            audit.audit_tensor([f"v_mfma_f32_32x32x64_f8f6f4 a[0:15], v[0:7], v[8:15], a[0:15] {modifier}"], "fp8")


def test_fp4_rule_needs_both_operands_in_e2m1():
    for modifier in ("cbsz:4", "blgp:4", ""):
        with pytest.raises(audit.TensorAuditError):
            audit.audit_tensor([f"v_mfma_scale_f32_32x32x64_f8f6f4 a[0:15], v[0:7], v[8:15], a[0:15], v1, v2 "
                                f"{modifier}"], "fp4")


def test_tf32_is_never_verified_without_xf32_instructions():
    with pytest.raises(audit.TensorAuditError):
        audit.audit_tensor(["v_mfma_f32_32x32x2_f32 a[0:15], v0, v1, a[0:15]"], "fp32", "tf32")
    with pytest.raises(audit.TensorAuditError):
        audit.audit_tensor(["v_mfma_f32_32x32x4_xf32 a[0:15], v[0:1], v[2:3], a[0:15]"], "fp32", "ieee")


def test_fp64_without_mfma_is_simt_and_no_instruction_is_an_error():
    result = audit.audit_tensor(["v_fma_f64 v[0:1], v[2:3], v[4:5], v[0:1]"], "fp64")
    assert (result["execution_kind"], result["native_tensor_verified"]) == ("simt", False)
    with pytest.raises(audit.TensorAuditError):
        audit.audit_tensor(["v_add_f32 v0, v1, v2"], "bf16")


def test_widened_rule_needs_fma_and_both_conversions():
    fp8 = ["v_cvt_pk_f32_fp8_e32 v[0:1], v2", "v_fma_f32 v0, v0, s4, s5", "v_cvt_pk_fp8_f32 v2, v0, v1"]
    assert audit.audit_widened(fp8, "fp8")["native_arithmetic_verified"] is False
    for missing in range(3):
        with pytest.raises(audit.VectorAuditError):
            audit.audit_widened(fp8[:missing] + fp8[missing + 1:], "fp8")
    with pytest.raises(audit.VectorAuditError):
        audit.audit_widened(fp8, "fp4")


def test_vector_rules():
    assert audit.audit_vector(["v_dot4_i32_i8 v0, v0, v1, v2"], "int8", "dp4a")["native_arithmetic_verified"]
    assert audit.audit_vector(["v_dot2_f32_bf16 v0, v1, v2, v3"], "bf16", "dot2")["native_arithmetic_verified"]
    promoted = audit.audit_vector(["v_fma_f32 v0, v1, v2, v3", "v_cvt_pk_bf16_f32 v0, v0, v4"], "bf16", "fma")
    assert promoted["native_arithmetic_verified"] is False and promoted["amdgcn_arithmetic_promoted"]
    with pytest.raises(audit.VectorAuditError):
        audit.audit_vector(["v_mul_lo_u32 v0, v1, v2", "v_add_u32 v0, v0, v3"], "int8", "dp4a")
    with pytest.raises(audit.VectorAuditError):
        audit.audit_vector(["v_mfma_f32_32x32x16_bf16 a[0:15], v[0:3], v[4:7], a[0:15]",
                            "v_fma_f32 v0, v1, v2, v3"], "fp32", "fma")


def test_registered_names_follow_the_mangled_template_arguments():
    symbol = "_ZN2mb12_GLOBAL__N_118tensor_peak_kernelINS_8MfmaBf16ELi128ELi128ELi64ELi2ELi2ELi2ELb0EEEvPKh"
    assert audit.registered_name(symbol) == "tensor_peak_bf16_128x128x64_c2_kn"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_111gemm_kernelINS_9MfmaMxfp4ELi128ELi128ELi256ELi2ELi2ELb1EEEv") \
        == "gemm_mxfp4_128x128x256_checked"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_111copy_kernelIDv4_jLi1ELi1EEEv") == "copy_dwordx4_vpt1_nt"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_111copy_kernelIjLi8ELi2EEEv") == "copy_dword_vpt8_stream"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_118gemm_staged_kernelINS_9MfmaMxfp4EEEvPKh") \
        == "gemm_mxfp4_256x256x256"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_115gemm_dma_kernelINS_11MfmaBf16x16EEEvPKh") \
        == "gemm_bf16_256x256x64"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_115gemm_dma_kernelINS_10MfmaFp8x16EEEvPKh") \
        == "gemm_fp8_256x256x128"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_119gemm_dma_f64_kernelINS_7MfmaF64EEEvPKh") \
        == "gemm_f64_256x128x16"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_117vector_f16_kernelILi8EEEv") == "vector_f16_u8"
    assert audit.registered_name("_ZN2mb12_GLOBAL__N_111fill_kernelILi2EEEvPDv4_jmj") == "fill_dwordx4_stream"
    assert audit.registered_name("unrelated_symbol") is None


# ---- the built library -----------------------------------------------------------

def test_every_registered_kernel_is_in_the_audited_code_object(listing):
    registered = set(_native.kernel_names())
    assert registered, "the library registry is empty"
    assert registered <= set(listing), sorted(registered - set(listing))


def test_every_peak_kernel_runs_only_its_mfma_in_the_timed_loop(listing):
    peak = [name for name in listing if name.startswith("tensor_peak_")]
    assert len(peak) >= 40
    for name in peak:
        fmt = _peak_format(name)
        expected = (PEAK_INSTRUCTION_16 if "_mfma16_" in name else PEAK_INSTRUCTION)[fmt]
        result = audit.audit_tensor(audit.instructions(name), fmt)
        assert result["tensor_instruction_types"] == [expected], name
        summary = audit.loop_summary(name)
        assert summary["timed_loop_matrix_types"] == [expected], name
        assert summary["timed_loop_matrix_instructions"] >= 2, name
        # Only scalar loop control and waits beside the MFMAs; FP64 also moves
        # accumulator halves between AGPRs and VGPRs.
        allowed = {"v_accvgpr_read_b32", "v_accvgpr_write_b32"} if fmt == "fp64" else set()
        assert set(summary["timed_loop_vector_memory_or_alu"]) <= allowed, (name, summary)


def test_every_gemm_kernel_uses_its_format_mfma(listing):
    gemm = [name for name in listing if name.startswith("gemm_")]
    assert gemm
    for name in gemm:
        fmt = FORMAT_OF[name.split("_")[1]]
        # The 256x256 DMA kernels (BF16/FP16/INT8/FP8/FP32) issue the 16x16 form.
        staged16 = fmt in ("bf16", "fp16", "int8", "fp8", "fp32") and "_256x256x" in name and not name.endswith("_checked")
        expected = (PEAK_INSTRUCTION_16 if staged16 else PEAK_INSTRUCTION)[fmt]
        result = audit.audit_tensor(audit.instructions(name), fmt)
        assert result["tensor_instruction_types"] == [expected], name


def test_every_vector_kernel_issues_its_native_instruction_and_no_mfma(listing):
    vector = [name for name in listing if name.startswith("vector_")]
    assert vector
    for name in vector:
        kind = re.match(r"vector_(\w+?)_u\d+$", name).group(1)
        lines = audit.instructions(name)
        if kind == "bf16fma":
            result = audit.audit_vector(lines, "bf16", "fma")
            assert result["native_arithmetic_verified"] is False
            continue
        if kind in ("fp8w", "fp4w"):
            result = audit.audit_widened(lines, kind[:3])
            assert result["native_arithmetic_verified"] is False
            unroll = int(name.rsplit("_u", 1)[1])
            # 8 chains: one FP32 FMA and one narrowing per update in the unrolled body.
            assert result["amdgcn_fp32_fma_instruction_sites"] >= 8 * unroll, (name, result)
            continue
        dtype, instruction = VECTOR_INSTRUCTION[kind]
        result = audit.audit_vector(lines, dtype, "native")
        assert instruction in result["amdgcn_instruction_types"], (name, result)


def test_no_kernel_spills_or_uses_scratch(listing):
    for name in listing:
        info = audit.resources(name)
        assert info["register_spills"] == 0, (name, info)
        assert not info["scratch_bytes"], (name, info)


def test_copy_policies_issue_their_cache_bits(listing):
    for name, load_bits, store_bits in (("copy_dwordx4_vpt1", "", ""), ("copy_dwordx4_vpt1_nt", "nt", "nt"),
                                        ("copy_dwordx4_vpt1_stream", "nt", "sc1")):
        lines = audit.instructions(name)
        loads = [l for l in lines if audit.mnemonic(l) == "global_load_dwordx4"]
        stores = [l for l in lines if audit.mnemonic(l) == "global_store_dwordx4"]
        assert loads and stores, name
        assert all(l.split()[-1] == (load_bits or "off") for l in loads), (name, loads)
        assert all(l.split()[-1] == (store_bits or "off") for l in stores), (name, stores)


def test_no_packed_fp32_valu_anywhere():
    text = native_build.DISASSEMBLY.read_text()
    assert not re.search(r"\bv_pk_(?:add|mul|fma|mov)_f32\b", text)


@pytest.mark.parametrize("name,instruction,mfmas", [("gemm_bf16_256x256x64", "v_mfma_f32_16x16x32_bf16", 256),
                                                     ("gemm_f16_256x256x64", "v_mfma_f32_16x16x32_f16", 256),
                                                     ("gemm_i8_256x256x128", "v_mfma_i32_16x16x64_i8", 256),
                                                     ("gemm_f32_256x256x32", "v_mfma_f32_16x16x4_f32", 1024),
                                                     ("gemm_fp8_256x256x128", "v_mfma_f32_16x16x128_f8f6f4", 128)])
def test_dma_gemm_loop_has_no_accumulator_copies(listing, name, instruction, mfmas):
    """The all-DMA fast path keeps every accumulator in its AGPRs through the
    in-place assembly of the 16x16 forms: the K loop (two 128-byte steps)
    issues its MFMAs, 64 fragment reads and 32 LDS-DMA loads (16 of A, 16 of
    B), no LDS writes, and nothing else on the vector side but the A slot
    address, with no spills."""
    assert name in listing
    resources = audit.resources(name)
    assert resources["register_spills"] == 0 and resources["scratch_bytes"] == 0
    summary = audit.loop_summary(name)
    assert summary["timed_loop_matrix_types"] == [instruction]
    assert summary["timed_loop_matrix_instructions"] == mfmas
    vector = dict(summary["timed_loop_vector_memory_or_alu"])
    assert {k: vector.pop(k, 0) for k in ("ds_read_b128", "ds_write_b128", "buffer_load_dwordx4")} == \
        {"ds_read_b128": 64, "ds_write_b128": 0, "buffer_load_dwordx4": 32}
    assert sum(line.rstrip().endswith(" lds") for line in audit.hot_loop(name)) == 32
    # What remains is the per-step A slot address (the ring of three slots is not a power of two).
    assert set(vector) <= {"v_or_b32_e32", "v_lshl_or_b32", "v_add_u32_e32", "v_readfirstlane_b32"} and \
        sum(vector.values()) <= 16, vector
    assert summary["timed_loop_other_instructions"]["s_barrier"] == 2


def _dma_coverage_violations(body: list[str], horizon=2, trips: int = 4) -> list[tuple[int, int]]:
    """Simulate gfx9's in-order vmcnt over `trips` passes of a loop body.

    An LDS-DMA issued after barrier e is read after barrier e + horizon, so when
    the wave reaches that barrier the waits before it must have retired it.
    `horizon` is a number, or a function of the DMA's ordinal among the DMAs
    issued since the last barrier. Returns (barrier, epoch) for every LDS-DMA
    still outstanding at a barrier its horizon or more barriers after its
    issue, from the second pass on (the first starts empty).
    """
    horizon_of = horizon if callable(horizon) else (lambda ordinal: horizon)
    outstanding: list[tuple[int | None, int]] = []  # (horizon of an LDS-DMA, barriers passed at issue), oldest first
    passed, violations, ordinal = 0, [], 0
    for trip in range(trips):
        for line in body:
            name = audit.mnemonic(line)
            if name.startswith(("buffer_load", "global_load", "buffer_store", "global_store")):
                dma = line.rstrip().endswith(" lds")
                outstanding.append((horizon_of(ordinal) if dma else None, passed))
                ordinal += dma
            elif name == "s_waitcnt":
                match = re.search(r"vmcnt\((\d+)\)", line)
                if match:
                    keep = int(match.group(1))
                    outstanding = outstanding[len(outstanding) - keep:] if keep < len(outstanding) else outstanding
            elif name == "s_barrier":
                reaching = passed + 1
                if trip:
                    violations += [(reaching, epoch) for h, epoch in outstanding if h and epoch <= reaching - h]
                passed, ordinal = reaching, 0
    return violations


def test_fp64_dma_gemm_loop_has_no_accumulator_copies(listing):
    """The 256x128 FP64 fast path: its K loop (two 128-byte steps) issues 256
    in-place v_mfma_f64_16x16x4_f64, 48 fragment reads (12 per wave per step,
    two 16-byte pieces each), 8 B stage writes and 24 buffer loads (8 of B, 16
    LDS-DMA of A), with no spills."""
    name = "gemm_f64_256x128x16"
    assert name in listing
    resources = audit.resources(name)
    assert resources["register_spills"] == 0 and resources["scratch_bytes"] == 0
    summary = audit.loop_summary(name)
    assert summary["timed_loop_matrix_types"] == ["v_mfma_f64_16x16x4_f64"]
    assert summary["timed_loop_matrix_instructions"] == 256
    vector = dict(summary["timed_loop_vector_memory_or_alu"])
    assert {k: vector.pop(k, 0) for k in ("ds_read_b128", "ds_write_b128", "buffer_load_dwordx4")} == \
        {"ds_read_b128": 48, "ds_write_b128": 8, "buffer_load_dwordx4": 24}
    assert set(vector) <= {"v_or_b32_e32", "v_lshl_or_b32", "v_add_u32_e32"} and sum(vector.values()) <= 8, vector
    assert summary["timed_loop_other_instructions"]["s_barrier"] == 2


@pytest.mark.parametrize("name", ["gemm_bf16_256x256x64", "gemm_f16_256x256x64", "gemm_i8_256x256x128",
                                  "gemm_fp8_256x256x128", "gemm_f32_256x256x32"])
def test_all_dma_gemm_loop_waits_cover_every_dma_before_its_reads(listing, name):
    """Both operands arrive by LDS-DMA issued as inline assembly, which the
    compiler's wait counts leave out: the kernel's own vmcnt(8) before each
    barrier orders them. After step kt's barrier a wave issues step kt+2's B
    (read after the next barrier: horizon 1) and then step kt+3's A (read
    after the barrier two steps on: horizon 2). In the compiled loop the waits
    retire every DMA within its horizon; giving A's DMAs B's horizon, or taking
    the waits out, leaves DMAs in flight, and the check sees it."""
    assert name in listing
    body = audit.hot_loop(name)
    assert sum(line.rstrip().endswith(" lds") for line in body) == 32
    b_then_a = lambda ordinal: 1 if ordinal < 8 else 2  # noqa: E731
    assert _dma_coverage_violations(body, horizon=b_then_a) == []
    assert _dma_coverage_violations(body, horizon=1), "A's DMAs are not retired within one barrier"
    unwaited = [line for line in body if not (audit.mnemonic(line) == "s_waitcnt" and "vmcnt" in line)]
    assert _dma_coverage_violations(unwaited, horizon=b_then_a), "the check must see DMAs left in flight"


def test_fp64_dma_gemm_loop_waits_cover_every_dma_before_its_reads(listing):
    """The FP64 kernel's A slots are filled by LDS-DMA issued as inline
    assembly, which the compiler's wait counts leave out: the kernel relies on
    the in-order vmcnt waits its B stage writes take for B loads. In the
    compiled loop, every DMA issued after a step's barrier is retired by the
    waits before the barrier two steps on, after which the step that reads it
    begins. Without those waits (a B path that no longer waits on loads, say)
    DMAs stay in flight, and the check sees it."""
    name = "gemm_f64_256x128x16"
    assert name in listing
    body = audit.hot_loop(name)
    assert sum(line.rstrip().endswith(" lds") for line in body) == 16
    assert _dma_coverage_violations(body) == []
    unwaited = [line for line in body if not (audit.mnemonic(line) == "s_waitcnt" and "vmcnt" in line)]
    assert _dma_coverage_violations(unwaited), "the check must see DMAs left in flight"


def test_mxfp4_gemm_loop_waits_cover_every_scale_dma_before_its_reads(listing):
    """The MXFP4 kernel's scale rows arrive by LDS-DMA three steps ahead: the DMA
    issued in step kt (after barrier kt-1) is read in step kt+2's last substep,
    after barrier kt+2, so the waits must retire it within three barriers. Two
    is too few (the check then reports it), and without the waits it stays in
    flight."""
    body = audit.hot_loop("gemm_mxfp4_256x256x256")
    assert sum(line.rstrip().endswith(" lds") for line in body) == 2
    assert _dma_coverage_violations(body, horizon=3) == []
    assert _dma_coverage_violations(body, horizon=2)
    unwaited = [line for line in body if not (audit.mnemonic(line) == "s_waitcnt" and "vmcnt" in line)]
    assert _dma_coverage_violations(unwaited, horizon=3)
