"""Build libmi355x_bench.so (gfx950) in-tree and record its audit artefacts.

Outputs, all inside the package directory:
  libmi355x_bench.so              the C-ABI library loaded through ctypes
  _build/<unit>.o                 per-translation-unit objects
  _build/<unit>.gfx950.s          device assembly with the AMDHSA metadata
                                  (VGPR/AGPR/SGPR counts, LDS, scratch, spills)
  _build/<unit>.gfx950.co         each object's gfx950 code object (embedded in the .so)
  _build/libmi355x_bench.gfx950.isa  llvm-objdump disassembly of all of them

The instruction audit reads the disassembly of the code object that the
library actually launches, so the audited instructions are the executed ones.
"""

from __future__ import annotations

import argparse
from concurrent.futures import ThreadPoolExecutor
import os
from pathlib import Path
import shutil
import subprocess
import sys

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
INCLUDE = PACKAGE.parent / "include"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libmi355x_bench.so"
DISASSEMBLY = BUILD / "libmi355x_bench.gfx950.isa"
ARCH = "gfx950"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
LLVM_BIN = ROCM / "llvm" / "bin"

# Packed FP32 VALU forms are kept out of every kernel: hipcc would otherwise
# form v_pk_{add,mul,fma}_f32 from ordinary float code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++17", f"--offload-arch={ARCH}", "-fPIC", f"-I{INCLUDE}",
                "-Wall", "-Wno-unused-command-line-argument", "-Wno-unknown-warning-option",
                *DEVICE_FLAGS]


def _hipcc() -> str:
    path = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    if not Path(path).exists():
        raise SystemExit("hipcc not found; a ROCm toolchain is required to build the gfx950 kernels")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _run(command: list[str], what: str) -> None:
    completed = subprocess.run(command, capture_output=True, text=True)
    if completed.returncode:
        # hipcc's host pass warns that it does not know the packed-fp32 feature;
        # only real failures reach this point.
        raise RuntimeError(f"{what} failed ({completed.returncode}):\n{' '.join(command)}\n"
                           f"{completed.stdout}\n{completed.stderr}")


# Per-source device flags. mb_tensor_peak_vgpr.hip holds resident-peak tiles
# that fit the architectural VGPRs; built with the VGPR form of v_mfma, their
# accumulators stay in one register file instead of being copied between AGPRs
# and VGPRs inside the timed loop. (The option is per compilation unit, and the
# larger tiles need AGPRs, so they stay in mb_tensor_peak.hip.)
SOURCE_FLAGS = {"mb_tensor_peak_vgpr.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _compile(source: Path) -> Path:
    flags = [*COMMON_FLAGS, *SOURCE_FLAGS.get(source.name, [])]
    obj = BUILD / (source.stem + ".o")
    _run([_hipcc(), *flags, "-c", str(source), "-o", str(obj)], f"compile {source.name}")
    asm = BUILD / f"{source.stem}.{ARCH}.s"
    _run([_hipcc(), *flags, "--offload-device-only", "-S", str(source), "-o", str(asm)],
         f"device assembly {source.name}")
    return obj


def _extract_code_objects(objects: list[Path]) -> None:
    """Unbundle each object's gfx950 code object and disassemble all of them.

    Every object file carries its own HIP fat binary, and the linked library
    embeds them side by side, so the per-object code objects are exactly the
    device code the library launches.
    """
    listings = []
    for obj in objects:
        fatbin = BUILD / f"{obj.stem}.hip_fatbin"
        code_object = BUILD / f"{obj.stem}.{ARCH}.co"
        dumped = subprocess.run([str(LLVM_BIN / "llvm-objcopy"), "--dump-section", f".hip_fatbin={fatbin}",
                                 str(obj), str(BUILD / "objcopy.discard")], capture_output=True, text=True)
        (BUILD / "objcopy.discard").unlink(missing_ok=True)
        if dumped.returncode and "not found" in dumped.stderr:
            continue  # a host-only translation unit has no device code
        if dumped.returncode:
            raise RuntimeError(f"extract the fat binary of {obj.name} failed:\n{dumped.stderr}")
        _run([str(LLVM_BIN / "clang-offload-bundler"), "--unbundle", "--type=o",
              f"--targets=hipv4-amdgcn-amd-amdhsa--{ARCH}", f"--input={fatbin}",
              f"--output={code_object}"], f"unbundle {obj.name}")
        fatbin.unlink()
        completed = subprocess.run([str(LLVM_BIN / "llvm-objdump"), "-d", f"--mcpu={ARCH}",
                                    "--no-show-raw-insn", str(code_object)],
                                   capture_output=True, text=True)
        if completed.returncode:
            raise RuntimeError(f"llvm-objdump failed on {code_object}:\n{completed.stderr}")
        listings.append(completed.stdout)
    DISASSEMBLY.write_text("\n".join(listings))


def build(verbose: bool = True) -> Path:
    """Compile every HIP source for gfx950 and link the C-ABI library."""
    BUILD.mkdir(exist_ok=True)
    units = sources()
    if not units:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = max(1, min(len(units), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(_compile, units))
    temporary = LIBRARY.with_name(LIBRARY.name + ".tmp")
    _run([_hipcc(), "-shared", f"--offload-arch={ARCH}", *objects_as_str(objects), "-o", str(temporary)],
         "link libmi355x_bench.so")
    temporary.replace(LIBRARY)
    _extract_code_objects(objects)
    if verbose:
        print(f"built {LIBRARY.relative_to(PACKAGE.parent)} from {len(units)} sources "
              f"({', '.join(unit.name for unit in units)})")
    return LIBRARY


def objects_as_str(objects: list[Path]) -> list[str]:
    return [str(obj) for obj in objects]


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    parser.add_argument("--quiet", action="store_true")
    args = parser.parse_args(argv)
    build(verbose=not args.quiet)
    return 0


if __name__ == "__main__":
    sys.exit(main())
