"""Compile the oracle's C restatement (oracle/c/*.c) into oracle/_build/.

Test infrastructure only. Built with gcc at -O2 with floating-point
contraction off, so every product and sum in the emulation rounds exactly as
written (no fused multiply-add is formed behind the code's back).
"""

from __future__ import annotations

from pathlib import Path
import shutil
import subprocess

HERE = Path(__file__).resolve().parent
SOURCES = sorted((HERE / "c").glob("*.c"))
BUILD = HERE / "_build"
LIBRARY = BUILD / "liboracle.so"


def build() -> Path:
    compiler = shutil.which("gcc") or shutil.which("cc")
    if compiler is None:
        raise RuntimeError("gcc is required to build the oracle's C restatement")
    BUILD.mkdir(exist_ok=True)
    temporary = LIBRARY.with_name(LIBRARY.name + ".tmp")
    command = [compiler, "-O2", "-std=c99", "-ffp-contract=off", "-fno-fast-math", "-shared", "-fPIC",
               *map(str, SOURCES), "-o", str(temporary), "-lm"]
    completed = subprocess.run(command, capture_output=True, text=True)
    if completed.returncode:
        raise RuntimeError(f"oracle build failed:\n{' '.join(command)}\n{completed.stderr}")
    temporary.replace(LIBRARY)
    return LIBRARY


def library_path() -> Path:
    """The built library, building it on first use when the sources are present."""
    if not LIBRARY.exists() or any(source.stat().st_mtime > LIBRARY.stat().st_mtime for source in SOURCES):
        build()
    return LIBRARY


if __name__ == "__main__":
    print(build())
