"""The C-ABI library loads, and exports exactly what include/*.h declares.

CPU-only: no entry point that launches work is called here.
"""

from pathlib import Path
import re

import pytest

from triton_chip_benchmarks_amd import _native

ROOT = Path(__file__).resolve().parent.parent
HEADERS = sorted((ROOT / "include").glob("*.h"))


def declared_functions():
    names = set()
    for header in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        for match in re.finditer(r"\b(mb_[a-z0-9_]+)\s*\(", text):
            names.add(match.group(1))
    return names


def test_headers_exist_and_declare_entry_points():
    assert HEADERS, "include/*.h must declare the C-ABI"
    assert {"mb_copy", "mb_read_sum", "mb_device_query", "mb_last_error"} <= declared_functions()


def test_library_exports_every_declared_symbol():
    library = _native.load()
    missing = [name for name in sorted(declared_functions()) if not hasattr(library, name)]
    assert not missing, f"declared but not exported: {missing}"


def test_python_binding_covers_exactly_the_header():
    assert set(_native.SIGNATURES) == declared_functions()


def test_abi_version_and_error_channel():
    library = _native.load()
    assert library.mb_abi_version() == _native.ABI_VERSION
    assert isinstance(_native.last_error(), str)


def test_kernel_registry_names_are_unique_and_cover_the_memory_kernels():
    names = _native.kernel_names()
    assert len(names) == len(set(names))
    assert {"copy_dwordx4_vpt4_nt", "copy_tail", "read_sum_f32_vec"} <= set(names)


def test_invalid_arguments_are_rejected_before_any_launch():
    # Argument checks run on the host before the HIP runtime is touched.
    library = _native.load()
    assert library.mb_copy(None, None, 64, 256, 4, 0, 0, None) == _native.MB_ERR_INVALID
    assert "NULL" in _native.last_error()
    assert library.mb_copy(1 << 20, 2 << 20, 64, 100, 4, 0, 0, None) == _native.MB_ERR_INVALID
    assert library.mb_copy(1 << 20, 2 << 20, 64, 256, 3, 0, 0, None) == _native.MB_ERR_INVALID
    assert library.mb_copy(1 << 20, (1 << 20) + 16, 64, 256, 4, 0, 0, None) == _native.MB_ERR_INVALID
    assert "overlap" in _native.last_error()
    assert library.mb_copy(1 << 20, 2 << 20, 64, 256, 4, 0, 4, None) == _native.MB_ERR_INVALID  # unknown flag
    assert "flags" in _native.last_error()
    assert library.mb_read_sum(0, 1 << 20, 2 << 20, 100, 100, 256, None) == _native.MB_ERR_INVALID
    assert library.mb_read_sum(7, 1 << 20, 2 << 20, 100, 1024, 256, None) == _native.MB_ERR_INVALID
    assert library.mb_copy(None, None, 0, 256, 4, 0, 0, None) == _native.MB_OK  # empty copy is a no-op


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_native.NativeLibraryMissing):
        _native.load(tmp_path / "absent.so")


def test_tensor_peak_tables_and_host_side_rejections():
    """Config enumeration and argument checks run on the host, before any launch."""
    import ctypes

    library = _native.load()
    for dtype in ("bf16", "fp16", "fp32", "int8", "fp64", "fp8", "fp4"):
        configs = _native.peak_configs(dtype)
        assert configs, dtype
        assert {c["b_nk"] for c in configs} == {0, 1}
        for config in configs:
            name = _native.peak_kernel_name(dtype, config)
            assert name and name in _native.kernel_names()
    tf32 = _native.MATRIX_FORMATS["tf32"]
    assert library.mb_tensor_peak_configs(tf32, None, 0) == _native.MB_ERR_UNSUPPORTED
    assert "xf32" in _native.last_error()
    config = _native.peak_config(_native.peak_configs("bf16")[0])
    bad = _native.peak_config({"tile_m": 48, "tile_n": 48, "tile_k": 48, "chains": 2})
    fake = 1 << 20  # never dereferenced: every call below fails its host-side checks
    assert library.mb_tensor_peak(tf32, ctypes.byref(config), fake, 1 << 30, fake, 1 << 30, None, 0, None, 0,
                                  fake, 1 << 30, 1, 1, None) == _native.MB_ERR_UNSUPPORTED
    assert library.mb_tensor_peak(0, ctypes.byref(bad), fake, 1 << 30, fake, 1 << 30, None, 0, None, 0,
                                  fake, 1 << 30, 1, 1, None) == _native.MB_ERR_INVALID
    assert library.mb_tensor_peak(0, ctypes.byref(config), fake, 16, fake, 1 << 30, None, 0, None, 0,
                                  fake, 1 << 30, 1, 1, None) == _native.MB_ERR_INVALID
    assert "too small" in _native.last_error()
    assert library.mb_tensor_peak(0, ctypes.byref(config), fake, 1 << 30, fake, 1 << 30, None, 0, None, 0,
                                  fake, 1 << 30, 1, 0, None) == _native.MB_ERR_INVALID
    fp4 = _native.peak_config(_native.peak_configs("fp4")[0])
    assert library.mb_tensor_peak(7, ctypes.byref(fp4), fake, 1 << 30, fake, 1 << 30, None, 0, None, 0,
                                  fake, 1 << 30, 1, 1, None) == _native.MB_ERR_INVALID
    assert "scales" in _native.last_error()


def test_vector_kernels_and_host_side_rejections():
    library = _native.load()
    for kind in (0, 1, 2, 3, 4, 5):
        for unroll in (1, 4, 8, 16):
            name = library.mb_vector_kernel_name(kind, unroll)
            assert name and name.decode() in _native.kernel_names()
    assert library.mb_vector_kernel_name(0, 3) is None
    fake = 1 << 20  # never dereferenced: every call below fails its host-side checks
    for kind in (6, 7):  # FP8 / FP4 have no VALU arithmetic on gfx950
        assert library.mb_vector_chains(kind, fake, fake, fake, 64, 1, 1, 64, 1 << 20, 1 << 20, 64,
                                        None) == _native.MB_ERR_UNSUPPORTED
    assert library.mb_vector_chains(0, fake, fake, fake, 100, 4, 1, 64, 1 << 20, 1 << 20, 64,
                                    None) == _native.MB_ERR_INVALID  # elements not a multiple of 64
    assert library.mb_vector_chains(0, fake, fake, fake, 64, 6, 4, 64, 1 << 20, 1 << 20, 64,
                                    None) == _native.MB_ERR_INVALID  # iterations not a multiple of unroll
    assert library.mb_vector_chains(0, fake, fake, fake, 64, 4, 4, 64, 16, 1 << 20, 64,
                                    None) == _native.MB_ERR_INVALID  # input too small
    assert "too small" in _native.last_error()
