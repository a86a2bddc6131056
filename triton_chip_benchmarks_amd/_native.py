"""ctypes binding of libmi355x_bench.so, the gfx950 C-ABI library.

Every compute entry point of the suite goes through this module. There is no
fallback: a missing or stale library raises NativeLibraryMissing, so a GPU run
can never silently measure something other than the hand-written kernels.
"""

from __future__ import annotations

import ctypes
from pathlib import Path
import threading

PACKAGE = Path(__file__).resolve().parent
LIBRARY_PATH = PACKAGE / "libmi355x_bench.so"
ABI_VERSION = 2  # 2: MXFP4 GEMM scales in K-step blocks (mb_gemm)

MB_OK = 0
MB_ERR_INVALID = -1
MB_ERR_UNSUPPORTED = -2
MB_ERR_HIP = -3
MB_ERR_ALIGNMENT = -4

MB_COPY_NONTEMPORAL = 1
MB_COPY_WRITE_THROUGH = 2

MB_DTYPE_F32 = 0
MB_DTYPE_F16 = 1
MB_DTYPE_BF16 = 2

_ERROR_NAMES = {MB_ERR_INVALID: "invalid argument", MB_ERR_UNSUPPORTED: "unsupported",
                MB_ERR_HIP: "HIP runtime error", MB_ERR_ALIGNMENT: "alignment"}


class NativeLibraryMissing(RuntimeError):
    """libmi355x_bench.so is absent, unloadable or built for another ABI."""


class NativeError(RuntimeError):
    """A C-ABI entry point returned a negative status."""

    def __init__(self, code: int, message: str):
        self.code = code
        super().__init__(f"{_ERROR_NAMES.get(code, 'error')} ({code}): {message}")


class UnsupportedNative(NativeError):
    """MB_ERR_UNSUPPORTED: a valid request without an implemented path."""


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64),
                ("compute_units", ctypes.c_int32), ("wavefront_size", ctypes.c_int32),
                ("clock_khz", ctypes.c_int32), ("memory_clock_khz", ctypes.c_int32),
                ("memory_bus_bits", ctypes.c_int32), ("reserved0", ctypes.c_int32),
                ("l2_cache_bytes", ctypes.c_int64), ("lds_bytes_per_cu", ctypes.c_int64),
                ("total_memory_bytes", ctypes.c_int64), ("free_memory_bytes", ctypes.c_int64)]


class KernelAttributes(ctypes.Structure):
    _fields_ = [("registers_per_thread", ctypes.c_int32), ("max_threads_per_block", ctypes.c_int32),
                ("lds_bytes", ctypes.c_int64), ("scratch_bytes", ctypes.c_int64)]


class PeakConfig(ctypes.Structure):
    _fields_ = [("tile_m", ctypes.c_uint32), ("tile_n", ctypes.c_uint32), ("tile_k", ctypes.c_uint32),
                ("chains", ctypes.c_uint32), ("b_nk", ctypes.c_uint32), ("mfma_m", ctypes.c_uint32),
                ("threads", ctypes.c_uint32)]

    def as_dict(self) -> dict:
        return {field: getattr(self, field) for field, _ in self._fields_}


class GemmConfig(ctypes.Structure):
    _fields_ = [("tile_m", ctypes.c_uint32), ("tile_n", ctypes.c_uint32), ("tile_k", ctypes.c_uint32),
                ("threads", ctypes.c_uint32)]

    def as_dict(self) -> dict:
        return {field: getattr(self, field) for field, _ in self._fields_}


# Matrix formats of the tensor entry points (MB_MATRIX_*).
MATRIX_FORMATS = {"bf16": 0, "fp16": 1, "fp32": 2, "tf32": 3, "int8": 4, "fp64": 5, "fp8": 6, "fp4": 7}

_u64, _u32, _i32, _ptr = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p

# name -> (restype, argtypes). Every symbol here is declared in
# include/mi355x_bench.h; tests check the two lists agree.
SIGNATURES: dict[str, tuple[object, list]] = {
    "mb_abi_version": (_i32, []),
    "mb_last_error": (ctypes.c_char_p, []),
    "mb_device_query": (_i32, [_i32, ctypes.POINTER(DeviceInfo)]),
    "mb_kernel_count": (_i32, []),
    "mb_kernel_name": (ctypes.c_char_p, [_i32]),
    "mb_kernel_attributes_query": (_i32, [ctypes.c_char_p, ctypes.POINTER(KernelAttributes)]),
    "mb_wall_clock_khz": (_i32, [ctypes.POINTER(_i32)]),
    "mb_clock_witness": (_i32, [_ptr, _u64, _u32, _ptr]),
    "mb_copy": (_i32, [_ptr, _ptr, _u64, _u32, _u32, _u32, _u32, _ptr]),
    "mb_fill": (_i32, [_ptr, _u64, _u32, _u32, _u32, _u32, _ptr]),
    "mb_read_sum": (_i32, [_i32, _ptr, _ptr, _u64, _u32, _u32, _ptr]),
    "mb_tensor_peak_configs": (_i32, [_i32, ctypes.POINTER(PeakConfig), _i32]),
    "mb_tensor_peak_kernel_name": (ctypes.c_char_p, [_i32, ctypes.POINTER(PeakConfig)]),
    "mb_tensor_peak": (_i32, [_i32, ctypes.POINTER(PeakConfig), _ptr, _u64, _ptr, _u64, _ptr, _u64, _ptr, _u64,
                              _ptr, _u64, _u32, _u32, _ptr]),
    "mb_gemm_configs": (_i32, [_i32, ctypes.POINTER(GemmConfig), _i32]),
    "mb_gemm_kernel_name": (ctypes.c_char_p, [_i32, ctypes.POINTER(GemmConfig)]),
    "mb_gemm_launched_kernel": (ctypes.c_char_p, [_i32, ctypes.POINTER(GemmConfig), _u32, _u32, _u32, _ptr, _ptr]),
    "mb_gemm": (_i32, [_i32, ctypes.POINTER(GemmConfig), _ptr, _u64, _ptr, _u64, _ptr, _u64, _ptr, _u64, _ptr, _u64,
                       _u32, _u32, _u32, _u32, _ptr]),
    "mb_vector_kernel_name": (ctypes.c_char_p, [_i32, _u32]),
    "mb_vector_chains": (_i32, [_i32, _ptr, _ptr, _ptr, _u64, _u32, _u32, _u32, _u64, _u64, _u64, _ptr]),
}

_lock = threading.Lock()
_library: ctypes.CDLL | None = None


def load(path: Path | None = None) -> ctypes.CDLL:
    """Load the library once and bind every declared signature."""
    global _library
    with _lock:
        if _library is not None and path is None:
            return _library
        target = Path(path) if path is not None else LIBRARY_PATH
        if not target.exists():
            raise NativeLibraryMissing(
                f"{target} is missing; build it with `python -m triton_chip_benchmarks_amd.build` "
                "(or __graft_entry__.build()) before running a benchmark")
        try:
            library = ctypes.CDLL(str(target))
        except OSError as exc:
            raise NativeLibraryMissing(f"cannot load {target}: {exc}") from exc
        missing = []
        for name, (restype, argtypes) in SIGNATURES.items():
            function = getattr(library, name, None)
            if function is None:
                missing.append(name)
                continue
            function.restype = restype
            function.argtypes = argtypes
        if missing:
            raise NativeLibraryMissing(f"{target} lacks {', '.join(missing)}; rebuild it")
        version = library.mb_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryMissing(f"{target} has ABI {version}, expected {ABI_VERSION}; rebuild it")
        if path is None:
            _library = library
        return library


def last_error() -> str:
    return (load().mb_last_error() or b"").decode(errors="replace")


def check(status: int) -> None:
    if status == MB_OK:
        return
    message = last_error()
    if status == MB_ERR_UNSUPPORTED:
        raise UnsupportedNative(status, message)
    raise NativeError(status, message)


def call(name: str, *arguments) -> None:
    check(getattr(load(), name)(*arguments))


def device_query(device: int) -> dict:
    info = DeviceInfo()
    call("mb_device_query", device, ctypes.byref(info))
    return {field: (getattr(info, field).decode(errors="replace") if isinstance(getattr(info, field), bytes)
                    else getattr(info, field)) for field, _ in DeviceInfo._fields_ if field != "reserved0"}


def wall_clock_khz() -> int:
    """Rate of the device's constant real-time counter (the clock witness's time base), in kHz."""
    khz = ctypes.c_int(0)
    call("mb_wall_clock_khz", ctypes.byref(khz))
    return khz.value


def clock_witness(out, microseconds: int, stream=None) -> None:
    """Enqueue the one-wave engine-clock witness on `stream` (a torch stream; default: the current one).

    out: int64 device tensor of 4 entries; after the stream completes it holds shader clock cycles, real-time
    ticks, polls and the starting real-time count (mb_clock_witness).
    """
    import torch

    if out.dtype != torch.int64 or out.numel() < 4 or not out.is_cuda or not out.is_contiguous():
        raise ValueError("clock witness output must be a contiguous int64 device tensor of 4 entries")
    handle = (stream or torch.cuda.current_stream()).cuda_stream
    call("mb_clock_witness", ctypes.c_void_p(out.data_ptr()), out.numel() * 8, int(microseconds),
         ctypes.c_void_p(handle))


def kernel_names() -> list[str]:
    library = load()
    return [library.mb_kernel_name(index).decode() for index in range(library.mb_kernel_count())]


def kernel_attributes(name: str) -> dict:
    attributes = KernelAttributes()
    call("mb_kernel_attributes_query", name.encode(), ctypes.byref(attributes))
    return {field: getattr(attributes, field) for field, _ in KernelAttributes._fields_}


def peak_configs(dtype: str) -> list[dict]:
    """Compiled resident-peak tiles of a matrix format."""
    library = load()
    code = MATRIX_FORMATS[dtype]
    count = library.mb_tensor_peak_configs(code, None, 0)
    if count < 0:
        check(count)
    configs = (PeakConfig * max(count, 1))()
    library.mb_tensor_peak_configs(code, configs, count)
    return [configs[index].as_dict() for index in range(count)]


def peak_config(config: dict) -> PeakConfig:
    return PeakConfig(config["tile_m"], config["tile_n"], config["tile_k"], config["chains"],
                      int(config.get("b_nk", 0)), int(config.get("mfma_m", 0)), int(config.get("threads", 0)))


def peak_kernel_name(dtype: str, config: dict) -> str | None:
    name = load().mb_tensor_peak_kernel_name(MATRIX_FORMATS[dtype], ctypes.byref(peak_config(config)))
    return name.decode() if name else None


def _buffer(tensor):
    if tensor is None:
        return None, 0
    return tensor.data_ptr(), tensor.numel() * tensor.element_size()


def tensor_peak(dtype: str, config: dict, a, b, c, blocks: int, iterations: int, scale_a=None, scale_b=None,
                stream=None) -> None:
    """One launch of the resident-operand peak kernel on the current stream."""
    a_ptr, a_bytes = _buffer(a)
    b_ptr, b_bytes = _buffer(b)
    sa_ptr, sa_bytes = _buffer(scale_a)
    sb_ptr, sb_bytes = _buffer(scale_b)
    c_ptr, c_bytes = _buffer(c)
    call("mb_tensor_peak", MATRIX_FORMATS[dtype], ctypes.byref(peak_config(config)), a_ptr, a_bytes, b_ptr,
         b_bytes, sa_ptr, sa_bytes, sb_ptr, sb_bytes, c_ptr, c_bytes, blocks, iterations,
         stream_handle(stream))


def gemm_configs(dtype: str) -> list[dict]:
    """Compiled GEMM tiles of a matrix format."""
    library = load()
    code = MATRIX_FORMATS[dtype]
    count = library.mb_gemm_configs(code, None, 0)
    if count < 0:
        check(count)
    configs = (GemmConfig * max(count, 1))()
    library.mb_gemm_configs(code, configs, count)
    return [configs[index].as_dict() for index in range(count)]


def _gemm_config(config: dict) -> GemmConfig:
    return GemmConfig(config["tile_m"], config["tile_n"], config["tile_k"], int(config.get("threads", 0)))


def gemm_kernel_name(dtype: str, config: dict) -> str | None:
    name = load().mb_gemm_kernel_name(MATRIX_FORMATS[dtype], ctypes.byref(_gemm_config(config)))
    return name.decode() if name else None


def gemm_launched_kernel(dtype: str, config: dict, m: int, n: int, k: int, scale_a=None, scale_b=None) -> str:
    """Registered name of the kernel mb_gemm launches for this shape (fast or checked path)."""
    name = load().mb_gemm_launched_kernel(MATRIX_FORMATS[dtype], ctypes.byref(_gemm_config(config)), m, n, k,
                                          _buffer(scale_a)[0], _buffer(scale_b)[0])
    if not name:
        raise NativeError(last_error())
    return name.decode()


def gemm(dtype: str, config: dict, a, b, c, m: int, n: int, k: int, scale_a=None, scale_b=None, group_m: int = 0,
         stream=None) -> None:
    """C = A . B^T-stored (both K-contiguous) on the current stream."""
    a_ptr, a_bytes = _buffer(a)
    b_ptr, b_bytes = _buffer(b)
    sa_ptr, sa_bytes = _buffer(scale_a)
    sb_ptr, sb_bytes = _buffer(scale_b)
    c_ptr, c_bytes = _buffer(c)
    call("mb_gemm", MATRIX_FORMATS[dtype], ctypes.byref(_gemm_config(config)), a_ptr, a_bytes, b_ptr, b_bytes,
         sa_ptr, sa_bytes, sb_ptr, sb_bytes, c_ptr, c_bytes, m, n, k, group_m, stream_handle(stream))


def stream_handle(stream=None) -> int | None:
    """The raw hipStream_t of a torch stream (the current one by default)."""
    import torch

    if stream is None:
        stream = torch.cuda.current_stream()
    handle = stream.cuda_stream
    return handle or None
