"""GPU parity of the memory kernels (mb_copy, mb_read_sum) against oracle.memory.

Copy is bit-exact; block sums stay within the reference's float32 summation
bound (bench_bandwidth.py:81-110). Cases cover ragged sizes, every access
width (16-byte, dword, byte), misaligned pointers, grid-stride launches and the
headline size of 2^28 fp32 through size-independent properties.
"""

import numpy as np
import pytest

from oracle import memory

pytestmark = pytest.mark.gpu


def _uniform(torch, n, seed, dtype=None, device="cuda"):
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    return torch.empty(n, device=device, dtype=dtype or torch.float32).uniform_(-1, 1, generator=generator)


def _bits(tensor):
    return tensor.cpu().contiguous().view(-1).numpy().view(np.uint8)


@pytest.mark.parametrize("elements", [1, 3, 63, 64, 1000, 4096 + 17, (1 << 20) + 5])
@pytest.mark.parametrize("vpt,nontemporal", [(1, False), (4, True), (16, False), (1, "stream"), (8, "stream")])
def test_copy_ragged_sizes_bit_exact(gpu, elements, vpt, nontemporal):
    import torch

    from triton_chip_benchmarks_amd.bench_bandwidth import launch_copy

    print(f"copy elements={elements} vpt={vpt} nt={nontemporal}", flush=True)
    src = _uniform(torch, elements, seed=elements)
    dst = torch.full_like(src, float("nan"))
    launch_copy(src, dst, 256, vpt, 0, nontemporal)
    torch.cuda.synchronize()
    assert (_bits(dst) == _bits(torch.from_numpy(memory.copy(src.cpu().numpy())))).all()


@pytest.mark.parametrize("flags", [0, 3])
@pytest.mark.parametrize("offset_bytes", [4, 1, 3])
def test_copy_misaligned_pointers_take_narrow_accesses(gpu, offset_bytes, flags):
    import torch

    from triton_chip_benchmarks_amd import _native

    print(f"misaligned copy offset={offset_bytes} flags={flags}", flush=True)
    raw = torch.randint(0, 256, (1 << 16,), dtype=torch.uint8, device="cuda")
    out = torch.zeros_like(raw)
    count = (1 << 16) - 64
    _native.call("mb_copy", raw.data_ptr() + offset_bytes, out.data_ptr() + offset_bytes, count, 256, 2, 0, flags,
                 _native.stream_handle())
    torch.cuda.synchronize()
    got, want = out.cpu().numpy(), raw.cpu().numpy()
    assert (got[offset_bytes:offset_bytes + count] == want[offset_bytes:offset_bytes + count]).all()
    assert not got[:offset_bytes].any() and not got[offset_bytes + count:].any()  # nothing outside the range


@pytest.mark.parametrize("grid_blocks", [1, 7, 512])
def test_copy_grid_stride_covers_every_vector(gpu, grid_blocks):
    import torch

    from triton_chip_benchmarks_amd.bench_bandwidth import launch_copy

    print(f"grid-stride copy grid={grid_blocks}", flush=True)
    src = _uniform(torch, (3 << 18) + 9, seed=grid_blocks)
    dst = torch.full_like(src, float("nan"))
    launch_copy(src, dst, 512, 2, grid_blocks, False)
    torch.cuda.synchronize()
    assert torch.equal(src.view(torch.int32), dst.view(torch.int32))


def test_copy_baseline_size_full_buffer(gpu):
    """2^28 fp32 (1 GiB): full bit equality on the device plus an oracle sample."""
    import torch

    from triton_chip_benchmarks_amd.bench_bandwidth import launch_copy

    print("copy 2^28 fp32", flush=True)
    src = _uniform(torch, 1 << 28, seed=0)
    dst = torch.full_like(src, float("nan"))
    launch_copy(src, dst, 256, 4, 0, True)
    torch.cuda.synchronize()
    assert torch.equal(src.view(torch.int32), dst.view(torch.int32))
    head, tail = slice(0, 1 << 16), slice((1 << 28) - (1 << 16), 1 << 28)
    for part in (head, tail):
        assert (_bits(dst[part]) == _bits(torch.from_numpy(memory.copy(src[part].cpu().numpy())))).all()
    del src, dst


@pytest.mark.parametrize("dtype_name", ["fp32", "fp16", "bf16"])
@pytest.mark.parametrize("block", [64, 1024, 16384])
@pytest.mark.parametrize("elements", [1, 1000, 65536 + 17])
def test_read_block_sums_within_reference_bound(gpu, dtype_name, block, elements):
    import torch

    from triton_chip_benchmarks_amd.bench_bandwidth import launch_read, torch_dtype

    print(f"read {dtype_name} block={block} elements={elements}", flush=True)
    src = _uniform(torch, elements, seed=block + elements, dtype=torch_dtype(dtype_name))
    sink = torch.full((-(-elements // block),), float("nan"), device="cuda")
    launch_read(src, sink, block, 256)
    torch.cuda.synchronize()
    memory.check_read(src.float().cpu().numpy(), sink.cpu().numpy(), block)


def test_read_exact_on_integer_lattice(gpu):
    """Small integers sum exactly in float32: any dropped or doubled element shows."""
    import torch

    from triton_chip_benchmarks_amd.bench_bandwidth import launch_read

    values = torch.randint(-8, 9, ((1 << 20) + 3,), device="cuda").float()
    sink = torch.full((-(-values.numel() // 4096),), float("nan"), device="cuda")
    launch_read(values, sink, 4096, 512)
    torch.cuda.synchronize()
    expected = memory.block_sums(values.cpu().numpy(), 4096)
    assert np.array_equal(sink.cpu().numpy().astype(np.float64), expected)


@pytest.mark.parametrize("nbytes", [1, 15, 16, 17, 4096 + 9, (1 << 22) + 3])
@pytest.mark.parametrize("threads,grid_blocks,policy", [(64, 0, "stream"), (256, 0, "off"), (1024, 0, "on"),
                                                        (256, 3, "stream")])
def test_fill_writes_every_byte_and_nothing_past_the_end(gpu, nbytes, threads, grid_blocks, policy):
    """mb_fill: every byte of a ragged buffer holds its byte of the little-endian pattern (the 16-byte body
    and the byte tail), and the guard bytes after the buffer are untouched; a small grid strides over all."""
    import torch

    from triton_chip_benchmarks_amd import _native
    from triton_chip_benchmarks_amd.bench_bandwidth import COPY_POLICIES

    print(f"fill bytes={nbytes} threads={threads} grid={grid_blocks} policy={policy}", flush=True)
    pattern = 0xA1B2C3D4
    buffer = torch.full((nbytes + 64,), 0x5A, dtype=torch.uint8, device="cuda")
    _native.call("mb_fill", buffer.data_ptr(), nbytes, pattern, threads, grid_blocks, COPY_POLICIES[policy],
                 _native.stream_handle())
    torch.cuda.synchronize()
    host = buffer.cpu().numpy()
    expected = np.frombuffer(np.array([pattern], dtype="<u4").tobytes(), dtype=np.uint8)[np.arange(nbytes) % 4]
    assert np.array_equal(host[:nbytes], expected)
    assert (host[nbytes:] == 0x5A).all()


def test_fill_refuses_bad_arguments(gpu):
    import torch

    from triton_chip_benchmarks_amd import _native

    library = _native.load()
    buffer = torch.zeros(64, dtype=torch.uint8, device="cuda")
    assert library.mb_fill(None, 16, 0, 64, 0, 0, None) == _native.MB_ERR_INVALID
    assert library.mb_fill(buffer.data_ptr() + 4, 16, 0, 64, 0, 0, None) == _native.MB_ERR_ALIGNMENT
    assert library.mb_fill(buffer.data_ptr(), 16, 0, 65, 0, 0, None) == _native.MB_ERR_INVALID
    assert library.mb_fill(buffer.data_ptr(), 16, 0, 64, 0, 8, None) == _native.MB_ERR_INVALID
    assert "mb_fill" in _native.last_error()
    assert library.mb_fill(buffer.data_ptr(), 0, 0, 64, 0, 0, None) == _native.MB_OK


def test_fill_baseline_size_full_buffer(gpu):
    """The write-only leg of the copy bound at the copy's size: 2^28 fp32 words all 1.0 afterwards."""
    import torch

    from triton_chip_benchmarks_amd.bench_bandwidth import check_fill, launch_fill

    print("fill 2^28 fp32", flush=True)
    dst = torch.full((1 << 28,), float("nan"), device="cuda")
    launch_fill(dst, 256, 0, "stream")
    torch.cuda.synchronize()
    check_fill(dst)
    assert bool((dst == 1.0).all())
