"""The staging rings against the reference's own transfer-layer tests
(reference tests/connector/test_gds_transfer.py:31-90: backend set, 1 MB
round trip with byte counts, two regions at different offsets, context
manager, missing file), run on device tensors for each ring (the native
ring also in its mapped mode)."""

import asyncio

import pytest
import torch

from daser_amd.store_io import NativeRingIO, PinnedRingIO, preallocate_store

pytestmark = pytest.mark.gpu

RINGS = {"native": NativeRingIO, "python": PinnedRingIO,
         "mmap": lambda path, dev, **kw: NativeRingIO(path, dev, mapped=True, **kw)}


@pytest.fixture()
def store_file(tmp_path):
    path = str(tmp_path / "test.store")
    preallocate_store(path, 4 * 1024 * 1024)
    return path


def _run(coro):
    return asyncio.run(coro)


@pytest.mark.parametrize("ring", RINGS)
def test_backend_is_set(gpu, store_file, ring):
    print(f"case: ring backend {ring}", flush=True)
    io = RINGS[ring](store_file, gpu)
    assert io.backend in ("io_uring", "posix", "threads", "mmap")
    io.close()


@pytest.mark.parametrize("ring", RINGS)
def test_write_and_read_roundtrip(gpu, store_file, ring):
    print(f"case: ring round trip {ring}", flush=True)
    nbytes = 1024 * 1024
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=gpu)
    io = RINGS[ring](store_file, gpu)
    assert _run(io.write_async(src, file_offset=0)) == nbytes
    dst = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
    assert _run(io.read_into_async(dst, file_offset=0)) == nbytes
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    io.close()


@pytest.mark.parametrize("ring", RINGS)
def test_multiple_offsets(gpu, store_file, ring):
    print(f"case: ring offsets {ring}", flush=True)
    size = 512 * 1024
    t1 = torch.ones(size, dtype=torch.uint8, device=gpu)
    t2 = torch.full((size,), 2, dtype=torch.uint8, device=gpu)
    io = RINGS[ring](store_file, gpu)
    _run(io.write_async(t1, file_offset=0))
    _run(io.write_async(t2, file_offset=size))
    r1 = torch.zeros(size, dtype=torch.uint8, device=gpu)
    r2 = torch.zeros(size, dtype=torch.uint8, device=gpu)
    _run(io.read_into_async(r1, file_offset=0))
    _run(io.read_into_async(r2, file_offset=size))
    torch.cuda.synchronize()
    assert torch.equal(t1, r1) and torch.equal(t2, r2)
    io.close()


@pytest.mark.parametrize("ring", RINGS)
def test_context_manager(gpu, store_file, ring):
    print(f"case: ring context manager {ring}", flush=True)
    with RINGS[ring](store_file, gpu) as io:
        assert io.backend
    with pytest.raises(Exception):
        io.read_into_device(torch.zeros(16, dtype=torch.uint8, device=gpu), 0)


@pytest.mark.parametrize("ring", RINGS)
def test_missing_file_raises(gpu, tmp_path, ring):
    print(f"case: ring missing file {ring}", flush=True)
    with pytest.raises(FileNotFoundError):
        RINGS[ring](str(tmp_path / "nonexistent.store"), gpu)


@pytest.mark.parametrize("ring", RINGS)
def test_read_waits_for_earlier_work_on_the_destination(gpu, store_file, ring):
    """A read into a buffer that earlier work on the consumer stream still
    writes (here a delayed fill) lands after that work: the ring's copies
    wait for the consumer stream, so the file's bytes are what remains."""
    print(f"case: ring read ordering {ring}", flush=True)
    nbytes = 2 * 1024 * 1024
    src = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device=gpu)
    io = RINGS[ring](store_file, gpu, slot_bytes=256 * 1024, n_slots=4)
    io.write_from_device(src, 0)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=gpu)
    torch.cuda.synchronize()
    torch.cuda._sleep(100_000_000)  # keeps the fill below pending while the file is read
    dst.fill_(7)
    io.read_into_device(dst, 0)
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    io.close()
