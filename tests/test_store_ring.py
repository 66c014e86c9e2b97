"""The native staging ring (dsr_ring_*) in host mode on the CPU: io_uring and
pread/pwrite paths, more pieces than slots, and its error reporting. The
device path is covered by tests/test_connector_gpu.py."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from daser_amd.store_io import NativeRingIO, StoreIOError, preallocate_store


@pytest.fixture()
def store(tmp_path):
    path = str(tmp_path / "daser.store")
    preallocate_store(path, 4 << 20)
    return path


MODES = {"io_uring": dict(use_io_uring=True), "posix": dict(use_io_uring=False),
         "mmap": dict(mapped=True)}


@pytest.mark.parametrize("mode", list(MODES))
def test_round_trip_many_pieces(store, mode):
    rng = np.random.default_rng(len(mode))
    src = torch.from_numpy(rng.integers(0, 256, 1_000_003, dtype=np.uint8))
    with NativeRingIO(store, "cpu", slot_bytes=65536, n_slots=3, **MODES[mode]) as io:
        if mode == "io_uring":
            assert io.uses_io_uring
        assert io.backend == ("mmap" if mode == "mmap" else io.backend)
        assert io.write_from_device(src, 8192) == src.numel()
        dst = torch.zeros_like(src)
        io.read_into_device(dst, 8192)
    assert torch.equal(src, dst)
    with open(store, "rb") as f:
        f.seek(8192)
        assert f.read(src.numel()) == src.numpy().tobytes()


def test_interleaved_transfers_and_single_slot(store):
    with NativeRingIO(store, "cpu", slot_bytes=4096, n_slots=1) as io:
        a = torch.arange(10_000, dtype=torch.int32)
        b = -torch.arange(7_000, dtype=torch.int32)
        io.write_from_device(a, 0)
        io.write_from_device(b, 65536)
        ra, rb = torch.zeros_like(a), torch.zeros_like(b)
        io.read_into_device(rb, 65536)
        io.read_into_device(ra, 0)
    assert torch.equal(a, ra) and torch.equal(b, rb)


def test_missing_file(tmp_path):
    with pytest.raises(FileNotFoundError):
        NativeRingIO(str(tmp_path / "absent"), "cpu")


@pytest.mark.parametrize("mode", list(MODES))
def test_read_past_end_is_an_error(store, mode):
    with NativeRingIO(store, "cpu", slot_bytes=8192, n_slots=2, **MODES[mode]) as io:
        with pytest.raises(StoreIOError):
            io.read_into_device(torch.zeros(100_000, dtype=torch.uint8), (4 << 20) - 5000)
        # the ring keeps working afterwards
        t = torch.ones(10, dtype=torch.uint8)
        io.write_from_device(t, 0)


@pytest.mark.skipif(not os.path.exists("/dev/full"), reason="needs /dev/full")
@pytest.mark.parametrize("uring", [True, False])
def test_write_failure_reports_errno(uring):
    with NativeRingIO("/dev/full", "cpu", slot_bytes=4096, n_slots=2, use_io_uring=uring) as io:
        with pytest.raises(StoreIOError, match="space"):
            io.write_from_device(torch.ones(20_000, dtype=torch.uint8), 0)


def test_closed_ring_refuses(store):
    io = NativeRingIO(store, "cpu")
    io.close()
    io.close()
    with pytest.raises(StoreIOError):
        io.write_from_device(torch.ones(4, dtype=torch.uint8), 0)


def _direct_ring(store, **kw):
    from daser_amd._lib import DSR_ERR_IO, DaserKVError

    try:
        return NativeRingIO(store, "cpu", direct=True, **kw)
    except DaserKVError as e:
        if e.code == DSR_ERR_IO:
            pytest.skip("file system without O_DIRECT")
        raise


@pytest.mark.parametrize("uring", [True, False])
def test_direct_io_round_trip_and_alignment(store, uring):
    """O_DIRECT mode: 4 KiB-aligned transfers round-trip through the file;
    unaligned offsets, sizes or slot sizes are DSR_ERR_ALIGN before any I/O."""
    from daser_amd._lib import DSR_ERR_ALIGN, DaserKVError

    src = torch.from_numpy(np.random.default_rng(4).integers(0, 256, 1 << 20, dtype=np.uint8))
    with _direct_ring(store, slot_bytes=65536, n_slots=3, use_io_uring=uring) as io:
        io.write_from_device(src, 8192)
        dst = torch.zeros_like(src)
        io.read_into_device(dst, 8192)
        assert torch.equal(src, dst)
        for n, off in ((4096, 100), (1000, 4096)):
            with pytest.raises(DaserKVError) as e:
                io.write_from_device(src[:n], off)
            assert e.value.code == DSR_ERR_ALIGN
        io.read_into_device(dst[:4096], 8192)  # still usable
    with open(store, "rb") as f:
        f.seek(8192)
        assert f.read(src.numel()) == src.numpy().tobytes()
    with pytest.raises(DaserKVError) as e:
        NativeRingIO(store, "cpu", slot_bytes=5000, direct=True)
    assert e.value.code == DSR_ERR_ALIGN


def test_mapped_write_past_the_end_extends_the_file(store):
    """A mapped ring writes beyond the end of the file through pwrite (the
    mapping cannot grow the file); later reads there are mapped."""
    rng = np.random.default_rng(8)
    data = torch.from_numpy(rng.integers(0, 256, 300_000, dtype=np.uint8))
    end = 4 << 20
    with NativeRingIO(store, "cpu", slot_bytes=65536, n_slots=4, mapped=True) as io:
        io.write_from_device(data, end - 1000)
        assert os.path.getsize(store) == end - 1000 + data.numel()
        back = torch.zeros_like(data)
        io.read_into_device(back, end - 1000)
        assert torch.equal(back, data)
        # inside the file again: overwrite part of it through the mapping
        io.write_from_device(data[:5000], 0)
        io.read_into_device(back[:5000], 0)
        assert torch.equal(back[:5000], data[:5000])


def test_mapped_write_keeps_neighbour_bytes(store):
    """A mapped write changes exactly its range: bytes of the pages at its
    ends that lie outside it keep their values."""
    rng = np.random.default_rng(9)
    base = torch.from_numpy(rng.integers(1, 256, 3 * 4096, dtype=np.uint8))
    with NativeRingIO(store, "cpu", slot_bytes=8192, n_slots=2) as plain:
        plain.write_from_device(base, 40960)
    patch = torch.zeros(4096 + 100, dtype=torch.uint8)
    with NativeRingIO(store, "cpu", slot_bytes=8192, n_slots=2, mapped=True) as io:
        io.write_from_device(patch, 40960 + 2000)
    want = base.clone()
    want[2000:2000 + patch.numel()] = 0
    with open(store, "rb") as f:
        f.seek(40960)
        got = np.frombuffer(f.read(want.numel()), np.uint8)
    assert np.array_equal(got, want.numpy())


def test_mapped_and_direct_are_exclusive(store):
    from daser_amd._lib import DSR_ERR_ARG, DaserKVError

    with pytest.raises(DaserKVError) as e:
        NativeRingIO(store, "cpu", slot_bytes=8192, mapped=True, direct=True)
    assert e.value.code == DSR_ERR_ARG


@pytest.mark.parametrize("mode", list(MODES))
def test_randomized_transfers_from_several_threads(tmp_path, mode):
    """Random sizes and offsets (pieces shorter and longer than a slot, odd
    lengths) from four threads, each with its own ring on one file over
    disjoint regions, and a shared ring used by two threads at once (its
    calls serialise): the file and every read back equal a host model."""
    import threading

    path = str(tmp_path / "daser.store")
    size = 8 << 20
    preallocate_store(path, size)
    model = np.zeros(size, np.uint8)
    shared = NativeRingIO(path, "cpu", slot_bytes=8192, n_slots=3, **MODES[mode])
    errors = []

    def worker(t: int, ring) -> None:
        try:
            rng = np.random.default_rng(100 + t)
            lo = t * (size // 6)
            for _ in range(40):
                n = int(rng.integers(1, 60_000))
                off = lo + int(rng.integers(0, size // 6 - n))
                data = rng.integers(0, 256, n, dtype=np.uint8)
                ring.write_from_device(torch.from_numpy(data), off)
                model[off:off + n] = data
                back = torch.zeros(n, dtype=torch.uint8)
                ring.read_into_device(back, off)
                assert np.array_equal(back.numpy(), data), f"thread {t}"
        except BaseException as e:  # reported on the main thread
            errors.append(e)

    own = [NativeRingIO(path, "cpu", slot_bytes=int(s), n_slots=int(k), **MODES[mode])
           for s, k in ((4096, 1), (16384, 2), (65536, 4), (5000 * 16, 3))]
    threads = [threading.Thread(target=worker, args=(t, r)) for t, r in enumerate(own)]
    threads += [threading.Thread(target=worker, args=(4 + t, shared)) for t in range(2)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    for r in own + [shared]:
        r.close()
    assert not errors, errors[0]
    with open(path, "rb") as f:
        assert np.array_equal(np.frombuffer(f.read(), np.uint8), model)


def test_ring_host_code_under_sanitizers():
    """The C++ ring's host path under ASan + UBSan (tests/c/ring_sanitize.cpp,
    built by the package build where the sanitizer runtimes exist)."""
    import subprocess

    exe = os.path.join(os.path.dirname(os.path.abspath(__file__)), "c", "ring_sanitize")
    if not os.path.exists(exe):
        pytest.skip("ring sanitizer driver not built (no sanitizer runtimes)")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0 and "ring sanitize ok" in r.stdout, r.stdout + r.stderr
