"""The HBM ceiling probes behind bench.py's hbm_ceilings move the bytes they
are timed for: the copy stream's destination equals its source, the write
stream fills every unit, and bad arguments are refused before any launch."""

from __future__ import annotations

import ctypes
import os

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "daser_amd", "libdaser_bwprobe.so")


def _probe():
    lib = ctypes.CDLL(LIB)
    fn = lib.dsr_bw_probe
    fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64,
                   ctypes.c_int64, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    return fn


def test_probe_refuses_bad_arguments():
    fn = _probe()
    assert fn(5, 16, 16, 1 << 20, 16384, 1, 16, None) == -1      # unknown stream
    assert fn(4, 16, 16, 8 * 16384, 16384, 1, 16, None) == -1    # 8 units: not 16 per group
    assert fn(3, None, 16, 1 << 20, 16384, 1, 16, None) == -1    # no permutation
    assert fn(2, 16, 16, 1 << 20, 1000, 1, 16, None) == -1       # unit not 4 KiB-aligned
    assert fn(2, 16, 16, 1 << 20 | 4096, 16384, 1, 16, None) == -1  # bytes not whole units
    assert fn(2, None, 16, 1 << 20, 16384, 1, 16, None) == -1    # copy without a source
    assert fn(0, 16, None, 1 << 20, 16384, 1, None, None) == -1  # read without a sink
    assert fn(1, None, 24, 1 << 20, 16384, 1, None, None) == -1  # misaligned


@pytest.mark.gpu
@pytest.mark.parametrize("unit", [4096, 16384, 32768, 65536])
def test_probe_streams_move_their_bytes(unit):
    fn = _probe()
    dev = torch.device("cuda:0")
    n = 64 << 20
    g = torch.Generator(device="cpu").manual_seed(unit)
    src = torch.randint(0, 256, (n,), generator=g, dtype=torch.uint8).to(dev)
    dst = torch.zeros(n, dtype=torch.uint8, device=dev)
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    print(f"bw probe unit={unit}", flush=True)
    assert fn(2, src.data_ptr(), dst.data_ptr(), n, unit, 2, sink.data_ptr(), stream) == 0
    torch.cuda.synchronize(dev)
    assert torch.equal(src, dst)
    assert fn(1, None, dst.data_ptr(), n, unit, 1, None, stream) == 0
    torch.cuda.synchronize(dev)
    words = dst.view(torch.int32).view(-1, 4)
    assert bool((words[:, 2] == 0x5a5a5a5a).all())  # every 16-byte vector written
    for op in (3, 4):  # every unit written once, at its permuted place
        dst.zero_()
        perm = torch.randperm(n // unit, generator=g, dtype=torch.int32).to(dev)
        assert fn(op, perm.data_ptr(), dst.data_ptr(), n, unit, 2, None, stream) == 0
        torch.cuda.synchronize(dev)
        assert bool((dst.view(torch.int32).view(-1, 4)[:, 2] == 0x5a5a5a5a).all())
    assert fn(0, src.data_ptr(), None, n, unit, 2, sink.data_ptr(), stream) == 0
    torch.cuda.synchronize(dev)
    assert int(sink.abs().sum()) == 0  # the read stream stores nothing
