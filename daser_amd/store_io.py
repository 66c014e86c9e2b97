"""Store-file I/O through a pinned-host staging ring.

Replaces the reference's kvikio layer (daser/connector/gds_transfer.py:22-127,
``GDSTransferLayer.write_async / read_into_async / close``) for a host without
GPUDirect Storage: the store file ``daser.store`` is read and written with
positional host I/O, and device data crosses PCIe through a ring of pinned
host slots with asynchronous copies on a side stream.

Save (device -> file), per slot-sized piece i:
    side stream waits for the producer stream (the gather is enqueued there),
    copies piece i device -> pinned slot, records event e_i;
    writer thread waits e_i, pwrite()s the slot at file_offset + i * slot.
Load (file -> device), per piece i:
    reader thread pread()s into a free slot;
    side stream copies slot -> device, records event e_i;
    the consumer stream waits on the last event before the scatter.

A slot is reused only after both its copy event and its host I/O have
completed; pieces of one transfer overlap (the copy of piece i runs while
piece i+1 is read or written). File format and offsets are the reference's:
the record of slot s begins at ``s * SLOT_SIZE`` (daser/server/ipc_server.py
file_offset = start_slot * slot_size).

With ``device="cpu"`` the same ring runs with plain host copies, which lets
its ordering and failure handling be tested without a GPU.
"""

from __future__ import annotations

import concurrent.futures
import os
import threading
from dataclasses import dataclass
from typing import Callable, Optional

import torch


class StoreIOError(RuntimeError):
    """A host read or write of the store file failed or came up short."""


def preallocate_store(path: str, nbytes: int) -> None:
    """Creates the store file zero-filled if it does not exist (reference
    register_kv_caches, daser/connector/daser_connector.py:415-428)."""
    if os.path.exists(path):
        return
    parent = os.path.dirname(path)
    if parent:
        os.makedirs(parent, exist_ok=True)
    with open(path, "wb") as f:
        f.truncate(nbytes)


@dataclass
class _Slot:
    host: torch.Tensor  # pinned uint8
    event: Optional[torch.cuda.Event]
    busy: Optional[concurrent.futures.Future] = None


class PinnedRingIO:
    """Pipelined device <-> file transfers through ``n_slots`` pinned slots.

    Args:
        path: store file (must exist, like GDSTransferLayer).
        device: device of the tensors transferred.
        slot_bytes: bytes per ring slot (one piece of a transfer).
        n_slots: ring depth (>= 2 for overlap).
        io_threads: host threads doing pread/pwrite.
        io_hook: optional callable(kind, offset, nbytes) run on the I/O
            thread before each host I/O (tests use it to slow or fail I/O).
    """

    def __init__(self, path: str, device: torch.device | str = "cuda",
                 slot_bytes: int = 64 << 20, n_slots: int = 4, io_threads: int = 2,
                 io_hook: Optional[Callable[[str, int, int], None]] = None) -> None:
        if not os.path.exists(path):
            raise FileNotFoundError(f"Store file not found: {path}")
        if n_slots < 1 or slot_bytes <= 0:
            raise ValueError("need at least one slot of positive size")
        self.path = path
        self.device = torch.device(device)
        self._gpu = self.device.type == "cuda"
        self._fd = os.open(path, os.O_RDWR)
        self._slot_bytes = int(slot_bytes)
        self._hook = io_hook
        pin = self._gpu
        self._slots = [
            _Slot(torch.empty(self._slot_bytes, dtype=torch.uint8, pin_memory=pin),
                  torch.cuda.Event() if self._gpu else None)
            for _ in range(n_slots)
        ]
        self._next = 0
        self._stream = torch.cuda.Stream(self.device) if self._gpu else None
        self._pool = concurrent.futures.ThreadPoolExecutor(io_threads, thread_name_prefix="daser-io")
        self._lock = threading.Lock()
        self._closed = False

    # ------------------------------------------------------------------ utils
    @property
    def slot_bytes(self) -> int:
        return self._slot_bytes

    @property
    def backend(self) -> str:
        """Threads doing pread/pwrite through pinned slots (counterpart of
        GDSTransferLayer.backend, gds_transfer.py:37-60)."""
        return "threads"

    def _take_slot(self) -> _Slot:
        """Next ring slot, after its previous host I/O (and so its copy) ended."""
        s = self._slots[self._next]
        self._next = (self._next + 1) % len(self._slots)
        if s.busy is not None:
            s.busy.result()  # re-raises a failed write of an earlier transfer
            s.busy = None
        return s

    def _pwrite(self, slot: _Slot, n: int, offset: int) -> int:
        if slot.event is not None:
            slot.event.synchronize()
        if self._hook:
            self._hook("write", offset, n)
        mv = memoryview(slot.host.numpy())[:n]
        done = 0
        while done < n:
            w = os.pwrite(self._fd, mv[done:], offset + done)
            if w <= 0:
                raise StoreIOError(f"pwrite returned {w} at offset {offset + done}")
            done += w
        return n

    def _pread(self, slot: _Slot, n: int, offset: int) -> int:
        if self._hook:
            self._hook("read", offset, n)
        mv = memoryview(slot.host.numpy())[:n]
        done = 0
        while done < n:
            r = os.preadv(self._fd, [mv[done:]], offset + done)
            if r <= 0:
                raise StoreIOError(
                    f"short read of {self.path}: {done} of {n} bytes at offset {offset}")
            done += r
        return n

    # --------------------------------------------------------------- transfers
    def write_from_device(self, src: torch.Tensor, file_offset: int,
                          producer: Optional[torch.cuda.Stream] = None) -> int:
        """Writes ``src`` (contiguous, any dtype) at ``file_offset``; returns
        when every byte is on its way to the file (host I/O submitted and the
        last piece's write finished). Work enqueued on ``producer`` (default:
        the current stream) before this call is complete before the copy."""
        self._check()
        flat = src.reshape(-1).view(torch.uint8)
        n = flat.numel()
        futs = []
        with self._lock:
            try:
                if self._gpu:
                    ready = torch.cuda.Event()
                    ready.record(producer or torch.cuda.current_stream(self.device))
                    self._stream.wait_event(ready)
                for off in range(0, n, self._slot_bytes):
                    m = min(self._slot_bytes, n - off)
                    slot = self._take_slot()
                    if self._gpu:
                        with torch.cuda.stream(self._stream):
                            slot.host[:m].copy_(flat[off:off + m], non_blocking=True)
                            slot.event.record(self._stream)
                    else:
                        slot.host[:m].copy_(flat[off:off + m])
                    slot.busy = self._pool.submit(self._pwrite, slot, m, file_offset + off)
                    futs.append(slot.busy)
                for f in futs:
                    f.result()
            except BaseException:
                self._abandon()
                raise
        return n

    def _abandon(self) -> None:
        """After a failed transfer: wait out its in-flight pieces and free
        their slots, so the error is reported once, by that transfer."""
        for s in self._slots:
            if s.busy is not None:
                concurrent.futures.wait([s.busy])
                s.busy = None

    def read_into_device(self, dst: torch.Tensor, file_offset: int,
                         consumer: Optional[torch.cuda.Stream] = None) -> int:
        """Reads ``dst.nbytes`` bytes at ``file_offset`` into ``dst``. Work
        enqueued on ``consumer`` (default: the current stream) before the call
        is complete before the first copy into ``dst``; on return the host
        reads are done and ``consumer`` is ordered after the last copy."""
        self._check()
        flat = dst.reshape(-1).view(torch.uint8)
        n = flat.numel()
        with self._lock:
            if self._gpu:  # earlier work on the consumer may still use dst
                before = torch.cuda.Event()
                before.record(consumer or torch.cuda.current_stream(self.device))
                self._stream.wait_event(before)
            try:
                # keep up to len(slots) reads in flight ahead of the copies
                pending = []
                for off in range(0, n, self._slot_bytes):
                    m = min(self._slot_bytes, n - off)
                    slot = self._take_slot()
                    slot.busy = self._pool.submit(self._pread, slot, m, file_offset + off)
                    pending.append((slot, off, m))
                    if len(pending) == len(self._slots):
                        self._drain_one(pending, flat)
                while pending:
                    self._drain_one(pending, flat)
            except BaseException:
                self._abandon()
                raise
            finally:
                if self._gpu:
                    done = torch.cuda.Event()
                    done.record(self._stream)
                    (consumer or torch.cuda.current_stream(self.device)).wait_event(done)
        return n

    def _drain_one(self, pending, flat) -> None:
        slot, off, m = pending.pop(0)
        slot.busy.result()
        slot.busy = None
        if self._gpu:
            # the slot's previous copy (if any) is ordered before this one on
            # the side stream; its host buffer is refilled only after this
            # copy's event, which _pwrite/_take_slot wait for
            with torch.cuda.stream(self._stream):
                flat[off:off + m].copy_(slot.host[:m], non_blocking=True)
                slot.event.record(self._stream)
            # the next pread into this slot must wait for the copy out of it
            ev = slot.event
            slot.busy = self._pool.submit(ev.synchronize)
        else:
            flat[off:off + m].copy_(slot.host[:m])

    # ------------------------------------------------- GDSTransferLayer shape
    async def write_async(self, buf: torch.Tensor, file_offset: int,
                          nbytes: Optional[int] = None) -> int:
        import asyncio

        src = buf.reshape(-1).view(torch.uint8)
        if nbytes is not None:
            src = src[:nbytes]
        loop = asyncio.get_running_loop()
        return await loop.run_in_executor(None, self.write_from_device, src, file_offset)

    async def read_into_async(self, buf: torch.Tensor, file_offset: int,
                              nbytes: Optional[int] = None) -> int:
        import asyncio

        dst = buf.reshape(-1).view(torch.uint8)
        if nbytes is not None:
            dst = dst[:nbytes]
        loop = asyncio.get_running_loop()
        n = await loop.run_in_executor(None, self.read_into_device, dst, file_offset)
        return n

    def flush(self) -> None:
        """Waits for every outstanding host write."""
        for s in self._slots:
            if s.busy is not None:
                s.busy.result()
                s.busy = None

    def _check(self) -> None:
        if self._closed:
            raise StoreIOError("store I/O is closed")

    def close(self) -> None:
        if self._closed:
            return
        try:
            self.flush()
        finally:
            self._closed = True
            self._pool.shutdown(wait=True)
            os.close(self._fd)

    def __enter__(self) -> "PinnedRingIO":
        return self

    def __exit__(self, *_: object) -> None:
        self.close()


class NativeRingIO:
    """The same transfers as :class:`PinnedRingIO`, done by the native ring of
    libdaser_kv (pinned slots, hipMemcpyAsync on a ring-owned stream,
    io_uring or pread/pwrite from the calling thread; ``dsr_ring_*`` in
    include/daser_kv.h). With ``device="cpu"`` the ring runs in host mode
    (memcpy, no HIP calls).
    """

    def __init__(self, path: str, device: torch.device | str = "cuda",
                 slot_bytes: int = 4 << 20, n_slots: int = 8, use_io_uring: bool = True,
                 direct: bool = False, mapped: bool = False) -> None:
        import ctypes

        from daser_amd import _lib

        self._lib = _lib
        self.path = path
        self.device = torch.device(device)
        flags = 0
        if self.device.type != "cuda":
            flags |= _lib.DSR_RING_HOST
        if not use_io_uring:
            flags |= _lib.DSR_RING_NO_URING
        if direct:
            flags |= _lib.DSR_RING_DIRECT
        if mapped:
            flags |= _lib.DSR_RING_MMAP
        h = ctypes.c_void_p()
        rc = _lib.lib().dsr_ring_open(path.encode(), int(slot_bytes), int(n_slots), flags,
                                      ctypes.byref(h))
        if rc == _lib.DSR_ERR_NOFILE:
            raise FileNotFoundError(f"Store file not found: {path}")
        _lib.check("dsr_ring_open", rc)
        self._h = h
        self._slot_bytes = int(slot_bytes)
        self._direct = bool(direct)

    @property
    def slot_bytes(self) -> int:
        return self._slot_bytes

    @property
    def uses_io_uring(self) -> bool:
        return bool(self._lib.lib().dsr_ring_uses_io_uring(self._handle()))

    @property
    def backend(self) -> str:
        """How file I/O is done ("mmap", "io_uring" or "posix", "+O_DIRECT");
        the counterpart of GDSTransferLayer.backend (gds_transfer.py:37-60).
        A mapped ring writes past the end of the file through io_uring or
        posix calls."""
        if self._lib.lib().dsr_ring_is_mapped(self._handle()):
            return "mmap"
        return ("io_uring" if self.uses_io_uring else "posix") + ("+O_DIRECT" if self._direct
                                                                  else "")

    def _handle(self):
        if self._h is None:
            raise StoreIOError("store I/O is closed")
        return self._h

    def _stream(self, s: Optional[torch.cuda.Stream]) -> Optional[int]:
        if self.device.type != "cuda":
            return None
        return (s or torch.cuda.current_stream(self.device)).cuda_stream

    def _raise(self, fn: str, rc: int) -> None:
        if rc == self._lib.DSR_ERR_IO:
            err = self._lib.lib().dsr_ring_last_errno(self._h)
            raise StoreIOError(f"{fn}: {os.strerror(err) if err else 'I/O error'} on {self.path}")
        self._lib.check(fn, rc)

    def write_from_device(self, src: torch.Tensor, file_offset: int,
                          producer: Optional[torch.cuda.Stream] = None) -> int:
        flat = src.reshape(-1).view(torch.uint8)
        if not flat.is_contiguous():
            raise ValueError("source must be contiguous")
        n = flat.numel()
        rc = self._lib.lib().dsr_ring_write(self._handle(), flat.data_ptr(), n, int(file_offset),
                                            self._stream(producer))
        if rc:
            self._raise("dsr_ring_write", rc)
        return n

    def read_into_device(self, dst: torch.Tensor, file_offset: int,
                         consumer: Optional[torch.cuda.Stream] = None) -> int:
        flat = dst.reshape(-1).view(torch.uint8)
        if not flat.is_contiguous():
            raise ValueError("destination must be contiguous")
        n = flat.numel()
        rc = self._lib.lib().dsr_ring_read(self._handle(), flat.data_ptr(), n, int(file_offset),
                                           self._stream(consumer))
        if rc:
            self._raise("dsr_ring_read", rc)
        return n

    async def write_async(self, buf: torch.Tensor, file_offset: int,
                          nbytes: Optional[int] = None) -> int:
        import asyncio

        src = buf.reshape(-1).view(torch.uint8)
        if nbytes is not None:
            src = src[:nbytes]
        return await asyncio.get_running_loop().run_in_executor(
            None, self.write_from_device, src, file_offset)

    async def read_into_async(self, buf: torch.Tensor, file_offset: int,
                              nbytes: Optional[int] = None) -> int:
        import asyncio

        dst = buf.reshape(-1).view(torch.uint8)
        if nbytes is not None:
            dst = dst[:nbytes]
        return await asyncio.get_running_loop().run_in_executor(
            None, self.read_into_device, dst, file_offset)

    def flush(self) -> None:
        """Writes complete before write_from_device returns; nothing pends."""

    def close(self) -> None:
        if self._h is not None:
            rc = self._lib.lib().dsr_ring_close(self._h)
            self._h = None
            self._lib.check("dsr_ring_close", rc)

    def __enter__(self) -> "NativeRingIO":
        return self

    def __exit__(self, *_: object) -> None:
        self.close()

    def __del__(self) -> None:  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass
