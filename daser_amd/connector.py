"""DaseR's vLLM connector (``KVConnectorBase_V1``) on the MI355X data path.

Same class name, constructor, hooks and metadata types as the reference
(daser/connector/daser_connector.py:60-711); the worker hooks run the HIP
kernels of libdaser_kv instead of per-(request, block, layer) torch copies:

  save_kv_layer   one gather launch per layer over every store request
                  (reference :574-632: 2 copies per block per layer);
  wait_for_save   device -> pinned ring -> store file, one transfer per
                  request, then commit_chunk (reference :634-684);
  start_load_kv   store file -> pinned ring -> device staging, then one
                  scatter launch for every load request, re-rotating K of
                  chunks whose position changed (reference :455-558, which
                  has no re-rotation).

Additions, all optional and defaulted so that reference metadata still
works: ``ReqLoadSpec.pos_offset`` (position the chunk was stored at,
``ChunkMeta.pos_offset``), ``ReqLoadSpec.new_pos`` (position of its first
token in this request) and ``ReqLoadSpec.segments`` (several cached chunks
assembled into one request, each with its own positions).

Extra ``kv_connector_extra_config`` keys: ``rope_theta`` (default 10000),
``rope_style`` ("neox" | "gptj"), ``rotary_dim`` (default head_dim),
``rope_scaling`` (the model's HF ``rope_scaling`` dict: linear, llama3, yarn,
mrope), ``rope_layers`` (per model layer: None for no RoPE, or
{"rope_theta", "rope_scaling"}; for models whose layers differ), all three
read from ``vllm_config.model_config.hf_config`` when not given,
``save_mode`` ("per_layer" | "deferred": one all-layer gather in
wait_for_save), ``io_slot_mb`` / ``io_slots`` (pinned ring geometry), ``io_readers``
(rings reading a load in parallel, default 4), ``io_timeout_s`` (a blocking
store read or write raises TimeoutError after this long, default 120 as in
the reference; None: wait forever),
``io_backend`` ("native": the C++ io_uring ring of libdaser_kv, default;
"direct": the same ring with the store file opened O_DIRECT;
"python": the threaded ring of store_io.PinnedRingIO), ``k_scale`` (one K
scale for every layer of an fp8 cache, when the attention modules' own
``_k_scale`` are not reachable), ``async_save`` (wait_for_save returns once
the gathers are enqueued and ordered before the next step's KV writes; file
writes and commits finish on a background writer; default False, the
reference's blocking behaviour), ``save_stream``
("side": per-layer gathers on a side stream after the layer's KV writes,
overlapping later layers, default; "current": on the model's stream).
"""

from __future__ import annotations

import array
import asyncio
import logging
import math
import threading
from dataclasses import dataclass, field
from typing import Any, Optional

import numpy as np
import torch

try:  # vLLM's base classes when vLLM is installed
    from vllm.distributed.kv_transfer.kv_connector.v1.base import (  # type: ignore
        KVConnectorBase_V1,
        KVConnectorMetadata,
        KVConnectorRole,
    )
except ImportError:  # pragma: no cover - exercised where vLLM is absent
    from daser_amd._vllm_base import KVConnectorBase_V1, KVConnectorMetadata, KVConnectorRole

logger = logging.getLogger("daser_amd.connector")


def hash_tokens(tokens: list[int]) -> str:
    """xxh3_128 hex of the int32 token array (reference :41-57)."""
    import xxhash

    return xxhash.xxh3_128(bytes(array.array("i", tokens))).hexdigest()


# ---------------------------------------------------------------------------
# metadata (reference :60-112, plus optional position fields)


@dataclass
class LoadSegment:
    """One cached chunk inside a load: ``num_slots`` records starting at
    store slot ``start_slot``, landing in ``block_ids[block_offset:
    block_offset + num_slots]``, stored at position ``pos_offset`` and
    placed at ``new_pos`` (None = as stored)."""

    start_slot: int
    num_slots: int
    block_offset: int
    pos_offset: int = 0
    new_pos: Optional[int] = None


@dataclass
class ReqLoadSpec:
    chunk_key: str
    start_slot: int
    num_slots: int
    block_ids: list[int]
    file_offset: int
    token_count: int
    pos_offset: int = 0
    new_pos: Optional[int] = None
    segments: list[LoadSegment] = field(default_factory=list)

    def resolved_segments(self) -> list[LoadSegment]:
        if self.segments:
            return self.segments
        return [LoadSegment(self.start_slot, len(self.block_ids), 0, self.pos_offset,
                            self.new_pos)]


@dataclass
class ReqStoreSpec:
    chunk_key: str
    start_slot: int
    num_slots: int
    block_ids: list[int]
    file_offset: int
    token_count: int


@dataclass
class DaserConnectorMeta(KVConnectorMetadata):
    reqs_to_load: dict[str, ReqLoadSpec] = field(default_factory=dict)
    reqs_to_store: dict[str, ReqStoreSpec] = field(default_factory=dict)


# ---------------------------------------------------------------------------
# planning (host side, no device work): which pages move where


@dataclass
class StorePlan:
    """Pages of every store request packed back to back in one arena."""

    page_ids: np.ndarray  # int32 block ids
    slot_offsets: np.ndarray  # int64 record offsets in the arena
    transfers: list[tuple[str, int, int, int]]  # (chunk_key, arena_off, nbytes, file_off)
    arena_bytes: int
    device_tables: Optional[tuple] = None  # (page_ids, slot_offsets) on the device


@dataclass
class LoadPlan:
    """Records read into one arena, then scattered into pages."""

    page_ids: np.ndarray
    src_offsets: np.ndarray
    rope_idx: np.ndarray  # int32, -1 = no rotation
    deltas: list[int]  # table order
    reads: list[tuple[int, int, int]]  # (arena_off, nbytes, file_off)
    arena_bytes: int
    page_read: np.ndarray = field(default_factory=lambda: np.zeros(0, np.int64))  # read of each page


def plan_store(reqs: dict[str, ReqStoreSpec], slot_bytes: int) -> StorePlan:
    """Record of request r's slot i at arena_r + i * SLOT, written to the file
    at start_slot * SLOT (reference :616-632, :652)."""
    ids, transfers = [], []
    base = 0
    for spec in reqs.values():
        n = len(spec.block_ids)
        if n == 0:
            continue
        ids.extend(spec.block_ids)
        transfers.append((spec.chunk_key, base, n * slot_bytes, spec.start_slot * slot_bytes))
        base += n * slot_bytes
    # records are packed back to back: page k of the step at k * SLOT
    offs = np.arange(len(ids), dtype=np.int64) * slot_bytes
    return StorePlan(np.asarray(ids, np.int32), offs, transfers, base)


def plan_load(reqs: dict[str, ReqLoadSpec], slot_bytes: int) -> LoadPlan:
    """Each segment's records are read once into the arena; page j of a
    segment scatters record j into block_ids[block_offset + j]. A segment
    whose new position differs from its stored one gets a rotation table for
    delta = new_pos - pos_offset (reference :498-551 for the unrotated part)."""
    ids: list[int] = []
    seg_pages, seg_table, reads = [], [], []
    table: dict[int, int] = {}
    base = 0
    for spec in reqs.values():
        blocks = spec.block_ids
        if not blocks:
            continue
        for seg in spec.resolved_segments():
            n = seg.num_slots
            if n <= 0:
                continue
            if seg.block_offset < 0 or seg.block_offset + n > len(blocks):
                raise ValueError(f"segment of {spec.chunk_key[:8]} exceeds its block list")
            reads.append((base, n * slot_bytes, seg.start_slot * slot_bytes))
            delta = 0 if seg.new_pos is None else int(seg.new_pos) - int(seg.pos_offset)
            seg_table.append(-1 if delta == 0 else table.setdefault(delta, len(table)))
            seg_pages.append(n)
            ids.extend(blocks[seg.block_offset:seg.block_offset + n])
            base += n * slot_bytes
    # segments' records are packed back to back: page k at k * SLOT
    counts = np.asarray(seg_pages, np.int64)
    return LoadPlan(np.asarray(ids, np.int32),
                    np.arange(len(ids), dtype=np.int64) * slot_bytes,
                    np.repeat(np.asarray(seg_table, np.int32), counts), list(table.keys()),
                    reads, base, np.repeat(np.arange(len(reads), dtype=np.int64), counts))


# ---------------------------------------------------------------------------
# worker data plane


class KVDataPlane:
    """Worker-side movement of KV pages between vLLM's caches and the store.

    Owns the layer table of the registered caches, the per-step staging
    arenas and the store I/O; every device operation is enqueued on torch's
    current stream of the caches' device.
    """

    def __init__(self, store_path: str, *, rope_theta: float = 10000.0,
                 rope_style: str = "neox", rotary_dim: Optional[int] = None,
                 inv_freq: Optional[np.ndarray] = None, rope_scaling: Optional[dict] = None,
                 save_mode: str = "per_layer",
                 io_slot_bytes: int = 4 << 20, io_slots: int = 8,
                 io_backend: str = "native", save_stream: str = "side",
                 k_scales: Optional[torch.Tensor] = None, io_readers: int = 4,
                 layer_rope: Optional[list] = None,
                 io_timeout: Optional[float] = 120.0) -> None:
        if save_mode not in ("per_layer", "deferred"):
            raise ValueError("save_mode must be 'per_layer' or 'deferred'")
        if io_backend not in ("native", "direct", "python"):
            raise ValueError("io_backend must be 'native', 'direct' or 'python'")
        if save_stream not in ("side", "current"):
            raise ValueError("save_stream must be 'side' or 'current'")
        self.io_backend = io_backend
        self.save_stream = save_stream
        self._side: Optional[torch.cuda.Stream] = None
        self.store_path = store_path
        self.rope_theta = float(rope_theta)
        self.rope_style = rope_style
        self.rotary_dim = rotary_dim
        self.inv_freq = inv_freq
        self.rope_scaling = rope_scaling
        # per model layer: None (no RoPE) or {"rope_theta", "rope_scaling"}
        self.layer_rope = layer_rope
        self._layer_group: Optional[torch.Tensor] = None
        self._group_inv: list[np.ndarray] = []
        if rope_scaling and inv_freq is None:
            from daser_amd.position import inv_freq_for

            # Unsupported scalings fail here, not at the first load.
            probe_dim = int(rotary_dim) if rotary_dim else 2
            scaled = inv_freq_for(rope_scaling, probe_dim, rope_theta)
            if rotary_dim:
                self.inv_freq = scaled
        self.save_mode = save_mode
        self._io_slot_bytes = io_slot_bytes
        self._io_slots = io_slots
        self.k_scales = k_scales
        self._writer = None  # background writer of flush_async, with its own ring
        self._wio = None
        self._io_readers = max(1, int(io_readers))  # parallel rings of load()
        self.io_timeout = io_timeout  # seconds a blocking transfer may take (None: no limit)
        self._sync_pool = None
        self._reader_pool = None
        self._readers: list = []
        self._idle_stream: Optional[torch.cuda.Stream] = None
        self._pending_writes: list = []
        self.table = None
        self.layer_names: list[str] = []
        self.layer_idx: dict[str, int] = {}
        self.slot_bytes = 0
        self.io = None

    # -- registration (reference register_kv_caches :383-429)
    def register(self, kv_caches: dict[str, torch.Tensor], slot_size: int = 0) -> int:
        from daser_amd import ops
        from daser_amd.store_io import preallocate_store

        self.layer_names = list(kv_caches.keys())
        self.layer_idx = {n: i for i, n in enumerate(self.layer_names)}
        self.table = ops.LayerTable([kv_caches[n] for n in self.layer_names])
        lay = self.table.layout
        derived = lay.slot_bytes
        if slot_size and slot_size != derived:
            raise ValueError(f"configured slot_size {slot_size} != derived {derived}")
        self.slot_bytes = derived
        if self.rotary_dim is None:
            self.rotary_dim = lay.head_dim
        if self.inv_freq is None and self.rope_scaling:
            from daser_amd.position import inv_freq_for

            self.inv_freq = inv_freq_for(self.rope_scaling, self.rotary_dim, self.rope_theta)
        if self.layer_rope is not None:
            self._register_layer_rope()
        preallocate_store(self.store_path, max(self.slot_bytes * 1024, 64 << 20))
        if self.save_stream == "side" and lay.device.type == "cuda" and self._side is None:
            self._side = torch.cuda.Stream(lay.device)  # default priority
        if self.io_backend == "direct" and self.slot_bytes % 4096:
            raise ValueError("io_backend='direct' needs a slot record size that is a "
                             "multiple of 4096 bytes")
        if self.io is None:
            self.io = self._open_ring(lay.device)
        return self.slot_bytes

    def _register_layer_rope(self) -> None:
        """Groups of layers sharing RoPE frequencies (layer_rope is indexed
        by the model's layer number, read from names like
        "model.layers.12.self_attn.attn", else by registration order)."""
        import re

        from daser_amd.position import layer_rope_groups

        specs = []
        for pos, name in enumerate(self.layer_names):
            m = re.search(r"layers\.(\d+)\.", name)
            idx = int(m.group(1)) if m else pos
            if idx >= len(self.layer_rope):
                raise ValueError(f"layer_rope has no entry for layer {idx} ({name})")
            specs.append(self.layer_rope[idx])
        groups, invs = layer_rope_groups(specs, self.rotary_dim, self.rope_theta)
        if len(invs) == 1 and (groups >= 0).all():
            self.inv_freq = invs[0]  # one RoPE after all: the single-table path
            return
        self._group_inv = invs
        self._layer_group = torch.from_numpy(groups).to(self.table.layout.device)

    def _open_ring(self, device: torch.device):
        from daser_amd.store_io import NativeRingIO, PinnedRingIO

        if self.io_backend == "python":
            return PinnedRingIO(self.store_path, device, slot_bytes=self._io_slot_bytes,
                                n_slots=self._io_slots)
        return NativeRingIO(self.store_path, device, slot_bytes=self._io_slot_bytes,
                            n_slots=self._io_slots, direct=self.io_backend == "direct")

    @property
    def device(self) -> torch.device:
        return self.table.layout.device

    # -- save
    def new_store_arena(self, plan: StorePlan) -> torch.Tensor:
        """Staging arena of a step's store requests. The plan's page tables are
        validated and uploaded once here and reused by every layer's gather."""
        from daser_amd import ops

        arena = torch.empty(max(plan.arena_bytes, 16), dtype=torch.uint8, device=self.device)
        if plan.page_ids.size:
            ops._validate(self.table.layout, plan.page_ids, plan.slot_offsets, arena, 0,
                          self.table.layout.num_layers, True)
            plan.device_tables = (torch.from_numpy(plan.page_ids).to(self.device),
                                  torch.from_numpy(plan.slot_offsets).to(self.device))
        return arena

    def _on_save_stream(self, arena: torch.Tensor):
        """Context for the gathers: the side stream, ordered after the work
        the model's stream has enqueued so far (the layer's KV writes)."""
        import contextlib

        if self._side is None:
            return contextlib.nullcontext()
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self._side.wait_event(ev)
        arena.record_stream(self._side)
        return torch.cuda.stream(self._side)

    def save_layer(self, layer_name: str, plan: StorePlan, arena: torch.Tensor) -> None:
        """Gathers one layer's pages of every store request. With
        save_stream="side" the gather runs on a side stream after the KV
        writes already enqueued, overlapping the model's later layers."""
        from daser_amd import ops

        if plan.page_ids.size == 0:
            return
        l = self.layer_idx[layer_name]
        ids, offs = plan.device_tables
        with self._on_save_stream(arena):
            ops.gather(self.table, ids, offs, arena, layers=(l, 1))

    def save_all(self, plan: StorePlan, arena: torch.Tensor) -> None:
        from daser_amd import ops

        if plan.page_ids.size == 0:
            return
        ids, offs = plan.device_tables
        with self._on_save_stream(arena):
            ops.gather(self.table, ids, offs, arena)

    def flush_async(self, plan: StorePlan, arena: torch.Tensor, done) -> None:
        """Like flush, but the file writes run on a background writer thread
        (one, so steps are written in order) and this returns at once. The
        current stream is first ordered after the step's gathers, so vLLM may
        reuse the cache blocks as soon as the gathers have run; the arena
        keeps the records until they are written. ``done(keys, error)`` is
        called on the writer thread with the chunk keys fully written (all
        of them unless ``error``)."""
        from concurrent.futures import ThreadPoolExecutor

        cur = torch.cuda.current_stream(self.device)
        ev = torch.cuda.Event()
        ev.record(self._side if self._side is not None else cur)
        if self._side is not None:
            cur.wait_event(ev)
        if self._writer is None:
            self._writer = ThreadPoolExecutor(max_workers=1, thread_name_prefix="daser-save")
            self._idle_stream = torch.cuda.Stream(self.device)  # never given work
            # its own ring: a load (start_load_kv) never waits behind a write
            self._wio = self._open_ring(self.table.layout.device)

        def job() -> None:
            keys: list[str] = []
            err: Optional[BaseException] = None
            try:
                ev.synchronize()  # the gathers into this arena have run
                for key, off, nbytes, file_off in plan.transfers:
                    self._wio.write_from_device(arena[off:off + nbytes], file_off,
                                                self._idle_stream)
                    keys.append(key)
            except BaseException as e:  # reported, never lost on the thread
                err = e
            done(keys, err)

        self._pending_writes.append(self._writer.submit(job))

    def drain(self, timeout: Optional[float] = None) -> None:
        """Waits for every write started by flush_async."""
        pending, self._pending_writes = self._pending_writes, []
        for f in pending:
            f.result(timeout=timeout)

    def flush(self, plan: StorePlan, arena: torch.Tensor) -> list[str]:
        """Writes each request's records at its file offset; returns the
        chunk keys written (to commit)."""
        keys: list[str] = []
        producer = self._side
        if producer is None and self.device.type == "cuda":
            producer = torch.cuda.current_stream(self.device)  # resolved on this thread

        def run() -> None:
            for key, off, nbytes, file_off in plan.transfers:
                self.io.write_from_device(arena[off:off + nbytes], file_off, producer)
                keys.append(key)

        self._io_call(run, "store write")
        return keys

    def _io_call(self, fn, what: str) -> None:
        """Runs a blocking store transfer; with io_timeout set it runs on a
        helper thread and raises TimeoutError if it does not return in time
        (the reference's worker I/O waits 120 s, daser_connector.py:526-528,
        670-672)."""
        if self.io_timeout is None:
            fn()
            return
        if self._sync_pool is None:
            from concurrent.futures import ThreadPoolExecutor

            self._sync_pool = ThreadPoolExecutor(max_workers=1, thread_name_prefix="daser-sync")
        self._wait(self._sync_pool.submit(fn), what)

    def _wait(self, fut, what: str) -> None:
        from concurrent.futures import TimeoutError as FutTimeout

        try:
            fut.result(timeout=self.io_timeout)
        except FutTimeout:
            raise TimeoutError(f"{what} did not finish within {self.io_timeout} s "
                               f"({self.store_path})") from None

    # -- load
    def load(self, plan: LoadPlan, batch_bytes: int = 256 << 20) -> None:
        """Reads the plan's records and scatters them. Reads are grouped into
        batches of about ``batch_bytes`` (a read larger than that is a batch
        of its own); each batch is scattered as soon as it has landed, so the
        GPU scatters batch i while the reader rings read batch i+1."""
        from daser_amd import ops, position

        if plan.page_ids.size == 0:
            return
        tabs = None
        if plan.deltas and self._layer_group is not None:
            if self._group_inv:  # [groups, tables, rot/2, 2]; layers in group -1 keep K
                tabs = torch.stack([position.delta_tables(plan.deltas, self.rotary_dim,
                                                          inv_freq=inv, device=self.device)
                                    for inv in self._group_inv])
        elif plan.deltas:
            tabs = position.delta_tables(plan.deltas, self.rotary_dim, self.rope_theta,
                                         inv_freq=self.inv_freq, device=self.device)
        page_read = plan.page_read if plan.page_read.size else np.zeros(plan.page_ids.size,
                                                                         np.int64)
        # Two batch buffers, alternating: batch k is read into buffer k % 2
        # once the scatter that last read that buffer (batch k - 2) has run,
        # so device staging stays near 2 * batch_bytes whatever the step
        # loads, and reading batch k overlaps scattering batch k - 1.
        bufs: list[Optional[torch.Tensor]] = [None, None]
        done: list[Optional[torch.cuda.Event]] = [None, None]
        first, acc, k = 0, 0, 0
        batch: list[tuple[int, int, int]] = []
        for r, (off, nbytes, file_off) in enumerate(plan.reads):
            batch.append((off, nbytes, file_off))
            acc += nbytes
            if acc < batch_bytes and r + 1 < len(plan.reads):
                continue
            base = batch[0][0]
            size = batch[-1][0] + batch[-1][1] - base  # reads are packed back to back
            i = k % 2
            if done[i] is not None:
                done[i].synchronize()
            if bufs[i] is None or bufs[i].numel() < size:
                bufs[i] = torch.empty(max(size, batch_bytes), dtype=torch.uint8,
                                      device=self.device)
            buf = bufs[i]
            self._read_batch(buf, [(o - base, n, f) for o, n, f in batch])
            batch = []
            sel = np.nonzero((page_read >= first) & (page_read <= r))[0]
            first, acc, k = r + 1, 0, k + 1
            if sel.size == 0:
                continue
            src = plan.src_offsets[sel] - base
            if tabs is None:
                ops.scatter(self.table, plan.page_ids[sel], src, buf)
            else:
                ops.scatter_rerotate(self.table, plan.page_ids[sel], src, buf, tabs,
                                     plan.rope_idx[sel], rot_dim=self.rotary_dim,
                                     style=self.rope_style, k_scale=self.k_scales,
                                     layer_group=self._layer_group)
            if self.device.type == "cuda":
                done[i] = torch.cuda.Event()
                done[i].record(torch.cuda.current_stream(self.device))

    def _read_batch(self, arena: torch.Tensor, reads: list[tuple[int, int, int]]) -> None:
        """Reads (arena_off, nbytes, file_off) ranges into the arena with the
        reader rings in parallel (page-cache reads measured 15-18 GB/s on
        one ring, 32-37 GB/s on four), in pieces of at most 16 MiB. On
        return the current stream is ordered after every copy."""
        piece = 16 << 20  # a multiple of 4 KiB: O_DIRECT reads stay aligned
        parts = [(o + k, min(piece, n - k), f + k) for o, n, f in reads
                 for k in range(0, n, piece)]
        consumer = torch.cuda.current_stream(self.device) if self.device.type == "cuda" else None
        if self._io_readers <= 1 or len(parts) == 1:
            def run_one() -> None:
                for o, n, f in parts:
                    self.io.read_into_device(arena[o:o + n], f, consumer)

            self._io_call(run_one, "store read")
            return
        if self._reader_pool is None:
            from concurrent.futures import ThreadPoolExecutor

            self._readers = [self.io] + [self._open_ring(self.device)
                                         for _ in range(self._io_readers - 1)]
            self._reader_pool = ThreadPoolExecutor(max_workers=self._io_readers,
                                                   thread_name_prefix="daser-load")

        def run(i: int) -> None:
            ring = self._readers[i]
            for o, n, f in parts[i::len(self._readers)]:
                ring.read_into_device(arena[o:o + n], f, consumer)

        for fut in [self._reader_pool.submit(run, i) for i in range(len(self._readers))]:
            self._wait(fut, "store read")

    def close(self) -> None:
        self.drain()
        if self._sync_pool is not None:
            self._sync_pool.shutdown(wait=False)
            self._sync_pool = None
        if self._reader_pool is not None:
            self._reader_pool.shutdown(wait=True)
            self._reader_pool = None
            for ring in self._readers[1:]:
                ring.close()
            self._readers = []
        if self._writer is not None:
            self._writer.shutdown(wait=True)
            self._writer = None
        if self._wio is not None:
            self._wio.close()
            self._wio = None
        if self.io is not None:
            self.io.close()
            self.io = None


# ---------------------------------------------------------------------------
# the connector


class _BgLoop:
    """Background asyncio loop for the async IPC client (reference :176-186)."""

    def __init__(self) -> None:
        self.loop = asyncio.new_event_loop()
        self.thread = threading.Thread(target=self._run, daemon=True, name="daser-io")
        self.thread.start()

    def _run(self) -> None:
        asyncio.set_event_loop(self.loop)
        self.loop.run_forever()

    def run(self, coro, timeout: Optional[float] = None):
        return asyncio.run_coroutine_threadsafe(coro, self.loop).result(timeout=timeout)

    def stop(self) -> None:
        self.loop.call_soon_threadsafe(self.loop.stop)
        self.thread.join(timeout=5)


def _default_ipc(kind: str, socket_path: str):
    """The reference's IPC clients, when its package is importable."""
    from daser.connector.ipc_client import IPCClientAsync, IPCClientSync  # type: ignore

    return (IPCClientSync if kind == "sync" else IPCClientAsync)(socket_path)


class DaserConnector(KVConnectorBase_V1):
    """vLLM ``KVConnectorBase_V1`` backed by DaseR, MI355X data path.

    ``ipc_client`` (scheduler role) and ``ipc_async`` (worker role) may be
    injected; by default the reference's IPC clients are used.
    """

    def __init__(self, vllm_config: Any, role: KVConnectorRole, kv_cache_config: Any = None,
                 *, ipc_client: Any = None, ipc_async: Any = None) -> None:
        super().__init__(vllm_config, role, kv_cache_config)
        extra: dict[str, Any] = {}
        ktc = getattr(vllm_config, "kv_transfer_config", None)
        if ktc is not None:
            extra = getattr(ktc, "kv_connector_extra_config", None) or {}
        self._socket_path: str = extra.get("socket_path", "/tmp/daser.sock")
        self._store_path: str = extra.get("store_path", "/tmp/daser/daser.store")
        self._slot_size: int = int(extra.get("slot_size", 0))
        self._block_tokens: int = int(extra.get("block_tokens", 16))
        self._model_id: str = extra.get("model_id", "default")
        self._role_kind = role
        if role == KVConnectorRole.SCHEDULER:
            self._ipc_sync = ipc_client if ipc_client is not None else _default_ipc(
                "sync", self._socket_path)
            self._pending_loads: dict[str, dict[str, Any]] = {}
            self._pending_stores: dict[str, dict[str, Any]] = {}
            self._pending_alloc: dict[str, dict[str, Any]] = {}
            self._req_tokens: dict[str, list[int]] = {}
        else:
            self._ipc_async = ipc_async if ipc_async is not None else _default_ipc(
                "async", self._socket_path)
            from daser_amd.position import layer_rope_from_hf, model_rope_from_hf

            hf = getattr(getattr(vllm_config, "model_config", None), "hf_config", None)
            hf_theta, hf_scaling = model_rope_from_hf(hf) if hf is not None else (None, None)
            self._plane = KVDataPlane(
                self._store_path,
                rope_theta=float(extra.get("rope_theta", hf_theta or 10000.0)),
                rope_style=extra.get("rope_style", "neox"),
                rotary_dim=extra.get("rotary_dim"),
                rope_scaling=extra.get("rope_scaling", hf_scaling),
                layer_rope=extra.get("rope_layers",
                                     layer_rope_from_hf(hf) if hf is not None else None),
                save_mode=extra.get("save_mode", "per_layer"),
                io_slot_bytes=int(float(extra.get("io_slot_mb", 4)) * (1 << 20)),
                io_slots=int(extra.get("io_slots", 8)),
                io_readers=int(extra.get("io_readers", 4)),
                io_timeout=extra.get("io_timeout_s", 120.0),
                io_backend=extra.get("io_backend", "native"),
                save_stream=extra.get("save_stream", "side"),
            )
            self._k_scale_cfg = extra.get("k_scale")  # uniform fp8 K scale, optional
            self._async_save = bool(extra.get("async_save", False))
            self._commit_futs: list = []
            cache_cfg = getattr(vllm_config, "cache_config", None)
            self._cache_dtype = str(getattr(cache_cfg, "cache_dtype", "auto"))
            self._meta: Optional[DaserConnectorMeta] = None
            self._store_plan: Optional[StorePlan] = None
            self._store_arena: Optional[torch.Tensor] = None
            self._saved_layers: set[int] = set()
            self._pending_commits: set[str] = set()
            self._flushed = False
            self._bg = _BgLoop()

    # ------------------------------------------------------------ scheduler
    def get_num_new_matched_tokens(self, request: Any, num_computed_tokens: int):
        """Reference :194-258 (match_and_alloc in one RPC), unchanged."""
        tokens = list(request.prompt_token_ids)
        self._req_tokens[request.request_id] = tokens
        available = len(tokens) - num_computed_tokens
        if available < self._block_tokens:
            return 0, False
        aligned = (available // self._block_tokens) * self._block_tokens
        prefix = tokens[: num_computed_tokens + aligned]
        full_aligned = (len(tokens) // self._block_tokens) * self._block_tokens
        store_key = hash_tokens(tokens[:full_aligned]) if full_aligned > 0 else ""
        try:
            resp = self._ipc_sync.match_and_alloc(prefix, store_key, self._model_id)
        except Exception as exc:  # a failed lookup degrades to a miss
            logger.warning("[CONNECTOR] match_and_alloc failed: %s", exc)
            return 0, False
        chunks = resp.get("chunks", [])
        alloc = resp.get("alloc")
        if alloc is not None:
            self._pending_alloc[request.request_id] = alloc
        if not chunks:
            return 0, False
        best = chunks[0]
        extra_tokens = best["token_count"] - num_computed_tokens
        if extra_tokens <= 0:
            return 0, False
        self._pending_loads[request.request_id] = best
        return extra_tokens, False

    def update_state_after_alloc(self, request: Any, blocks: Any, num_external_tokens: int) -> None:
        """Reference :260-298."""
        req_id = request.request_id
        block_ids = [blk.block_id for blk in blocks.blocks[0]]
        if num_external_tokens > 0 and req_id in self._pending_loads:
            chunk = self._pending_loads[req_id]
            chunk["block_ids"] = block_ids[: math.ceil(num_external_tokens / self._block_tokens)]
        else:
            alloc = self._pending_alloc.pop(req_id, None)
            if alloc is None:
                return
            alloc["block_ids"] = block_ids[: math.ceil(alloc["token_count"] / self._block_tokens)]
            self._pending_stores[req_id] = alloc

    def build_connector_meta(self, scheduler_output: Any) -> DaserConnectorMeta:
        """Reference :300-357; also forwards the chunk's stored position
        (``pos_offset`` of the lookup reply) and, when the reply names one, the
        position to place it at (``new_pos``) and its segments."""
        meta = DaserConnectorMeta()
        scheduled = set(scheduler_output.num_scheduled_tokens.keys())
        for req_id, chunk in list(self._pending_loads.items()):
            if req_id in scheduled and "block_ids" in chunk:
                segs = [LoadSegment(**s) for s in chunk.get("segments", [])]
                meta.reqs_to_load[req_id] = ReqLoadSpec(
                    chunk_key=chunk["chunk_key"], start_slot=chunk["start_slot"],
                    num_slots=chunk["num_slots"], block_ids=chunk["block_ids"],
                    file_offset=chunk["file_offset"], token_count=chunk["token_count"],
                    pos_offset=int(chunk.get("pos_offset", 0)), new_pos=chunk.get("new_pos"),
                    segments=segs)
                del self._pending_loads[req_id]
        for req_id, alloc in list(self._pending_stores.items()):
            if req_id in scheduled and "block_ids" in alloc:
                meta.reqs_to_store[req_id] = ReqStoreSpec(
                    chunk_key=alloc["chunk_key"], start_slot=alloc["start_slot"],
                    num_slots=alloc["num_slots"], block_ids=alloc["block_ids"],
                    file_offset=alloc["file_offset"], token_count=alloc["token_count"])
                del self._pending_stores[req_id]
        return meta

    def request_finished(self, request: Any, block_ids: list[int]):
        for d in (self._req_tokens, self._pending_loads, self._pending_stores, self._pending_alloc):
            d.pop(request.request_id, None)
        return False, None

    # --------------------------------------------------------------- worker
    def register_kv_caches(self, kv_caches: dict[str, torch.Tensor]) -> None:
        if self._cache_dtype in ("fp8", "fp8_e4m3"):
            # vLLM may hold an fp8 cache as raw uint8; the re-rotation needs the
            # element format (OCP e4m3fn on gfx950). A view, no copy.
            kv_caches = {n: t.view(torch.float8_e4m3fn) if t.dtype == torch.uint8 else t
                         for n, t in kv_caches.items()}
        self._slot_size = self._plane.register(kv_caches, self._slot_size)
        logger.info("[CONNECTOR] %d layers, slot_size=%d", len(kv_caches), self._slot_size)

    def bind_connector_metadata(self, connector_metadata: DaserConnectorMeta) -> None:
        super().bind_connector_metadata(connector_metadata)
        self._meta = connector_metadata
        self._store_plan = None
        self._store_arena = None
        self._saved_layers = set()
        self._pending_commits = set()
        self._flushed = False

    def clear_connector_metadata(self) -> None:
        super().clear_connector_metadata()
        self._meta = None

    def start_load_kv(self, forward_context: Any, **kwargs: Any) -> None:
        """Reads every load request's records, then one scatter (with
        re-rotation where positions moved). All device work is enqueued on
        the current stream before returning, so it precedes the forward pass
        (also under full graph replay, which skips per-layer hooks)."""
        if self._meta is None or not self._meta.reqs_to_load or self._plane.table is None:
            return
        plan = plan_load(self._meta.reqs_to_load, self._slot_size)
        if plan.deltas and self._plane.table.layout.dtype == torch.float8_e4m3fn:
            self._plane.k_scales = self._fp8_k_scales(forward_context)
        self._plane.load(plan)

    def _fp8_k_scales(self, forward_context: Any) -> torch.Tensor:
        """Per-layer K scales of an e4m3 cache, in registration order: the
        attention modules' ``_k_scale`` (vLLM keeps them there; the forward
        context maps layer names to the modules in ``no_compile_layers``), or
        ``kv_connector_extra_config["k_scale"]`` for one scale everywhere.
        Read at every load, since vLLM may recompute them after its first
        pass. Rotating e4m3 codes needs them; without them this raises."""
        dev = self._plane.device
        names = self._plane.layer_names
        layers = getattr(forward_context, "no_compile_layers", None) or {}
        found = [getattr(layers.get(n), "_k_scale", None) for n in names]
        if all(t is not None for t in found):
            return torch.stack([torch.as_tensor(t, dtype=torch.float32, device=dev).reshape(())
                                for t in found])
        if self._k_scale_cfg is not None:
            return torch.full((len(names),), float(self._k_scale_cfg), dtype=torch.float32,
                              device=dev)
        missing = [n for n, t in zip(names, found) if t is None]
        raise ValueError(
            "re-rotating an fp8 KV cache needs each layer's K scale: none found for "
            f"{missing[:3]}{'...' if len(missing) > 3 else ''} in "
            "forward_context.no_compile_layers[layer]._k_scale, and no "
            "kv_connector_extra_config['k_scale']")

    def wait_for_layer_load(self, layer_name: str) -> None:
        return

    def _ensure_store_plan(self) -> bool:
        if (self._meta is None or not self._meta.reqs_to_store or self._plane.table is None
                or self._flushed):
            return False
        if self._store_plan is None:
            self._store_plan = plan_store(self._meta.reqs_to_store, self._slot_size)
            self._store_arena = self._plane.new_store_arena(self._store_plan)
        return True

    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, attn_metadata: Any,
                      **kwargs: Any) -> None:
        """Enqueues this layer's gather for every store request."""
        if not self._ensure_store_plan():
            return
        for spec in self._meta.reqs_to_store.values():
            self._pending_commits.add(spec.chunk_key)
        if layer_name not in self._plane.layer_idx:
            logger.warning("[CONNECTOR] save_kv_layer: unknown layer %s, skipping", layer_name)
            return
        if self._plane.save_mode == "per_layer":
            self._plane.save_layer(layer_name, self._store_plan, self._store_arena)
        self._saved_layers.add(self._plane.layer_idx[layer_name])

    def wait_for_save(self) -> None:
        """Writes each request's records to the store, then commits. Layers
        whose save_kv_layer never ran this step (all of them under full
        graph replay, which skips per-layer hooks) are gathered here, so no
        record is written with unset bytes."""
        if self._flushed or not self._ensure_store_plan():
            return
        for spec in self._meta.reqs_to_store.values():
            self._pending_commits.add(spec.chunk_key)
        if self._plane.save_mode == "deferred":
            self._plane.save_all(self._store_plan, self._store_arena)
        else:
            for name, idx in self._plane.layer_idx.items():
                if idx not in self._saved_layers:
                    self._plane.save_layer(name, self._store_plan, self._store_arena)
        if self._async_save:
            self._plane.flush_async(self._store_plan, self._store_arena, self._commit_written)
        else:
            self._plane.flush(self._store_plan, self._store_arena)
        self._store_plan = None
        self._store_arena = None
        self._flushed = True
        if self._pending_commits and not self._async_save:
            keys = list(self._pending_commits)
            self._bg.run(self._commit_keys(keys), timeout=120.0)
        self._pending_commits.clear()

    async def _commit_keys(self, keys: list[str]) -> None:
        await asyncio.gather(*(self._ipc_async.commit_chunk(k) for k in keys))

    def _commit_written(self, keys: list[str], err: Optional[BaseException]) -> None:
        """async_save: runs on the writer thread once a step's records are in
        the file; commits the chunks written (a failed write is logged and
        its chunk stays uncommitted, so lookups keep missing it)."""
        if err is not None:
            logger.error("[CONNECTOR] async save failed after %d chunk(s): %s", len(keys), err)
        if keys:
            self._commit_futs.append(
                asyncio.run_coroutine_threadsafe(self._commit_keys(keys), self._bg.loop))

    def shutdown(self) -> None:
        if self._role_kind != KVConnectorRole.WORKER:
            return
        self._plane.drain(timeout=120.0)  # async_save: the last steps' writes
        for f in self._commit_futs:
            try:
                f.result(timeout=120.0)
            except Exception as exc:  # noqa: BLE001 - reported, shutdown continues
                logger.error("[CONNECTOR] commit failed: %s", exc)
        self._commit_futs = []
        self._plane.close()
        self._bg.stop()
