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
``allow_chunk_assembly`` (default False: only the first chunk of a lookup
reply is loaded, the reference's single prefix hit; True: consecutive
chunks of the reply are assembled, see :func:`place_chunks`; their tokens
then lack the attention between chunks that a full prefill would have),
``store_path`` may hold ``{rank}``, replaced by the worker's tensor-parallel
rank (one store file per rank; the reference's single path would make ranks
overwrite each other's records at the same offsets),
``io_backend`` ("mmap", default: the C++ ring of libdaser_kv copying
between its pinned slots and a shared mapping of the store file on worker
threads: buffered writes to one file serialise in the kernel, page faults
on a mapping do not; a disk read error or an outside truncation of the
store file then faults the process instead of failing the call;
"native": the same ring with io_uring (pread/pwrite) file calls;
"direct": the same ring with the store file opened O_DIRECT;
"python": the threaded ring of store_io.PinnedRingIO), ``k_scale`` (one K
scale for every layer of an fp8 cache, when the attention modules' own
``_k_scale`` are not reachable), ``async_save`` (wait_for_save returns once
the gathers are enqueued and ordered before the next step's KV writes; file
writes and commits finish on a background writer; default False, the
reference's blocking behaviour), ``save_stream``
("side": per-layer gathers on a side stream after the layer's KV writes,
overlapping later layers; "current": on the model's stream; "auto", default:
the side stream when one layer's gather moves at least 32 MiB, else the
model's stream, where a small gather costs less than ordering a side stream),
``block_size`` / ``head_dim`` / ``kv_layout`` (head geometry of caches whose
shape does not carry it: the 3-D (2, NB, block_size * H * D) caches of vLLM's
PagedAttention backend, whose K pages use the split-x layout, "kx"; read
from cache_config.block_size and the hf_config when not given; copies of
such caches need none of it).
"""

from __future__ import annotations

import array
import asyncio
import logging
import threading
from dataclasses import dataclass, field
from typing import Any, Optional

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

# the data path; re-exported here, where the reference keeps its connector
from daser_amd.data_plane import (  # noqa: E402
    KVDataPlane,
    LoadPlan,
    StorePlan,
    plan_load,
    plan_store,
)

__all__ = ["DaserConnector", "DaserConnectorMeta", "KVDataPlane", "LoadPlan", "LoadSegment",
           "ReqLoadSpec", "ReqStoreSpec", "StorePlan", "hash_tokens", "load_spec",
           "place_chunks", "plan_load", "plan_store", "rank_store_path"]


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
# placing looked-up chunks in the prompt (scheduler side)


def place_chunks(tokens: list[int], chunks: list[dict], block_tokens: int,
                 max_chunks: Optional[int] = None) -> list[tuple[int, dict]]:
    """(first token position, chunk) of each chunk of a lookup reply that the
    prompt can use, in prompt order, at most ``max_chunks`` of them (None: no
    limit).

    The first chunk goes at position 0, as the reference loads its single
    prefix hit (daser_connector.py:240-258, daser/retrieval/prefix.py:49-72).
    Each further chunk goes where the previous one ends, if that is a block
    boundary and its key is the hash of exactly the prompt tokens it would
    cover: a reply that lists alternatives rather than consecutive pieces
    stops after the first.
    Positions here are prompt positions; a chunk's stored position is its
    ``pos_offset``."""
    placed: list[tuple[int, dict]] = []
    pos = 0
    for i, ch in enumerate(chunks):
        if max_chunks is not None and i >= max_chunks:
            break
        n = int(ch.get("token_count", 0))
        if n <= 0 or pos + n > len(tokens) and i > 0:
            break
        if i > 0 and (pos % block_tokens or
                      hash_tokens(tokens[pos:pos + n]) != ch.get("chunk_key")):
            break
        placed.append((pos, ch))
        pos += n
    return placed


def load_spec(placed: list[tuple[int, dict]], block_ids: list[int], block_tokens: int,
              first_block: int = 0) -> Optional[ReqLoadSpec]:
    """The worker's load of placed chunks into the request's blocks: chunk
    i's records go to the blocks from ``position_i / block_size``, as far as
    the blocks reach, each with ``new_pos`` = its position. ``block_ids``
    are all of the request's blocks from token 0; those below
    ``first_block`` already hold vLLM's own KV (its local prefix cache hit,
    ``num_computed_tokens``) and receive nothing. A single chunk keeps the
    reference's flat fields; several become segments, indexing the returned
    ``block_ids``, which start at ``first_block``."""
    segs = []
    end = 0  # token after the last one loaded
    for pos, ch in placed:
        first = pos // block_tokens
        n = min(int(ch["num_slots"]), len(block_ids) - first)
        if n <= 0:
            break
        end = min(pos + int(ch["token_count"]), (first + n) * block_tokens)
        skip = max(0, first_block - first)  # pages vLLM computed itself
        if skip >= n:
            continue
        # the segment's first page moves by `skip`, both positions with it:
        # the rotation delta new_pos - pos_offset is unchanged
        segs.append(LoadSegment(start_slot=int(ch["start_slot"]) + skip, num_slots=n - skip,
                                block_offset=first + skip - first_block,
                                pos_offset=int(ch.get("pos_offset", 0)) + skip * block_tokens,
                                new_pos=pos + skip * block_tokens))
    if not segs:
        return None
    head = placed[0][1]
    used = block_ids[first_block:first_block + segs[-1].block_offset + segs[-1].num_slots]
    return ReqLoadSpec(
        chunk_key=head["chunk_key"], start_slot=segs[0].start_slot, num_slots=segs[0].num_slots,
        # file_offset stays the head chunk's: loads read start_slot * slot_size
        block_ids=used, file_offset=int(head["file_offset"]),
        token_count=end, pos_offset=segs[0].pos_offset, new_pos=segs[0].new_pos,
        segments=segs if len(segs) > 1 or segs[0].block_offset else [])


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


def _tp_rank() -> int:
    """This worker's tensor-parallel rank: vLLM's, when vLLM is running it,
    else LOCAL_RANK / RANK from the environment, else 0."""
    try:
        from vllm.distributed.parallel_state import get_tensor_model_parallel_rank  # type: ignore

        return int(get_tensor_model_parallel_rank())
    except Exception:  # vLLM absent or its groups not initialised
        import os

        return int(os.environ.get("LOCAL_RANK", os.environ.get("RANK", "0")))


def rank_store_path(path: str, rank: Optional[int] = None) -> str:
    """``store_path`` with ``{rank}`` replaced by the tensor-parallel rank.
    Under tensor parallelism every rank saves its own heads' records at the
    same slot offsets, so ranks need one store file each; the reference
    keeps one path for all ranks. A path without the placeholder is used as
    given."""
    if "{rank}" not in path:
        return path
    return path.replace("{rank}", str(_tp_rank() if rank is None else rank))


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
        # several separately prefilled chunks in one prompt skip the
        # attention between them: opt in, else only the first (the
        # reference's single prefix hit) is loaded
        self._allow_assembly = bool(extra.get("allow_chunk_assembly", False))
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
            from daser_amd.position import head_dim_from_hf, layer_rope_from_hf, model_rope_from_hf

            hf = getattr(getattr(vllm_config, "model_config", None), "hf_config", None)
            hf_theta, hf_scaling = model_rope_from_hf(hf) if hf is not None else (None, None)
            cache_cfg = getattr(vllm_config, "cache_config", None)
            # head geometry of caches whose shape does not carry it (3-D)
            geometry = {
                "block_size": extra.get("block_size", getattr(cache_cfg, "block_size", None)
                                        or self._block_tokens),
                "head_dim": extra.get("head_dim", head_dim_from_hf(hf) if hf is not None
                                      else None),
                "k_layout": extra.get("kv_layout"),
            }
            self._store_path = rank_store_path(self._store_path)
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
                io_backend=extra.get("io_backend", "mmap"),
                save_stream=extra.get("save_stream", "auto"),
                cache_geometry=geometry,
            )
            self._k_scale_cfg = extra.get("k_scale")  # uniform fp8 K scale, optional
            self._async_save = bool(extra.get("async_save", False))
            self._commit_futs: list = []
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
        """Asks the server for cached chunks of the prompt (one
        ``match_and_alloc`` RPC, as the reference does at :194-258: the
        block-aligned part of the prompt to look up, and the key under which
        a miss stores the whole aligned prompt) and places the chunks it
        returns (:func:`place_chunks`). Returns the tokens the placed chunks
        add beyond those vLLM already computed. A failed RPC is a miss."""
        rid = request.request_id
        tokens = list(request.prompt_token_ids)
        self._req_tokens[rid] = tokens
        bs = self._block_tokens
        lookup_len = num_computed_tokens + (len(tokens) - num_computed_tokens) // bs * bs
        if lookup_len - num_computed_tokens <= 0:
            return 0, False
        whole = len(tokens) // bs * bs
        try:
            reply = self._ipc_sync.match_and_alloc(
                tokens[:lookup_len], hash_tokens(tokens[:whole]) if whole else "",
                self._model_id)
        except Exception as exc:  # a failed lookup degrades to a miss
            logger.warning("[CONNECTOR] match_and_alloc failed: %s", exc)
            return 0, False
        if reply.get("alloc") is not None:
            self._pending_alloc[rid] = reply["alloc"]
        placed = place_chunks(tokens[:lookup_len], reply.get("chunks") or [], bs,
                              None if self._allow_assembly else 1)
        if not placed:
            return 0, False
        matched = placed[-1][0] + int(placed[-1][1]["token_count"])
        # vLLM computes at least the last prompt token itself (its logits
        # start the decode): a hit covering the whole prompt reports one token
        # less. The load still fills the last page; the recomputed token's
        # KV overwrites its own slot.
        new_tokens = min(matched, len(tokens) - 1) - num_computed_tokens
        if new_tokens <= 0:
            return 0, False
        self._pending_loads[rid] = {"placed": placed, "computed": num_computed_tokens}
        return new_tokens, False

    def update_state_after_alloc(self, request: Any, blocks: Any, num_external_tokens: int) -> None:
        """Records the blocks vLLM gave the request: those of tokens
        [num_computed_tokens, num_computed_tokens + num_external_tokens)
        receive a load, or those of the aligned prompt receive its store
        (reference :260-298, which counts the load's blocks from block 0
        and so assumes num_computed_tokens == 0)."""
        rid = request.request_id
        block_ids = [blk.block_id for blk in blocks.blocks[0]]
        bs = self._block_tokens
        pending = self._pending_loads.get(rid)
        if num_external_tokens > 0 and pending is not None:
            # vLLM's blocks start at token 0; its own prefix-cache hit (the
            # first num_computed_tokens, whole blocks) keeps its KV and the
            # external tokens follow it
            computed = pending["computed"]
            pending["block_ids"] = block_ids[:-(-(computed + num_external_tokens) // bs)]
            pending["first_block"] = computed // bs
            return
        alloc = self._pending_alloc.pop(rid, None)
        if alloc is not None:
            alloc["block_ids"] = block_ids[:-(-int(alloc["token_count"]) // bs)]
            self._pending_stores[rid] = alloc

    def build_connector_meta(self, scheduler_output: Any) -> DaserConnectorMeta:
        """Turns the scheduled requests' pending loads and stores into the
        worker's metadata (reference :300-357). Every load names the position
        its records go to: segment i lands at the token where chunk i was
        placed, so a chunk stored at ``pos_offset`` is re-rotated when that
        differs, including the reference's single prefix chunk (placed at 0)."""
        meta = DaserConnectorMeta()
        scheduled = scheduler_output.num_scheduled_tokens
        for rid in [r for r, p in self._pending_loads.items()
                    if r in scheduled and "block_ids" in p]:
            pending = self._pending_loads.pop(rid)
            spec = load_spec(pending["placed"], pending["block_ids"], self._block_tokens,
                             pending["first_block"])
            if spec is not None:
                meta.reqs_to_load[rid] = spec
        for rid in [r for r, a in self._pending_stores.items()
                    if r in scheduled and "block_ids" in a]:
            a = self._pending_stores.pop(rid)
            meta.reqs_to_store[rid] = ReqStoreSpec(
                chunk_key=a["chunk_key"], start_slot=a["start_slot"], num_slots=a["num_slots"],
                block_ids=a["block_ids"], file_offset=a["file_offset"],
                token_count=a["token_count"])
        return meta

    def request_finished(self, request: Any, block_ids: list[int]):
        for d in (self._req_tokens, self._pending_loads, self._pending_stores, self._pending_alloc):
            d.pop(request.request_id, None)
        return False, None

    # --------------------------------------------------------------- worker
    def register_kv_caches(self, kv_caches: dict[str, torch.Tensor]) -> None:
        fp8 = {"fp8": torch.float8_e4m3fn, "fp8_e4m3": torch.float8_e4m3fn,
               "fp8_e5m2": torch.float8_e5m2}.get(self._cache_dtype)
        if fp8 is not None:
            # vLLM may hold an fp8 cache as raw uint8; the re-rotation needs the
            # element format (OCP e4m3fn or e5m2 on gfx950). A view, no copy.
            kv_caches = {n: t.view(fp8) if t.dtype == torch.uint8 else t
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
        if plan.deltas and self._plane.table.layout.dtype in (torch.float8_e4m3fn,
                                                               torch.float8_e5m2):
            self._plane.k_scales = self._fp8_k_scales(forward_context)
        self._plane.load(plan)

    def _fp8_k_scales(self, forward_context: Any) -> torch.Tensor:
        """Per-layer K scales of an fp8 (e4m3 or e5m2) cache, in registration order: the
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
            self._pending_commits.update(s.chunk_key for s in self._meta.reqs_to_store.values())
        return True

    def save_kv_layer(self, layer_name: str, kv_layer: torch.Tensor, attn_metadata: Any,
                      **kwargs: Any) -> None:
        """Enqueues this layer's gather for every store request."""
        if not self._ensure_store_plan():
            return
        if layer_name not in self._plane.layer_idx:
            logger.warning("[CONNECTOR] save_kv_layer: unknown layer %s, skipping", layer_name)
            return
        if self._plane.save_mode == "per_layer":
            self._plane.save_layer(layer_name, self._store_plan, self._store_arena, kv_layer)
        self._saved_layers.add(self._plane.layer_idx[layer_name])

    def wait_for_save(self) -> None:
        """Writes each request's records to the store, then commits. Layers
        whose save_kv_layer never ran this step (all of them under full
        graph replay, which skips per-layer hooks) are gathered here, so no
        record is written with unset bytes."""
        if self._flushed or not self._ensure_store_plan():
            return
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
