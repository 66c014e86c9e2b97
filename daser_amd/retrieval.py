"""Retrieval indexes for the DaseR server, keyed the reference's way.

The reference server asks a pluggable ``RetrievalIndex`` (lookup / insert /
remove, daser/retrieval/base.py:10-48) for the cached chunks matching a
prompt; its only implementation, ``PrefixHashIndex``
(daser/retrieval/prefix.py:33-90), hashes every block-aligned prefix from
scratch, longest first, and returns at most one chunk: the longest cached
prefix. A chunk's key is ``xxh3_128`` of its int32 token ids
(daser/retrieval/prefix.py:17-30, daser/service/chunker.py:10-25), whether it
was stored as a whole prompt's aligned prefix by the connector or as one
fixed-size piece of a document by the service's chunker.

Two indexes with the same interface, both driven by the one-pass prefix keys
of :mod:`daser_amd.prefix_hash` (the xxh3 streaming state yields the key of
every aligned prefix while the tokens are fed once):

``IncrementalPrefixIndex``
    the reference's lookup (same hit, same single-element result) in one
    hashing pass instead of one pass per candidate length.
``ChunkAssemblyIndex``
    a RAG prompt is usually several cached pieces back to back (retrieved
    document chunks, each prefilled on its own at position 0) followed by
    the question. This index tiles the prompt from its first token: at
    position p it takes the longest cached chunk whose tokens are exactly
    ``tokens[p:p + n]``, then continues at ``p + n``, until nothing matches.
    The chunks come back in prompt order; the first one is the reference's
    longest-prefix hit. The connector's scheduler places chunk i at the
    position where the previous ones end (checking each chunk's key against
    those tokens) and the worker re-rotates its K from the stored position
    to that one. Reusing separately prefilled chunks drops the attention
    between them; that is the reuse this path serves (the chunk-reuse
    workloads it is measured on), not an exact prefix hit.

Both accept the reference's ``ChunkMeta`` or any object with its fields
(``chunk_key``, ``token_count``, ``model_id``, ...), so the reference server
can host them in place of ``PrefixHashIndex``: they subclass its
``RetrievalIndex`` when that package is importable.
"""

from __future__ import annotations

import array
from abc import ABC, abstractmethod
from dataclasses import dataclass, field
from typing import Any

import numpy as np

from daser_amd.prefix_hash import prefix_keys

try:  # the reference's interface, when its package is installed
    from daser.retrieval.base import RetrievalIndex  # type: ignore
except ImportError:  # pragma: no cover - the reference is not installed here

    class RetrievalIndex(ABC):  # type: ignore[no-redef]
        """The reference's retrieval interface (daser/retrieval/base.py:10-48)."""

        @abstractmethod
        async def lookup(self, tokens: list[int], model_id: str) -> list[Any]:
            """Chunks matching ``tokens``, best first; may be empty."""

        @abstractmethod
        async def insert(self, meta: Any) -> None:
            """Adds a committed chunk."""

        @abstractmethod
        async def remove(self, chunk_key: str) -> None:
            """Drops an evicted chunk (unknown keys are ignored)."""


__all__ = ["ChunkAssemblyIndex", "ChunkMeta", "IncrementalPrefixIndex", "RetrievalIndex",
           "chunk_key"]


@dataclass
class ChunkMeta:
    """The fields of the reference's ChunkMeta (daser/server/metadata_store.py:18-45)
    that a lookup reply carries; used where the reference is not installed."""

    chunk_key: str
    start_slot: int
    num_slots: int
    token_count: int
    pos_offset: int
    model_id: str
    created_at: float = 0.0
    doc_ids: list[str] = field(default_factory=list)


def chunk_key(tokens) -> str:
    """xxh3_128 hex of the int32 token ids: the key every DaseR component
    gives a chunk (reference daser/retrieval/prefix.py:17-30)."""
    import xxhash

    return xxhash.xxh3_128(bytes(array.array("i", [int(t) for t in tokens]))).hexdigest()


class _KeyedIndex(RetrievalIndex):
    """Committed chunks by key (insert replaces, remove ignores unknown keys,
    as the reference's dict does)."""

    def __init__(self, block_tokens: int = 16) -> None:
        if block_tokens <= 0:
            raise ValueError("block_tokens must be positive")
        self._block_tokens = int(block_tokens)
        self._index: dict[str, Any] = {}

    async def insert(self, meta: Any) -> None:
        self._index[meta.chunk_key] = meta

    async def remove(self, chunk_key: str) -> None:
        self._index.pop(chunk_key, None)

    def __len__(self) -> int:
        return len(self._index)

    def _longest_at(self, toks: np.ndarray, start: int, model_id: str,
                    limit: int) -> tuple[int, Any]:
        """(tokens, chunk) of the longest cached chunk of this model that is
        exactly ``toks[start:start + n]`` for an aligned n <= limit; (0, None)
        if none is."""
        bs = self._block_tokens
        keys = prefix_keys(toks[start:start + limit], bs)
        for i in range(len(keys) - 1, -1, -1):
            meta = self._index.get(keys[i])
            if meta is not None and meta.model_id == model_id:
                return (i + 1) * bs, meta
        return 0, None


class IncrementalPrefixIndex(_KeyedIndex):
    """Longest cached block-aligned prefix of the prompt, at most one chunk:
    the reference's PrefixHashIndex.lookup (daser/retrieval/prefix.py:49-72)
    with all candidate keys from one streaming pass."""

    async def lookup(self, tokens: list[int], model_id: str) -> list[Any]:
        toks = np.asarray(tokens, dtype=np.int32)
        n, meta = self._longest_at(toks, 0, model_id, toks.size)
        return [meta] if n else []


class ChunkAssemblyIndex(_KeyedIndex):
    """Cached chunks tiling the prompt from token 0, in prompt order (see the
    module docstring). ``max_chunks`` bounds the reply. A chunk is at most
    as long as the longest one ever inserted, so each position's scan hashes
    at most that many tokens."""

    def __init__(self, block_tokens: int = 16, max_chunks: int = 256) -> None:
        super().__init__(block_tokens)
        self._max_chunks = int(max_chunks)
        self._longest = 0

    async def insert(self, meta: Any) -> None:
        await super().insert(meta)
        self._longest = max(self._longest, int(meta.token_count))

    async def lookup(self, tokens: list[int], model_id: str) -> list[Any]:
        toks = np.asarray(tokens, dtype=np.int32)
        out: list[Any] = []
        pos = 0
        while len(out) < self._max_chunks and pos < toks.size:
            n, meta = self._longest_at(toks, pos, model_id, self._longest)
            if not n:
                break
            out.append(meta)
            pos += n
        return out
