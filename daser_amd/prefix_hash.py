"""Block-aligned prefix keys in one pass.

The reference keys a cached chunk by ``xxh3_128(bytes(array('i', tokens)))``
(daser/connector/daser_connector.py:41-57, daser/retrieval/prefix.py:17-30)
and finds the longest cached prefix by hashing every block-aligned prefix
from scratch, longest first (daser/retrieval/prefix.py:49-72): O(n^2 / bs)
bytes hashed per lookup, a cold-path cost its own notes list as open. The
xxh3 streaming state gives the digest of each prefix as the tokens are fed
once, so all n / bs keys cost one pass, and they are the same keys.
"""

from __future__ import annotations

from typing import Iterable, Mapping, Optional

import numpy as np


def prefix_keys(tokens: Iterable[int], block_tokens: int) -> list[str]:
    """Keys of the prefixes of length bs, 2 bs, ..., floor(n / bs) * bs, equal
    to ``hash_tokens(tokens[:k])`` of the reference for each k."""
    import xxhash

    if block_tokens <= 0:
        raise ValueError("block_tokens must be positive")
    buf = np.ascontiguousarray(np.asarray(list(tokens), dtype=np.int32)).tobytes()
    step = 4 * block_tokens
    h = xxhash.xxh3_128()
    keys = []
    for off in range(0, len(buf) - step + 1, step):
        h.update(buf[off:off + step])
        keys.append(h.hexdigest())
    return keys


def longest_prefix(index: Mapping[str, object], tokens: Iterable[int], block_tokens: int,
                   accept=None) -> tuple[int, Optional[object]]:
    """(matched tokens, entry) of the longest block-aligned prefix present in
    ``index`` (and accepted by ``accept(entry)``, e.g. a model_id check),
    else (0, None); the result of the reference's longest-first scan."""
    keys = prefix_keys(tokens, block_tokens)
    for i in range(len(keys) - 1, -1, -1):
        entry = index.get(keys[i])
        if entry is not None and (accept is None or accept(entry)):
            return (i + 1) * block_tokens, entry
    return 0, None
