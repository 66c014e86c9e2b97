"""ops.whole_pages: the host-side split of a token-form scatter into whole
record pages (page kernel) and ragged rows (token kernel), checked against a
per-block brute force on random slot tables."""

from __future__ import annotations

import numpy as np
import pytest

from daser_amd import ops


def _brute(sm, ro, bs, row, ri):
    """Whole blocks by definition: every slot of the block listed, in
    consecutive entries, in slot order, record rows stepping by row, one
    table index."""
    pages, offs, rope, rest = [], [], [], np.ones(sm.size, bool)
    for i in range(sm.size - bs + 1):
        s = sm[i:i + bs]
        if s[0] < 0 or s[0] % bs:
            continue
        if not np.array_equal(s, s[0] + np.arange(bs)):
            continue
        if not np.array_equal(ro[i:i + bs], ro[i] + np.arange(bs) * row):
            continue
        if ri is not None and np.any(ri[i:i + bs] != ri[i]):
            continue
        pages.append(s[0] // bs)
        offs.append(ro[i])
        rope.append(-9 if ri is None else ri[i])
        rest[i:i + bs] = False
    return pages, offs, rope, rest


@pytest.mark.parametrize("seed", range(12))
@pytest.mark.parametrize("bs", [4, 16])
def test_whole_pages_match_brute_force(seed, bs):
    rng = np.random.default_rng(seed)
    row = 256
    nreq = int(rng.integers(1, 9))
    toks = rng.integers(1, 6 * bs, size=nreq)
    pages = -(-toks // bs)
    perm = rng.permutation(int(pages.sum()) + 5)
    tables, k = [], 0
    for p in pages:
        tables.append(perm[k:k + p].tolist())
        k += p
    sm = ops.slot_mapping_for(tables, toks, bs)
    ro = ops.token_row_offsets(toks, 1 << 16, bs, row)
    ri = np.repeat(rng.integers(-1, 3, size=nreq), toks)
    # damage: padding, a record row out of step, a mid-request table change
    sm[rng.random(sm.size) < 0.03] = -1
    if sm.size > 5:
        ro[int(rng.integers(0, sm.size))] += 16
        ri[int(rng.integers(0, sm.size))] = 7
    order = np.argsort(sm, kind="stable")
    sm, ro, ri = sm[order], ro[order], ri[order]
    for r in (None, ri):
        got = ops.whole_pages(sm, ro, bs, row, r)
        want = _brute(sm, ro, bs, row, r)
        assert got[0].tolist() == want[0]
        assert got[1].tolist() == want[1]
        if r is not None:
            assert got[2].tolist() == want[2]
        assert np.array_equal(got[3], want[3])


def test_whole_pages_small_and_empty():
    e = ops.whole_pages(np.zeros(0, np.int64), np.zeros(0, np.int64), 16, 256)
    assert e[0].size == 0 and e[3].size == 0
    got = ops.whole_pages(np.arange(3, dtype=np.int64), np.arange(3) * 256, 4, 256)
    assert got[0].size == 0 and got[3].all()
    sm = np.arange(8, dtype=np.int64)
    got = ops.whole_pages(sm, sm * 256 + 4096, 4, 256)
    assert got[0].tolist() == [0, 1] and got[1].tolist() == [4096, 5120] and not got[3].any()


def test_last_per_slot_keeps_the_last_entry():
    sm = np.array([5, 9, 5, -1, 9, 2], np.int64)
    assert ops._last_per_slot(sm).tolist() == [-1, -1, 5, -1, 9, 2]
    assert ops._last_per_slot(np.array([1, 2], np.int64)).tolist() == [1, 2]
