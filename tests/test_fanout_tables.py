"""ops.fanout_tables groups a scatter's host tables by source record: every
destination appears once, under the source it reads, in block order."""

from __future__ import annotations

import numpy as np

from daser_amd import ops


def test_fanout_tables_group_every_destination_under_its_source():
    rng = np.random.default_rng(3)
    for n_src, n in ((1, 1), (3, 50), (40, 41), (7, 500)):
        page_ids = rng.permutation(4 * n)[:n]
        offs = rng.integers(0, n_src, n) * 2 ** 21
        ridx = rng.integers(-1, 4, n)
        ids_o, offs_o, ridx_o = ops.dest_order(page_ids, offs, ridx)
        src, start, dpages, drope = ops.fanout_tables(ids_o, offs_o, ridx_o)
        assert start[0] == 0 and start[-1] == n and np.all(np.diff(start) > 0)
        assert np.all(np.diff(src) > 0)  # distinct sources, ascending
        assert sorted(dpages.tolist()) == sorted(page_ids.tolist())
        want = {int(p): (int(o), int(r)) for p, o, r in zip(page_ids, offs, ridx)}
        for s in range(src.size):
            block = dpages[start[s]:start[s + 1]]
            assert np.all(np.diff(block) > 0)  # block order inside a source
            for p, r in zip(block, drope[start[s]:start[s + 1]]):
                assert want[int(p)] == (int(src[s]), int(r))


def test_fanout_tables_without_rotation():
    src, start, dpages, drope = ops.fanout_tables(np.array([5, 2, 9]), np.array([64, 0, 64]))
    assert src.tolist() == [0, 64] and start.tolist() == [0, 1, 3]
    assert dpages.tolist() == [2, 5, 9] and drope is None
