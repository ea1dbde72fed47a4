"""The native page-pool allocator (libpal_hip.so, host side; no GPU needed)
against its specification and the oracle's compaction plan.

Pinned by: lowest-first allocation, atomic failure on exhaustion and on bad
frees, and a compaction plan that equals the oracle's on random
allocate/free histories and satisfies the invariants that fix it (the live
set becomes [0, L), ids already below L stay, each mover lands in a hole).
"""

from __future__ import annotations

import numpy as np
import pytest

import proxy_attention_lab as pal
from oracle import pal_oracle as orc


def test_allocate_lowest_first_and_free():
    pool = pal.PagePool(10)
    assert pool.num_free == 10
    a = pool.allocate(4)
    assert a.tolist() == [0, 1, 2, 3]
    pool.free([1, 2])
    assert pool.allocate(3).tolist() == [1, 2, 4]
    assert pool.num_used == 5


def test_exhaustion_and_bad_frees_change_nothing():
    pool = pal.PagePool(5)
    pool.allocate(3)
    with pytest.raises(RuntimeError, match="out of pages"):
        pool.allocate(3)
    assert pool.num_free == 2
    for bad, msg in (([7], "out of range"), ([3], "not allocated"), ([0, 0], "twice"), ([1, 4], "not allocated")):
        with pytest.raises(ValueError, match=msg):
            pool.free(bad)
        assert pool.num_free == 2
    pool.free([0, 1, 2])
    assert pool.num_free == 5


@pytest.mark.parametrize("seed", range(6))
def test_compaction_plan_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 400))
    pool = pal.PagePool(n)
    live = set()
    for _ in range(40):  # random allocate / free history
        if live and rng.random() < 0.45:
            k = int(rng.integers(1, len(live) + 1))
            drop = rng.choice(sorted(live), size=k, replace=False)
            pool.free(drop)
            live -= set(int(x) for x in drop)
        else:
            k = int(rng.integers(0, pool.num_free + 1))
            live |= set(int(x) for x in pool.allocate(k))
    used = np.array(sorted(live), np.int64)
    src, dst = pool.compaction_plan()
    esrc, edst = orc.compaction_plan(used, n)
    assert np.array_equal(src, esrc) and np.array_equal(dst, edst)
    # invariants: the live set becomes [0, L); nothing below L moves; holes are filled
    L = len(used)
    after = (set(live) - set(src.tolist())) | set(dst.tolist())
    assert after == set(range(L))
    assert np.all(src >= L) and np.all(dst < L)
    # the allocator agrees: exactly the ids [0, L) are taken
    assert pool.num_used == L
    if L < n:
        assert pool.allocate(1)[0] == L
    # a second plan has nothing left to move
    pool2 = pal.PagePool(n)
    pool2.allocate(L)
    s2, _ = pool2.compaction_plan()
    assert s2.size == 0


def test_oracle_apply_and_remap():
    pool = np.arange(6 * 3).reshape(6, 3)
    src, dst = np.array([4, 5], np.uint32), np.array([0, 2], np.uint32)
    out = orc.apply_moves(pool, src, dst)
    assert np.array_equal(out[0], pool[4]) and np.array_equal(out[2], pool[5]) and np.array_equal(out[1], pool[1])
    t = np.array([[4, 1, 5], [3, 9, 0]], np.uint32)
    assert orc.remap_table(t, src, dst, 6).tolist() == [[0, 1, 2], [3, 9, 0]]


def test_rejected_compact_changes_nothing():
    """compact() checks its pools and tables before it plans: a rejected call
    leaves the allocator's state (and the caller's tables) as they were."""
    import torch

    pool = pal.PagePool(8)
    pool.allocate(6)
    pool.free([1, 2])
    free_before = pool.num_free
    k = torch.zeros((8, 1, 2, 16, 8), dtype=torch.bfloat16)  # host tensors: not a HIP device
    v = torch.zeros((8, 1, 16, 16), dtype=torch.bfloat16)
    table = torch.tensor([[0, 3, 4, 5]], dtype=torch.int64)
    with pytest.raises(ValueError, match="HIP device"):
        pool.compact(k, v, [table])
    assert pool.num_free == free_before
    assert table.tolist() == [[0, 3, 4, 5]]
    # the plan is still the one the allocator held before the rejected call
    src, dst = pool.compaction_plan()
    assert src.tolist() == [4, 5] and dst.tolist() == [1, 2]
