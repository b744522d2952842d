"""Host allocator (libpkv pkv_pool_*) against the allocator restatement
(oracle/alloc.py) and the reference scheduler's own constants. CPU only."""
import numpy as np
import pytest

import pkv
from oracle.alloc import BlockPool


def test_fresh_pool_order_matches_reference():
    # free list [n-1 .. 0] (sched.rs:515); take_blocks splits off the tail
    # (sched.rs:801-807): a fresh pool's first request of 2 gets [1, 0].
    for P in (pkv.Pool, BlockPool):
        p = P(64)
        assert p.take(2) == [1, 0]
        assert p.take(3) == [4, 3, 2]
    p = pkv.Pool(8)
    assert p.free_list() == [7, 6, 5, 4, 3, 2, 1, 0]


def test_admission_counts_restated():
    """Restates sched.rs:1687-1697 (admission_reserves_the_whole_request):
    a pool of 2 blocks holds one request of 20 prompt + 12 output tokens
    (ceil(32 / 16) = 2 blocks) and nothing more."""
    p = pkv.Pool(2)
    assert len(p.take((20 + 12 + 15) // 16)) == 2
    with pytest.raises(pkv.PkvError) as e:
        p.take(1)
    assert e.value.status == pkv.ERR_NO_BLOCKS


def test_prefix_sharing_counts_restated():
    """Restates the block counts of sched.rs:1563-1622
    (prefixes_are_kept_reused_and_evicted) at the allocator level: a 150+2
    token request takes 10 blocks; its 128-token prefix entry keeps 8; after
    release 64 - 8 are free; a 250+1 token request reusing the 8 takes 8 more
    (ceil(251/16) = 16 - 8); its own 192-token entry refs 12; after release
    64 - 12 are free."""
    p = pkv.Pool(64)
    a = p.take((150 + 2 + 15) // 16)
    assert len(a) == 10
    entry1 = a[:128 // 16]
    p.ref(entry1)          # add_entry
    p.unref(a)             # release
    assert p.free_count() == 64 - 8
    p.ref(entry1)          # admit hit: share the prefix's pages
    own = p.take((250 + 1 + 15) // 16 - 8)
    seq = entry1 + own
    entry2 = seq[:192 // 16]
    p.ref(entry2)
    p.unref(seq)
    assert p.free_count() == 64 - 12
    # evicting both entries frees everything
    p.unref(entry1)
    p.unref(entry2)
    assert p.free_count() == 64


def test_random_ops_match_restatement():
    rng = np.random.default_rng(0)
    a, b = pkv.Pool(200), BlockPool(200)
    held = []
    for _ in range(3000):
        op = rng.integers(0, 3)
        if op == 0:
            n = int(rng.integers(0, 12))
            if n <= len(b.free):
                x, y = a.take(n), b.take(n)
                assert x == y
                held.extend(x)
        elif op == 1 and held:
            k = int(rng.integers(1, min(6, len(held)) + 1))
            idx = sorted(rng.choice(len(held), size=k, replace=False), reverse=True)
            ids = [held.pop(i) for i in idx]
            a.unref(ids)
            b.unref(ids)
        elif op == 2 and held:
            ids = [held[int(i)] for i in rng.choice(len(held), size=min(3, len(held)), replace=False)]
            a.ref(ids)
            b.ref(ids)
            held.extend(ids)
        assert a.free_list() == b.free
    assert [a.refs(i) for i in range(200)] == b.refs


def test_bad_unref_changes_nothing():
    p = pkv.Pool(4)
    ids = p.take(2)
    before = p.free_list()
    with pytest.raises(pkv.PkvError):
        p.unref([ids[0], ids[0]])  # underflow on the second
    assert p.free_list() == before and p.refs(ids[0]) == 1
    with pytest.raises(pkv.PkvError):
        p.unref([99])
    with pytest.raises(pkv.PkvError):
        p.ref([3 if 3 not in ids else 0 if 0 not in ids else 2])  # a free page cannot gain refs
