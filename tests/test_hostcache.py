"""Host-tier page cache (wave_buffer_cpu_hotcold.cpp:54-372, 850-949).

CPU tests: the oracle's restatement against scenarios worked by hand from the
reference's steps, its invariants over random runs, and the library's
imi_hostcache_* (host code, no GPU call) against the oracle, list for list.
"""
import ctypes
import random

import numpy as np
import pytest

from oracle import hostcache as O


def _group(sizes, capacity, block_size, max_consider, ratio):
    offsets = np.concatenate([[0], np.cumsum(sizes)]).tolist()
    return O.Group(sizes, offsets, capacity, block_size, max_consider, ratio)


def test_oracle_worked_scenario():
    # capacity 4 blocks of 2 rows, hot capacity int(4 * 0.5) = 2; cells of
    # 3, 2, 0, 4, 1 rows: blocks 2, 1, 0, 2, 1; list rows 0, 3, 5, 5, 9
    g = _group([3, 2, 0, 4, 1], capacity=4, block_size=2, max_consider=10, ratio=0.5)
    # step 1: both miss; cell 0 takes free[3], free[2] (the back of the free
    # list, last block first), cell 1 takes free[1]; cold = [1, 0]
    h, m = g.access([0, 1])
    assert h == [] and m == [(0, 2, 0), (2, 1, 2), (3, 2, 3)]
    assert g.update() == [(3, 2, 0), (2, 1, 2), (1, 2, 3)]
    assert g.cold_list == [1, 0] and g.hot_list == [] and g.free == [0]
    # step 2: cell 1 hits and is promoted to hot; cell 3 misses and needs 2
    # blocks: the cold tail (cell 0) is evicted, freeing 3, 2 -> free
    # [0, 3, 2]; cell 3 takes free[2], free[1]
    h, m = g.access([1, 3])
    assert h == [(1, 2, 0)] and m == [(5, 2, 0), (7, 2, 2)]
    assert g.update() == [(2, 2, 0), (3, 2, 2)]
    assert g.hot_list == [1] and g.cold_list == [3] and g.free == [0]
    # step 3: cells 3 and 1 hit, 0 and 4 miss.  Hits are touched last to
    # first: cell 1 (already the hot head), then cell 3 promoted: hot
    # [3, 1] holds 3 blocks > 2, so cell 1 spills to the cold front.  The
    # misses need 3 blocks: evict the cold tail (cell 1: free [0, 1]), then
    # the hot tail (cell 3: free [0, 1, 2, 3]); cell 0 takes 3, 2, cell 4
    # takes 1
    h, m = g.access([0, 3, 1, 4])
    assert h == [(2, 2, 0), (3, 2, 2), (1, 2, 4)]
    assert m == [(0, 2, 0), (2, 1, 2), (9, 1, 3)]
    assert g.update() == [(3, 2, 0), (2, 1, 2), (1, 1, 3)]
    assert g.hot_list == [] and g.cold_list == [4, 0] and g.free == [0]
    assert g.cached == [True, False, False, False, True]


def test_oracle_page_rule_and_capacity():
    g = _group([4, 4, 2], capacity=2, block_size=2, max_consider=3, ratio=0.3)
    # blocks 2, 2, 1: the second cell takes the consideration to 4 > 3 and
    # stops the access (the page rule); the third is never looked at
    h, m = g.access([0, 1, 2])
    assert h == [] and m == [(0, 2, 0), (2, 2, 2)]
    assert g.update() == [(1, 2, 0), (0, 2, 2)]
    # capacity: misses 1 (2 blocks) then 2 (1 block): only the first fits
    g2 = _group([4, 4, 2], capacity=2, block_size=2, max_consider=10, ratio=0.3)
    g2.access([1, 2])
    assert g2.update() == [(1, 2, 0), (0, 2, 2)]
    assert g2.cached == [False, True, False]


def test_oracle_oversized_hit_stays_cold():
    # hot capacity int(4 * 0.3) = 1 block: a 2-block hit is refreshed in the
    # cold list instead of promoted
    g = _group([4, 2], capacity=4, block_size=2, max_consider=10, ratio=0.3)
    g.access([0, 1])
    g.update()
    assert g.cold_list == [1, 0]
    g.access([0])
    g.update()
    assert g.hot_list == [] and g.cold_list == [0, 1]
    g.access([1])
    g.update()
    assert g.hot_list == [1] and g.cold_list == [0]


def test_oracle_invariants_random():
    rng = random.Random(5)
    for trial in range(20):
        n = rng.randint(5, 40)
        sizes = [rng.choice([0, 1, 2, 3, 5, 8, 13]) for _ in range(n)]
        cap, bs = rng.randint(1, 12), rng.choice([1, 2, 4])
        g = _group(sizes, cap, bs, rng.randint(1, 20), rng.choice([0.0, 0.1, 0.5, 1.0]))
        for step in range(30):
            keys = rng.sample(range(n), rng.randint(0, n))
            g.access(keys)
            g.update()
            own = g.owned_blocks()
            assert len(own) + len(g.free) == cap
            assert set(own).isdisjoint(g.free)
            assert sorted(g.hot_list + g.cold_list) == sorted(k for k in range(n) if g.cached[k])


@pytest.fixture(scope="module")
def L():
    from adaptiveimi_amd import _lib
    return _lib.lib()


def _lists(mb, groups):
    return [np.zeros(groups * mb, np.int32) for _ in range(3)] + [np.zeros(groups, np.int32)]


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_library_matches_oracle(L, seed):
    from adaptiveimi_amd import _lib
    rng = np.random.default_rng(seed)
    groups, n = 3, 48
    bs = int(rng.choice([2, 8]))
    cap = int(rng.integers(4, 24))
    mb = int(rng.integers(6, 30))
    ratio = float(rng.choice([0.0, 0.25, 0.6]))
    nkeys = 20
    sizes = rng.choice([0, 1, 3, 7, 8, 9, 17], size=(groups, n)).astype(np.int32)
    sizes[:, -1] = 0                                   # the padding cell
    offsets = np.zeros((groups, n + 1), np.int32)
    offsets[:, 1:] = np.cumsum(sizes, axis=1)
    h = ctypes.c_void_p()
    _lib.check(L.imi_hostcache_create(groups, n, cap, bs, mb, nkeys, ratio, ctypes.byref(h)), "create")
    try:
        _lib.check(L.imi_hostcache_set_metadata(h, _p(sizes), _p(offsets)), "set_metadata")
        ref = [O.Group(sizes[g].tolist(), offsets[g].tolist(), cap, bs, mb, ratio) for g in range(groups)]
        for step in range(40):
            keys = np.stack([rng.permutation(n)[:nkeys] for _ in range(groups)]).astype(np.int64)
            keys[:, rng.integers(0, nkeys)] = n - 1    # a padding entry in the list
            hit = _lists(mb, groups)
            miss = _lists(mb, groups)
            _lib.check(L.imi_hostcache_access(h, _p(keys), nkeys, *map(_p, hit), *map(_p, miss)), "access")
            upd = _lists(mb, groups)
            _lib.check(L.imi_hostcache_update(h, *map(_p, upd)), "update")
            hb, mbk = ctypes.c_int64(), ctypes.c_int64()
            _lib.check(L.imi_hostcache_stats(h, ctypes.byref(hb), ctypes.byref(mbk)), "stats")
            tot_h = tot_m = 0
            for g in range(groups):
                eh, em = ref[g].access(keys[g].tolist())
                eu = ref[g].update()
                nh, nm, nu = hit[3][g], miss[3][g], upd[3][g]
                got_h = list(zip(*(hit[i][g * mb:g * mb + nh].tolist() for i in range(3))))
                got_m = list(zip(*(miss[i][g * mb:g * mb + nm].tolist() for i in range(3))))
                got_u = list(zip(*(upd[i][g * mb:g * mb + nu].tolist() for i in range(3))))
                assert got_h == eh, (step, g)
                assert got_m == em, (step, g)
                assert got_u == eu, (step, g)
                tot_h += nh
                tot_m += nm
            assert (hb.value, mbk.value) == (tot_h, tot_m)
    finally:
        L.imi_hostcache_destroy(h)


def test_library_rejects_bad_arguments(L):
    from adaptiveimi_amd import _lib
    h = ctypes.c_void_p()
    assert L.imi_hostcache_create(0, 4, 4, 2, 4, 4, 0.3, ctypes.byref(h)) == 1
    assert "positive" in L.imi_last_error().decode()
    _lib.check(L.imi_hostcache_create(1, 4, 4, 2, 4, 4, 0.3, ctypes.byref(h)), "create")
    try:
        sizes = np.array([2, 2, 2, 0], np.int32)
        offsets = np.array([0, 2, 4, 6, 6], np.int32)
        _lib.check(L.imi_hostcache_set_metadata(h, _p(sizes), _p(offsets)), "set_metadata")
        lists = _lists(4, 1) + _lists(4, 1)
        keys = np.array([7], np.int64)
        assert L.imi_hostcache_access(h, _p(keys), 1, *map(_p, lists)) == 1
        assert "outside" in L.imi_last_error().decode()
        keys = np.zeros(5, np.int64)
        assert L.imi_hostcache_access(h, _p(keys), 5, *map(_p, lists)) == 1
    finally:
        L.imi_hostcache_destroy(h)
    # two groups: a bad key in the second group rejects the whole access
    # before the first group's outputs or lists change, and an update after
    # the rejection admits nothing
    _lib.check(L.imi_hostcache_create(2, 4, 4, 2, 4, 4, 0.3, ctypes.byref(h)), "create")
    try:
        sizes = np.array([2, 2, 2, 0] * 2, np.int32)
        offsets = np.array([0, 2, 4, 6, 6] * 2, np.int32)
        _lib.check(L.imi_hostcache_set_metadata(h, _p(sizes), _p(offsets)), "set_metadata")
        lists = _lists(4, 2) + _lists(4, 2)
        good = np.array([0, 1, 2, 1], np.int64)
        _lib.check(L.imi_hostcache_access(h, _p(good), 2, *map(_p, lists)), "access")
        assert lists[7].tolist() == [2, 2]   # misses per group (nothing cached yet)
        for a in lists:
            a.fill(-5)
        bad = np.array([0, 1, 2, 9], np.int64)
        assert L.imi_hostcache_access(h, _p(bad), 2, *map(_p, lists)) == 1
        assert "outside" in L.imi_last_error().decode()
        assert all((a == -5).all() for a in lists)
        upd = _lists(4, 2)
        _lib.check(L.imi_hostcache_update(h, *map(_p, upd)), "update")
        assert upd[3].tolist() == [0, 0]
        # a valid access afterwards still sees an empty cache
        _lib.check(L.imi_hostcache_access(h, _p(good), 2, *map(_p, lists)), "access")
        assert lists[3].tolist() == [0, 0] and lists[7].tolist() == [2, 2]
    finally:
        L.imi_hostcache_destroy(h)
