"""Test infrastructure only: a CPU restatement of the reference's host-tier
page cache, the checker for imi_hostcache_* and the host-tier decode step.
Nothing under adaptiveimi_amd/ imports it.

Reference: library/AdaptiveIMI/cpp_extensions/src/wave_buffer_cpu_hotcold.cpp
  BufferManager               54-372
    resolve_hot_capacity      75-95    (IMI_HOTCOLD_HOT_RATIO, default 0.3)
    list_remove / push_front  97-125
    demote_hot_if_needed      127-137
    touch_hot / touch_cold    139-151
    promote_to_hot            153-165
    removeLeastRecentlyUsed   167-188
    batch_update              216-293
    batch_access              295-371
  AdpIMI_Index::set_cluster_metadata  850-895

Pinned by tests/test_hostcache.py: hand-worked scenarios (a miss, its
admission, a hit and its promotion, hot-list spill, LRU eviction order,
capacity-bounded admission, the page rule, oversized clusters) whose
expected lists follow from the reference's steps, and invariants (every
cache block owned at most once, owned + free = capacity) over random runs.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple


class Group:
    """BufferManager of one group (KV head) over its cells (clusters)."""

    def __init__(self, sizes: Sequence[int], offsets: Sequence[int], capacity: int, block_size: int,
                 max_consider: int, hot_ratio: float = 0.0):
        self.capacity, self.block_size, self.max_consider = capacity, block_size, max_consider
        ratio = hot_ratio if hot_ratio > 0.0 else 0.3          # :75-95
        ratio = min(ratio, 1.0)
        target = int(capacity * ratio)
        self.hot_capacity = target if target > 0 else min(capacity, 1)
        self.start = [int(o) for o in offsets[:len(sizes)]]   # set_cluster_metadata :868-891
        self.blocks = [(int(s) + block_size - 1) // block_size if s > 0 else 0 for s in sizes]
        self.last = [(int(s) % block_size or block_size) if s > 0 else 0 for s in sizes]
        n = len(sizes)
        self.cached = [False] * n
        self.hot = [False] * n
        self.ids: List[List[int]] = [[] for _ in range(n)]
        self.free = list(range(capacity))                      # constructor :196-199
        self.hot_list: List[int] = []    # front = most recent
        self.cold_list: List[int] = []
        self.hit_keys: List[int] = []
        self.miss_keys: List[int] = []

    def _hot_blocks(self) -> int:
        return sum(self.blocks[k] for k in self.hot_list)

    def access(self, keys: Sequence[int]):
        """batch_access :295-371 -> (hit blocks, miss blocks) as lists of
        (cache block id | first list row, rows, row prefix)."""
        self.hit_keys, self.miss_keys = [], []
        hits, misses = [], []
        hrow = mrow = consider = 0
        for key in keys:
            key = int(key)
            if self.blocks[key] == 0 or self.last[key] == 0:
                continue
            consider += self.blocks[key]
            if consider > self.max_consider:
                break
            nb = self.blocks[key]
            if not self.cached[key]:
                self.miss_keys.append(key)
                for j in range(nb):
                    span = self.last[key] if j + 1 == nb else self.block_size
                    misses.append((self.start[key] + j * self.block_size, span, mrow))
                    mrow += span
            else:
                self.hit_keys.append(key)
                for j in range(nb):
                    span = self.last[key] if j + 1 == nb else self.block_size
                    hits.append((self.ids[key][j], span, hrow))
                    hrow += span
        return hits, misses

    def _promote(self, key: int) -> None:
        """promote_to_hot :153-165 with demote_hot_if_needed :127-137."""
        if self.blocks[key] > self.hot_capacity:
            self.cold_list.remove(key)
            self.cold_list.insert(0, key)                      # touch_cold
            return
        self.cold_list.remove(key)
        self.hot[key] = True
        self.hot_list.insert(0, key)
        while self._hot_blocks() > self.hot_capacity and self.hot_list:
            d = self.hot_list.pop()
            self.hot[d] = False
            self.cold_list.insert(0, d)

    def _evict(self) -> None:
        """removeLeastRecentlyUsed :167-188."""
        if self.cold_list:
            v = self.cold_list.pop()
        elif self.hot_list:
            v = self.hot_list.pop()
        else:
            return
        self.hot[v] = False
        self.free.extend(self.ids[v][:self.blocks[v]])
        self.cached[v] = False

    def update(self):
        """batch_update :216-293 -> admitted blocks as (cache block id, rows,
        row prefix in the miss region)."""
        for key in reversed(self.hit_keys):
            if self.blocks[key] == 0 or self.last[key] == 0:
                continue
            if self.hot[key]:
                self.hot_list.remove(key)
                self.hot_list.insert(0, key)                   # touch_hot
            else:
                self._promote(key)
        admit = need = 0
        for key in self.miss_keys:
            if need + self.blocks[key] > self.capacity:
                break
            admit += 1
            need += self.blocks[key]
        out = []
        if admit:
            while len(self.free) < need:
                self._evict()
            row = 0
            for key in self.miss_keys[:admit]:
                nb = self.blocks[key]
                if len(self.free) < nb:
                    continue
                self.cached[key] = True
                self.hot[key] = False
                base = len(self.free) - nb
                self.ids[key] = [0] * nb
                for j in range(nb):
                    bid = self.free[base + nb - 1 - j]
                    span = self.last[key] if j + 1 == nb else self.block_size
                    self.ids[key][j] = bid
                    out.append((bid, span, row))
                    row += span
                del self.free[base:]
                self.cold_list.insert(0, key)
        self.hit_keys, self.miss_keys = [], []
        return out

    def owned_blocks(self) -> Dict[int, int]:
        """cache block -> owning cell, over the cached cells."""
        own = {}
        for k, c in enumerate(self.cached):
            if c:
                for b in self.ids[k][:self.blocks[k]]:
                    assert b not in own, "cache block owned twice"
                    own[b] = k
        return own


def run(groups: Sequence[Group], steps: Sequence[Sequence[Sequence[int]]]):
    """Per step: access with each group's keys, then update; returns per step
    and group (hits, misses, admitted)."""
    out = []
    for keys in steps:
        step = []
        for gr, k in zip(groups, keys):
            h, m = gr.access(k)
            u = gr.update()
            step.append((h, m, u))
        out.append(step)
    return out
