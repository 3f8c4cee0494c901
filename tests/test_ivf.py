"""IVF indexing (subspace_parts = 0), host side: the library's limits and
the oracle's one-subspace restatement.

Reference: kmeans_core.cpp:503-595 (KmeansExecutorIVF), reorganize_core.cpp
:178-231 (build_compact_reorg_input_ivf), layer_pipeline.cpp:177-228 and
1142-1148 (k = runtime k1 or round(T / 16)), indexing.py:179-181 (sizing).
"""
import ctypes

import numpy as np
import pytest

from oracle import oracle as orc


@pytest.fixture(scope="module")
def L():
    from adaptiveimi_amd import _lib
    return _lib.lib()


def test_ivf_sizing_and_adaptive_k():
    # round(T / 16) clusters (std::round, half away from zero), n_c = k + 1
    assert orc.adaptive_k(16384, subspace_parts=0) == [1024]
    assert orc.adaptive_k(24, subspace_parts=0) == [2]          # round(1.5) = 2
    assert orc.adaptive_k(8, subspace_parts=0) == [1]           # round(0.5) = 1
    sz = orc.sizing(16384, 0.1, subspace_parts=0)
    assert sz["n_centroids"] == 1025 and sz["nprobe"] == 102 and sz["padding_cluster_id"] == 1024


def test_ivf_compaction_is_rank_of_used_labels():
    """build_compact_reorg_input_ivf: compact id = rank of the label among the
    used labels, offsets = exclusive prefix of the counts, tokens of a cell
    in ascending order (checked against a direct numpy restatement)."""
    rng = np.random.default_rng(3)
    T, k = 5000, 700
    lab = rng.integers(0, k, T).astype(np.int32)
    lab[lab % 7 == 3] = 5            # some labels unused, one crowded
    r = orc.compact_reorg([lab], [k])
    used = np.unique(lab)
    assert r["n_active"] == len(used) and np.array_equal(r["gids"], used)
    counts = np.array([(lab == g).sum() for g in used])
    assert np.array_equal(np.diff(r["offsets"]), counts) and r["offsets"][0] == 0
    assert np.array_equal(r["perm"], np.argsort(lab, kind="stable"))


def test_ivf_kmeans_head_is_one_full_width_run():
    """kmeans_head with one k: one Lloyd run over all 128 dims (no subvector
    split), kmeans++ seeded with 42 as KmeansExecutorIVF does."""
    rng = np.random.default_rng(4)
    x = rng.standard_normal((400, 128)).astype(np.float32)
    labs, cents, _ = orc.kmeans_head(x, [20], 2, init="kmeans++")
    c0 = orc.kmeanspp_init(x, 20, 42)
    c, lab, _ = orc.lloyd(x, c0, 2)
    assert np.array_equal(cents[0], c) and np.array_equal(labs[0], lab)
    assert cents[0].shape == (20, 128)


def _kargs(parts, k, dim=128):
    from adaptiveimi_amd import _lib
    a = _lib.KmeansArgs(keys=16, head_stride=128 * 1000, token_stride=128, kv_heads=2, n_tokens=1000, dim=dim,
                        parts=parts, max_iters=2, init_mode=0, centroids=16, labels=16)
    for i in range(parts):
        a.k[i] = k
    return a


def test_ivf_library_limits(L):
    from adaptiveimi_amd import _lib
    need = ctypes.c_size_t()
    assert L.imi_kmeans_workspace_size(ctypes.byref(_kargs(1, 700)), ctypes.byref(need)) == 0
    big = _kargs(1, 4097)
    big.n_tokens = 5000
    assert L.imi_kmeans_workspace_size(ctypes.byref(big), ctypes.byref(need)) != 0
    assert "4096" in L.imi_last_error().decode()
    # subspaces of 2 / 4 keep their 512 limit
    assert L.imi_kmeans_workspace_size(ctypes.byref(_kargs(2, 512)), ctypes.byref(need)) == 0
    assert L.imi_kmeans_workspace_size(ctypes.byref(_kargs(2, 513)), ctypes.byref(need)) != 0
    assert "512" in L.imi_last_error().decode()
    # selection: IVF through the ranking pipeline, with or without the online update
    a = _lib.SelectArgs(query=16, centroids=16, cell_count=16, cell_offset=16, kv_heads=2, groups=4, dim=128,
                        parts=1, nprobe=10, max_tokens=100, buffer_pages=20, page_size=8, tile_mode=0)
    a.k[0] = 100
    a.sel_cap = 10
    assert L.imi_select_workspace_size(ctypes.byref(a), ctypes.byref(need)) == 0 and need.value > 0
    a.ring_cap, a.ring_cell, a.ring_row, a.ring_n = 1, 16, 16, 16
    assert L.imi_select_workspace_size(ctypes.byref(a), ctypes.byref(need)) == 0
    a.k[0] = 4097
    assert L.imi_select_workspace_size(ctypes.byref(a), ctypes.byref(need)) != 0
    assert "IVF" in L.imi_last_error().decode()
