"""CPU oracle for the AdaptiveIMI sparse-decode path (numpy + liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py``, never by the product package
``adaptiveimi_amd``.  Each function restates a step of the reference and cites
the file:line it follows (paths relative to the reference repository root).

Parity status per function (what pins it is in tests/test_oracle.py):
  sizing()              pinned: formula table + hand-computed cases
  kmeans E-step         pinned: brute force, integer-valued exact cases, tie rule
  kmeans M-step         pinned: closed-form mean, partition invariance on
                        integer data, constructed empty-cluster case
  kmeans++ init         pinned only on the same libstdc++ (mt19937_64 and the
                        distributions are replayed through <random>)
  compact/reorganize    pinned: invariants (offsets, ranks, stability)
  scores                pinned: exact on integer data, fp64 tolerance otherwise
  select                pinned: brute-force enumeration of the three rules
  attention             parity unpinned against the (unvendored)
                        weighted_flash_decoding; pinned against closed-form
                        softmax attention (uniform / one-hot cases)
  update_assign         the reference's torch.bmm summation order is parity
                        unpinned; the arg-max and its lowest-row tie rule are
                        pinned on integer data (exact dot products) and
                        against an fp64 arg-max away from near-ties
  OnlineUpdateOracle    pinned: closed-form running means on integer data,
                        the threshold/reset rule, ring order, and the
                        delta-match rules (kept cells, padding id) on
                        constructed cases
"""
from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path
from typing import Dict, List, Optional, Sequence

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_BASE_PATH = _HERE / "libcpudecode.so"
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i32p = ctypes.POINTER(ctypes.c_int32)
_i64p = ctypes.POINTER(ctypes.c_int64)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_u8p = ctypes.POINTER(ctypes.c_uint8)


def build(force: bool = False) -> Path:
    """Compile liboracle.so (the checker) and libcpudecode.so (the CPU
    baseline) with oracle/Makefile."""
    stale = any(not lib_.exists() or lib_.stat().st_mtime < (_HERE / src).stat().st_mtime
                for lib_, src in ((_LIB_PATH, "imi_oracle.cpp"), (_BASE_PATH, "cpu_decode.cpp")))
    if force or stale:
        subprocess.run(["make", "-B" if force else "-s", "-C", str(_HERE), "all"], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        build()
        L = ctypes.CDLL(str(_LIB_PATH))
        L.orc_l2.restype = ctypes.c_float
        L.orc_l2.argtypes = [_f32p, _f32p, ctypes.c_int]
        L.orc_estep.restype = ctypes.c_float
        L.orc_estep.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _f32p, ctypes.c_int, _i32p, _f32p, ctypes.c_int]
        L.orc_mstep.restype = None
        L.orc_mstep.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, _i32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_reseed_draws.restype = None
        L.orc_reseed_draws.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int, _i32p]
        L.orc_kmeanspp_init.restype = None
        L.orc_kmeanspp_init.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_uint64, _f32p]
        L.orc_lloyd_p.restype = ctypes.c_int
        L.orc_lloyd_p.argtypes = [_f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, _f32p, _i32p, ctypes.c_int,
                                  ctypes.c_float, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.orc_compact_reorg.restype = ctypes.c_int32
        L.orc_compact_reorg.argtypes = [_i32p, _i32p, ctypes.c_int, ctypes.c_int64, _i32p, _i32p, _i32p, _i32p]
        L.orc_scores.restype = None
        L.orc_scores.argtypes = [_u16p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p]
        L.orc_select.restype = None
        L.orc_select.argtypes = [_f32p, _i32p, _u8p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_int, _i32p, _i32p, _i64p]
        L.orc_update_assign.restype = None
        L.orc_update_assign.argtypes = [_f32p, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int, _i32p]
        L.orc_mt32_outputs.restype = None
        L.orc_mt32_outputs.argtypes = [ctypes.c_uint32, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint32)]
        L.orc_mt64_outputs.restype = None
        L.orc_mt64_outputs.argtypes = [ctypes.c_uint64, ctypes.c_int64, ctypes.POINTER(ctypes.c_uint64)]
        L.orc_attention.restype = None
        L.orc_attention.argtypes = [_u16p, _u16p, _u16p, ctypes.c_int64, _i64p, _i32p, ctypes.c_int64,
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_double, _f64p]
        _lib = L
    return _lib


def _p(a: np.ndarray, t):
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(t)


# ---------------------------------------------------------------- bf16 ----

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """Exact widen (kmeans_core.cpp:811-815): u16 << 16 reinterpreted as fp32."""
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit pattern (NaN kept quiet)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        rounded[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


# -------------------------------------------------------------- sizing ----

def sizing(list_capacity: int, retrieval_budget: float, subspace_parts: int = 2,
           buffer_cluster_num: int = 32, page_size: int = 8,
           k_override: Optional[Sequence[int]] = None) -> Dict[str, int]:
    """Decode sizing rules, cache_hub/adaptive_imi/runtime.py:31-63 and
    indexing.py:175-192.  ``k_override`` (runtime kmeans.k1..k4) replaces the
    Python k so that n_centroids matches the cells the index actually has
    (layer_pipeline.cpp:1131-1163 uses the runtime k1/k2 when given)."""
    n_tokens = max(int(list_capacity), 1)
    total_clusters = max(int(n_tokens / 16), 1)
    if k_override:
        ncells = 1
        for k in k_override:
            ncells *= int(k)
        n_centroids = ncells + 1
    elif subspace_parts == 0:
        n_centroids = max(int(round(n_tokens / 16.0)), 1) + 1
    elif subspace_parts == 4:
        total_f = max(n_tokens / 16.0, 1.0)
        k = max(int(round(total_f ** 0.25)), 2)
        n_centroids = k ** 4 + 1
    else:
        k = max(int(math.sqrt(total_clusters)), 32)
        n_centroids = k * k + 1
    nprobe = max(round((n_centroids - 1) * retrieval_budget), 1)
    nprobe = min(nprobe, n_centroids - 1)
    max_tokens = max(int(retrieval_budget * list_capacity), 1)
    retrieval_pages = max((max_tokens + page_size - 1) // page_size, 1) if max_tokens > 0 else 0
    buffer_pages = max(int(max(buffer_cluster_num, retrieval_pages)), 1)
    return dict(n_centroids=n_centroids, padding_cluster_id=n_centroids - 1, nprobe=int(nprobe),
                max_tokens=int(max_tokens), buffer_pages=int(buffer_pages), page_size=page_size)


def adaptive_k(seq_len: int, target_cluster_size: int = 16, subspace_parts: int = 2) -> List[int]:
    """layer_pipeline.cpp:177-228 (calculate_adaptive_k_values)."""
    if seq_len <= 0:
        return [1] if subspace_parts == 0 else [1] * (4 if subspace_parts == 4 else 2)
    if target_cluster_size <= 0:
        target_cluster_size = 16
    total = float(seq_len) / target_cluster_size
    if subspace_parts == 0:
        return [max(int(_round_half_away(total)), 1)]
    if subspace_parts == 4:
        k = max(int(_round_half_away(total ** 0.25)), 2)
        return [k, k, k, k]
    k = max(int(math.sqrt(total)), 32)
    return [k, k]


def _round_half_away(x: float) -> float:
    """std::round semantics (half away from zero)."""
    return math.floor(x + 0.5) if x >= 0 else math.ceil(x - 0.5)


def reference_threads_per_phase(cores: int, kv_heads: int, parts: int) -> int:
    """Threads each (head, subspace) Lloyd run uses in the reference:
    cache.py:113-124 (min_threads_per_phase, worker_threads) feeding
    kmeans_core.cpp:433-443 with one k-means job active."""
    tasks = kv_heads * max(parts, 1)
    min_threads = max(1, cores // max(1, tasks))
    available = max(1, cores)
    min_threads = max(1, min(min_threads, available))
    max_concurrent = max(1, min(tasks, available // min_threads))
    tpp = max(1, available // max_concurrent)
    return max(tpp, min_threads)


# -------------------------------------------------------------- k-means ----

def estep(data: np.ndarray, cent: np.ndarray, nthreads: int = 0):
    """kmeans_core.cpp:222-242. Returns (labels int32[n], mind f32[n], inertia)."""
    data = np.ascontiguousarray(data, np.float32)
    cent = np.ascontiguousarray(cent, np.float32)
    n, dim = data.shape
    k = cent.shape[0]
    labels = np.empty(n, np.int32)
    mind = np.empty(n, np.float32)
    inertia = lib().orc_estep(_p(data, _f32p), n, dim, _p(cent, _f32p), k, _p(labels, _i32p),
                              _p(mind, _f32p), nthreads or os.cpu_count() or 1)
    return labels, mind, float(inertia)


def mstep(data: np.ndarray, labels: np.ndarray, k: int, iteration: int, nthreads: int = 1) -> np.ndarray:
    """kmeans_core.cpp:265-312 with `nthreads` static OpenMP chunks."""
    data = np.ascontiguousarray(data, np.float32)
    labels = np.ascontiguousarray(labels, np.int32)
    n, dim = data.shape
    cent = np.empty((k, dim), np.float32)
    lib().orc_mstep(_p(data, _f32p), n, dim, _p(labels, _i32p), k, nthreads, iteration, _p(cent, _f32p))
    return cent


def reseed_draws(iteration: int, n: int, count: int) -> np.ndarray:
    out = np.empty(count, np.int32)
    lib().orc_reseed_draws(iteration, n, count, _p(out, _i32p))
    return out


def mt_outputs(seed: int, n: int, bits: int = 64) -> np.ndarray:
    """The first n outputs of std::mt19937 (bits=32) or std::mt19937_64 seeded
    with `seed` (the engines of kmeans_core.cpp:150 and :293)."""
    if bits == 64:
        out = np.empty(n, np.uint64)
        lib().orc_mt64_outputs(seed, n, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)))
    else:
        out = np.empty(n, np.uint32)
        lib().orc_mt32_outputs(seed, n, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return out


def kmeanspp_init(data: np.ndarray, k: int, seed: int) -> np.ndarray:
    """kmeans_core.cpp:138-186."""
    data = np.ascontiguousarray(data, np.float32)
    n, dim = data.shape
    cent = np.empty((k, dim), np.float32)
    lib().orc_kmeanspp_init(_p(data, _f32p), n, dim, k, seed, _p(cent, _f32p))
    return cent


def lloyd(data: np.ndarray, cent0: np.ndarray, max_iters: int, tol: float = 5e-4,
          early_stop_min_iter: Optional[int] = None, early_stop_rel_tol: float = 5e-4,
          mstep_threads: int = 1, estep_threads: int = 0):
    """kmeans_core.cpp:190-314; early stop disabled by default
    (early_stop_min_iter = max_iters + 1).  Returns (centroids, labels, iters)."""
    data = np.ascontiguousarray(data, np.float32)
    cent = np.array(cent0, np.float32, copy=True, order="C")
    n, dim = data.shape
    labels = np.empty(n, np.int32)
    es = max_iters + 1 if early_stop_min_iter is None else early_stop_min_iter
    iters = lib().orc_lloyd_p(_p(data, _f32p), n, dim, cent.shape[0], _p(cent, _f32p), _p(labels, _i32p),
                              max(1, max_iters), max(tol, 0.0), max(1, es), max(early_stop_rel_tol, 0.0),
                              mstep_threads, estep_threads or os.cpu_count() or 1)
    return cent, labels, iters


def subspace_slices(dim: int, parts: int):
    """extract_subvectors / extract_subvectors_4 (kmeans_core.cpp:316-348)."""
    p = max(parts, 1)
    w = dim // p
    return [slice(i * w, (i + 1) * w) for i in range(p)]


# seeds per subspace phase: kmeans_core.cpp:459,469 (2-way), 702-735 (4-way)
PHASE_SEEDS = (42, 43, 44, 45)


def kmeans_head(keys_f32: np.ndarray, ks: Sequence[int], max_iters: int, init: str = "first",
                mstep_threads: int = 1, tol: float = 5e-4, early_stop_min_iter: Optional[int] = None,
                early_stop_rel_tol: float = 5e-4, init_centroids: Optional[List[np.ndarray]] = None):
    """One KV head of KmeansExecutor::execute (kmeans_core.cpp:384-501):
    independent Lloyd runs per subspace.  init: 'first' (first k rows of the
    subspace, the BASELINE configs), 'kmeans++' (the reference default) or
    'given' (init_centroids)."""
    parts = len(ks)
    sl = subspace_slices(keys_f32.shape[1], parts if parts > 1 else 0)
    labels, cents, iters = [], [], []
    for p in range(parts):
        sub = np.ascontiguousarray(keys_f32[:, sl[p]])
        if init == "first":
            c0 = sub[: ks[p]].copy()
        elif init == "kmeans++":
            c0 = kmeanspp_init(sub, ks[p], PHASE_SEEDS[p])
        else:
            c0 = np.array(init_centroids[p], np.float32)
        c, lab, it = lloyd(sub, c0, max_iters, tol, early_stop_min_iter, early_stop_rel_tol, mstep_threads)
        labels.append(lab)
        cents.append(c)
        iters.append(it)
    return labels, cents, iters


# ---------------------------------------------------------- reorganize ----

def compact_reorg(labels: Sequence[np.ndarray], ks: Sequence[int]):
    """reorganize_core.cpp:18-231 + 234-311 (token permutation only)."""
    T = labels[0].shape[0]
    P = len(labels)
    lab = np.ascontiguousarray(np.stack(labels).astype(np.int32))
    ksa = np.asarray(ks, np.int32)
    ncells = int(np.prod(ksa.astype(np.int64)))
    cap = min(ncells, T)
    final = np.empty(T, np.int32)
    gids = np.empty(cap, np.int32)
    offsets = np.empty(cap + 1, np.int32)
    perm = np.empty(T, np.int32)
    n_active = lib().orc_compact_reorg(_p(lab, _i32p), _p(ksa, _i32p), P, T, _p(final, _i32p),
                                       _p(gids, _i32p), _p(offsets, _i32p), _p(perm, _i32p))
    return dict(n_active=int(n_active), final_labels=final, gids=gids[:n_active].copy(),
                offsets=offsets[: n_active + 1].copy(), perm=perm)


def merged_centroids(cents: Sequence[np.ndarray], gids: np.ndarray, ks: Sequence[int]) -> np.ndarray:
    """Concatenate the subspace centroids of each occupied cell in compact
    order (reorganize_core.cpp:66-82 and 149-173)."""
    parts = len(cents)
    idx = []
    rem = gids.astype(np.int64)
    for p in reversed(range(parts)):
        idx.append(rem % ks[p])
        rem = rem // ks[p]
    idx = idx[::-1]
    return np.concatenate([cents[p][idx[p]] for p in range(parts)], axis=1).astype(np.float32)


def build_index(keys_bits: np.ndarray, values_bits: np.ndarray, ks: Sequence[int], max_iters: int,
                init: str = "first", mstep_threads: int = 1, **lloyd_kw):
    """Whole-layer index build (layer_pipeline.cpp merge_all_chunks 1077-1401):
    keys/values bf16 bits [H, T, D].  Returns per-head dicts."""
    H, T, D = keys_bits.shape
    heads = []
    for h in range(H):
        kf = bf16_to_f32(keys_bits[h])
        labels, cents, iters = kmeans_head(kf, ks, max_iters, init, mstep_threads, **lloyd_kw)
        reorg = compact_reorg(labels, ks)
        merged = merged_centroids(cents, reorg["gids"], ks)
        perm = reorg["perm"]
        heads.append(dict(labels=labels, centroids=cents, iters=iters, merged=merged,
                          list_keys=keys_bits[h][perm], list_values=values_bits[h][perm], **reorg))
    return heads


def pad_metadata(heads: List[dict], n_centroids: int, D: int):
    """pipeline_bindings.cpp:206-276 + indexing.py:108-174: pad per-head CSR
    metadata to n_centroids slots.  Returns (sizes i32[H,n_c],
    offsets i32[H,n_c+1], centroids f32[H,n_c,D], mask bool[H,n_c])."""
    H = len(heads)
    sizes = np.zeros((H, n_centroids), np.int32)
    offsets = np.zeros((H, n_centroids + 1), np.int32)
    cent = np.zeros((H, n_centroids, D), np.float32)
    mask = np.ones((H, n_centroids), bool)
    for h, hd in enumerate(heads):
        n = hd["n_active"]
        if n > n_centroids:
            raise ValueError(f"head {h}: {n} occupied cells exceed n_centroids {n_centroids}")
        off = hd["offsets"]
        sizes[h, :n] = np.diff(off)
        offsets[h, : n + 1] = off
        offsets[h, n + 1:] = off[-1]
        cent[h, :n] = hd["merged"]
        mask[h, :n] = sizes[h, :n] == 0
    return sizes, offsets, cent, mask


# -------------------------------------------------------------- decode ----

def scores(q_bits: np.ndarray, cent: np.ndarray) -> np.ndarray:
    """compute_impl.cu:62-103; q_bits [H,G,D] bf16 bits, cent [H,N,D] f32."""
    q_bits = np.ascontiguousarray(q_bits, np.uint16)
    cent = np.ascontiguousarray(cent, np.float32)
    H, G, D = q_bits.shape
    N = cent.shape[1]
    out = np.empty((H, N), np.float32)
    lib().orc_scores(_p(q_bits, _u16p), _p(cent, _f32p), H, G, N, D, _p(out, _f32p))
    return out


def select(sc: np.ndarray, sizes: np.ndarray, mask: np.ndarray, nprobe: int, max_tokens: int,
           buffer_pages: int, page_size: int = 8):
    """retrieval.py:295-303,357 + wave_buffer_cpu_hotcold.cpp:303-371.
    Returns (sel i32[H,nprobe] compact ids in rank order, -1 padded; m i32[H];
    tokens i64[H])."""
    sc = np.ascontiguousarray(sc, np.float32)
    sizes = np.ascontiguousarray(sizes, np.int32)
    mk = np.ascontiguousarray(mask, np.uint8)
    H, N = sc.shape
    sel = np.empty((H, nprobe), np.int32)
    m = np.empty(H, np.int32)
    tok = np.empty(H, np.int64)
    lib().orc_select(_p(sc, _f32p), _p(sizes, _i32p), _p(mk, _u8p), H, N, nprobe, max_tokens, buffer_pages,
                     page_size, _p(sel, _i32p), _p(m, _i32p), _p(tok, _i64p))
    return sel, m, tok


def select_tiles(sc: np.ndarray, sizes: np.ndarray, mask: np.ndarray, nprobe: int, max_tokens: int,
                 buffer_pages: int, page_size: int = 8):
    """Tile mode (IMI_MAX_TILES != 0): retrieval.py:295-303 (topk + token
    budget) then _build_cluster_tiles (retrieval.py:30-112).  Tiles group the
    kept cells in rank order so that each tile holds at most buffer_pages
    pages; a cell whose own page count exceeds buffer_pages can join no tile,
    so its head stops there.  Every tile is attended and the tiles are merged
    by LSE (retrieval.py:452-527), i.e. the attended set is the union of the
    tiles.  Returns (sel, m, tokens) like select()."""
    big = np.iinfo(np.int32).max // 2
    sel, m, _ = select(sc, sizes, mask, nprobe, max_tokens, big, page_size)
    H = sel.shape[0]
    tok = np.zeros(H, np.int64)
    for h in range(H):
        cut = int(m[h])
        for r in range(int(m[h])):
            pages = (int(sizes[h, sel[h, r]]) + page_size - 1) // page_size
            if pages > buffer_pages:
                cut = r
                break
        sel[h, cut:] = -1
        m[h] = cut
        tok[h] = int(sum(int(sizes[h, c]) for c in sel[h, :cut]))
    return sel, m, tok


def build_cluster_tiles(sel: np.ndarray, counts: np.ndarray, sizes: np.ndarray, buffer_pages: int, page_size: int,
                        padding_id: int) -> List[np.ndarray]:
    """_build_cluster_tiles (retrieval.py:30-112) over every head at once.
    sel [H, nprobe]: cells in rank order, the first counts[h] of them
    selected (the rest ignored); sizes [H, n]: cell sizes.  Each tile is an
    [H, max_take] array: head h's next run of cells that fits buffer_pages
    pages, padded with padding_id where the head took fewer than the head
    that took most.  A head stops at a cell whose own pages exceed
    buffer_pages (it can join no tile)."""
    sel = np.asarray(sel, np.int64)
    H, nprobe = sel.shape
    counts = np.asarray(counts, np.int64)
    pos = np.arange(nprobe)[None, :]
    ids = np.where(pos < counts[:, None], sel, padding_id)
    szs = np.zeros((H, nprobe), np.int64)
    for h in range(H):
        live = ids[h] != padding_id
        szs[h, live] = sizes[h, ids[h, live]]
    pages = np.where(szs > 0, np.maximum((szs + page_size - 1) // page_size, 1), 0)
    prefix = np.cumsum(pages, axis=1)
    offs = np.zeros(H, np.int64)
    tiles = []
    while np.any(offs < counts):
        valid = offs < counts
        start = np.where(offs > 0, prefix[np.arange(H), np.maximum(offs - 1, 0)], 0)
        rel = prefix - start[:, None]
        cand = (pos >= offs[:, None]) & (pos < counts[:, None]) & (rel <= buffer_pages)
        take = cand.sum(axis=1)
        force = valid & (take == 0)
        cur_pages = pages[np.arange(H), np.minimum(offs, nprobe - 1)]
        take = np.where(force & (cur_pages <= buffer_pages), 1, take)
        take = np.minimum(take, counts - offs)
        mt = int(take.max())
        if mt <= 0:
            break
        tile = np.full((H, mt), padding_id, np.int64)
        for h in range(H):
            tile[h, : take[h]] = ids[h, offs[h]: offs[h] + take[h]]
        tiles.append(tile)
        offs = offs + take
    return tiles


def selected_rows(sel: np.ndarray, m: np.ndarray, offsets: np.ndarray) -> List[np.ndarray]:
    """CSR rows of the selected cells per head, in rank order."""
    out = []
    for h in range(sel.shape[0]):
        rows = [np.arange(offsets[h, c], offsets[h, c + 1], dtype=np.int64) for c in sel[h, : m[h]]]
        out.append(np.concatenate(rows) if rows else np.zeros(0, np.int64))
    return out


def attention(q_bits: np.ndarray, k_bits: np.ndarray, v_bits: np.ndarray, rows: List[np.ndarray],
              scale: Optional[float] = None) -> np.ndarray:
    """fp64 softmax attention over the listed rows of each KV head.
    q_bits [H,G,D]; k_bits/v_bits [H,L,D]; returns f64 [H,G,D]."""
    q_bits = np.ascontiguousarray(q_bits, np.uint16)
    k_bits = np.ascontiguousarray(k_bits, np.uint16)
    v_bits = np.ascontiguousarray(v_bits, np.uint16)
    H, G, D = q_bits.shape
    L = k_bits.shape[1]
    width = max(1, max(len(r) for r in rows))
    rl = np.zeros((H, width), np.int64)
    nr = np.zeros(H, np.int32)
    for h, r in enumerate(rows):
        rl[h, : len(r)] = r
        nr[h] = len(r)
    out = np.empty((H, G, D), np.float64)
    sc = 1.0 / math.sqrt(D) if scale is None else scale
    lib().orc_attention(_p(q_bits, _u16p), _p(k_bits, _u16p), _p(v_bits, _u16p), L * D, _p(rl, _i64p),
                        _p(nr, _i32p), width, H, G, D, sc, _p(out, _f64p))
    return out


def decode_step(q_bits: np.ndarray, heads: List[dict], steady_k: np.ndarray, steady_v: np.ndarray,
                static_len: int, n_centroids: int, nprobe: int, max_tokens: int, buffer_pages: int,
                page_size: int = 8, tile_mode: bool = False):
    """One sparse_attention call (retrieval.py:320-602): scores -> mask ->
    select (select_tiles in tile mode) -> execution buffer [static rows |
    selected rows]
    (copy_kernel.cuh:220-335) -> attention.  steady_k/v: bf16 bits
    [H, static_cap, D].  Returns (out f64 [H,G,D], sel, m, rows per head as
    indices into the per-head CSR list)."""
    H, G, D = q_bits.shape
    sizes, offsets, cent, mask = pad_metadata(heads, n_centroids, D)
    sc = scores(q_bits, cent)
    pick = select_tiles if tile_mode else select
    sel, m, tok = pick(sc, sizes, mask, nprobe, max_tokens, buffer_pages, page_size)
    rows = selected_rows(sel, m, offsets)
    width = max(static_len + len(r) for r in rows)
    ek = np.zeros((H, max(width, 1), D), np.uint16)
    ev = np.zeros_like(ek)
    nr = []
    for h, hd in enumerate(heads):
        n = static_len + len(rows[h])
        ek[h, :static_len] = steady_k[h, :static_len]
        ev[h, :static_len] = steady_v[h, :static_len]
        ek[h, static_len:n] = hd["list_keys"][rows[h]]
        ev[h, static_len:n] = hd["list_values"][rows[h]]
        nr.append(np.arange(n, dtype=np.int64))
    out = attention(q_bits, ek, ev, nr)
    return out, sel, m, rows


_base = None


def base_lib():
    """libcpudecode.so: the CPU baseline's own vectorized build."""
    global _base
    if _base is None:
        build()
        L = ctypes.CDLL(str(_BASE_PATH))
        L.cpu_decode_step_f32.restype = None
        L.cpu_decode_step_f32.argtypes = [_u16p, _f32p, _i32p, _u8p, _i32p, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_int, _u16p, _u16p, ctypes.c_int64, _u16p, _u16p,
                                          ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.c_int, ctypes.c_float, _f32p, _i32p]
        _base = L
    return _base


class DecodeBaselineF32:
    """CPU BASELINE, not a checker: the decode step of every KV head in fp32
    (cpu_decode_step_f32, AVX2 + OpenMP: each K/V row read once for the G
    queries of its KV head, row chunks over the threads), on metadata padded
    once (pad_metadata).  list_keys / values: [H, L, D] bf16 bits;
    steady_k / v: [H, S, D] bf16 bits."""

    def __init__(self, heads: List[dict], list_keys: np.ndarray, list_values: np.ndarray, steady_k: np.ndarray,
                 steady_v: np.ndarray, n_centroids: int, D: int = 128):
        self.sizes, self.offsets, self.cent, mask = pad_metadata(heads, n_centroids, D)
        self.cent_t = np.ascontiguousarray(self.cent.transpose(0, 2, 1))   # [H, D, N]
        self.mask = np.ascontiguousarray(mask, np.uint8)
        self.lk = np.ascontiguousarray(list_keys, np.uint16)
        self.lv = np.ascontiguousarray(list_values, np.uint16)
        self.sk = np.ascontiguousarray(steady_k, np.uint16)
        self.sv = np.ascontiguousarray(steady_v, np.uint16)
        self.H, self.N, self.D = self.cent.shape

    def step(self, q_bits: np.ndarray, static_len: int, nprobe: int, max_tokens: int, buffer_pages: int,
             page_size: int = 8, scale: Optional[float] = None):
        q_bits = np.ascontiguousarray(q_bits, np.uint16)
        G = q_bits.shape[1]
        out = np.empty((self.H, G, self.D), np.float32)
        m = np.empty(self.H, np.int32)
        sc = 1.0 / math.sqrt(self.D) if scale is None else scale
        if G > 16 or self.D % 8 or self.D > 256:
            raise ValueError("the CPU baseline takes G <= 16 and D a multiple of 8 up to 256")
        base_lib().cpu_decode_step_f32(_p(q_bits, _u16p), _p(self.cent_t, _f32p), _p(self.sizes, _i32p),
                                  _p(self.mask, _u8p), _p(self.offsets, _i32p), self.H, G, self.N, self.D,
                                  _p(self.lk, _u16p), _p(self.lv, _u16p), self.lk.shape[1], _p(self.sk, _u16p),
                                  _p(self.sv, _u16p), self.sk.shape[1], static_len, nprobe, max_tokens,
                                  buffer_pages, page_size, sc, _p(out, _f32p), _p(m, _i32p))
        return out, m


# ------------------------------------------------ online index update ----

def update_assign(keys_f32: np.ndarray, rows: np.ndarray) -> np.ndarray:
    """async_update.py:125-127: arg-max over rows of keys @ rows^T, first
    index on ties, dot products as sequential fp32 FMA chains (the
    reference's bmm order is the BLAS library's).  keys [B, D], rows [N, D]."""
    keys_f32 = np.ascontiguousarray(keys_f32, np.float32)
    rows = np.ascontiguousarray(rows, np.float32)
    B, D = keys_f32.shape
    out = np.empty(B, np.int32)
    lib().orc_update_assign(_p(keys_f32, _f32p), B, _p(rows, _f32p), rows.shape[0], D, _p(out, _i32p))
    return out


class OnlineUpdateOracle:
    """The reference's async centroid update and delta ring, per KV head
    (async_update.py:77-162; state from runtime.py:115-166), with the update
    applied at the next step (the reference applies it once its side stream
    has finished, async_update.py:7-19).

    shadow [H, n_c, D] f32: merged centroids by compact id, zero past
    n_active; sizes [H, n_c]: the cell sizes (centroid_counts)."""

    def __init__(self, shadow: np.ndarray, sizes: np.ndarray, padding_id: int, threshold: int, ring_cap: int):
        H, n_c, D = shadow.shape
        self.shadow = np.array(shadow, np.float32)
        self.cc = np.array(sizes, np.int64)
        self.dc = np.zeros((H, n_c), np.int64)
        self.ds = np.zeros((H, n_c, D), np.float32)
        self.padding_id, self.threshold, self.cap = int(padding_id), int(threshold), int(ring_cap)
        self.ring_id = np.full((H, ring_cap), padding_id, np.int64)
        self.ring_row = np.zeros((H, ring_cap), np.int64)
        self.pos = np.zeros(H, np.int64)
        self.n = np.zeros(H, np.int64)
        self.last_ids: Optional[np.ndarray] = None
        self.replaced: List[List[int]] = [[] for _ in range(H)]   # compact rows, first-replacement order

    def assign(self, keys_bits: np.ndarray, rows: Sequence[int]) -> np.ndarray:
        """async_update.py:119-134 (scatter_add in batch order) and 146-161
        (ring write).  keys_bits [H, B, D] bf16 bits; rows: steady rows."""
        H, B, _ = keys_bits.shape
        ids = np.empty((H, B), np.int64)
        for h in range(H):
            x = bf16_to_f32(keys_bits[h])
            ids[h] = update_assign(x, self.shadow[h])
            for s_ in range(B):
                c = ids[h, s_]
                self.ds[h, c] = self.ds[h, c] + x[s_]
                self.dc[h, c] += 1
            for s_ in range(B):
                p = (self.pos[h] + s_) % self.cap
                self.ring_id[h, p] = ids[h, s_]
                self.ring_row[h, p] = rows[s_]
            self.pos[h] = (self.pos[h] + B) % self.cap
            self.n[h] = min(self.n[h] + B, self.cap)
        self.last_ids = ids
        return ids

    def refresh(self) -> None:
        """async_update.py:135-143 for the rows the last batch touched."""
        ids = self.last_ids
        if ids is None:
            return
        for h in range(ids.shape[0]):
            for c in dict.fromkeys(int(v) for v in ids[h]):
                if self.dc[h, c] < self.threshold:
                    continue
                total = self.cc[h, c] + self.dc[h, c]
                num = self.shadow[h, c] * np.float32(self.cc[h, c]) + self.ds[h, c]
                self.shadow[h, c] = num / np.float32(max(total, 1))
                self.cc[h, c] = total
                self.dc[h, c] = 0
                self.ds[h, c] = 0.0
                if c not in self.replaced[h]:
                    self.replaced[h].append(c)
        self.last_ids = None

    def delta_rows(self, h: int, kept: Sequence[int], nprobe: int, exec_rows: int, rows_sel: int) -> List[int]:
        """async_update.py:41-76 for one head: ring entries (index order, the
        first n valid) whose cluster is one of the kept compact ids (the cells
        passing nprobe and the token budget), or the padding id when fewer
        than nprobe pass; at most exec_rows - rows_sel of them."""
        ks = set(int(c) for c in kept)
        pad = len(ks) < nprobe
        out = [int(self.ring_row[h, p]) for p in range(int(self.n[h]))
               if int(self.ring_id[h, p]) in ks or (pad and int(self.ring_id[h, p]) == self.padding_id)]
        return out[: max(exec_rows - rows_sel, 0)]


    def delta_rows_tiles(self, h: int, tiles: Sequence[np.ndarray], exec_rows: int, sizes_h: np.ndarray) -> List[int]:
        """async_update.py:41-76 once per tile, as retrieval.py:480-509 calls
        it: for each tile (build_cluster_tiles, padded with the padding id)
        the ring entries (index order, the first n valid) whose cluster is in
        head h's row of the tile -- the padding id included when that row is
        padded -- at most exec_rows minus the rows of that row's cells.  An
        entry can be appended once per tile it matches."""
        out = []
        for tile in tiles:
            ids = set(int(c) for c in tile[h])
            rows_t = int(sum(int(sizes_h[c]) for c in tile[h] if int(c) != self.padding_id))
            got = [int(self.ring_row[h, p]) for p in range(int(self.n[h])) if int(self.ring_id[h, p]) in ids]
            out += got[: max(exec_rows - rows_t, 0)]
        return out


def decode_step_online(q_bits: np.ndarray, sizes: np.ndarray, offsets: np.ndarray, mask: np.ndarray,
                       list_keys: np.ndarray, list_values: np.ndarray, steady_k: np.ndarray, steady_v: np.ndarray,
                       static_len: int, upd: OnlineUpdateOracle, nprobe: int, max_tokens: int, buffer_pages: int,
                       exec_rows: int, page_size: int = 8, tile_mode: bool = False):
    """sparse_attention with the async update on (retrieval.py:320-447 with
    async_update.py:7-76): scores over the current centroids (the shadow),
    selection, execution buffer [static rows | selected rows | delta rows]
    and attention.  sizes/offsets/mask padded per head ([H, n_c(+1)]);
    list_keys/values [H, L, D] bf16 bits.  Returns (out f64 [H, G, D], sel,
    m, list rows per head, delta steady rows per head)."""
    H, G, D = q_bits.shape
    sc = scores(q_bits, upd.shadow)
    big = np.iinfo(np.int32).max // 2
    sel_t, m_t, _ = select(sc, sizes, mask, nprobe, max_tokens, big, page_size)
    if tile_mode:   # retrieval.py:452-527: every tile, its delta rows, LSE-merged
        sel, m, _ = select_tiles(sc, sizes, mask, nprobe, max_tokens, buffer_pages, page_size)
        rows = selected_rows(sel, m, offsets)
        tiles = build_cluster_tiles(sel_t, m_t, sizes, buffer_pages, page_size, upd.padding_id)
        drows = [upd.delta_rows_tiles(h, tiles, exec_rows, sizes[h]) for h in range(H)]
    else:
        sel, m, _ = select(sc, sizes, mask, nprobe, max_tokens, buffer_pages, page_size)
        rows = selected_rows(sel, m, offsets)
        drows = [upd.delta_rows(h, sel_t[h, : m_t[h]], nprobe, exec_rows, len(rows[h])) for h in range(H)]
    width = max(static_len + len(rows[h]) + len(drows[h]) for h in range(H))
    ek = np.zeros((H, max(width, 1), D), np.uint16)
    ev = np.zeros_like(ek)
    nr = []
    for h in range(H):
        a, b = static_len, static_len + len(rows[h])
        n = b + len(drows[h])
        ek[h, :a], ev[h, :a] = steady_k[h, :a], steady_v[h, :a]
        ek[h, a:b], ev[h, a:b] = list_keys[h][rows[h]], list_values[h][rows[h]]
        ek[h, b:n], ev[h, b:n] = steady_k[h][drows[h]], steady_v[h][drows[h]]
        nr.append(np.arange(n, dtype=np.int64))
    out = attention(q_bits, ek, ev, nr)
    return out, sel, m, rows, drows

