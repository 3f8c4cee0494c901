"""Decode sizing rules of the reference cache.

cache_hub/adaptive_imi/runtime.py:31-63 (prepare_cache) and
indexing.py:175-192 (_ensure_metadata_buffers): n_centroids, padding id,
nprobe, token budget and page budget.  One deliberate difference: when the
k-means runs with explicit per-subspace k (runtime kmeans.k1/k2, which the
reference's LayerPipeline honours at layer_pipeline.cpp:1147-1156),
n_centroids is derived from those k so the padded metadata has room for every
cell; the reference derives it from list_capacity only and would fail to pad
(indexing.py:130) whenever the two disagree.
"""
from __future__ import annotations

import math
from typing import Dict, Optional, Sequence


def tokens_to_pages(tokens: int, page_size: int = 8) -> int:
    """retrieval.py:16-19."""
    if tokens <= 0:
        return 0
    return max((int(tokens) + page_size - 1) // page_size, 1)


def n_centroids_for(list_capacity: int, subspace_parts: int = 2,
                    k_override: Optional[Sequence[int]] = None) -> int:
    n_tokens = max(int(list_capacity), 1)
    total_clusters = max(int(n_tokens / 16), 1)
    if k_override:
        cells = 1
        for k in k_override:
            cells *= int(k)
        return cells + 1
    if subspace_parts == 0:
        return max(int(round(n_tokens / 16.0)), 1) + 1
    if subspace_parts == 4:
        k = max(int(round(max(n_tokens / 16.0, 1.0) ** 0.25)), 2)
        return k ** 4 + 1
    k = max(int(math.sqrt(total_clusters)), 32)
    return k * k + 1


def decode_sizing(list_capacity: int, retrieval_budget: float, subspace_parts: int = 2,
                  buffer_cluster_num: int = 32, page_size: int = 8,
                  k_override: Optional[Sequence[int]] = None) -> Dict[str, int]:
    n_c = n_centroids_for(list_capacity, subspace_parts, k_override)
    nprobe = max(round((n_c - 1) * retrieval_budget), 1)   # Python round (half to even)
    nprobe = min(nprobe, n_c - 1)
    max_tokens = max(int(retrieval_budget * list_capacity), 1)
    buffer_pages = max(int(max(buffer_cluster_num, tokens_to_pages(max_tokens, page_size))), 1)
    return dict(n_centroids=n_c, padding_cluster_id=n_c - 1, nprobe=int(nprobe), max_tokens=int(max_tokens),
                buffer_pages=int(buffer_pages), page_size=page_size)


def adaptive_k(seq_len: int, target_cluster_size: int = 16, subspace_parts: int = 2):
    """layer_pipeline.cpp:177-228 (calculate_adaptive_k_values), the k the
    index build uses when no runtime k is configured."""
    if seq_len <= 0:
        return [1] if subspace_parts == 0 else [1] * (4 if subspace_parts == 4 else 2)
    if target_cluster_size <= 0:
        target_cluster_size = 16
    total = float(seq_len) / target_cluster_size
    half_away = lambda x: math.floor(x + 0.5)  # std::round for x >= 0
    if subspace_parts == 0:
        return [max(int(half_away(total)), 1)]
    if subspace_parts == 4:
        return [max(int(half_away(total ** 0.25)), 2)] * 4
    return [max(int(math.sqrt(total)), 32)] * 2
