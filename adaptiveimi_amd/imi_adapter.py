"""``get_imi_kernels()`` of the reference adapter
(library/AdaptiveIMI/imi_adapter.py:88-111): the GPU scoring op the cache
calls, here backed by imi_fused_query_group_similarities."""
from __future__ import annotations

from types import SimpleNamespace

from . import ops


def get_imi_kernels():
    """Namespace with fused_query_group_similarities(query_grouped [H, G, D]
    bf16, centroids [H, N, D] fp32, out=None) -> [H, N] fp32
    (gpu_bindings.cpp:21-43)."""
    return SimpleNamespace(fused_query_group_similarities=ops.fused_query_group_similarities)
