"""AdaptiveIMI cache (reference: cache_hub/adaptive_imi)."""
from .cache import adpimi_cache

__all__ = ["adpimi_cache"]
