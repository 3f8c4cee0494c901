"""KV caches of the sparse-decode path (mirrors the reference's cache_hub)."""
