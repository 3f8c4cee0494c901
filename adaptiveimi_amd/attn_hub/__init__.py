"""Decode attention entry points (mirrors the reference's attn_hub)."""
