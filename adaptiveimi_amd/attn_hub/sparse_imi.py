"""attn_hub/sparse_imi.py:1-10 of the reference, unchanged in behaviour."""


def imi_decode_attn(query_states, key_states, value_states, layer_idx, imi_cache):
    """query_states: (batch_size, 1, head_num, dim) device tensor.  Every layer
    but the last also attends the token appended to the steady zone in this
    step (the cache's static_pattern_total advances after the last layer)."""
    static_len = (
        imi_cache.static_pattern_total
        if layer_idx == imi_cache.layer_num - 1
        else imi_cache.static_pattern_total + 1
    )
    return imi_cache.attn_func(query_states.contiguous(), layer_idx, static_len)
