"""MI355X-native (gfx950) AdaptiveIMI retrieval-guided sparse-decode path.

Drop-in for the reference's cache_hub/adaptive_imi cache and
attn_hub/sparse_imi.py attention call; the index build, selection and
gather + attention run as hand-written HIP kernels in libimi_hip.so
(C ABI: include/imi_hip.h).
"""
__version__ = "0.1.0"
