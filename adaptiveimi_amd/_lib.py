"""ctypes binding of libimi_hip.so (declared in include/imi_hip.h).

The library is loaded after torch so both share torch's HIP runtime.  There is
no fallback: if the library is missing or fails to load, every entry point
raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(__file__).resolve().parent / "libimi_hip.so"

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class KmeansArgs(ctypes.Structure):
    _fields_ = [
        ("keys", _vp), ("head_stride", _i64), ("token_stride", _i64),
        ("kv_heads", _i32), ("n_tokens", _i32), ("dim", _i32), ("parts", _i32),
        ("k", _i32 * 4), ("max_iters", _i32), ("tol", _f32), ("early_stop_min_iter", _i32),
        ("early_stop_rel_tol", _f32), ("init_mode", _i32),
        ("centroids", _vp), ("labels", _vp), ("iters_run", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


class IndexArgs(ctypes.Structure):
    _fields_ = [
        ("keys", _vp), ("values", _vp), ("head_stride", _i64), ("token_stride", _i64),
        ("kv_heads", _i32), ("n_tokens", _i32), ("dim", _i32), ("parts", _i32),
        ("k", _i32 * 4), ("centroids", _vp), ("labels", _vp),
        ("cell_count", _vp), ("cell_offset", _vp), ("perm", _vp),
        ("list_keys", _vp), ("list_values", _vp), ("list_rows", _i64),
        ("n_centroids", _i32), ("n_active", _vp), ("compact_gid", _vp), ("compact_size", _vp),
        ("compact_offset", _vp), ("compact_centroids", _vp), ("compact_mask", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


class SelectArgs(ctypes.Structure):
    _fields_ = [
        ("query", _vp), ("centroids", _vp), ("cell_count", _vp), ("cell_offset", _vp),
        ("kv_heads", _i32), ("groups", _i32), ("dim", _i32), ("parts", _i32),
        ("k", _i32 * 4), ("nprobe", _i32), ("max_tokens", _i32), ("buffer_pages", _i32), ("page_size", _i32),
        ("sel_cell", _vp), ("sel_offset", _vp), ("sel_count", _vp), ("sel_prefix", _vp),
        ("n_selected", _vp), ("n_rows", _vp), ("sel_cap", _i32),
        ("compact_gid", _vp), ("compact_size", _vp), ("compact_offset", _vp), ("n_active", _vp),
        ("compact_cap", _i32), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("head_max_tokens", _vp), ("head_buffer_pages", _vp), ("tile_mode", _i32),
        ("shadow", _vp), ("shadow_rows", _i32), ("upd_slot", _vp), ("upd_row", _vp), ("upd_n", _vp),
        ("ring_cell", _vp), ("ring_row", _vp), ("ring_n", _vp), ("ring_cap", _i32), ("exec_rows", _i32),
        ("delta_rows", _vp), ("n_delta", _vp),
    ]


class AttentionArgs(ctypes.Structure):
    _fields_ = [
        ("query", _vp), ("steady_keys", _vp), ("steady_values", _vp), ("steady_stride", _i64),
        ("static_len", _i32), ("list_keys", _vp), ("list_values", _vp), ("list_rows", _i64),
        ("sel_offset", _vp), ("sel_count", _vp), ("sel_prefix", _vp), ("n_selected", _vp), ("n_rows", _vp),
        ("sel_cap", _i32), ("max_rows", _i32), ("kv_heads", _i32), ("groups", _i32), ("dim", _i32),
        ("scale", _f32), ("out", _vp), ("out_lse", _vp),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("delta_rows", _vp), ("n_delta", _vp), ("delta_cap", _i32), ("head_rows_bound", _vp),
        ("rows_hint", _i32),
    ]


class UpdateArgs(ctypes.Structure):
    _fields_ = [
        ("steady_keys", _vp), ("steady_stride", _i64), ("row0", _i32), ("count", _i32),
        ("kv_heads", _i32), ("dim", _i32), ("shadow", _vp), ("n_rows", _i32), ("padding_id", _i32),
        ("n_active", _vp), ("compact_gid", _vp), ("centroid_counts", _vp), ("delta_counts", _vp),
        ("delta_sums", _vp), ("threshold", _i32), ("ring_id", _vp), ("ring_cell", _vp), ("ring_row", _vp),
        ("ring_pos", _vp), ("ring_n", _vp), ("ring_cap", _i32), ("upd_slot", _vp), ("upd_row", _vp),
        ("upd_n", _vp), ("n_index", _i32), ("index_by_gid", _i32),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [("sel", SelectArgs), ("attn", AttentionArgs), ("phases", _i32)]


class HostcacheGatherArgs(ctypes.Structure):
    _fields_ = [("host_keys", _vp), ("host_values", _vp), ("list_rows", _i64),
                ("cache_keys", _vp), ("cache_values", _vp), ("cache_rows", _i64),
                ("exec_keys", _vp), ("exec_values", _vp), ("exec_rows", _i64),
                ("groups", _i32), ("max_blocks", _i32), ("block_size", _i32),
                ("hit_ids", _vp), ("hit_sizes", _vp), ("hit_prefix", _vp), ("hit_nums", _vp),
                ("miss_ids", _vp), ("miss_sizes", _vp), ("miss_prefix", _vp), ("miss_nums", _vp),
                ("sel_offset", _vp), ("sel_count", _vp), ("sel_prefix", _vp), ("n_selected", _vp),
                ("n_rows", _vp), ("sel_cap", _i32)]


EXPORTS = {
    "imi_last_error": (ctypes.c_char_p, []),
    "imi_version": (ctypes.c_int, []),
    "imi_kmeans_workspace_size": (ctypes.c_int, [ctypes.POINTER(KmeansArgs), ctypes.POINTER(ctypes.c_size_t)]),
    "imi_kmeans_execute": (ctypes.c_int, [ctypes.POINTER(KmeansArgs), _vp]),
    "imi_kmeans_assign": (ctypes.c_int, [_vp, _i64, _i64, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _vp]),
    "imi_index_workspace_size": (ctypes.c_int, [ctypes.POINTER(IndexArgs), ctypes.POINTER(ctypes.c_size_t)]),
    "imi_build_index": (ctypes.c_int, [ctypes.POINTER(IndexArgs), _vp]),
    "imi_fused_query_group_similarities": (ctypes.c_int, [_vp, _vp, _vp, _i64, _vp, _i32, _i32, _i32, _i32, _vp]),
    "imi_select_workspace_size": (ctypes.c_int, [ctypes.POINTER(SelectArgs), ctypes.POINTER(ctypes.c_size_t)]),
    "imi_select": (ctypes.c_int, [ctypes.POINTER(SelectArgs), _vp]),
    "imi_attention_workspace_size": (ctypes.c_int, [ctypes.POINTER(AttentionArgs), ctypes.POINTER(ctypes.c_size_t)]),
    "imi_sparse_attention": (ctypes.c_int, [ctypes.POINTER(AttentionArgs), _vp]),
    "imi_decode_workspace_size": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), ctypes.POINTER(ctypes.c_size_t)]),
    "imi_decode_step": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _vp]),
    "imi_decode_step_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), _vp]),
    "imi_update_workspace_size": (ctypes.c_int, [ctypes.POINTER(UpdateArgs), ctypes.POINTER(ctypes.c_size_t)]),
    "imi_update_assign": (ctypes.c_int, [ctypes.POINTER(UpdateArgs), _vp]),
    "imi_update_refresh": (ctypes.c_int, [ctypes.POINTER(UpdateArgs), _vp]),
    "imi_hostcache_create": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32, _i32, ctypes.c_double,
                                            ctypes.POINTER(_vp)]),
    "imi_hostcache_destroy": (None, [_vp]),
    "imi_hostcache_set_metadata": (ctypes.c_int, [_vp, _vp, _vp]),
    "imi_hostcache_access": (ctypes.c_int, [_vp, _vp, _i32] + [_vp] * 8),
    "imi_hostcache_update": (ctypes.c_int, [_vp, _vp, _vp, _vp, _vp]),
    "imi_hostcache_stats": (ctypes.c_int, [_vp, ctypes.POINTER(_i64), ctypes.POINTER(_i64)]),
    "imi_hostcache_gather": (ctypes.c_int, [ctypes.POINTER(HostcacheGatherArgs), _vp]),
    "imi_hostcache_admit": (ctypes.c_int, [_vp, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _vp,
                                           _vp]),
    "imi_host_device_pointer": (ctypes.c_int, [_vp, ctypes.POINTER(_vp)]),
}

_lib = None


class IMIError(RuntimeError):
    """Error reported by libimi_hip (status code + imi_last_error text)."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m adaptiveimi_amd.build` "
                "(there is no CPU fallback for the sparse-decode path)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in EXPORTS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().imi_last_error().decode(errors="replace")
        raise IMIError(f"{what} failed (status {rc}): {msg}")
