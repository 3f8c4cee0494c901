"""Drop-in ``adpimi_cache`` for the AdaptiveIMI sparse-decode path on MI355X.

Mirrors the public surface of the reference cache
(cache_hub/adaptive_imi/cache.py:44-455, indexing.py:316-611,
runtime.py:9-402, retrieval.py:320-602) that the model code calls:
constructor arguments, ``prefill_update_kv_cache``, ``sync``,
``prepare_cache``, ``decode_update_kv_cache``, ``attn_func`` (=
``sparse_attention`` / ``dense_attention``), ``capture_cuda_graph``,
``cleanup``, ``can_reuse_for_next_sequence`` / ``reset_for_next_sequence``,
``get_index_stats`` and the attributes callers read (``static_pattern_total``,
``layer_num``, ``context``, ``valid_start_list``).

What differs inside: the index is built on the GPU at prefill (k-means +
stable CSR reorganisation, ``imi_kmeans_execute`` / ``imi_build_index``) and
the list stays in HBM; a decode step is one ``imi_decode_step`` call (scores,
selection with the page rule, in-place gather and attention) with no host
round trip.  By default nothing lives on the host, so the reference's
thread pool and prefetch warm-up have no counterpart (their constructor
arguments are accepted and recorded).  runtime_config["host_tier"] =
{"enabled": True} keeps each layer's lists in pinned host memory instead,
as the reference always does (indexing.py:98-107): each layer's build
writes its lists to a device buffer that an asynchronous copy moves to the
pinned lists and that is freed at once, so the device never holds more than
one layer's lists.  Decode then runs with a GPU block cache of
round(n_centroids * cache_ratio) clusters of pages_per_cluster pages per
head and the reference's hot / cold policy (IMI_HOTCOLD_HOT_RATIO, default
0.3): ops.HostTierPlan, for lists that do not fit in HBM (2-way, 4-way IMI
or IVF, async_update included; not with tile mode).  A host-tier step
synchronises with the host (its selected cells go to the cache manager), so
it cannot be captured in a graph.

subspace_parts = 0 builds an IVF index (kmeans_core.cpp:503-595: one
k-means over the 128 dims per KV head, k = runtime kmeans.k1 or
round(T / 16), at most 4096) whose clusters are the cells of the same
selection and attention path, async_update and host_tier included.

Online index maintenance (runtime_config["async_update"], async_update.py)
runs on the device as well: every `batch` decode keys of a layer are
assigned to clusters and enter the delta ring (imi_update_assign, at
decode_update_kv_cache), the centroids whose delta count reached
`threshold` are replaced before that layer's next selection
(imi_update_refresh), and the selection scores replaced centroids over their
new values and appends the matching ring tokens to the attended rows.  The
reference applies a finished side-stream update at the next step; here the
update is stream-ordered and always lands at the next step.
"""
from __future__ import annotations

import math
import os
from typing import Dict, List, Optional, Sequence

import torch

from ... import ops
from ...sizing import adaptive_k, decode_sizing

_KMEANS_DEFAULTS = {  # LayerPipelineRuntimeConfig defaults (layer_pipeline.hpp:148-153)
    "max_iters": 25,
    "tol": 5e-4,
    "early_stop_min_iter": 5,
    "early_stop_rel_tol": 5e-4,
    "target_cluster_size": 16,
    "init": "kmeans++",   # kmeans_plusplus_init_inplace, as the reference; "first" = first k rows
}


class adpimi_cache:  # noqa: N801  (reference class name)
    def __init__(
        self,
        valid_start,
        layer_num: int,
        batch_size: int,
        max_length: int,
        num_key_value_heads: int,
        num_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        layer_mapping: dict,
        max_new_length: int,
        input_length: Optional[int],
        static_pattern_start: int,
        static_pattern_end: int,
        core: int,
        pages_per_cluster: int,
        retrieval_budget: float,
        cache_ratio: float,
        buffer_cluster_num: int,
        prefill_bsz: int,
        num_gpus: int,
        model_size: int,
        subspace_parts: int = 4,
        runtime_config: Optional[Dict[str, Dict[str, object]]] = None,
    ) -> None:
        # KV_Cache fields (cache_hub/base.py)
        self.layer_num = layer_num
        self.batch_size = batch_size
        self.max_length = max_length
        self.kv_head = num_key_value_heads
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.layer_mapping = layer_mapping
        self.prefill_bsz = min(prefill_bsz, batch_size)
        self.num_gpus = num_gpus
        self.model_size = model_size
        self.context = 0
        if batch_size != 1:
            raise ValueError("IMI cache currently supports batch_size=1.")
        if head_dim != 128:
            raise ValueError("the gfx950 kernels implement head_dim 128")
        if num_heads % num_key_value_heads != 0:
            raise ValueError("num_heads must be a multiple of num_key_value_heads")
        if subspace_parts not in (0, 2, 4):
            raise ValueError("subspace_parts must be 0, 2 or 4")

        self.device_list = sorted(set(self.layer_mapping.values()),
                                  key=lambda x: (x.split(":")[0], int(x.split(":")[1]) if ":" in x else 0))
        self.valid_start_list = valid_start
        self.static_pattern_start = static_pattern_start
        self.static_pattern_end = static_pattern_end
        self.static_pattern_total = static_pattern_start + static_pattern_end
        self.group_size = num_heads // num_key_value_heads
        self.batch_groups = batch_size * num_key_value_heads
        self.page_size = 8
        self.pages_per_cluster = pages_per_cluster
        self.retrieval_budget = retrieval_budget
        self.cache_ratio = cache_ratio
        self.buffer_cluster_num = buffer_cluster_num
        self.subspace_parts = subspace_parts
        self.core = core

        runtime_config = runtime_config or {}
        kmeans_cfg = dict(_KMEANS_DEFAULTS)
        kmeans_cfg.update(runtime_config.get("kmeans") or {})
        self.runtime_config = {
            "kmeans": kmeans_cfg,
            "prefetch": dict(runtime_config.get("prefetch") or {}),
            "async_update": dict(runtime_config.get("async_update") or {}),
            "pipeline": dict(runtime_config.get("pipeline") or {}),
            "host_tier": dict(runtime_config.get("host_tier") or {}),
        }
        self.host_tier = bool(self.runtime_config["host_tier"].get("enabled", False))
        # The reference builds each layer's index on host worker threads while
        # the next layers prefill (LayerPipeline); here the build runs on a
        # side HIP stream and the first use of the index waits for it on the
        # device (no host synchronisation).
        self.async_build = bool(self.runtime_config["pipeline"].get("async_build", True))
        self._build_stream: Optional[torch.cuda.Stream] = None
        self._build_events: List[Optional[torch.cuda.Event]] = [None] * layer_num
        # online index maintenance (cache.py:305-311 defaults)
        acfg = self.runtime_config["async_update"]
        self.async_update_enabled = bool(acfg.get("enabled", False))
        self.async_update_batch = max(int(acfg.get("batch", 16)), 1)
        self.async_update_threshold = max(int(acfg.get("threshold", 16)), 1)
        self.async_update_delta_tokens = max(int(acfg.get("delta_tokens", 512)), 1)
        if self.async_update_enabled and self.async_update_batch > min(64, self.async_update_delta_tokens):
            raise ValueError("async_update: batch must be at most 64 and at most delta_tokens")
        if self.async_update_enabled and self.async_update_delta_tokens > 1024:
            raise ValueError("async_update: delta_tokens must be at most 1024")
        self._updates: List[Optional[ops.OnlineUpdate]] = [None] * layer_num
        self._upd_count = [0] * layer_num
        self._upd_pending: List[Optional[int]] = [None] * layer_num   # decode step of an unapplied refresh
        self._decode_step = 0
        self.execution_stride = 0

        # sizes (cache.py:133-153)
        self.input_length = int(input_length) if input_length is not None else self.max_length - max_new_length
        self.actual_gen_len = max_new_length - 1
        self.capacity_input_length = int(self.max_length - max_new_length)
        self.capacity_actual_gen_len = self.actual_gen_len
        if self.input_length <= 0:
            raise ValueError(f"input length({self.input_length}) should be larger than 0")
        if self.capacity_input_length <= 0:
            raise ValueError(f"capacity input length({self.capacity_input_length}) should be larger than 0")
        self.list_capacity = max(self.capacity_input_length - self.static_pattern_total, 0)
        self.list_stride = max(self.input_length - self.static_pattern_total, 0)
        self.build_index_when_prefilling = self.list_capacity > 0
        if self.build_index_when_prefilling:
            self.static_capacity = self.static_pattern_total + self.capacity_actual_gen_len
            self.static_stride = self.static_pattern_total + self.actual_gen_len
        else:
            self.static_capacity = self.capacity_input_length + self.capacity_actual_gen_len
            self.static_stride = self.input_length + self.actual_gen_len

        self.attn_func = self.dense_attention
        self.n_centroids = 0
        self.padding_cluster_id = -1
        self.nprobe = 0
        self.max_retrieval_tokens = 0
        self.buffer_size = 0
        self.cache_prepared = False
        self.layer_ready = [False] * layer_num
        self.layer_started = [False] * layer_num
        self._expected_middle_len: List[Optional[int]] = [None] * layer_num

        self.steady_zone_keys = []
        self.steady_zone_values = []
        for ldx in range(layer_num):
            dev = self.layer_mapping[str(ldx)]
            shape = (batch_size, num_key_value_heads, self.static_capacity, head_dim)
            self.steady_zone_keys.append(torch.zeros(shape, dtype=dtype, device=dev))
            self.steady_zone_values.append(torch.zeros(shape, dtype=dtype, device=dev))

        # per-layer index state (device tensors)
        self.layer_ks: List[Optional[List[int]]] = [None] * layer_num
        self.centroids: List[Optional[torch.Tensor]] = [None] * layer_num      # [H, P, kmax, Dp]
        self.cell_count: List[Optional[torch.Tensor]] = [None] * layer_num     # [H, ncells]
        self.cell_offset: List[Optional[torch.Tensor]] = [None] * layer_num    # [H, ncells + 1]
        self.token_perm: List[Optional[torch.Tensor]] = [None] * layer_num     # [H, T] list row -> token
        # 4-way only: the occupied cells in cell order (n_active, gid, size, offset)
        self.compact_cells: List[Optional[Dict[str, torch.Tensor]]] = [None] * layer_num
        # online update only: the compact metadata with merged centroids
        self.compact_meta: List[Optional[Dict[str, torch.Tensor]]] = [None] * layer_num
        self.list_keys: List[Optional[torch.Tensor]] = [None] * layer_num      # [1, H, list_capacity, D]
        self.list_values: List[Optional[torch.Tensor]] = [None] * layer_num
        # host tier: each layer's lists in pinned host memory ([H, rows, D] keys, values)
        self.host_lists: List[Optional[tuple]] = [None] * layer_num
        self._plans: List[Optional[ops.DecodePlan]] = [None] * layer_num
        # the reference's execution-buffer views; the gather here reads rows in place
        self.execution_buffer_keys_dict: Dict[str, torch.Tensor] = {}
        self.execution_buffer_values_dict: Dict[str, torch.Tensor] = {}
        self.valid_lengths_dict: Dict[str, torch.Tensor] = {}

    # ------------------------------------------------------------ prefill --
    def _k_names(self) -> Sequence[str]:
        """Runtime k knobs by index type; IVF takes its cluster count from
        k1 (layer_pipeline.cpp:1142-1148)."""
        return {0: ("k1",), 2: ("k1", "k2")}.get(self.subspace_parts, ("k1", "k2", "k3", "k4"))

    def _layer_ks(self, n_tokens: int) -> List[int]:
        cfg = self.runtime_config["kmeans"]
        ks = [int(cfg.get(n, 0) or 0) for n in self._k_names()]
        if all(k > 0 for k in ks):   # layer_pipeline.cpp:1137-1156
            return ks
        return adaptive_k(n_tokens, int(cfg.get("target_cluster_size", 16)), self.subspace_parts)

    def _decode_budget(self, ks: Sequence[int]) -> Dict[str, int]:
        """runtime.py:31-63 with this cache's list capacity and budget."""
        explicit = all(int(self.runtime_config["kmeans"].get(n, 0) or 0) > 0 for n in self._k_names())
        return decode_sizing(self.list_capacity, self.retrieval_budget, self.subspace_parts, self.buffer_cluster_num,
                             self.page_size, k_override=ks if explicit else None)

    def _check_decode_limits(self, ks: Sequence[int]) -> None:
        """Fail before the index build, not at the first decode step, when the
        selection kernels cannot rank this shape (e.g. too many cells to
        rank for the 4-way path)."""
        sz = self._decode_budget(ks)
        tiles = int(os.getenv("IMI_MAX_TILES", "0") or 0) != 0
        if tiles and self.host_tier:
            raise NotImplementedError("host_tier runs without tile mode (IMI_MAX_TILES)")
        bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"], self.page_size, tile_mode=tiles)
        ops.check_decode_limits(self.batch_groups, self.group_size, ks, bud, online=self.async_update_enabled)

    def _build_layer_index(self, layer_idx: int, middle_k: torch.Tensor, middle_v: torch.Tensor) -> None:
        """k-means + reorganisation of one layer's middle keys ([H, T, D]
        strided views of the prefill tensors; nothing is copied first)."""
        cfg = self.runtime_config["kmeans"]
        H, T, D = middle_k.shape
        ks = self._layer_ks(T)
        if T < max(ks) and cfg["init"] == "first":
            raise ValueError(f"IMI layer {layer_idx}: {T} middle tokens < k = {max(ks)} (first-k initialisation)")
        self._check_decode_limits(ks)
        km_kw = dict(tol=float(cfg["tol"]), early_stop_min_iter=int(cfg["early_stop_min_iter"]),
                     early_stop_rel_tol=float(cfg["early_stop_rel_tol"]), init=str(cfg["init"]))
        sample = int(cfg.get("sample_keys", 0) or 0)
        if 0 < sample < T:   # 1M-token build: Lloyd on a strided sample, then every key assigned
            cent, labels, _ = ops.kmeans_sampled(middle_k, ks, int(cfg["max_iters"]), sample, **km_kw)
        else:
            cent, labels, _ = ops.kmeans(middle_k, ks, int(cfg["max_iters"]), **km_kw)
        dev = middle_k.device
        rows = max(self.list_capacity, T)
        lk = torch.empty((1, H, rows, D), dtype=middle_k.dtype, device=dev)
        lv = torch.empty_like(lk)
        four_way = self.subspace_parts == 4
        ncells = 1
        for k in ks:
            ncells *= int(k)
        # 4-way scoring walks the occupied cells only (at most min(T, k^4) of
        # them); the online update keeps merged centroids by compact id (the
        # reference's padded n_centroids = k^2 + 1 slots for 2-way)
        online = self.async_update_enabled
        idx = ops.build_index(middle_k, middle_v, cent, labels, ks, list_keys=lk[0], list_values=lv[0],
                              compact=four_way or online, merged=online,
                              n_centroids=min(T, ncells) + 1 if four_way else ncells + 1)
        if self.host_tier:
            # the lists go to pinned host memory on this (the build's) stream;
            # the device buffer is freed now, and the allocator hands its block
            # to the next build on the same stream only after this copy
            hk = torch.empty((H, rows, D), dtype=middle_k.dtype, pin_memory=True)
            hv = torch.empty_like(hk, pin_memory=True)
            hk.copy_(lk[0], non_blocking=True)
            hv.copy_(lv[0], non_blocking=True)
            self.host_lists[layer_idx] = (hk, hv)
            lk = lv = None
        self.compact_cells[layer_idx] = (
            {n: idx[n] for n in ("n_active", "compact_gid", "compact_size", "compact_offset")} if four_way else None)
        self.compact_meta[layer_idx] = (
            {n: idx[n] for n in ("n_active", "compact_gid", "compact_size", "compact_centroids")} if online else None)
        self._updates[layer_idx] = None
        self.layer_ks[layer_idx] = ks
        self.centroids[layer_idx] = cent
        self.cell_count[layer_idx] = idx["cell_count"]
        self.cell_offset[layer_idx] = idx["cell_offset"]
        self.token_perm[layer_idx] = idx["perm"]
        self.list_keys[layer_idx] = lk
        self.list_values[layer_idx] = lv
        self._plans[layer_idx] = None
        self.layer_ready[layer_idx] = True

    def prefill_update_kv_cache(self, query_states, key_states, value_states, layer_idx, start_bdx):
        """indexing.py:548-611.  key_states / value_states: [1, S, H, D]."""
        bsz, seq_len, _, _ = key_states.shape
        if bsz != 1:
            raise ValueError("IMI cache currently supports batch_size=1 for prefilling.")
        valid_start = self.valid_start_list[start_bdx]
        end_bdx = start_bdx + bsz
        if self.build_index_when_prefilling:
            middle_start = valid_start + self.static_pattern_start
            middle_end = seq_len - self.static_pattern_end
            middle_len = max(middle_end - middle_start, 0)
            if middle_len <= 0:
                raise ValueError("IMI cache requires a non-empty middle segment.")
            self._expected_middle_len[layer_idx] = int(middle_len)
            if not self.layer_started[layer_idx]:
                mk = key_states[0, middle_start:middle_end].transpose(0, 1)     # [H, T, D] view
                mv = value_states[0, middle_start:middle_end].transpose(0, 1)
                if self.async_build and key_states.is_cuda:
                    main = torch.cuda.current_stream(key_states.device)
                    if self._build_stream is None:
                        self._build_stream = torch.cuda.Stream(key_states.device)   # default priority
                    side = self._build_stream
                    side.wait_stream(main)
                    with torch.cuda.stream(side):
                        self._build_layer_index(layer_idx, mk, mv)
                    # the prefill tensors stay allocated until the build has read them
                    key_states.record_stream(side)
                    value_states.record_stream(side)
                    ev = torch.cuda.Event()
                    ev.record(side)
                    self._build_events[layer_idx] = ev
                else:
                    self._build_layer_index(layer_idx, mk, mv)
                self.layer_started[layer_idx] = True
            ss, se = self.static_pattern_start, self.static_pattern_end
            self.steady_zone_keys[layer_idx][start_bdx:end_bdx, :, :ss, :] = (
                key_states[:, valid_start:valid_start + ss, :, :].transpose(1, 2))
            self.steady_zone_values[layer_idx][start_bdx:end_bdx, :, :ss, :] = (
                value_states[:, valid_start:valid_start + ss, :, :].transpose(1, 2))
            self.steady_zone_keys[layer_idx][start_bdx:end_bdx, :, ss:ss + se, :] = (
                key_states[:, seq_len - se:seq_len, :, :].transpose(1, 2))
            self.steady_zone_values[layer_idx][start_bdx:end_bdx, :, ss:ss + se, :] = (
                value_states[:, seq_len - se:seq_len, :, :].transpose(1, 2))
        else:
            self.steady_zone_keys[layer_idx][start_bdx:end_bdx, :, :seq_len, :].copy_(key_states.transpose(1, 2))
            self.steady_zone_values[layer_idx][start_bdx:end_bdx, :, :seq_len, :].copy_(value_states.transpose(1, 2))

        if layer_idx == self.layer_num - 1 and start_bdx + bsz == self.batch_size:
            self.context += seq_len
            if self.build_index_when_prefilling:
                self.attn_func = self.sparse_attention
            else:
                self.static_pattern_total = seq_len
        return key_states[:, valid_start:, :, :], value_states[:, valid_start:, :, :]

    def sync(self, layer_idx, start_bdx):
        """indexing.py:612.  Returns at once, as the reference's does once the
        chunk copy is done: the build keeps running on the side stream, and
        every use of the index (prepare_cache, the decode plans, the index
        statistics) first makes the caller's stream wait for it."""
        return None

    def _await_index(self, layer_idx: int) -> None:
        """Order the caller's stream after layer_idx's side-stream build and
        tie the layer's tensors to that stream for the allocator."""
        ev = self._build_events[layer_idx]
        if ev is None:
            return
        main = torch.cuda.current_stream(self.centroids[layer_idx].device)
        main.wait_event(ev)
        for t in (self.centroids[layer_idx], self.cell_count[layer_idx], self.cell_offset[layer_idx],
                  self.token_perm[layer_idx], self.list_keys[layer_idx], self.list_values[layer_idx]):
            if t is not None:
                t.record_stream(main)
        for t in list((self.compact_cells[layer_idx] or {}).values()) + list((self.compact_meta[layer_idx] or {}).values()):
            t.record_stream(main)
        self._build_events[layer_idx] = None

    # ------------------------------------------------------------- decode --
    def prepare_cache(self, skip_prefetch: bool = False):
        """runtime.py:11-63: decode budgets, then one decode plan per layer."""
        if not self.build_index_when_prefilling:
            return
        for layer in range(self.layer_num):
            self._await_index(layer)
        if self.cache_prepared:
            return
        ks = next((k for k in self.layer_ks if k is not None), None)
        if ks is None:
            raise RuntimeError("prepare_cache: no layer index has been built")
        sz = self._decode_budget(ks)
        self._check_decode_limits(ks)
        self.n_centroids = sz["n_centroids"]
        self.padding_cluster_id = sz["padding_cluster_id"]
        self.nprobe = sz["nprobe"]
        self.max_retrieval_tokens = sz["max_tokens"]
        self.budget_tokens = self.max_retrieval_tokens
        self.buffer_size = sz["buffer_pages"]
        self.buffer_budget_pages = self.buffer_size
        self.execution_stride = self.buffer_size * self.page_size + self.static_capacity   # runtime.py:62
        self.cache_prepared = True

    def _update_state(self, layer_idx: int) -> Optional[ops.OnlineUpdate]:
        """runtime.py:106-166: the layer's update state, made on first use."""
        if not self.async_update_enabled or self.compact_meta[layer_idx] is None:
            return None
        upd = self._updates[layer_idx]
        if upd is None:
            if not self.cache_prepared:
                self.prepare_cache()
            self._await_index(layer_idx)
            meta = self.compact_meta[layer_idx]
            four_way = self.subspace_parts == 4
            ncells = int(self.cell_count[layer_idx].shape[1])
            upd = ops.OnlineUpdate(meta["compact_centroids"], meta["compact_size"], meta["compact_gid"],
                                   meta["n_active"], self.padding_cluster_id, self.async_update_threshold,
                                   self.async_update_delta_tokens,
                                   n_index=meta["compact_gid"].shape[1] if four_way else ncells,
                                   index_by_gid=not four_way)
            self._updates[layer_idx] = upd
            self._plans[layer_idx] = None
        return upd

    def _plan(self, layer_idx: int) -> ops.DecodePlan:
        upd = self._update_state(layer_idx)   # (re)builds the plan when the state is new
        plan = self._plans[layer_idx]
        if plan is None:
            if not self.cache_prepared:
                self.prepare_cache()
            self._await_index(layer_idx)
            # IMI_MAX_TILES != 0 selects the reference's tile mode (retrieval.py:373-382)
            tiles = int(os.getenv("IMI_MAX_TILES", "0") or 0) != 0
            bud = ops.Budget(self.nprobe, self.max_retrieval_tokens, self.buffer_size, self.page_size,
                             tile_mode=tiles)
            if self.host_tier:
                plan = self._host_plan(layer_idx, bud, upd)
                self._plans[layer_idx] = plan
                return plan
            plan = ops.DecodePlan(self.centroids[layer_idx], self.cell_count[layer_idx], self.cell_offset[layer_idx],
                                  self.layer_ks[layer_idx], bud, self.list_keys[layer_idx][0],
                                  self.list_values[layer_idx][0], self.steady_zone_keys[layer_idx][0],
                                  self.steady_zone_values[layer_idx][0], self.group_size,
                                  compact=self.compact_cells[layer_idx], update=upd)
            self._plans[layer_idx] = plan
        return plan

    def _host_plan(self, layer_idx: int, bud: "ops.Budget", upd) -> "ops.HostTierPlan":
        """Decode over the layer's pinned host lists; the device holds the
        block cache and the execution buffer (retrieval.py:200-290)."""
        if bud.tile_mode:
            raise NotImplementedError("host_tier runs without tile mode (IMI_MAX_TILES)")
        env = os.getenv("IMI_HOTCOLD_HOT_RATIO", "")
        try:
            ratio = float(env) if env else 0.0   # wave_buffer_cpu_hotcold.cpp:75-95
        except ValueError:
            ratio = 0.0
        pages = ops.host_cache_pages(self.n_centroids, self.nprobe, self.pages_per_cluster, self.cache_ratio)
        hk, hv = self.host_lists[layer_idx]
        return ops.HostTierPlan(self.centroids[layer_idx], self.cell_count[layer_idx], self.cell_offset[layer_idx],
                                self.layer_ks[layer_idx], bud, hk, hv, self.steady_zone_keys[layer_idx][0],
                                self.steady_zone_values[layer_idx][0], self.group_size, cache_pages=pages,
                                hot_ratio=ratio, compact=self.compact_cells[layer_idx], update=upd)

    def ensure_layer_ready(self, layer_idx: int) -> None:
        if not self.layer_ready[layer_idx]:
            raise RuntimeError(f"IMI index for layer {layer_idx} has not been built")

    def sparse_attention(self, queries, layer_idx, static_len):
        """retrieval.py:320-602 (tile mode off): scores, selection with the
        token and page budgets, gather and GQA attention in one call."""
        self.ensure_layer_ready(layer_idx)
        plan = self._plan(layer_idx)
        pending = self._upd_pending[layer_idx]
        if pending is not None and pending < self._decode_step:   # async_update.py:7-19, one step later
            self._updates[layer_idx].refresh(self.async_update_batch)
            self._upd_pending[layer_idx] = None
        q = queries.reshape(self.batch_groups, self.group_size, self.head_dim)
        if not q.is_contiguous():
            q = q.contiguous()
        out = torch.empty((self.batch_size, 1, self.num_heads, self.head_dim), dtype=queries.dtype,
                          device=queries.device)
        if isinstance(plan, ops.HostTierPlan):
            plan.step(q, out, int(static_len), exec_rows=self.execution_stride - int(static_len))
        else:
            plan.run(q, out, int(static_len), exec_rows=self.execution_stride - int(static_len))
        return out

    def dense_attention(self, queries, layer_idx, static_len):
        """runtime.py:393-402: attention over the steady zone only."""
        q = queries.reshape(self.batch_groups, self.group_size, self.head_dim)
        out = ops.dense_attention(q.contiguous(), self.steady_zone_keys[layer_idx][0],
                                  self.steady_zone_values[layer_idx][0], int(static_len))
        return out.view(self.batch_size, 1, self.num_heads, self.head_dim)

    def decode_update_kv_cache(self, key_states, value_states, layer_idx):
        """runtime.py:378-392.  key_states / value_states: [1, 1, H, D]."""
        if layer_idx == 0:
            self._decode_step += 1
        row = self.static_pattern_total
        self.steady_zone_keys[layer_idx][:, :, row, :] = key_states[:, 0, :, :]
        self.steady_zone_values[layer_idx][:, :, row, :] = value_states[:, 0, :, :]
        upd = self._update_state(layer_idx) if self.attn_func == self.sparse_attention else None
        if upd is not None:   # async_update.py:77-162
            self._upd_count[layer_idx] += 1
            if self._upd_count[layer_idx] == self.async_update_batch:
                if self._upd_pending[layer_idx] is not None:   # the previous batch's refresh comes first
                    upd.refresh(self.async_update_batch)
                n = self.async_update_batch
                upd.assign(self.steady_zone_keys[layer_idx][0], row - n + 1, n)
                self._upd_pending[layer_idx] = self._decode_step
                self._upd_count[layer_idx] = 0
        if layer_idx == self.layer_num - 1:
            self.context += 1
            self.static_pattern_total += 1
        return None, None

    def capture_cuda_graph(self):
        """runtime.py:9 (a no-op there too).  HBM-resident decode steps are
        graph-capturable; host-tier steps are not (each one hands its
        selected cells to the host cache manager)."""
        return None

    # ----------------------------------------------------------- lifecycle --
    def get_index_stats(self) -> Dict[str, object]:
        """indexing.py:316-350."""
        for layer in range(self.layer_num):
            self._await_index(layer)
        ideal_per_head = max(float(self.list_capacity) / 16.0, 0.0)
        total_heads = int(self.layer_num * self.batch_groups)
        ideal_total = ideal_per_head * float(total_heads)
        non_empty = 0
        ready = 0
        for cnt in self.cell_count:
            if cnt is None:
                continue
            ready += 1
            non_empty += int((cnt > 0).sum().item())
        return {
            "n_centroids": int(self.n_centroids),
            "ready_layers": int(ready),
            "total_heads": total_heads,
            "ideal_clusters_per_head": float(ideal_per_head),
            "ideal_clusters_total": float(ideal_total),
            "non_empty_clusters_total": int(non_empty),
            "non_empty_ratio": float(non_empty) / float(ideal_total) if ideal_total > 0 else 0.0,
            # indexing.py:333-334: padded merged centroids (n_centroids x head_dim fp32 per KV head) per ready
            # layer, the metadata the reference keeps on the GPU; the decode kernels here read the
            # subspace centroids instead (subspace_centroid_bytes_gpu)
            "total_centroid_bytes_gpu": int(ready * self.batch_groups * self.n_centroids * self.head_dim * 4),
            "subspace_centroid_bytes_gpu": int(sum(c.numel() * 4 for c in self.centroids if c is not None)),
        }

    def can_reuse_for_next_sequence(self, valid_start, max_new_length: int, input_length: int) -> bool:
        """cache.py:380-395."""
        new_list_stride = max(int(input_length) - self.static_pattern_total, 0)
        if new_list_stride > self.list_capacity:
            return False
        new_gen = int(max_new_length) - 1
        if self.build_index_when_prefilling:
            new_static_stride = self.static_pattern_total + new_gen
        else:
            new_static_stride = int(input_length) + new_gen
        if new_static_stride > self.static_capacity:
            return False
        return len(valid_start) == len(self.valid_start_list)

    def reset_for_next_sequence(self, valid_start, max_new_length: int, input_length: int) -> None:
        """cache.py:396-455 (the index state of every layer is dropped)."""
        if not self.can_reuse_for_next_sequence(valid_start, max_new_length, input_length):
            raise ValueError('AdaptiveIMI cache shape mismatch; cannot reuse across samples')
        self.valid_start_list = valid_start
        self.input_length = int(input_length)
        self.actual_gen_len = int(max_new_length) - 1
        self.list_stride = max(self.input_length - self.static_pattern_total, 0)
        if self.build_index_when_prefilling:
            self.static_stride = self.static_pattern_total + self.actual_gen_len
        else:
            self.static_stride = self.input_length + self.actual_gen_len
        self.context = 0
        self.attn_func = self.dense_attention
        self.layer_ready = [False] * self.layer_num
        self.layer_started = [False] * self.layer_num
        self._expected_middle_len = [None] * self.layer_num
        self._plans = [None] * self.layer_num
        self._updates = [None] * self.layer_num
        self._upd_count = [0] * self.layer_num
        self._upd_pending = [None] * self.layer_num
        for layer in range(self.layer_num):
            if self.centroids[layer] is not None:
                self._await_index(layer)

    def cleanup(self):
        """indexing.py:453: drop every device buffer the cache holds."""
        n = self.layer_num
        self._plans = [None] * n
        self._build_events = [None] * n
        self.centroids = [None] * n
        self.cell_count = [None] * n
        self.cell_offset = [None] * n
        self.token_perm = [None] * n
        self.compact_cells = [None] * n
        self.compact_meta = [None] * n
        self._updates = [None] * n
        self._upd_count = [0] * n
        self._upd_pending = [None] * n
        self.list_keys = [None] * n
        self.list_values = [None] * n
        self.host_lists = [None] * n
        self.layer_ks = [None] * n
        self.layer_ready = [False] * n

    def __del__(self):
        try:
            self.cleanup()
        except Exception:
            pass
