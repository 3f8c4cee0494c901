"""torch-facing wrappers over the C ABI (include/imi_hip.h).

All tensors must live on a HIP device; every call enqueues on the current
torch stream and returns without a host synchronisation.  Workspaces come
from the torch caching allocator and are zero-filled once on allocation (the
kernels leave them reusable).
"""
from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Dict, Optional, Sequence, Tuple

import torch

from . import _lib
from ._lib import AttentionArgs, DecodeArgs, IndexArgs, KmeansArgs, SelectArgs, UpdateArgs, check

_WS: Dict[Tuple[str, int], torch.Tensor] = {}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_device(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError("adaptiveimi_amd kernels need HIP device tensors (no CPU path)")
        dev = t.device if dev is None else dev
    return dev


def workspace(name: str, nbytes: int, device: torch.device) -> torch.Tensor:
    """Zero-filled byte buffer reused across calls (grown on demand), one per
    (name, device, stream): calls on one stream are ordered, calls on two
    streams (an index build on a side stream) never share a buffer."""
    key = (name, device.index if device.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(device).cuda_stream)
    buf = _WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device=device)
        _WS[key] = buf
    return buf


def _ks(ks: Sequence[int]):
    arr = (ctypes.c_int32 * 4)()
    for i, k in enumerate(ks):
        arr[i] = int(k)
    return arr


def _as_bits(t: torch.Tensor) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise TypeError(f"expected bfloat16 tensor, got {t.dtype}")
    return t


def _head_token_strides(x: torch.Tensor) -> Tuple[int, int]:
    if x.dim() != 3 or x.stride(2) != 1:
        raise ValueError("expected a [heads, tokens, dim] view with unit stride on dim")
    return x.stride(0), x.stride(1)


# ----------------------------------------------------------------- k-means --

_INIT_MODES = {"first": 0, "kmeans++": 2}


def kmeans(keys: torch.Tensor, ks: Sequence[int], max_iters: int, tol: float = 5e-4,
           early_stop_min_iter: Optional[int] = None, early_stop_rel_tol: float = 5e-4,
           init_centroids: Optional[torch.Tensor] = None, init: str = "first"):
    """Per-(head, subspace) Lloyd k-means (kmeans_core.cpp:384-501).
    init: 'first' (first k rows of each subspace), 'kmeans++' (the
    reference's kmeans_plusplus_init_inplace, seeds 42 + subspace) or, when
    init_centroids is given, those centroids.
    keys: bf16 [H, T, D] view.  Returns (centroids f32 [H, P, kmax, D/P],
    labels i32 [H, P, T], iters i32 [H, P])."""
    dev = _require_device(keys, init_centroids)
    _as_bits(keys)
    H, T, D = keys.shape
    P = len(ks)
    kmax = max(ks)
    hs, ts = _head_token_strides(keys)
    if init_centroids is not None:
        cent = init_centroids.to(device=dev, dtype=torch.float32).contiguous().clone()
        if cent.shape != (H, P, kmax, D // P):
            raise ValueError(f"init_centroids must be [{H}, {P}, {kmax}, {D // P}]")
    else:
        cent = torch.zeros((H, P, kmax, D // P), dtype=torch.float32, device=dev)
    labels = torch.empty((H, P, T), dtype=torch.int32, device=dev)
    iters = torch.zeros((H, P), dtype=torch.int32, device=dev)
    a = KmeansArgs(keys=keys.data_ptr(), head_stride=hs, token_stride=ts, kv_heads=H, n_tokens=T, dim=D,
                   parts=P, k=_ks(ks), max_iters=int(max_iters), tol=float(tol),
                   early_stop_min_iter=int(max_iters + 1 if early_stop_min_iter is None else early_stop_min_iter),
                   early_stop_rel_tol=float(early_stop_rel_tol),
                   init_mode=1 if init_centroids is not None else _INIT_MODES[init],
                   centroids=cent.data_ptr(), labels=labels.data_ptr(), iters_run=iters.data_ptr())
    need = ctypes.c_size_t()
    check(_lib.lib().imi_kmeans_workspace_size(ctypes.byref(a), ctypes.byref(need)), "imi_kmeans_workspace_size")
    ws = workspace("kmeans", need.value, dev)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    check(_lib.lib().imi_kmeans_execute(ctypes.byref(a), _stream(dev)), "imi_kmeans_execute")
    return cent, labels, iters


def kmeans_assign(keys: torch.Tensor, centroids: torch.Tensor, ks: Sequence[int], with_distance: bool = True):
    """One E-step with given centroids [H, P, kmax, D/P] (kmeans_core.cpp:222-242).
    Returns (labels i32 [H, P, T], min distance f32 [H, P, T]); the distance
    is None with ``with_distance=False`` (the labels alone are cheaper)."""
    dev = _require_device(keys, centroids)
    _as_bits(keys)
    H, T, D = keys.shape
    P = len(ks)
    hs, ts = _head_token_strides(keys)
    cent = centroids.to(torch.float32).contiguous()
    labels = torch.empty((H, P, T), dtype=torch.int32, device=dev)
    mind = torch.empty((H, P, T), dtype=torch.float32, device=dev) if with_distance else None
    check(_lib.lib().imi_kmeans_assign(keys.data_ptr(), hs, ts, H, T, D, P, ctypes.cast(_ks(ks), ctypes.c_void_p),
                                       cent.data_ptr(), labels.data_ptr(),
                                       mind.data_ptr() if with_distance else None, _stream(dev)),
          "imi_kmeans_assign")
    return labels, mind


def kmeans_sampled(keys: torch.Tensor, ks: Sequence[int], max_iters: int, sample_tokens: int, **kw):
    """K-means on an evenly strided sample of at most ``sample_tokens`` keys
    per head (a strided view: every ceil(T / sample_tokens)-th token, nothing
    copied), then one assignment pass of every key with the final centroids
    (the 1M-token build: 20 iterations on 65536 keys, then all keys).  The
    batch-1 reference has no sampling; each half is its own reference step
    (kmeans_core.cpp:190-314, then the E-step 222-242).  Returns
    (centroids f32 [H, P, kmax, D/P], labels i32 [H, P, T], iters i32 [H, P])."""
    if sample_tokens <= 0:
        raise ValueError("sample_tokens must be positive")
    H, T, D = keys.shape
    step = max(1, -(-T // int(sample_tokens)))
    cent, _, iters = kmeans(keys[:, ::step], ks, max_iters, **kw)
    labels, _ = kmeans_assign(keys, cent, ks, with_distance=False)
    return cent, labels, iters


# -------------------------------------------------------------- cell index --

def build_index(keys: torch.Tensor, values: torch.Tensor, centroids: torch.Tensor, labels: torch.Tensor,
                ks: Sequence[int], n_centroids: Optional[int] = None, list_rows: Optional[int] = None,
                list_keys: Optional[torch.Tensor] = None, list_values: Optional[torch.Tensor] = None,
                compact: bool = True, merged: bool = True) -> Dict[str, torch.Tensor]:
    """Cell order + CSR + K/V permutation (reorganize_core.cpp:18-394).
    compact: also list the occupied cells (gid, size, offset, n_active);
    merged: with them the padded merged centroids and mask (the metadata the
    reference uploads; not needed by the decode kernels)."""
    dev = _require_device(keys, values, centroids, labels)
    _as_bits(keys)
    _as_bits(values)
    H, T, D = keys.shape
    if values.shape != keys.shape or values.stride() != keys.stride():
        raise ValueError("keys and values must share shape and strides")
    hs, ts = _head_token_strides(keys)
    P = len(ks)
    ncells = 1
    for k in ks:
        ncells *= int(k)
    rows = int(list_rows or T)
    out: Dict[str, torch.Tensor] = {}
    out["cell_count"] = torch.empty((H, ncells), dtype=torch.int32, device=dev)
    out["cell_offset"] = torch.empty((H, ncells + 1), dtype=torch.int32, device=dev)
    out["perm"] = torch.empty((H, T), dtype=torch.int32, device=dev)
    out["list_keys"] = list_keys if list_keys is not None else torch.empty((H, rows, D), dtype=keys.dtype, device=dev)
    out["list_values"] = (list_values if list_values is not None
                          else torch.empty((H, rows, D), dtype=keys.dtype, device=dev))
    for name in ("list_keys", "list_values"):
        t = out[name]
        if t.shape[0] != H or t.shape[2] != D or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous [H, rows, D]")
    rows = out["list_keys"].shape[1]
    a = IndexArgs(keys=keys.data_ptr(), values=values.data_ptr(), head_stride=hs, token_stride=ts, kv_heads=H,
                  n_tokens=T, dim=D, parts=P, k=_ks(ks), centroids=centroids.data_ptr(), labels=labels.data_ptr(),
                  cell_count=out["cell_count"].data_ptr(), cell_offset=out["cell_offset"].data_ptr(),
                  perm=out["perm"].data_ptr(), list_keys=out["list_keys"].data_ptr(),
                  list_values=out["list_values"].data_ptr(), list_rows=rows)
    if compact:
        n_c = int(n_centroids if n_centroids is not None else ncells + 1)
        out["n_active"] = torch.empty((H,), dtype=torch.int32, device=dev)
        out["compact_gid"] = torch.empty((H, n_c), dtype=torch.int32, device=dev)
        out["compact_size"] = torch.empty((H, n_c), dtype=torch.int32, device=dev)
        out["compact_offset"] = torch.empty((H, n_c + 1), dtype=torch.int32, device=dev)
        a.n_centroids = n_c
        a.n_active = out["n_active"].data_ptr()
        a.compact_gid = out["compact_gid"].data_ptr()
        a.compact_size = out["compact_size"].data_ptr()
        a.compact_offset = out["compact_offset"].data_ptr()
        if merged:
            out["compact_centroids"] = torch.empty((H, n_c, D), dtype=torch.float32, device=dev)
            out["compact_mask"] = torch.empty((H, n_c), dtype=torch.bool, device=dev)
            a.compact_centroids = out["compact_centroids"].data_ptr()
            a.compact_mask = out["compact_mask"].data_ptr()
    need = ctypes.c_size_t()
    check(_lib.lib().imi_index_workspace_size(ctypes.byref(a), ctypes.byref(need)), "imi_index_workspace_size")
    ws = workspace("index", need.value, dev)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    check(_lib.lib().imi_build_index(ctypes.byref(a), _stream(dev)), "imi_build_index")
    return out


# ------------------------------------------------------------------ decode --

def fused_query_group_similarities(query_grouped: torch.Tensor, centroids: torch.Tensor,
                                   out: Optional[torch.Tensor] = None,
                                   mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gpu_bindings.cpp:21-43 signature; optional mask fuses retrieval.py:357."""
    dev = _require_device(query_grouped, centroids, out, mask)
    _as_bits(query_grouped)
    if query_grouped.dim() != 3 or centroids.dim() != 3:
        raise ValueError("query_grouped and centroids must be 3D tensors")
    H, G, D = query_grouped.shape
    if centroids.shape[0] != H or centroids.shape[2] != D:
        raise ValueError("kv_heads / head_dim mismatch between query_grouped and centroids")
    if centroids.dtype != torch.float32:
        raise TypeError("centroids must be float32")
    q = query_grouped.contiguous()
    c = centroids.contiguous()
    N = c.shape[1]
    if out is None:
        res = torch.empty((H, N), dtype=torch.float32, device=dev)
    else:
        if out.dtype != torch.float32 or out.dim() != 2 or out.shape[0] < H or out.shape[1] < N:
            raise ValueError("out tensor shape insufficient")
        res = out.narrow(0, 0, H).narrow(1, 0, N)
        if res.stride(1) != 1:
            raise ValueError("out must have unit stride on its last dim")
    m = None if mask is None else mask.to(torch.bool).contiguous()
    check(_lib.lib().imi_fused_query_group_similarities(q.data_ptr(), c.data_ptr(), res.data_ptr(), res.stride(0),
                                                        _ptr(m), H, G, N, D, _stream(dev)),
          "imi_fused_query_group_similarities")
    return res


@dataclass
class Budget:
    """Decode budgets (runtime.py:31-63).  head_max_tokens / head_buffer_pages
    give per-KV-head budgets for a ragged batch (the heads of several
    sequences in one launch); the scalars are then their maxima."""
    nprobe: int
    max_tokens: int
    buffer_pages: int
    page_size: int = 8
    head_max_tokens: Optional[Sequence[int]] = None
    head_buffer_pages: Optional[Sequence[int]] = None
    tile_mode: bool = False   # IMI_MAX_TILES != 0 (retrieval.py:30-112, 452-527)

    @property
    def sel_cap(self) -> int:
        if self.tile_mode:
            return max(1, self.nprobe)
        return max(1, min(self.nprobe, self.buffer_pages))

    @property
    def max_rows(self) -> int:
        if self.tile_mode:   # the token budget plus one cell of at most buffer_pages pages
            return self.max_tokens + self.buffer_pages * self.page_size
        return self.buffer_pages * self.page_size

    @classmethod
    def ragged(cls, per_sequence: Sequence["Budget"], heads_per_sequence: int) -> "Budget":
        """One launch over the KV heads of several sequences (sequence-major):
        same nprobe and page size, each sequence's own token and page budget."""
        if not per_sequence:
            raise ValueError("ragged budget needs at least one sequence")
        nprobe = {b.nprobe for b in per_sequence}
        page = {b.page_size for b in per_sequence}
        if len(nprobe) != 1 or len(page) != 1:
            raise ValueError("sequences of one ragged launch share nprobe and page_size")
        mt = [b.max_tokens for b in per_sequence for _ in range(heads_per_sequence)]
        bp = [b.buffer_pages for b in per_sequence for _ in range(heads_per_sequence)]
        tiles = {b.tile_mode for b in per_sequence}
        if len(tiles) != 1:
            raise ValueError("sequences of one ragged launch share tile_mode")
        return cls(nprobe.pop(), max(mt), max(bp), page.pop(), head_max_tokens=mt, head_buffer_pages=bp,
                   tile_mode=tiles.pop())


def _budget_fields(a, budget: Budget, H: int, dev) -> Tuple[torch.Tensor, ...]:
    """Per-head budget arrays of a ragged launch (device int32 [H]); the
    returned tensors must outlive the call."""
    keep = []
    for name, vals in (("head_max_tokens", budget.head_max_tokens), ("head_buffer_pages", budget.head_buffer_pages)):
        if vals is None:
            continue
        t = torch.as_tensor(list(vals), dtype=torch.int32).to(dev)
        if t.numel() != H:
            raise ValueError(f"{name} has {t.numel()} entries for {H} KV heads")
        setattr(a, name, t.data_ptr())
        keep.append(t)
    return tuple(keep)


def _compact_fields(a, compact: Optional[Dict[str, torch.Tensor]]) -> None:
    """Point SelectArgs at the occupied-cell arrays of build_index (4-way)."""
    if compact is None:
        return
    a.compact_gid = compact["compact_gid"].data_ptr()
    a.compact_size = compact["compact_size"].data_ptr()
    a.compact_offset = compact["compact_offset"].data_ptr()
    a.n_active = compact["n_active"].data_ptr()
    a.compact_cap = compact["compact_gid"].shape[1]


class OnlineUpdate:
    """One layer's online index maintenance: the reference's async centroid
    update and delta ring (async_update.py:77-162; state of runtime.py:106-166).

    shadow [H, n_rows, D] f32 starts as the merged centroids by compact id
    (rows past n_active zero), centroid_counts as the cell sizes.  assign()
    takes a batch of decode keys from the steady zone (cluster = arg-max dot
    product over the shadow, delta counts and sums, ring entries); refresh()
    replaces the centroids whose delta count reached the threshold.  The
    selection reads the shadow rows of replaced cells and matches the ring
    against the kept cells (select / DecodePlan with ``update=``).  Call
    refresh() before the next step's selection, and before the next assign().
    index_by_gid: the override slots are indexed by global cell id (2-way
    selection) instead of compact id (4-way)."""

    def __init__(self, compact_centroids: torch.Tensor, compact_size: torch.Tensor, compact_gid: torch.Tensor,
                 n_active: torch.Tensor, padding_id: int, threshold: int, ring_cap: int, n_index: int,
                 index_by_gid: bool):
        dev = _require_device(compact_centroids, compact_size, compact_gid, n_active)
        H, n_rows, D = compact_centroids.shape
        if D != 128:
            raise ValueError("online update needs head_dim 128")
        self.device, self.H, self.n_rows, self.D = dev, H, n_rows, D
        self.padding_id, self.threshold, self.ring_cap = int(padding_id), int(threshold), int(ring_cap)
        self.n_index, self.index_by_gid = int(n_index), bool(index_by_gid)
        i32 = dict(dtype=torch.int32, device=dev)
        self.shadow = compact_centroids.to(torch.float32).contiguous().clone()
        self.centroid_counts = compact_size.to(torch.int32).contiguous().clone()
        self.delta_counts = torch.zeros((H, n_rows), **i32)
        self.delta_sums = torch.zeros((H, n_rows, D), dtype=torch.float32, device=dev)
        self.compact_gid = compact_gid.to(torch.int32).contiguous()
        self.n_active = n_active.to(torch.int32).contiguous()
        self.ring_id = torch.full((H, ring_cap), int(padding_id), **i32)
        self.ring_cell = torch.full((H, ring_cap), -2, **i32)
        self.ring_row = torch.zeros((H, ring_cap), **i32)
        self.ring_pos = torch.zeros((H,), **i32)
        self.ring_n = torch.zeros((H,), **i32)
        self.upd_slot = torch.full((H, self.n_index), -1, **i32)
        self.upd_row = torch.zeros((H, n_rows), **i32)
        self.upd_n = torch.zeros((H,), **i32)
        self._ws: Optional[torch.Tensor] = None

    def _args(self, steady_keys: Optional[torch.Tensor], row0: int, count: int) -> UpdateArgs:
        a = UpdateArgs(steady_stride=0, row0=int(row0), count=int(count), kv_heads=self.H, dim=self.D,
                       shadow=self.shadow.data_ptr(), n_rows=self.n_rows, padding_id=self.padding_id,
                       n_active=self.n_active.data_ptr(), compact_gid=self.compact_gid.data_ptr(),
                       centroid_counts=self.centroid_counts.data_ptr(), delta_counts=self.delta_counts.data_ptr(),
                       delta_sums=self.delta_sums.data_ptr(), threshold=self.threshold,
                       ring_id=self.ring_id.data_ptr(), ring_cell=self.ring_cell.data_ptr(),
                       ring_row=self.ring_row.data_ptr(), ring_pos=self.ring_pos.data_ptr(),
                       ring_n=self.ring_n.data_ptr(), ring_cap=self.ring_cap, upd_slot=self.upd_slot.data_ptr(),
                       upd_row=self.upd_row.data_ptr(), upd_n=self.upd_n.data_ptr(), n_index=self.n_index,
                       index_by_gid=int(self.index_by_gid))
        if steady_keys is not None:
            if steady_keys.dim() != 3 or steady_keys.shape[0] != self.H or not steady_keys.is_contiguous():
                raise ValueError(f"steady_keys must be a contiguous [{self.H}, rows, {self.D}] tensor")
            _as_bits(steady_keys)
            a.steady_keys = steady_keys.data_ptr()
            a.steady_stride = steady_keys.shape[1]
        return a

    def assign(self, steady_keys: torch.Tensor, row0: int, count: int) -> None:
        """async_update.py:119-134, 146-161 for the keys at steady rows
        [row0, row0 + count) of steady_keys [H, rows, D] (bf16)."""
        a = self._args(steady_keys, row0, count)
        need = ctypes.c_size_t()
        check(_lib.lib().imi_update_workspace_size(ctypes.byref(a), ctypes.byref(need)), "imi_update_workspace_size")
        if self._ws is None or self._ws.numel() < need.value:
            self._ws = torch.empty(max(int(need.value), 256), dtype=torch.uint8, device=self.device)
        a.workspace = self._ws.data_ptr()
        a.workspace_bytes = self._ws.numel()
        check(_lib.lib().imi_update_assign(ctypes.byref(a), _stream(self.device)), "imi_update_assign")

    def refresh(self, count: int) -> None:
        """async_update.py:135-143 for the batch of the last assign(count)."""
        a = self._args(None, 0, count)
        check(_lib.lib().imi_update_refresh(ctypes.byref(a), _stream(self.device)), "imi_update_refresh")

    def wire(self, s: SelectArgs, exec_rows: int) -> None:
        """Point selection arguments at this state (replaced centroids and
        the delta ring)."""
        s.shadow = self.shadow.data_ptr()
        s.shadow_rows = self.n_rows
        s.upd_slot = self.upd_slot.data_ptr()
        s.upd_row = self.upd_row.data_ptr()
        s.upd_n = self.upd_n.data_ptr()
        s.ring_cell = self.ring_cell.data_ptr()
        s.ring_row = self.ring_row.data_ptr()
        s.ring_n = self.ring_n.data_ptr()
        s.ring_cap = self.ring_cap
        s.exec_rows = int(exec_rows)


def check_decode_limits(kv_heads: int, groups: int, ks: Sequence[int], budget: Budget,
                        online: bool = False) -> None:
    """Raise IMIError now if the selection kernels cannot rank this shape
    (cells per head, cells to rank, heads, groups), before any index is built:
    imi_select_workspace_size validates the same limits a decode step would.
    online: the delta match ranks all of nprobe (async update on)."""
    ncells = 1
    for k in ks:
        ncells *= int(k)
    a = SelectArgs(query=16, centroids=16, cell_count=16, cell_offset=16, kv_heads=int(kv_heads),
                   groups=int(groups), dim=128, parts=len(ks), nprobe=budget.nprobe, max_tokens=budget.max_tokens,
                   buffer_pages=budget.buffer_pages, page_size=budget.page_size,
                   tile_mode=int(bool(budget.tile_mode)))
    a.k = _ks(ks)
    rank_all = online or budget.tile_mode
    a.sel_cap = budget.nprobe if rank_all else min(budget.nprobe, budget.buffer_pages)
    if online:
        a.ring_cap, a.ring_cell, a.ring_row, a.ring_n, a.exec_rows = 1, 16, 16, 16, 0
    if len(ks) == 4:
        a.compact_gid = a.compact_size = a.compact_offset = a.n_active = 16
        a.compact_cap = ncells + 1
    need = ctypes.c_size_t()
    check(_lib.lib().imi_select_workspace_size(ctypes.byref(a), ctypes.byref(need)),
          f"decode selection for k={list(ks)}, nprobe={budget.nprobe}, buffer_pages={budget.buffer_pages}")


def _sel_cap(budget: Budget, update: Optional[OnlineUpdate]) -> int:
    """Ranks the selection keeps: the delta match needs all of nprobe."""
    return max(budget.sel_cap, budget.nprobe) if update is not None else budget.sel_cap


def select(query: torch.Tensor, centroids: torch.Tensor, cell_count: torch.Tensor, cell_offset: torch.Tensor,
           ks: Sequence[int], budget: Budget, compact: Optional[Dict[str, torch.Tensor]] = None,
           update: Optional[OnlineUpdate] = None, exec_rows: int = 0) -> Dict[str, torch.Tensor]:
    """Scores + top-nprobe + token prefix + page rule, per KV head
    (retrieval.py:295-303,357; wave_buffer_cpu_hotcold.cpp:303-371).
    A 4-way IMI needs ``compact`` (the build_index outputs with compact=True).
    With ``update`` the replaced centroids are scored and the delta ring is
    matched (outputs delta_rows [H, ring_cap], n_delta [H]); exec_rows =
    execution-buffer rows after the static rows."""
    dev = _require_device(query, centroids, cell_count, cell_offset)
    _as_bits(query)
    H, G, D = query.shape
    cap = _sel_cap(budget, update)
    out = {
        "sel_cell": torch.full((H, cap), -1, dtype=torch.int32, device=dev),
        "sel_offset": torch.zeros((H, cap), dtype=torch.int32, device=dev),
        "sel_count": torch.zeros((H, cap), dtype=torch.int32, device=dev),
        "sel_prefix": torch.zeros((H, cap + 1), dtype=torch.int32, device=dev),
        "n_selected": torch.zeros((H,), dtype=torch.int32, device=dev),
        "n_rows": torch.zeros((H,), dtype=torch.int32, device=dev),
    }
    q = query.contiguous()
    a = SelectArgs(query=q.data_ptr(), centroids=centroids.data_ptr(), cell_count=cell_count.data_ptr(),
                   cell_offset=cell_offset.data_ptr(), kv_heads=H, groups=G, dim=D, parts=len(ks), k=_ks(ks),
                   nprobe=budget.nprobe, max_tokens=budget.max_tokens, buffer_pages=budget.buffer_pages,
                   page_size=budget.page_size, sel_cell=out["sel_cell"].data_ptr(),
                   sel_offset=out["sel_offset"].data_ptr(), sel_count=out["sel_count"].data_ptr(),
                   sel_prefix=out["sel_prefix"].data_ptr(), n_selected=out["n_selected"].data_ptr(),
                   n_rows=out["n_rows"].data_ptr(), sel_cap=cap)
    _compact_fields(a, compact)
    keep = _budget_fields(a, budget, H, dev)
    a.tile_mode = int(bool(budget.tile_mode))
    if update is not None:
        update.wire(a, exec_rows)
        out["delta_rows"] = torch.zeros((H, update.ring_cap), dtype=torch.int32, device=dev)
        out["n_delta"] = torch.zeros((H,), dtype=torch.int32, device=dev)
        a.delta_rows = out["delta_rows"].data_ptr()
        a.n_delta = out["n_delta"].data_ptr()
    need = ctypes.c_size_t()
    check(_lib.lib().imi_select_workspace_size(ctypes.byref(a), ctypes.byref(need)), "imi_select_workspace_size")
    if need.value:
        ws = workspace("select", need.value, dev)
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel()
    check(_lib.lib().imi_select(ctypes.byref(a), _stream(dev)), "imi_select")
    return out


def sparse_attention(query: torch.Tensor, steady_keys: Optional[torch.Tensor], steady_values: Optional[torch.Tensor],
                     static_len: int, list_keys: torch.Tensor, list_values: torch.Tensor, sel: Dict[str, torch.Tensor],
                     max_rows: int, scale: Optional[float] = None, return_lse: bool = False):
    """Gather + GQA decode attention over [static rows | selected rows |
    delta rows]; the delta rows (steady-zone rows) come from a selection
    made with ``update`` (sel["delta_rows"], sel["n_delta"]), and max_rows
    must then also cover them."""
    dev = _require_device(query, list_keys, list_values)
    _as_bits(query)
    H, G, D = query.shape
    out = torch.empty((H * G, D), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((H * G,), dtype=torch.float32, device=dev) if return_lse else None
    ss = steady_keys.shape[1] if steady_keys is not None else 0
    cap = sel["sel_cell"].shape[1]
    a = AttentionArgs(query=query.contiguous().data_ptr(), steady_keys=_ptr(steady_keys),
                      steady_values=_ptr(steady_values), steady_stride=ss, static_len=int(static_len),
                      list_keys=list_keys.data_ptr(), list_values=list_values.data_ptr(),
                      list_rows=list_keys.shape[1], sel_offset=sel["sel_offset"].data_ptr(),
                      sel_count=sel["sel_count"].data_ptr(), sel_prefix=sel["sel_prefix"].data_ptr(),
                      n_selected=sel["n_selected"].data_ptr(), n_rows=sel["n_rows"].data_ptr(), sel_cap=cap,
                      max_rows=int(max_rows), kv_heads=H, groups=G, dim=D,
                      scale=float(scale if scale is not None else 1.0 / math.sqrt(D)), out=out.data_ptr(),
                      out_lse=_ptr(lse))
    if "delta_rows" in sel:
        a.delta_rows = sel["delta_rows"].data_ptr()
        a.n_delta = sel["n_delta"].data_ptr()
        a.delta_cap = sel["delta_rows"].shape[1]
    need = ctypes.c_size_t()
    check(_lib.lib().imi_attention_workspace_size(ctypes.byref(a), ctypes.byref(need)),
          "imi_attention_workspace_size")
    ws = workspace("attention", need.value, dev)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    check(_lib.lib().imi_sparse_attention(ctypes.byref(a), _stream(dev)), "imi_sparse_attention")
    return (out, lse) if return_lse else out


def _rows_hint(cell_count: torch.Tensor, compact: Optional[Dict[str, torch.Tensor]], budget: "Budget",
               steady_rows: int) -> int:
    """Expected attended rows per head, for the attention's choice of split
    pass only (one device sync, at plan time): cells of the index's mean
    occupied size, as many as nprobe, the token rule and the page rule allow
    (wave_buffer_cpu_hotcold.cpp:303-371), plus the steady zone; the largest
    over the heads.  0 (unknown) in tile mode."""
    if budget.tile_mode:
        return 0
    if compact is not None:
        rows = compact["compact_size"].sum(1).double()
        occ = compact["n_active"].double()
    else:
        rows = cell_count.sum(1).double()
        occ = (cell_count > 0).sum(1).double()
    mean = (rows / occ.clamp(min=1)).clamp(min=1).cpu().tolist()
    est = 0.0
    for m in mean:
        cells = min(budget.nprobe, budget.buffer_pages // max(1, math.ceil(m / budget.page_size)))
        est = max(est, min(budget.max_tokens + m, cells * m))
    return int(min(est + steady_rows, 2 ** 30))


class DecodePlan:
    """Pre-built arguments of imi_decode_step for one layer: only the query,
    output and static_len change between steps, so a step costs one ctypes
    call.  The plan owns its workspace (zero-filled once)."""

    def __init__(self, centroids: torch.Tensor, cell_count: torch.Tensor, cell_offset: torch.Tensor,
                 ks: Sequence[int], budget: Budget, list_keys: torch.Tensor, list_values: torch.Tensor,
                 steady_keys: Optional[torch.Tensor], steady_values: Optional[torch.Tensor], groups: int,
                 scale: Optional[float] = None, query: Optional[torch.Tensor] = None,
                 out: Optional[torch.Tensor] = None, out_lse: Optional[torch.Tensor] = None,
                 compact: Optional[Dict[str, torch.Tensor]] = None, update: Optional[OnlineUpdate] = None):
        dev = _require_device(centroids, cell_count, cell_offset, list_keys, list_values)
        self.device = dev
        H, _, D = list_keys.shape
        self.H, self.G, self.D = H, groups, D
        self.budget = budget
        self.update = update
        self.sel_cap = _sel_cap(budget, update)
        self.query = query if query is not None else torch.zeros((H, groups, D), dtype=torch.bfloat16, device=dev)
        self.out = out if out is not None else torch.empty((H * groups, D), dtype=torch.bfloat16, device=dev)
        self._keep = (centroids, cell_count, cell_offset, list_keys, list_values, steady_keys, steady_values,
                      out_lse, compact, update)
        a = DecodeArgs()
        s = a.sel
        s.query = self.query.data_ptr()
        s.centroids = centroids.data_ptr()
        s.cell_count = cell_count.data_ptr()
        s.cell_offset = cell_offset.data_ptr()
        s.kv_heads, s.groups, s.dim, s.parts = H, groups, D, len(ks)
        s.k = _ks(ks)
        s.nprobe, s.max_tokens = budget.nprobe, budget.max_tokens
        s.buffer_pages, s.page_size = budget.buffer_pages, budget.page_size
        s.sel_cap = self.sel_cap
        _compact_fields(s, compact)
        self._keep_budget = _budget_fields(s, budget, H, dev)
        s.tile_mode = int(bool(budget.tile_mode))
        if update is not None:
            update.wire(s, 0)
        t = a.attn
        t.query = self.query.data_ptr()
        t.steady_keys = _ptr(steady_keys)
        t.steady_values = _ptr(steady_values)
        t.steady_stride = steady_keys.shape[1] if steady_keys is not None else 0
        t.static_len = 0
        t.list_keys, t.list_values = list_keys.data_ptr(), list_values.data_ptr()
        t.list_rows = list_keys.shape[1]
        t.max_rows = budget.max_rows + (update.ring_cap if update is not None else 0)
        t.kv_heads, t.groups, t.dim = H, groups, D
        t.scale = float(scale if scale is not None else 1.0 / math.sqrt(D))
        t.out = self.out.data_ptr()
        t.out_lse = _ptr(out_lse)
        # a ragged batch: per-head row bounds (host memory, read at each call),
        # so that the attention gives each sequence's heads splits in
        # proportion to their budgets
        self._head_bounds = None
        if budget.head_buffer_pages is not None:
            rc = update.ring_cap if update is not None else 0
            mt = budget.head_max_tokens or [budget.max_tokens] * H
            bounds = [t.steady_stride + bp * budget.page_size + (m if budget.tile_mode else 0) + rc
                      for bp, m in zip(budget.head_buffer_pages, mt)]
            self._head_bounds = (ctypes.c_int32 * H)(*bounds)
            t.head_rows_bound = ctypes.addressof(self._head_bounds)
        t.rows_hint = _rows_hint(cell_count, compact, budget, t.steady_stride)
        need = ctypes.c_size_t()
        check(_lib.lib().imi_decode_workspace_size(ctypes.byref(a), ctypes.byref(need)), "imi_decode_workspace_size")
        self.ws = torch.zeros(max(need.value, 256), dtype=torch.uint8, device=dev)
        t.workspace = self.ws.data_ptr()
        t.workspace_bytes = self.ws.numel()
        self.args = a
        self._fn = _lib.lib().imi_decode_step
        self._ref = ctypes.byref(a)
        self.selection = self._selection_views()

    def _selection_views(self) -> Dict[str, torch.Tensor]:
        """Views of the workspace where the selection outputs land."""
        H, cap = self.H, self.sel_cap
        i32 = self.ws.view(torch.int32)
        off = 0
        views = {}
        rc = self.update.ring_cap if self.update is not None else 0
        for name, n in (("sel_cell", H * cap), ("sel_offset", H * cap), ("sel_count", H * cap),
                        ("sel_prefix", H * (cap + 1)), ("n_selected", H), ("n_rows", H),
                        ("delta_rows", H * max(rc, 1)), ("n_delta", H)):
            off = (off + 63) // 64 * 64  # 256-byte alignment in int32 units
            views[name] = i32[off:off + n]
            off += n
        if rc:
            views["delta_rows"] = views["delta_rows"].view(H, rc)
        else:
            del views["delta_rows"], views["n_delta"]
        views["sel_cell"] = views["sel_cell"].view(H, cap)
        views["sel_offset"] = views["sel_offset"].view(H, cap)
        views["sel_count"] = views["sel_count"].view(H, cap)
        views["sel_prefix"] = views["sel_prefix"].view(H, cap + 1)
        return views

    def set_static_len(self, static_len: int) -> None:
        self.args.attn.static_len = int(static_len)

    def set_exec_rows(self, exec_rows: int) -> None:
        """Execution-buffer rows left after the static rows (the delta
        append's bound, retrieval.py via async_update.py:57-72)."""
        self.args.sel.exec_rows = int(exec_rows)

    def run(self, query: torch.Tensor, out: torch.Tensor, static_len: int, stream: Optional[int] = None,
            exec_rows: Optional[int] = None, phases: int = 3) -> torch.Tensor:
        """One step (phases as in step(); 3 = all of it) on caller-owned query
        [H, G, D] and out [H * G, D] buffers (no copies: the plan's pointers
        are redirected)."""
        _as_bits(query)
        if not query.is_contiguous() or tuple(query.shape) != (self.H, self.G, self.D):
            raise ValueError(f"query must be a contiguous [{self.H}, {self.G}, {self.D}] tensor")
        if not out.is_contiguous() or out.numel() != self.H * self.G * self.D or out.dtype != torch.bfloat16:
            raise ValueError("out must be a contiguous bf16 tensor of H * G * D elements")
        a = self.args
        a.sel.query = a.attn.query = query.data_ptr()
        a.attn.out = out.data_ptr()
        a.attn.static_len = int(static_len)
        if exec_rows is not None:
            a.sel.exec_rows = int(exec_rows)
        a.phases = int(phases)
        try:
            check(self._fn(self._ref, stream if stream is not None else _stream(self.device)), "imi_decode_step")
        finally:
            a.sel.query = a.attn.query = self.query.data_ptr()
            a.attn.out = self.out.data_ptr()
        return out

    def step(self, stream: Optional[int] = None, phases: int = 3) -> torch.Tensor:
        """Enqueue one step.  phases (bits): 1 selection, 2 attention (split
        pass + merge), 4 split pass only, 8 merge only; 3 = the whole step."""
        self.args.phases = phases
        check(self._fn(self._ref, stream if stream is not None else _stream(self.device)), "imi_decode_step")
        return self.out


def dense_attention(query: torch.Tensor, steady_keys: torch.Tensor, steady_values: torch.Tensor, static_len: int,
                    scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """GQA decode attention over the first static_len rows of the steady zone
    only (runtime.py:393-402): the gather kernel with an empty selection."""
    dev = _require_device(query, steady_keys, steady_values)
    _as_bits(query)
    H, G, D = query.shape
    if steady_keys.shape[0] != H or steady_keys.shape[2] != D or not steady_keys.is_contiguous():
        raise ValueError("steady_keys must be contiguous [H, rows, D]")
    if steady_values.shape != steady_keys.shape or not steady_values.is_contiguous():
        raise ValueError("steady_values must match steady_keys")
    key = ("dense_sel", dev.index if dev.index is not None else torch.cuda.current_device(), H)
    zeros = _WS.get(key)
    if zeros is None:
        # sel_offset [H][1], sel_count [H][1], sel_prefix [H][2], counts [H]: all zero
        zeros = torch.zeros((4, 2 * H + 2), dtype=torch.int32, device=dev)
        _WS[key] = zeros
    if out is None:
        out = torch.empty((H * G, D), dtype=torch.bfloat16, device=dev)
    a = AttentionArgs(query=query.contiguous().data_ptr(), steady_keys=steady_keys.data_ptr(),
                      steady_values=steady_values.data_ptr(), steady_stride=steady_keys.shape[1],
                      static_len=int(static_len), list_keys=steady_keys.data_ptr(),
                      list_values=steady_values.data_ptr(), list_rows=steady_keys.shape[1],
                      sel_offset=zeros[0].data_ptr(), sel_count=zeros[1].data_ptr(), sel_prefix=zeros[2].data_ptr(),
                      n_selected=zeros[3].data_ptr(), n_rows=zeros[3].data_ptr(), sel_cap=1, max_rows=0,
                      kv_heads=H, groups=G, dim=D,
                      scale=float(scale if scale is not None else 1.0 / math.sqrt(D)), out=out.data_ptr(),
                      out_lse=None)
    need = ctypes.c_size_t()
    check(_lib.lib().imi_attention_workspace_size(ctypes.byref(a), ctypes.byref(need)),
          "imi_attention_workspace_size")
    ws = workspace("dense_attention", need.value, dev)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = ws.numel()
    check(_lib.lib().imi_sparse_attention(ctypes.byref(a), _stream(dev)), "imi_sparse_attention")
    return out


def host_cache_pages(n_centroids: int, nprobe: int, pages_per_cluster: int = 2, cache_ratio: float = 0.05) -> int:
    """GPU cache size in pages (runtime.py:48-53): round(n_centroids *
    cache_ratio) clusters (nprobe * 3 when cache_ratio <= 0) of
    pages_per_cluster pages, at least one."""
    clusters = round(n_centroids * cache_ratio) if cache_ratio > 0.0 else nprobe * 3
    return max(int(clusters) * int(pages_per_cluster), 1)


class HostTierPlan:
    """Decode over KV lists in pinned host memory with a GPU block cache per
    KV head (the reference's wave buffer: wave_buffer_cpu_hotcold.cpp:54-372,
    retrieval.py:200-290 _run_retrieval_full).  Per step: the selection runs
    on the GPU and its ranked cells come to the host (the reference's
    retrieval.py:377 copy); the host cache manager splits their pages into
    hits (cache blocks) and misses (list rows in host memory); the gather
    kernel builds the execution buffer [miss rows | hit rows] and a one-cell
    selection over it; the host admits the missed clusters that fit; the
    admission kernel copies them into the cache; the attention runs over
    [steady rows | buffer | matched delta-ring rows].

    Cells: the global cells of the CSR for a 2-way IMI and IVF; for a 4-way
    IMI (``compact``, the occupied cells of build_index) the manager keeps
    the occupied cells by compact id and the host maps each selected global
    id to its compact id (the reference's clusters are its compact cells).
    ``update``: the online index update (async_update.py), whose replaced
    centroids the selection scores and whose matched ring tokens (steady
    rows) are attended after the buffer.  Not with tile mode.

    list_keys / list_values: pinned host tensors [H, rows, D], used in place
    (the drop-in cache writes each layer's lists there during its build), or
    device tensors, copied once into pinned host memory.  The device holds
    the cache (cache_pages x page_size rows per head) and the execution
    buffer (buffer_pages x page_size rows per head)."""

    def __init__(self, centroids: torch.Tensor, cell_count: torch.Tensor, cell_offset: torch.Tensor,
                 ks: Sequence[int], budget: Budget, list_keys: torch.Tensor, list_values: torch.Tensor,
                 steady_keys: Optional[torch.Tensor], steady_values: Optional[torch.Tensor], groups: int,
                 cache_pages: int, hot_ratio: float = 0.0, scale: Optional[float] = None,
                 compact: Optional[Dict[str, torch.Tensor]] = None, update: Optional[OnlineUpdate] = None):
        import numpy as np

        if len(ks) not in (1, 2, 4):
            raise ValueError("the host tier serves IVF, 2-way and 4-way IMI")
        if len(ks) == 4 and compact is None:
            raise ValueError("a 4-way host tier needs the occupied cells (build_index compact outputs)")
        if budget.tile_mode or budget.head_buffer_pages is not None:
            raise ValueError("the host tier runs without tile mode and with one budget for every head")
        if cache_pages < 1:
            raise ValueError("cache_pages must be >= 1")
        dev = _require_device(centroids, cell_count, cell_offset)
        H, list_rows, D = list_keys.shape
        if tuple(list_values.shape) != (H, list_rows, D):
            raise ValueError("list_keys and list_values must have the same [H, rows, D] shape")
        ps, bp = budget.page_size, budget.buffer_pages
        self.device, self.H, self.G, self.D = dev, H, groups, D
        self.budget, self.cache_pages = budget, int(cache_pages)
        # pinned host lists (taken as they are when already pinned) and their device mapping
        host = [t if (not t.is_cuda and t.is_pinned() and t.is_contiguous()) else None
                for t in (list_keys, list_values)]
        if host[0] is None or host[1] is None:
            host = [torch.empty((H, list_rows, D), dtype=t.dtype, pin_memory=True) for t in (list_keys, list_values)]
            host[0].copy_(list_keys)
            host[1].copy_(list_values)
        self.h_keys, self.h_values = host
        _as_bits(self.h_keys)
        _as_bits(self.h_values)
        L = _lib.lib()
        dk, dv = ctypes.c_void_p(), ctypes.c_void_p()
        check(L.imi_host_device_pointer(ctypes.c_void_p(self.h_keys.data_ptr()), ctypes.byref(dk)),
              "imi_host_device_pointer")
        check(L.imi_host_device_pointer(ctypes.c_void_p(self.h_values.data_ptr()), ctypes.byref(dv)),
              "imi_host_device_pointer")
        self.exec_rows = bp * ps
        self.cache_rows = self.cache_pages * ps
        self.exec_keys = torch.zeros((H, self.exec_rows, D), dtype=torch.bfloat16, device=dev)
        self.exec_values = torch.zeros_like(self.exec_keys)
        self.cache_keys = torch.zeros((H, self.cache_rows, D), dtype=torch.bfloat16, device=dev)
        self.cache_values = torch.zeros_like(self.cache_keys)
        # the selection and the attention of one DecodePlan whose list is the buffer
        self.plan = DecodePlan(centroids, cell_count, cell_offset, ks, budget, self.exec_keys, self.exec_values,
                               steady_keys, steady_values, groups, scale=scale, compact=compact, update=update)
        self.cap = self.plan.sel_cap
        # the manager's cells: sizes and CSR offsets per head, then one empty
        # padding cell that closes each key list
        if compact is not None:
            na = compact["n_active"].cpu().numpy().astype(np.int64)
            n = int(na.max()) if na.size else 0
            self._gids = compact["compact_gid"].cpu().numpy()
            self._na = na
            csz = compact["compact_size"].cpu().numpy()
            coff = compact["compact_offset"].cpu().numpy()
            sizes = np.zeros((H, n + 1), np.int32)
            offs = np.zeros((H, n + 2), np.int32)
            for h in range(H):
                sizes[h, :na[h]] = csz[h, :na[h]]
                offs[h, :na[h] + 1] = coff[h, :na[h] + 1]
                offs[h, na[h] + 1:] = coff[h, na[h]]
        else:
            self._gids = None
            n = int(cell_count.shape[1])
            sizes = np.zeros((H, n + 1), np.int32)
            offs = np.zeros((H, n + 2), np.int32)
            sizes[:, :n] = cell_count.cpu().numpy()
            offs[:, :n + 1] = cell_offset.cpu().numpy()
            offs[:, n + 1] = offs[:, n]
        self.pad = n
        self._h = ctypes.c_void_p()
        check(L.imi_hostcache_create(H, n + 1, self.cache_pages, ps, bp, self.cap, float(hot_ratio),
                                     ctypes.byref(self._h)), "imi_hostcache_create")
        check(L.imi_hostcache_set_metadata(self._h, sizes.ctypes.data_as(ctypes.c_void_p),
                                           offs.ctypes.data_as(ctypes.c_void_p)), "imi_hostcache_set_metadata")
        # pinned host lists (8 access + 4 update arrays) and their device copies
        n = H * bp
        self.h_lists = torch.zeros((12, n), dtype=torch.int32, pin_memory=True)
        self.h_nums = torch.zeros((3, 2, H), dtype=torch.int32, pin_memory=True)   # hit, miss, update counts
        self.d_lists = torch.zeros((12, n), dtype=torch.int32, device=dev)
        self.d_nums = torch.zeros((3, 2, H), dtype=torch.int32, device=dev)
        self.h_sel = torch.zeros((H, self.cap), dtype=torch.int32, pin_memory=True)
        self.h_nsel = torch.zeros(H, dtype=torch.int32, pin_memory=True)
        self.keys = np.full((H, self.cap), self.pad, np.int64)
        self.hits = self.misses = 0     # blocks over all steps
        self.miss_rows = 0              # rows read from host memory over all steps
        sel = self.plan.selection
        g = _lib.HostcacheGatherArgs()
        g.host_keys, g.host_values, g.list_rows = dk.value, dv.value, list_rows
        g.cache_keys, g.cache_values, g.cache_rows = self.cache_keys.data_ptr(), self.cache_values.data_ptr(), self.cache_rows
        g.exec_keys, g.exec_values, g.exec_rows = self.exec_keys.data_ptr(), self.exec_values.data_ptr(), self.exec_rows
        g.groups, g.max_blocks, g.block_size = H, bp, ps
        row = lambda i: self.d_lists[i].data_ptr()
        g.hit_ids, g.hit_sizes, g.hit_prefix = row(0), row(1), row(2)
        g.miss_ids, g.miss_sizes, g.miss_prefix = row(3), row(4), row(5)
        g.hit_nums, g.miss_nums = self.d_nums[0, 0].data_ptr(), self.d_nums[0, 1].data_ptr()
        g.sel_offset, g.sel_count = sel["sel_offset"].data_ptr(), sel["sel_count"].data_ptr()
        g.sel_prefix, g.n_selected, g.n_rows = sel["sel_prefix"].data_ptr(), sel["n_selected"].data_ptr(), sel["n_rows"].data_ptr()
        g.sel_cap = self.cap
        self._gather = g

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _lib.lib().imi_hostcache_destroy(h)
            self._h = None

    def step(self, query: torch.Tensor, out: torch.Tensor, static_len: int,
             exec_rows: Optional[int] = None) -> torch.Tensor:
        """One decode step (host-synchronous, as the reference's).  exec_rows:
        execution-buffer rows left after the static rows, the bound of the
        delta append (with the online update)."""
        import numpy as np

        L = _lib.lib()
        stream = _stream(self.device)
        H, cap, bp = self.H, self.cap, self.budget.buffer_pages
        self.plan.run(query, out, static_len, stream=stream, phases=1, exec_rows=exec_rows)   # selection
        sel = self.plan.selection
        self.h_sel.copy_(sel["sel_cell"], non_blocking=True)
        self.h_nsel.copy_(sel["n_selected"], non_blocking=True)
        torch.cuda.current_stream(self.device).synchronize()
        cells, m = self.h_sel.numpy(), self.h_nsel.numpy()
        keys = self.keys
        keys.fill(self.pad)
        if self._gids is None:
            live = np.arange(cap)[None, :] < np.clip(m, 0, cap)[:, None]
            keys[live] = cells[live]
        else:   # 4-way: selected global ids -> compact ids (occupied cells in ascending global id)
            for h in range(H):
                mh = int(np.clip(m[h], 0, cap))
                keys[h, :mh] = np.searchsorted(self._gids[h, :self._na[h]], cells[h, :mh])
        hl, hn = self.h_lists.numpy(), self.h_nums.numpy()
        p = lambda a: a.ctypes.data_as(ctypes.c_void_p)
        check(L.imi_hostcache_access(self._h, p(keys), cap, p(hl[0]), p(hl[1]), p(hl[2]), p(hn[0, 0]),
                                     p(hl[3]), p(hl[4]), p(hl[5]), p(hn[0, 1])), "imi_hostcache_access")
        self.d_lists[:6].copy_(self.h_lists[:6], non_blocking=True)
        self.d_nums[0].copy_(self.h_nums[0], non_blocking=True)
        check(L.imi_hostcache_gather(ctypes.byref(self._gather), stream), "imi_hostcache_gather")
        hb, mbk = ctypes.c_int64(), ctypes.c_int64()
        check(L.imi_hostcache_stats(self._h, ctypes.byref(hb), ctypes.byref(mbk)), "imi_hostcache_stats")
        self.hits += hb.value
        self.misses += mbk.value
        nm = hn[0, 1]
        self.miss_rows += int(sum(int(hl[4][g * bp:g * bp + int(nm[g])].sum()) for g in range(H)))
        # admission (host) while the gather runs, then its copy into the cache
        check(L.imi_hostcache_update(self._h, p(hl[6]), p(hl[7]), p(hl[8]), p(hn[1, 0])), "imi_hostcache_update")
        self.d_lists[6:9].copy_(self.h_lists[6:9], non_blocking=True)
        self.d_nums[1].copy_(self.h_nums[1], non_blocking=True)
        row = lambda i: self.d_lists[i].data_ptr()
        check(L.imi_hostcache_admit(self.exec_keys.data_ptr(), self.exec_values.data_ptr(), self.exec_rows,
                                    self.cache_keys.data_ptr(), self.cache_values.data_ptr(), self.cache_rows,
                                    self.budget.page_size, H, bp, row(6), row(7), row(8),
                                    self.d_nums[1, 0].data_ptr(), stream), "imi_hostcache_admit")
        self.plan.run(query, out, static_len, stream=stream, phases=2, exec_rows=exec_rows)   # attention + merge
        return out
