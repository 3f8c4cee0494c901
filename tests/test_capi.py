"""Host-side checks of the C ABI that need no GPU: the library loads, exports
every entry point declared in include/imi_hip.h, and rejects bad arguments
with a status code and a message (no kernel is launched on these paths)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def declared_functions():
    text = (ROOT / "include" / "imi_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|void|const char\*)\s+(imi_\w+)\s*\(", text, re.M)))


@pytest.fixture(scope="module")
def L():
    from adaptiveimi_amd import _lib

    return _lib.lib()


def test_exports_every_declared_symbol(L):
    names = declared_functions()
    assert len(names) >= 12
    for n in names:
        assert hasattr(L, n), n
    from adaptiveimi_amd import _lib

    assert set(names) == set(_lib.EXPORTS), "ctypes prototypes out of sync with the header"


def test_version(L):
    assert L.imi_version() == 5


def _kmeans_args(**over):
    from adaptiveimi_amd._lib import KmeansArgs

    a = KmeansArgs(keys=16, head_stride=4096 * 128, token_stride=128, kv_heads=8, n_tokens=4096, dim=128, parts=2,
                   max_iters=10, early_stop_min_iter=11, init_mode=0, centroids=16, labels=16)
    a.k[0] = a.k[1] = 64
    for k, v in over.items():
        if k == "k":
            for i, x in enumerate(v):
                a.k[i] = x
        else:
            setattr(a, k, v)
    return a


@pytest.mark.parametrize("over,code,text", [
    (dict(parts=3), 3, "parts"),
    (dict(k=(0, 64)), 3, "k[0]"),
    (dict(k=(513, 64)), 3, "k[0]"),
    (dict(n_tokens=0), 1, "empty"),
    (dict(n_tokens=32), 1, "first-k"),
    (dict(max_iters=0), 1, "max_iters"),
    (dict(token_stride=100), 1, "strides"),
    (dict(dim=96, parts=2), 3, "subspace width"),
])
def test_kmeans_rejects_bad_arguments(L, over, code, text):
    a = _kmeans_args(**over)
    need = ctypes.c_size_t()
    rc = L.imi_kmeans_workspace_size(ctypes.byref(a), ctypes.byref(need))
    assert rc == code
    assert text in L.imi_last_error().decode()


def test_kmeans_workspace_and_too_small_workspace(L):
    a = _kmeans_args()
    need = ctypes.c_size_t()
    assert L.imi_kmeans_workspace_size(ctypes.byref(a), ctypes.byref(need)) == 0
    assert need.value > 8 * 2 * 4096 * 4
    a.workspace = 256
    a.workspace_bytes = need.value - 1
    assert L.imi_kmeans_execute(ctypes.byref(a), None) == 4
    assert "workspace" in L.imi_last_error().decode()


def test_select_and_decode_argument_checks(L):
    from adaptiveimi_amd._lib import AttentionArgs, DecodeArgs, SelectArgs

    s = SelectArgs(query=16, centroids=16, cell_count=16, cell_offset=16, kv_heads=8, groups=4, dim=128, parts=4,
                   nprobe=410, max_tokens=3276, buffer_pages=410, page_size=8, sel_cap=410)
    s.k[0] = s.k[1] = 64
    assert L.imi_select(ctypes.byref(s), None) == 3          # 4-way needs every k in [1, 64]
    assert "k[2]=0" in L.imi_last_error().decode()
    s.k[2] = s.k[3] = 64
    assert L.imi_select(ctypes.byref(s), None) == 1          # ... and the occupied-cell arrays
    assert "compact cell arrays" in L.imi_last_error().decode()
    s.compact_gid = s.compact_size = s.compact_offset = s.n_active = 16
    s.compact_cap = 20000
    s.nprobe = s.buffer_pages = 9000
    assert L.imi_select(ctypes.byref(s), None) == 3          # top-k beyond the ranking capacity
    assert "exceed 8192" in L.imi_last_error().decode()
    s.compact_cap = 4096
    s.nprobe = s.buffer_pages = 9000                         # ... bounded by the occupied cells
    assert L.imi_select(ctypes.byref(s), None) == 1 and "sel_cap" in L.imi_last_error().decode()
    s.nprobe = s.buffer_pages = 410
    s.sel_cell = s.sel_offset = s.sel_count = s.sel_prefix = s.n_selected = s.n_rows = 16
    need = ctypes.c_size_t()
    assert L.imi_select_workspace_size(ctypes.byref(s), ctypes.byref(need)) == 0 and need.value > 0
    assert L.imi_select(ctypes.byref(s), None) == 4          # no workspace given
    assert "workspace" in L.imi_last_error().decode()
    s.parts = 2   # 2-way within the one-kernel bounds (k <= 128, K' <= 2048): no workspace
    assert L.imi_select_workspace_size(ctypes.byref(s), ctypes.byref(need)) == 0 and need.value == 0
    s.k[0], s.nprobe, s.buffer_pages = 200, 3000, 3000   # beyond them: the ranking pipeline's candidate list
    s.sel_cap = 3000
    assert L.imi_select_workspace_size(ctypes.byref(s), ctypes.byref(need)) == 0
    assert need.value >= 8 * 200 * 64 * 12   # room for every cell as a candidate: 64-bit key + cell index
    s.k[0], s.nprobe, s.buffer_pages, s.sel_cap = 64, 410, 410, 410
    s.sel_cap = 100
    assert L.imi_select(ctypes.byref(s), None) == 1
    assert "sel_cap" in L.imi_last_error().decode()
    d = DecodeArgs()
    d.sel = s
    d.sel.sel_cap = 410
    d.attn = AttentionArgs(query=16, out=16, list_keys=16, list_values=16, list_rows=4096, kv_heads=8, groups=4,
                           dim=128, max_rows=100)
    need = ctypes.c_size_t()
    assert L.imi_decode_workspace_size(ctypes.byref(d), ctypes.byref(need)) == 1
    assert "max_rows" in L.imi_last_error().decode()
    d.attn.max_rows = 410 * 8
    assert L.imi_decode_workspace_size(ctypes.byref(d), ctypes.byref(need)) == 0
    d.attn.workspace = 256                                    # never touched: the call stops at the check
    d.attn.workspace_bytes = need.value
    d.phases = 16
    assert L.imi_decode_step(ctypes.byref(d), None) == 1
    assert "phases" in L.imi_last_error().decode()
    d.phases = 0
    for g, rc in ((5, 0), (6, 0), (16, 0), (9, 3), (17, 3)):   # 1..8 and 16 query heads per KV head
        d.attn.groups = g
        d.sel.groups = g
        assert L.imi_decode_workspace_size(ctypes.byref(d), ctypes.byref(need)) == rc, g


def test_online_update_argument_checks(L):
    from adaptiveimi_amd._lib import AttentionArgs, DecodeArgs, SelectArgs, UpdateArgs

    u = UpdateArgs(steady_keys=16, steady_stride=1000, row0=980, count=16, kv_heads=8, dim=128, shadow=16,
                   n_rows=4097, padding_id=4096, n_active=16, compact_gid=16, centroid_counts=16, delta_counts=16,
                   delta_sums=16, threshold=16, ring_id=16, ring_cell=16, ring_row=16, ring_pos=16, ring_n=16,
                   ring_cap=512, upd_slot=16, upd_row=16, upd_n=16, n_index=4096, index_by_gid=1)
    need = ctypes.c_size_t()
    assert L.imi_update_workspace_size(ctypes.byref(u), ctypes.byref(need)) == 0 and need.value >= 8 * 16 * 17 * 8
    assert L.imi_update_assign(ctypes.byref(u), None) == 4          # no workspace given
    u.row0 = 990
    assert L.imi_update_assign(ctypes.byref(u), None) == 1          # rows past the steady zone
    assert "steady zone" in L.imi_last_error().decode()
    u.row0, u.count = 0, 65
    assert L.imi_update_refresh(ctypes.byref(u), None) == 3         # batch above 64 keys
    u.count, u.ring_cap = 16, 2000
    assert L.imi_update_refresh(ctypes.byref(u), None) == 3
    assert "ring_cap" in L.imi_last_error().decode()
    u.ring_cap, u.delta_sums = 512, None
    assert L.imi_update_refresh(ctypes.byref(u), None) == 1
    assert "null state" in L.imi_last_error().decode()
    # selection: the delta append needs the ring and must rank all of nprobe;
    # in tile mode it needs the workspace of its tile scratch (the one-kernel
    # selection needs none otherwise)
    s = SelectArgs(query=16, centroids=16, cell_count=16, cell_offset=16, kv_heads=8, groups=4, dim=128, parts=2,
                   nprobe=410, max_tokens=3276, buffer_pages=300, page_size=8, sel_cap=300, ring_cap=512,
                   tile_mode=1)
    s.k[0] = s.k[1] = 64
    assert L.imi_select(ctypes.byref(s), None) == 1
    assert "delta ring" in L.imi_last_error().decode()
    s.ring_cell = s.ring_row = s.ring_n = 16
    assert L.imi_select(ctypes.byref(s), None) == 1
    assert "sel_cap 300 < 410 (nprobe)" in L.imi_last_error().decode()
    s.sel_cap = 410
    assert L.imi_select_workspace_size(ctypes.byref(s), ctypes.byref(need)) == 0 and need.value >= 8 * 411 * 4
    s.sel_cell = s.sel_offset = s.sel_count = s.sel_prefix = s.n_selected = s.n_rows = 16
    s.delta_rows = s.n_delta = 16
    assert L.imi_select(ctypes.byref(s), None) == 4
    assert "workspace" in L.imi_last_error().decode()
    s.tile_mode = 0
    assert L.imi_select_workspace_size(ctypes.byref(s), ctypes.byref(need)) == 0 and need.value == 0
    s.sel_cell = s.sel_offset = s.sel_count = s.sel_prefix = s.n_selected = s.n_rows = None
    s.delta_rows = s.n_delta = None
    s.upd_slot = 16
    assert L.imi_select(ctypes.byref(s), None) == 1
    assert "shadow" in L.imi_last_error().decode()
    s.upd_slot = None
    d = DecodeArgs()
    d.sel = s
    d.attn = AttentionArgs(query=16, out=16, list_keys=16, list_values=16, list_rows=4096, kv_heads=8, groups=4,
                           dim=128, max_rows=300 * 8, steady_keys=16, steady_values=16, steady_stride=200)
    assert L.imi_decode_workspace_size(ctypes.byref(d), ctypes.byref(need)) == 1   # max_rows misses the ring
    assert "max_rows" in L.imi_last_error().decode()
    d.attn.max_rows = 300 * 8 + 512
    assert L.imi_decode_workspace_size(ctypes.byref(d), ctypes.byref(need)) == 0


def test_ops_refuse_cpu_tensors():
    import torch

    from adaptiveimi_amd import ops

    k = torch.zeros((2, 64, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        ops.kmeans(k, [8, 8], 2)


def test_noalloc_rejects_shapes_beyond_its_scratch(L):
    """The no-alloc step checks its workspace need against the static array
    (64 MiB) before touching the device."""
    from adaptiveimi_amd._lib import AttentionArgs, DecodeArgs, SelectArgs

    s = SelectArgs(query=16, centroids=16, cell_count=16, cell_offset=16, kv_heads=16384, groups=4, dim=128, parts=2,
                   nprobe=410, max_tokens=3276, buffer_pages=410, page_size=8, sel_cap=410)
    s.k[0] = s.k[1] = 64
    d = DecodeArgs()
    d.sel = s
    d.attn = AttentionArgs(query=16, out=16, list_keys=16, list_values=16, list_rows=4096, kv_heads=16384, groups=4,
                           dim=128, max_rows=410 * 8, steady_stride=512)
    need = ctypes.c_size_t()
    assert L.imi_decode_workspace_size(ctypes.byref(d), ctypes.byref(need)) == 0
    assert need.value > 64 << 20
    assert L.imi_decode_step_noalloc(ctypes.byref(d), None) == 3
    assert "scratch" in L.imi_last_error().decode()


def test_check_decode_limits_rejects_before_any_build(L):
    """ops.check_decode_limits runs the selection's argument checks alone (no
    device, no index), so a cache can refuse an unsupported shape before it
    spends the prefill on an index build."""
    from adaptiveimi_amd import ops
    from adaptiveimi_amd._lib import IMIError

    ops.check_decode_limits(8, 4, (64, 64), ops.Budget(410, 13097, 1638))
    ops.check_decode_limits(8, 4, (181, 90), ops.Budget(1638, 52000, 1638))      # 2-way k above 128
    ops.check_decode_limits(8, 4, (32, 32, 32, 32), ops.Budget(16390, 4096, 512))
    ops.check_decode_limits(8, 4, (256, 256), ops.Budget(6554, 100000, 6554))  # 2-way at 1M
    ops.check_decode_limits(8, 4, (362, 362), ops.Budget(2621, 41943, 5243))   # 2-way at 2M, budget 0.02
    ops.check_decode_limits(8, 4, (512, 512), ops.Budget(5243, 83886, 10486))  # 2-way at 4M, budget 0.02
    ops.check_decode_limits(8, 4, (16, 16, 16, 16), ops.Budget(6554, 100000, 2000), online=True)   # 4-way 1M, async
    with pytest.raises(IMIError, match="rank"):
        ops.check_decode_limits(8, 4, (128, 128), ops.Budget(9000, 90000, 9000))  # K' above the ranking capacity
    with pytest.raises(IMIError, match="k"):
        ops.check_decode_limits(8, 4, (513, 64), ops.Budget(410, 13097, 1638))    # 2-way k above 512
