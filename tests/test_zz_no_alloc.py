"""imi_decode_step_noalloc (workspace in the library's static device array)
against imi_decode_step (caller workspace), through the C ABI: identical
selection and output bits, on calls in a row of decreasing size and changing
shape (2-way, then 4-way, then a smaller 2-way), so that each call starts from
what the previous one left in the shared array."""
import ctypes

import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")]

DEV = "cuda:0"


def _plan(ops, H, T, ks, G, seed, static_len):
    from adaptiveimi_amd import synthetic
    from adaptiveimi_amd.sizing import decode_sizing

    keys, values = synthetic.make_kv(H, T, seed=seed)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 4)
    ncells = int(np.prod(ks))
    idx = ops.build_index(kd, vd, cent, labels, list(ks), compact=True, merged=False,
                          n_centroids=min(T, ncells) + 1)
    sz = decode_sizing(T, 0.1, subspace_parts=len(ks), k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    sk, sv = synthetic.make_kv(H, static_len + 8, seed=seed + 1)
    plan = ops.DecodePlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, idx["list_keys"],
                          idx["list_values"], sk.to(DEV), sv.to(DEV), G,
                          compact=idx if len(ks) == 4 else None)
    plan.set_static_len(static_len)
    q = synthetic.make_queries(keys, G, seed=seed + 2)[0]
    plan.query.copy_(q.to(DEV))
    return plan, (idx, cent, sk, sv)


def _both(ops, plan):
    """The same step through imi_decode_step and imi_decode_step_noalloc;
    the selection outputs of the no-alloc call go to caller buffers."""
    from adaptiveimi_amd import _lib

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    ref_out = plan.step().clone()
    ref_sel = {k: v.clone() for k, v in plan.selection.items()}
    H, cap = plan.H, plan.sel_cap
    outs = {name: torch.full(shape, -7, dtype=torch.int32, device=DEV)
            for name, shape in (("sel_cell", (H, cap)), ("sel_offset", (H, cap)), ("sel_count", (H, cap)),
                                ("sel_prefix", (H, cap + 1)), ("n_selected", (H,)), ("n_rows", (H,)))}
    out = torch.full_like(ref_out, 0)
    a = plan.args
    saved = (a.attn.out, a.attn.workspace, a.attn.workspace_bytes)
    a.sel.sel_cell, a.sel.sel_offset = outs["sel_cell"].data_ptr(), outs["sel_offset"].data_ptr()
    a.sel.sel_count, a.sel.sel_prefix = outs["sel_count"].data_ptr(), outs["sel_prefix"].data_ptr()
    a.sel.n_selected, a.sel.n_rows = outs["n_selected"].data_ptr(), outs["n_rows"].data_ptr()
    a.attn.out = out.data_ptr()
    a.attn.workspace, a.attn.workspace_bytes = None, 0   # ignored by the no-alloc entry point
    a.phases = 3
    try:
        _lib.check(L.imi_decode_step_noalloc(ctypes.byref(a), stream), "imi_decode_step_noalloc")
        torch.cuda.synchronize()
    finally:
        a.sel.sel_cell = a.sel.sel_offset = a.sel.sel_count = a.sel.sel_prefix = None
        a.sel.n_selected = a.sel.n_rows = None
        a.attn.out, a.attn.workspace, a.attn.workspace_bytes = saved
    n_sel = ref_sel["n_selected"].cpu().numpy()
    assert np.array_equal(outs["n_selected"].cpu().numpy(), n_sel)
    assert np.array_equal(outs["n_rows"].cpu().numpy(), ref_sel["n_rows"].cpu().numpy())
    for h in range(H):
        m = int(n_sel[h])
        for name in ("sel_cell", "sel_offset", "sel_count"):
            assert np.array_equal(outs[name][h, :m].cpu().numpy(), ref_sel[name][h, :m].cpu().numpy()), name
        assert np.array_equal(outs["sel_prefix"][h, :m + 1].cpu().numpy(),
                              ref_sel["sel_prefix"][h, :m + 1].cpu().numpy())
    assert torch.equal(out.view(torch.int16), ref_out.view(torch.int16))
    return n_sel


def test_noalloc_matches_decode_step_on_calls_of_decreasing_size():
    from adaptiveimi_amd import ops

    cases = [(8, 24000, (32, 32), 4, 96), (8, 9000, (6, 6, 6, 6), 8, 40), (4, 3000, (16, 16), 4, 0)]
    for H, T, ks, G, static_len in cases:
        print(f"[noalloc] H={H} T={T} ks={ks} G={G} static={static_len}", flush=True)
        plan, keep = _plan(ops, H, T, ks, G, seed=T, static_len=static_len)
        n_sel = _both(ops, plan)
        assert n_sel.min() > 0
        _both(ops, plan)   # a second call of the same shape sees what the first left behind
        del plan, keep
