"""Host tier on the GPU: lists in pinned host memory, a GPU block cache.

Per step, against the CPU restatement of the reference's cache manager
(oracle/hostcache.py, wave_buffer_cpu_hotcold.cpp:54-372):
  - the execution buffer holds exactly the rows of the missed blocks (from
    the host lists) then of the hit blocks (from the cache), bit for bit;
  - the attention equals the HBM-resident decode step of the same selection
    within 2e-2 abs / 1e-2 rel (same rows, another summation order);
  - after the run, every cached cluster's cache blocks hold its list rows.
"""
import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")]

DEV = "cuda:0"


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.parametrize("T,ks,G,cache_pages,ratio", [(12000, (32, 32), 4, 60, 0.0), (9000, (16, 16), 8, 400, 0.5),
                                                       (9000, (560,), 4, 200, 0.3),   # (560,): IVF
                                                       (12000, (8, 8, 8, 8), 4, 150, 0.0)])   # 4-way: compact cells
def test_host_tier_decode_matches(T, ks, G, cache_pages, ratio):
    from adaptiveimi_amd import ops, synthetic
    from oracle import hostcache as O
    from oracle import oracle as orc

    print(f"[host tier] T={T} ks={ks} G={G} cache_pages={cache_pages}", flush=True)
    H, static_len = 4, 64
    keys, values = synthetic.make_kv(H, T, seed=41)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 3)
    four = len(ks) == 4
    ncells = int(np.prod(ks))
    idx = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=min(T, ncells) + 1 if four else ncells + 1)
    compact = {n: idx[n] for n in ("n_active", "compact_gid", "compact_size", "compact_offset")} if four else None
    sk, sv = synthetic.make_kv(H, static_len + 8, seed=7)
    sk, sv = sk.to(DEV), sv.to(DEV)
    sz = orc.sizing(T, 0.1, subspace_parts=len(ks) if len(ks) > 1 else 0, k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    plan = ops.DecodePlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, idx["list_keys"],
                          idx["list_values"], sk, sv, G, compact=compact)
    # the lists handed over in pinned host memory, as the drop-in cache does
    hk = torch.empty(tuple(idx["list_keys"].shape), dtype=torch.bfloat16, pin_memory=True)
    hv = torch.empty_like(hk, pin_memory=True)
    hk.copy_(idx["list_keys"])
    hv.copy_(idx["list_values"])
    host = ops.HostTierPlan(cent, idx["cell_count"], idx["cell_offset"], ks, bud, hk, hv, sk, sv, G,
                            cache_pages=cache_pages, hot_ratio=ratio, compact=compact)
    assert host.h_keys.data_ptr() == hk.data_ptr()   # used in place
    lk, lv = bits(idx["list_keys"]), bits(idx["list_values"])
    ps = bud.page_size
    if four:   # the manager's cells are the occupied cells by compact id
        na = idx["n_active"].cpu().numpy()
        csz, coff = idx["compact_size"].cpu().numpy(), idx["compact_offset"].cpu().numpy()
        groups = [O.Group(list(csz[h, :na[h]]) + [0] * (host.pad + 1 - na[h]),
                          list(coff[h, :na[h] + 1]) + [coff[h, na[h]]] * (host.pad + 1 - na[h]),
                          cache_pages, ps, bud.buffer_pages, ratio) for h in range(H)]
    else:
        counts = idx["cell_count"].cpu().numpy()
        offs = idx["cell_offset"].cpu().numpy()
        groups = [O.Group(list(counts[h]) + [0], list(offs[h]) + [offs[h][-1]], cache_pages, ps, bud.buffer_pages,
                          ratio) for h in range(H)]
    out_h = torch.empty((H * G, 128), dtype=torch.bfloat16, device=DEV)
    out_r = torch.empty_like(out_h)
    hits = 0
    for step, seed in enumerate([1, 2, 1, 3, 1, 2, 4, 1]):   # repeated queries select cached cells again
        q = synthetic.make_queries(keys, G, seed=seed)[0].to(DEV).contiguous()
        host.step(q, out_h, static_len)
        plan.run(q, out_r, static_len)
        torch.cuda.synchronize()
        ex_k, ex_v = bits(host.exec_keys), bits(host.exec_values)
        for h in range(H):
            ks_h = host.keys[h].tolist()
            own = {b: c for b, c in groups[h].owned_blocks().items()}
            hl, ml = groups[h].access(ks_h)
            rows = [r for (rid, n, _) in ml for r in range(rid, rid + n)]
            for (bid, n, _) in hl:
                cell = own[bid]
                j = groups[h].ids[cell].index(bid)
                start = groups[h].start[cell] + j * ps
                rows += list(range(start, start + n))
            groups[h].update()
            hits += len(hl)
            total = len(rows)
            assert int(host.plan.selection["n_rows"][h]) == total, (step, h)
            assert np.array_equal(ex_k[h, :total], lk[h, rows]), (step, h)
            assert np.array_equal(ex_v[h, :total], lv[h, rows]), (step, h)
        a, b = out_h.float().cpu().numpy(), out_r.float().cpu().numpy()
        assert np.all(np.abs(a - b) <= 2e-2 + 1e-2 * np.abs(b)), (step, float(np.abs(a - b).max()))
    assert hits > 0 and host.hits == hits
    # the cache holds each cached cluster's list rows
    ck, cv = bits(host.cache_keys), bits(host.cache_values)
    for h in range(H):
        for bid, cell in groups[h].owned_blocks().items():
            j = groups[h].ids[cell].index(bid)
            n = groups[h].last[cell] if j + 1 == groups[h].blocks[cell] else ps
            start = groups[h].start[cell] + j * ps
            assert np.array_equal(ck[h, bid * ps:bid * ps + n], lk[h, start:start + n]), (h, bid)
            assert np.array_equal(cv[h, bid * ps:bid * ps + n], lv[h, start:start + n]), (h, bid)
