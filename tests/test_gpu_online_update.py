"""GPU parity of the online index maintenance (the reference's async centroid
update and delta append, cache_hub/adaptive_imi/async_update.py) against
oracle.OnlineUpdateOracle / oracle.decode_step_online, through the C ABI.

Bit-exact: batch cluster ids, delta counts and sums, ring entries, replaced
centroids and counts, override slots, the selection over replaced centroids
and the appended delta rows.  Attention: within 2e-2 abs + 1e-2 rel."""
import numpy as np
import pytest
import torch

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")]

DEV = "cuda:0"


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def note(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def ops():
    from adaptiveimi_amd import ops as o

    return o


def _built(ops, H, T, ks, seed):
    """Index of synthetic keys with the compact metadata the update needs."""
    from adaptiveimi_amd import synthetic

    keys, values = synthetic.make_kv(H, T, seed=seed)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 3)
    ncells = int(np.prod(ks))
    n_c = min(T, ncells) + 1 if len(ks) == 4 else ncells + 1
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=n_c, compact=True, merged=True)
    return keys, values, cent, out, ncells


def _state(ops, oracle, out, ks, ncells, threshold, ring_cap):
    """The GPU state and its oracle twin, padding id = the reference's
    n_centroids - 1 (k^2 for 2-way, k^4 for 4-way)."""
    four = len(ks) == 4
    padding_id = ncells
    upd = ops.OnlineUpdate(out["compact_centroids"], out["compact_size"], out["compact_gid"], out["n_active"],
                           padding_id, threshold, ring_cap,
                           n_index=out["compact_gid"].shape[1] if four else ncells, index_by_gid=not four)
    orc = oracle.OnlineUpdateOracle(out["compact_centroids"].cpu().numpy(), out["compact_size"].cpu().numpy(),
                                    padding_id, threshold, ring_cap)
    return upd, orc


def _decode_keys(keys, H, n, seed):
    """Decode keys that revisit a few prompt keys (so that cells reach the
    threshold), as a steady zone [H, n, D] bf16."""
    g = torch.Generator().manual_seed(seed)
    picks = torch.randint(0, keys.shape[1], (H, 5), generator=g)
    idx = picks[:, torch.randint(0, 5, (n,), generator=g)]
    return torch.stack([keys[h, idx[h]] for h in range(H)]).contiguous()


def _compare_state(upd, orc, out, four, ncells):
    H = upd.H
    assert np.array_equal(upd.ring_id.cpu().numpy(), orc.ring_id), "ring cluster ids differ"
    assert np.array_equal(upd.ring_row.cpu().numpy(), orc.ring_row)
    assert np.array_equal(upd.ring_pos.cpu().numpy(), orc.pos) and np.array_equal(upd.ring_n.cpu().numpy(), orc.n)
    assert np.array_equal(upd.delta_counts.cpu().numpy(), orc.dc)
    assert np.array_equal(upd.delta_sums.cpu().numpy(), orc.ds), "delta sums differ"
    assert np.array_equal(upd.shadow.cpu().numpy(), orc.shadow), "replaced centroids differ"
    assert np.array_equal(upd.centroid_counts.cpu().numpy(), orc.cc)
    gid = out["compact_gid"].cpu().numpy()
    na = out["n_active"].cpu().numpy()
    codes = upd.ring_cell.cpu().numpy()
    un = upd.upd_n.cpu().numpy()
    urow = upd.upd_row.cpu().numpy()
    uslot = upd.upd_slot.cpu().numpy()
    for h in range(H):
        for p in range(int(orc.n[h])):
            c = int(orc.ring_id[h, p])
            want = gid[h, c] if c < na[h] else (-1 if c == ncells else -2)
            assert codes[h, p] == want
        rep = [c for c in orc.replaced[h] if c < na[h]]
        assert list(urow[h, : un[h]]) == rep, f"head {h}: override slots differ"
        for s_, c in enumerate(rep):
            assert uslot[h, c if four else gid[h, c]] == s_
        assert (uslot[h] >= 0).sum() == len(rep)


@pytest.mark.parametrize("ks", [(32, 32), (6, 6, 6, 6), (8, 8, 8, 8), (300,)])   # (8,8,8,8): power-of-two digits; (300,): IVF
def test_update_kernels_match_oracle(ops, oracle, ks):
    note(f"[online] update kernels ks={ks}")
    H, T, B = 8, 5000, 8
    keys, _, _, out, ncells = _built(ops, H, T, ks, 61)
    upd, orc = _state(ops, oracle, out, ks, ncells, threshold=3, ring_cap=40)
    steady = _decode_keys(keys, H, 7 * B, seed=5)
    sd = steady.to(DEV)
    for b in range(7):
        rows = list(range(b * B, (b + 1) * B))
        upd.assign(sd, rows[0], B)
        orc.assign(bits(steady[:, rows[0]:rows[0] + B]), rows)
        torch.cuda.synchronize()
        _compare_state(upd, orc, out, len(ks) == 4, ncells)
        upd.refresh(B)
        orc.refresh()
        torch.cuda.synchronize()
        _compare_state(upd, orc, out, len(ks) == 4, ncells)
    assert sum(len(r) for r in orc.replaced) > 0, "no centroid reached the threshold"
    assert int(orc.n.min()) == 40   # the ring wrapped


def test_update_zero_rows_and_padding_code(ops, oracle):
    """Keys with negative similarity to every occupied row go to the first zero
    row: the padding id (match code -1) when it is the first zero row, another
    empty slot (-2) otherwise; a zero row that reaches the threshold is
    replaced like any other but gets no override slot."""
    note("[online] zero rows")
    H, n_rows, D = 2, 10, 128
    cent = torch.zeros((H, n_rows, D), dtype=torch.float32)
    n_active = torch.tensor([9, 7], dtype=torch.int32)
    for h in range(H):
        cent[h, : int(n_active[h]), 0] = torch.arange(1, int(n_active[h]) + 1, dtype=torch.float32)
        cent[h, : int(n_active[h]), 1:] = 0.25
    sizes = torch.zeros((H, n_rows), dtype=torch.int32)
    for h in range(H):
        sizes[h, : int(n_active[h])] = 5
    gid = torch.arange(n_rows, dtype=torch.int32).repeat(H, 1) * 3 + 1
    upd = ops.OnlineUpdate(cent.to(DEV), sizes.to(DEV), gid.to(DEV), n_active.to(DEV), 9, 2, 8, n_index=40,
                           index_by_gid=True)
    orc = oracle.OnlineUpdateOracle(cent.numpy(), sizes.numpy(), 9, 2, 8)
    steady = torch.zeros((H, 4, D))
    steady[:, 0, 0] = -1.0      # negative against every occupied row
    steady[:, 1, 0] = -2.0
    steady[:, 2, 0] = 3.0       # the largest occupied row
    steady[:, 3, 0] = -1.5
    steady = steady.to(torch.bfloat16)
    upd.assign(steady.to(DEV), 0, 4)
    orc.assign(bits(steady), [0, 1, 2, 3])
    torch.cuda.synchronize()
    ids = upd.ring_id.cpu().numpy()
    assert list(ids[0, :4]) == [9, 9, 8, 9] and list(ids[1, :4]) == [7, 7, 6, 7]
    assert list(upd.ring_cell.cpu().numpy()[0, :4]) == [-1, -1, 25, -1]
    assert list(upd.ring_cell.cpu().numpy()[1, :4]) == [-2, -2, 19, -2]
    upd.refresh(4)
    orc.refresh()
    torch.cuda.synchronize()
    assert np.array_equal(upd.shadow.cpu().numpy(), orc.shadow)
    assert np.array_equal(upd.centroid_counts.cpu().numpy(), orc.cc)
    assert upd.shadow[0, 9, 0].item() == pytest.approx(-1.5) and upd.upd_n.cpu().tolist() == [0, 0]


def _select_oracle(oracle, orc, q, out, sz, bud, exec_rows, ncells):
    """Oracle selection over the current shadow: (cells in rank order as
    global ids, m, rows, delta rows) per head."""
    sizes = out["compact_size"].cpu().numpy()
    mask = out["compact_mask"].cpu().numpy()
    gid = out["compact_gid"].cpu().numpy()
    sc = oracle.scores(bits(q), orc.shadow)
    rs, rm, rtok = oracle.select(sc, sizes, mask, bud.nprobe, bud.max_tokens, bud.buffer_pages)
    big = np.iinfo(np.int32).max // 2
    ts, tm, _ = oracle.select(sc, sizes, mask, bud.nprobe, bud.max_tokens, big)
    dr = [orc.delta_rows(h, ts[h, : tm[h]], bud.nprobe, exec_rows, int(rtok[h])) for h in range(q.shape[0])]
    cells = [gid[h][rs[h, : rm[h]]] for h in range(q.shape[0])]
    return cells, rm, rtok, dr


@pytest.mark.parametrize("ks,T", [((32, 32), 6000), ((128, 128), 6000), ((6, 6, 6, 6), 6000), ((8, 8, 8, 8), 6000),
                                  # the 1M 4-way config's sizing (adaptive k 16, budget 0.1): nprobe 6554, all of it
                                  # ranked for the delta match; 2-way past the one-kernel selection (k 181)
                                  ((16, 16, 16, 16), 120000), ((181, 181), 60000),
                                  ((375,), 6000)])   # IVF
def test_select_with_replaced_centroids_and_delta(ops, oracle, ks, T):
    from adaptiveimi_amd import synthetic

    note(f"[online] selection ks={ks} T={T}")
    H, B, G = 8, 8, 4
    keys, _, cent, out, ncells = _built(ops, H, T, ks, 71)
    upd, orc = _state(ops, oracle, out, ks, ncells, threshold=2, ring_cap=64)
    steady = _decode_keys(keys, H, 6 * B, seed=9)
    sd = steady.to(DEV)
    for b in range(6):
        upd.assign(sd, b * B, B)
        orc.assign(bits(steady[:, b * B:(b + 1) * B]), list(range(b * B, (b + 1) * B)))
        upd.refresh(B)
        orc.refresh()
    sz = oracle.sizing(T, 0.1, subspace_parts=len(ks), k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    if ks == (16, 16, 16, 16):
        assert bud.nprobe == 6554
    compact = out if len(ks) == 4 else None
    # queries aimed at the decode keys (so replaced cells rank high) and plain ones
    qs = [(steady[:, :G].float() * 2).to(torch.bfloat16), synthetic.make_queries(keys, G, seed=4)[0]]
    hit_replaced = 0
    for qi, q in enumerate(qs):
        for exec_rows in (10 ** 6, None):
            base = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud, compact=compact)
            rows_sel = base["n_rows"].cpu().numpy()
            er = exec_rows if exec_rows is not None else int(rows_sel.min()) + 5   # truncates the delta rows
            sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud, compact=compact,
                             update=upd, exec_rows=er)
            cells, rm, rtok, dr = _select_oracle(oracle, orc, q, out, sz, bud, er, ncells)
            m = sel["n_selected"].cpu().numpy()
            assert np.array_equal(m, rm), (qi, er)
            got = sel["sel_cell"].cpu().numpy()
            nd = sel["n_delta"].cpu().numpy()
            drow = sel["delta_rows"].cpu().numpy()
            for h in range(H):
                assert np.array_equal(got[h, : m[h]], cells[h]), (qi, h)
                assert list(drow[h, : nd[h]]) == dr[h], (qi, h, er)
            assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)
            gid = out["compact_gid"].cpu().numpy()
            for h in range(H):
                rep = set(gid[h][orc.replaced[h]]) if orc.replaced[h] else set()
                hit_replaced += len(rep & set(cells[h].tolist()))
    assert hit_replaced > 0, "no replaced centroid was selected: the test covers nothing"


def _pad_ring(upd, orc, ncells, seed, per_head=6):
    """Turn a few valid ring entries of every head into padding entries (the
    padding id, match code -1), on the GPU state and its oracle twin."""
    rng = np.random.default_rng(seed)
    torch.cuda.synchronize()
    rc = upd.ring_cell.cpu().numpy()
    for h in range(rc.shape[0]):
        n = int(orc.n[h])
        for p in rng.choice(n, min(per_head, n), replace=False):
            orc.ring_id[h, p] = ncells
            rc[h, p] = -1
    upd.ring_cell.copy_(torch.from_numpy(rc).to(DEV))


@pytest.mark.parametrize("ks,T", [((32, 32), 6000), ((181, 181), 60000), ((8, 8, 8, 8), 6000), ((375,), 6000)])
def test_select_tile_mode_with_delta(ops, oracle, ks, T):
    """Tile mode with the delta append (retrieval.py:480-509): per tile, the
    ring entries of the tile's cells and -- where the head's row of the tile
    is padded -- the padding entries, each tile's list cut at the buffer rows
    its cells leave; checked against the oracle's literal tile builder and
    per-tile append, with page budgets that make several tiles."""
    from adaptiveimi_amd import synthetic

    note(f"[online] tile-mode delta ks={ks} T={T}")
    H, B, G, cap = 8, 8, 4, 64
    keys, _, cent, out, ncells = _built(ops, H, T, ks, 71)
    upd, orc = _state(ops, oracle, out, ks, ncells, threshold=2, ring_cap=cap)
    steady = _decode_keys(keys, H, 6 * B, seed=9)
    sd = steady.to(DEV)
    for b in range(6):
        upd.assign(sd, b * B, B)
        orc.assign(bits(steady[:, b * B:(b + 1) * B]), list(range(b * B, (b + 1) * B)))
        upd.refresh(B)
        orc.refresh()
    _pad_ring(upd, orc, ncells, seed=3)
    sizes = out["compact_size"].cpu().numpy()
    mask = out["compact_mask"].cpu().numpy()
    gid = out["compact_gid"].cpu().numpy()
    sz = oracle.sizing(T, 0.1, subspace_parts=len(ks), k_override=ks)
    compact = out if len(ks) == 4 else None
    qs = [(steady[:, :G].float() * 2).to(torch.bfloat16), synthetic.make_queries(keys, G, seed=4)[0]]
    big = np.iinfo(np.int32).max // 2
    several = 0
    for bp in (max(6, sz["buffer_pages"] // 6), sz["buffer_pages"]):
        bud = ops.Budget(sz["nprobe"], sz["max_tokens"], bp, tile_mode=True)
        for qi, q in enumerate(qs):
            sc = oracle.scores(bits(q), orc.shadow)
            rs, rm, rtok = oracle.select_tiles(sc, sizes, mask, bud.nprobe, bud.max_tokens, bp)
            st, mt, _ = oracle.select(sc, sizes, mask, bud.nprobe, bud.max_tokens, big)
            tiles = oracle.build_cluster_tiles(st, mt, sizes, bp, bud.page_size, ncells)
            several += len(tiles) > 1
            for er in (10 ** 6, bp * bud.page_size - 30, bp * bud.page_size // 2):
                sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud, compact=compact,
                                 update=upd, exec_rows=er)
                m = sel["n_selected"].cpu().numpy()
                assert np.array_equal(m, rm), (bp, qi, er)
                got = sel["sel_cell"].cpu().numpy()
                nd = sel["n_delta"].cpu().numpy()
                drow = sel["delta_rows"].cpu().numpy()
                assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)
                for h in range(H):
                    assert np.array_equal(got[h, : m[h]], gid[h][rs[h, : rm[h]]]), (bp, qi, h)
                    want = orc.delta_rows_tiles(h, tiles, er, sizes[h])[:cap]
                    assert list(drow[h, : nd[h]]) == want, (bp, qi, h, er)
    assert several > 0, "no call made more than one tile"


def test_select_many_replaced_centroids(ops, oracle):
    """More than 64 replaced centroids in a head (the selection then scores
    them in several passes of 64): threshold 1 and batches of 64 keys drawn
    over the whole prompt."""
    note("[online] selection with > 64 replaced cells")
    H, T, B, G, ks = 8, 8000, 64, 4, (32, 32)
    keys, _, cent, out, ncells = _built(ops, H, T, ks, 91)
    upd, orc = _state(ops, oracle, out, ks, ncells, threshold=1, ring_cap=256)
    g = torch.Generator().manual_seed(17)
    idx = torch.randint(0, T, (H, 4 * B), generator=g)
    steady = torch.stack([keys[h, idx[h]] for h in range(H)]).contiguous()
    sd = steady.to(DEV)
    for b in range(4):
        upd.assign(sd, b * B, B)
        orc.assign(bits(steady[:, b * B:(b + 1) * B]), list(range(b * B, (b + 1) * B)))
        upd.refresh(B)
        orc.refresh()
    torch.cuda.synchronize()
    assert int(upd.upd_n.min()) > 64 and int(upd.upd_n.max()) > 128
    sz = oracle.sizing(T, 0.1, k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    from adaptiveimi_amd import synthetic

    for q in ((steady[:, :G].float() * 2).to(torch.bfloat16), synthetic.make_queries(keys, G, seed=8)[0]):
        sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud, update=upd,
                         exec_rows=10 ** 6)
        cells, rm, rtok, dr = _select_oracle(oracle, orc, q, out, sz, bud, 10 ** 6, ncells)
        m = sel["n_selected"].cpu().numpy()
        assert np.array_equal(m, rm)
        got = sel["sel_cell"].cpu().numpy()
        nd = sel["n_delta"].cpu().numpy()
        drow = sel["delta_rows"].cpu().numpy()
        for h in range(H):
            assert np.array_equal(got[h, : m[h]], cells[h]), h
            assert list(drow[h, : nd[h]]) == dr[h], h
        assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)


@pytest.mark.parametrize("tile", [False, True])
def test_decode_step_online_matches_oracle(ops, oracle, tile):
    note(f"[online] decode step tile={tile}")
    H, T, B, G, ks = 8, 9000, 8, 4, (32, 32)
    keys, values, cent, out, ncells = _built(ops, H, T, ks, 81)
    upd, orc = _state(ops, oracle, out, ks, ncells, threshold=2, ring_cap=48)
    static_len = 96 + 4 * B
    from adaptiveimi_amd import synthetic

    sk, sv = synthetic.make_kv(H, static_len + 8, seed=13)
    sk[:, 96:96 + 4 * B] = _decode_keys(keys, H, 4 * B, seed=3)
    skd, svd = sk.contiguous().to(DEV), sv.contiguous().to(DEV)
    for b in range(4):
        r0 = 96 + b * B
        upd.assign(skd, r0, B)
        orc.assign(bits(sk[:, r0:r0 + B]), list(range(r0, r0 + B)))
        upd.refresh(B)
        orc.refresh()
    if tile:
        _pad_ring(upd, orc, ncells, seed=4, per_head=3)
    sz = oracle.sizing(T, 0.1, k_override=ks)
    bp = sz["buffer_pages"] // 5 if tile else sz["buffer_pages"]   # tile mode: several tiles
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], bp, tile_mode=tile)
    plan = ops.DecodePlan(cent, out["cell_count"], out["cell_offset"], ks, bud, out["list_keys"],
                          out["list_values"], skd, svd, G, update=upd)
    exec_rows = bud.buffer_pages * bud.page_size + 64
    q = (sk[:, 96:96 + G].float() * 2).to(torch.bfloat16).contiguous()
    res = torch.empty((H * G, 128), dtype=torch.bfloat16, device=DEV)
    plan.run(q.to(DEV), res, static_len, exec_rows=exec_rows)
    torch.cuda.synchronize()
    sizes = out["compact_size"].cpu().numpy()
    offs = np.zeros((H, sizes.shape[1] + 1), np.int64)
    offs[:, 1:] = np.cumsum(sizes, axis=1)
    ref, rs, rm, rows, dr = oracle.decode_step_online(bits(q), sizes, offs, out["compact_mask"].cpu().numpy(),
                                                      bits(out["list_keys"]), bits(out["list_values"]), bits(sk),
                                                      bits(sv), static_len, orc, bud.nprobe, bud.max_tokens,
                                                      bud.buffer_pages, exec_rows, tile_mode=tile)
    sel = plan.selection
    assert np.array_equal(sel["n_selected"].cpu().numpy(), rm)
    nd = sel["n_delta"].cpu().numpy()
    assert max(len(d) for d in dr) <= upd.ring_cap, "the oracle's list would be cut: the case checks less"
    assert [int(x) for x in nd] == [len(d) for d in dr]
    assert sum(len(d) for d in dr) > 0, "no delta row was appended"
    got = res.float().cpu().numpy().reshape(H, G, 128)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), float(err.max())


@pytest.mark.parametrize("ks,steps,batch,thr,ring,host,tiles", [
    ((32, 32), 14, 4, 2, 24, False, False), ((6, 6, 6, 6), 14, 4, 2, 24, False, False),
    ((8, 8, 8, 8), 14, 4, 2, 24, False, False),
    ((32, 32), 50, 16, 3, 40, False, False), ((256,), 14, 4, 2, 24, False, False),   # (256,): IVF
    # the host tier (lists in pinned host memory, GPU block cache) with the update
    # on: the reference's shipped 1M configuration is a 4-way index with async_update
    ((8, 8, 8, 8), 14, 4, 2, 24, True, False), ((32, 32), 50, 16, 3, 40, True, False),
    # tile mode (IMI_MAX_TILES != 0) with the per-tile delta append
    ((32, 32), 14, 4, 2, 24, False, True), ((8, 8, 8, 8), 14, 4, 2, 24, False, True)])
def test_cache_with_async_update_matches_oracle(ops, oracle, monkeypatch, ks, steps, batch, thr, ring, host,
                                                tiles):
    """The drop-in with async_update on, driven like model_hub drives it,
    against a step-by-step oracle replay (update applied at the next step);
    the 50-step cases use the reference's batch of 16 keys over three batches
    with a ring that wraps.  host: the same with runtime_config["host_tier"]."""
    from adaptiveimi_amd import synthetic
    from adaptiveimi_amd.attn_hub.sparse_imi import imi_decode_attn
    from adaptiveimi_amd.cache_hub.adaptive_imi import adpimi_cache

    L, S, H, G, D = 2, 4096, 8, 4, 128
    note(f"[online] drop-in ks={ks} {steps} decode steps host_tier={host}")
    kcfg = {f"k{i + 1}": k for i, k in enumerate(ks)}
    kcfg.update(max_iters=3, early_stop_min_iter=3, init="first")
    monkeypatch.setenv("IMI_MAX_TILES", "4" if tiles else "0")
    cache = adpimi_cache(valid_start=[0], layer_num=L, batch_size=1, max_length=S + steps + 1,
                         num_key_value_heads=H, num_heads=H * G, head_dim=D, dtype=torch.bfloat16,
                         layer_mapping={"0": DEV, "1": DEV}, max_new_length=steps + 1, input_length=S,
                         static_pattern_start=32, static_pattern_end=64, core=4, pages_per_cluster=2,
                         retrieval_budget=0.1, cache_ratio=0.05, buffer_cluster_num=32, prefill_bsz=1, num_gpus=1,
                         model_size=8, subspace_parts=len(ks) if len(ks) > 1 else 0,
                         runtime_config={"kmeans": kcfg, "async_update": {"enabled": True, "batch": batch,
                                                                          "threshold": thr, "delta_tokens": ring},
                                         "host_tier": {"enabled": host}})
    kv = []
    for layer in range(L):
        k, v = synthetic.make_kv(H, S, seed=50 + layer)
        kv.append((k, v))
        cache.prefill_update_kv_cache(None, k.transpose(0, 1).unsqueeze(0).contiguous().to(DEV),
                                      v.transpose(0, 1).unsqueeze(0).contiguous().to(DEV), layer, 0)
    cache.prepare_cache()
    torch.cuda.synchronize()   # the host tier's list copies are done
    ncells = int(np.prod(ks))
    # oracle twins of each layer's index (from the device build, whose parity
    # is tested on its own) and update state
    twins = []
    for layer in range(L):
        lists = cache.host_lists[layer] if host else (cache.list_keys[layer][0], cache.list_values[layer][0])
        if host:
            assert cache.list_keys[layer] is None and not lists[0].is_cuda
        meta = cache.compact_meta[layer]
        sizes = meta["compact_size"].cpu().numpy()
        offs = np.zeros((H, sizes.shape[1] + 1), np.int64)
        offs[:, 1:] = np.cumsum(sizes, axis=1)
        na = meta["n_active"].cpu().numpy()
        mask = (sizes == 0) | (np.arange(sizes.shape[1])[None, :] >= na[:, None])
        orc = oracle.OnlineUpdateOracle(meta["compact_centroids"].cpu().numpy(), sizes, cache.padding_cluster_id,
                                        thr, ring)
        twins.append(dict(sizes=sizes, offs=offs, mask=mask, orc=orc, count=0, pending=None,
                          lk=bits(lists[0]), lv=bits(lists[1])))
    assert cache.padding_cluster_id == ncells
    g = torch.Generator().manual_seed(7)
    appended = 0
    for step in range(1, steps + 1):
        for layer in range(L):
            k, _ = kv[layer]
            tw = twins[layer]
            picks = torch.randint(0, S, (H,), generator=g)
            nk = torch.stack([k[h, picks[h]] for h in range(H)]).reshape(1, 1, H, D)
            nv = torch.randn((1, 1, H, D), generator=g).to(torch.bfloat16)
            row = cache.static_pattern_total
            cache.decode_update_kv_cache(nk.to(DEV), nv.to(DEV), layer)
            # oracle replay of decode_update_kv_cache (async_update.py:77-162)
            tw["count"] += 1
            if tw["count"] == batch:
                if tw["pending"] is not None:
                    tw["orc"].refresh()
                steady_now = bits(cache.steady_zone_keys[layer][0])
                tw["orc"].assign(steady_now[:, row - batch + 1:row + 1], list(range(row - batch + 1, row + 1)))
                tw["pending"], tw["count"] = step, 0
            q = synthetic.make_queries(k, G, seed=100 * step + layer)[0]
            out = imi_decode_attn(q.reshape(1, 1, H * G, D).to(DEV), nk, nv, layer, cache)
            static_len = cache.static_pattern_total + (1 if layer < L - 1 else 0)
            if tw["pending"] is not None and tw["pending"] < step:
                tw["orc"].refresh()
                tw["pending"] = None
            exec_rows = cache.execution_stride - static_len
            ref, _, rm, rrows, dr = oracle.decode_step_online(
                bits(q), tw["sizes"], tw["offs"], tw["mask"], tw["lk"],
                tw["lv"], bits(cache.steady_zone_keys[layer][0]), bits(cache.steady_zone_values[layer][0]),
                static_len, tw["orc"], cache.nprobe, cache.max_retrieval_tokens, cache.buffer_size, exec_rows,
                tile_mode=tiles)
            plan = cache._plans[layer]
            if host:   # the buffer's one-cell selection replaced the ranked one in the workspace
                assert isinstance(plan, ops.HostTierPlan)
                sel = plan.plan.selection
                assert np.array_equal(plan.h_nsel.numpy(), rm), (step, layer)
                assert np.array_equal(sel["n_rows"].cpu().numpy(), [len(r) for r in rrows]), (step, layer)
            else:
                sel = plan.selection
                assert np.array_equal(sel["n_selected"].cpu().numpy(), rm), (step, layer)
            assert [int(x) for x in sel["n_delta"].cpu().numpy()] == [len(d) for d in dr], (step, layer)
            appended += sum(len(d) for d in dr)
            got = out.float().cpu().numpy().reshape(H, G, D)
            err = np.abs(got - ref)
            assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), f"step {step} layer {layer}: {err.max()}"
        if step == steps:
            for layer in range(L):
                upd = cache._updates[layer]
                assert np.array_equal(upd.shadow.cpu().numpy(), twins[layer]["orc"].shadow)
    assert appended > 0
    if host:
        assert all(cache._plans[layer].hits > 0 for layer in range(L))
