"""IVF indexing (subspace_parts = 0) on the GPU against the CPU oracle.

Reference: kmeans_core.cpp:503-595 (KmeansExecutorIVF: one k-means over the
full 128 dims per head, kmeans++ with seed 42), reorganize_core.cpp:178-231
(build_compact_reorg_input_ivf: compact ids = ranks of the used labels), and
the decode path shared with the IMI modes (compute_impl.cu:62-103 over the
merged centroid, which for IVF is the centroid itself; retrieval.py:295-303;
wave_buffer_cpu_hotcold.cpp:303-371).

Bit-exact: E-step labels and distances, full Lloyd runs (first-k and
kmeans++ initialisation (one launch per pick), more than 256
empty clusters re-seeded in one iteration), cell order, CSR, permutation,
selected cells and row totals.  Attention within 2e-2 abs / 1e-2 rel.
"""
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


def _kv(H, T, seed=0, integer=False):
    from adaptiveimi_amd import synthetic

    if integer:
        return synthetic.integer_kv(H, T, seed=seed)
    return synthetic.make_kv(H, T, seed=seed)


@pytest.mark.parametrize("T,k,integer", [(1500, 100, False), (1200, 700, False), (1000, 300, True),
                                           (6000, 4096, False), (5000, 4096, True)])   # the 4096-cluster limit
def test_ivf_assign_bit_exact(ops, oracle, T, k, integer):
    """E-step over 128 dims with the centroids streamed through LDS in tiles
    (kmeans_core.cpp:222-242)."""
    note(f"[ivf assign] T={T} k={k} integer={integer}")
    H = 3
    keys, _ = _kv(H, T, seed=T, integer=integer)
    rng = np.random.default_rng(k)
    cent = rng.standard_normal((H, 1, k, 128)).astype(np.float32) * 2
    if integer:
        cent = np.round(cent).astype(np.float32)
        cent[:, :, k // 2:] = cent[:, :, : k - k // 2]   # duplicated centroids: exact ties, lowest index wins
    labels, mind = ops.kmeans_assign(keys.to(DEV), torch.from_numpy(cent).to(DEV), [k])
    labels, mind = labels.cpu().numpy(), mind.cpu().numpy()
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        ref, rmind, _ = oracle.estep(np.ascontiguousarray(kf[h]), cent[h, 0])
        assert np.array_equal(labels[h, 0], ref), h
        assert np.array_equal(mind[h, 0], rmind), h


@pytest.mark.parametrize("T,k,iters,init,dup", [
    (3000, 200, 4, "first", 0),
    (2500, 600, 3, "first", 0),
    (2000, 900, 2, "first", 700),     # 699 identical first rows: > 256 clusters re-seeded in iteration 0
    (3000, 300, 2, "kmeans++", 0),    # 300 picks
    (1800, 520, 2, "kmeans++", 0),    # 520 picks
    (6000, 4096, 2, "first", 0),      # the 4096-cluster limit (kIvfMaxK): 64 LDS tiles, 16 draw batches
])
def test_ivf_kmeans_bit_exact(ops, oracle, T, k, iters, init, dup):
    """KmeansExecutorIVF (kmeans_core.cpp:503-595): labels and centroids equal
    the oracle's run with threads_per_phase = 1."""
    note(f"[ivf kmeans] T={T} k={k} iters={iters} init={init} dup={dup}")
    H = 2
    keys, _ = _kv(H, T, seed=11 + T)
    if dup:
        keys[:, 1:dup] = keys[:, :1]
    cent, labels, it = ops.kmeans(keys.to(DEV), [k], iters, init=init)
    cent, labels = cent.cpu().numpy(), labels.cpu().numpy()
    assert cent.shape == (H, 1, k, 128)
    assert (it.cpu().numpy() == iters).all()
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        labs, cents, _ = oracle.kmeans_head(kf[h], [k], iters, init=init)
        assert np.array_equal(labels[h, 0], labs[0]), h
        assert np.array_equal(cent[h, 0], cents[0]), h
    if dup:   # the case really re-seeds beyond the first 256 draws
        lab0, _, _ = oracle.estep(np.ascontiguousarray(kf[0]), np.ascontiguousarray(kf[0][:k]))
        assert k - len(np.unique(lab0)) > 256


def _ivf_index(ops, H, T, k, seed, iters=3):
    keys, values = _kv(H, T, seed=seed)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, [k], iters)
    out = ops.build_index(kd, vd, cent, labels, [k], n_centroids=k + 1)
    out["labels"] = labels
    return keys, values, cent, out


@pytest.mark.parametrize("T,k", [(5000, 400), (9000, 3000)])
def test_ivf_build_index_bit_exact(ops, oracle, T, k):
    """build_compact_reorg_input_ivf (reorganize_core.cpp:178-231) and the
    stable permutation (234-311)."""
    note(f"[ivf index] T={T} k={k}")
    H = 3
    keys, values, cent, out = _ivf_index(ops, H, T, k, T + 3)
    lab = out["labels"].cpu().numpy()
    centn = cent.cpu().numpy()
    kb, vb = bits(keys), bits(values)
    for h in range(H):
        r = oracle.compact_reorg([lab[h, 0]], [k])
        assert np.array_equal(out["perm"][h].cpu().numpy(), r["perm"]), h
        na = int(out["n_active"][h])
        assert na == r["n_active"] == len(np.unique(lab[h, 0]))
        assert np.array_equal(out["compact_gid"][h, :na].cpu().numpy(), r["gids"])
        assert np.array_equal(out["compact_offset"][h, : na + 1].cpu().numpy(), r["offsets"])
        assert np.array_equal(out["compact_centroids"][h, :na].cpu().numpy(), centn[h, 0][r["gids"]])
        assert np.array_equal(bits(out["list_keys"][h]), kb[h][r["perm"]])
        assert np.array_equal(bits(out["list_values"][h]), vb[h][r["perm"]])
        cnt = out["cell_count"][h].cpu().numpy()
        assert np.array_equal(np.flatnonzero(cnt), r["gids"])


@pytest.mark.parametrize("T,k,budget,G,seed", [
    (20000, 1250, 0.1, 4, 0),     # adaptive IVF k = round(T / 16)
    (16384, 1024, 0.2, 8, 1),     # the largest T the reference's IVF metadata holds (k <= 1024)
    (40000, 4000, 0.05, 4, 2),    # near the IVF cluster limit
])
def test_ivf_select_bit_exact(ops, oracle, T, k, budget, G, seed):
    note(f"[ivf select] T={T} k={k} budget={budget} G={G}")
    H = 4
    keys, _, cent, out = _ivf_index(ops, H, T, k, 400 + seed)
    from adaptiveimi_amd import synthetic

    sz = oracle.sizing(T, budget, subspace_parts=0, k_override=[k])
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    qs = synthetic.make_queries(keys, G, seed=seed, n_queries=2)
    sizes = out["compact_size"].cpu().numpy()
    mask = out["compact_mask"].cpu().numpy()
    gids = out["compact_gid"].cpu().numpy()
    merged = out["compact_centroids"].cpu().numpy()
    coff = out["compact_offset"].cpu().numpy()
    for qi in range(qs.shape[0]):
        q = qs[qi]
        sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], [k], bud)
        sc = oracle.scores(bits(q), merged)
        rs, rm, rtok = oracle.select(sc, sizes, mask, bud.nprobe, bud.max_tokens, bud.buffer_pages)
        m = sel["n_selected"].cpu().numpy()
        assert np.array_equal(m, rm), (qi, m, rm)
        cells = sel["sel_cell"].cpu().numpy()
        offs = sel["sel_offset"].cpu().numpy()
        for h in range(H):
            assert np.array_equal(cells[h, : m[h]], gids[h][rs[h, : rm[h]]]), (qi, h)
            assert np.array_equal(offs[h, : m[h]], coff[h][rs[h, : rm[h]]]), (qi, h)
        assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)


@pytest.mark.parametrize("T,k,G,static_len,tiles", [(16000, 1000, 4, 96, False), (12000, 750, 8, 0, True)])
def test_ivf_decode_step_matches_oracle(ops, oracle, T, k, G, static_len, tiles):
    note(f"[ivf decode] T={T} k={k} G={G} static={static_len} tiles={tiles}")
    H = 8
    keys, values, cent, out = _ivf_index(ops, H, T, k, 500 + G)
    from adaptiveimi_amd import synthetic

    sk, sv = synthetic.make_kv(H, max(static_len, 1) + 8, seed=78)
    sz = oracle.sizing(T, 0.1, subspace_parts=0, k_override=[k])
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], 12 if tiles else sz["buffer_pages"], tile_mode=tiles)
    plan = ops.DecodePlan(cent, out["cell_count"], out["cell_offset"], [k], bud, out["list_keys"],
                          out["list_values"], sk.to(DEV), sv.to(DEV), G)
    plan.set_static_len(static_len)
    q = synthetic.make_queries(keys, G, seed=6)[0]
    plan.query.copy_(q.to(DEV))
    res = plan.step().clone()
    torch.cuda.synchronize()
    heads = []
    for h in range(H):
        na = int(out["n_active"][h])
        heads.append(dict(n_active=na, offsets=out["compact_offset"][h, : na + 1].cpu().numpy(),
                          merged=out["compact_centroids"][h, :na].cpu().numpy(),
                          list_keys=bits(out["list_keys"][h]), list_values=bits(out["list_values"][h])))
    ref, rs, rm, rrows = oracle.decode_step(bits(q), heads, bits(sk), bits(sv), static_len, sz["n_centroids"],
                                            bud.nprobe, bud.max_tokens, bud.buffer_pages, tile_mode=tiles)
    sel = plan.selection
    assert np.array_equal(sel["n_selected"].cpu().numpy(), rm)
    gids = out["compact_gid"].cpu().numpy()
    cells = sel["sel_cell"].cpu().numpy()
    nrows = sel["n_rows"].cpu().numpy()
    for h in range(H):
        assert np.array_equal(cells[h, : rm[h]], gids[h][rs[h, : rm[h]]]), h
        assert nrows[h] == len(rrows[h]), h
    got = res.float().cpu().numpy().reshape(ref.shape)
    err = np.abs(got - ref)
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), float(err.max())
