"""GPU parity of the HIP path against the CPU oracle, through the C ABI.

Bit-exact: assignments (given identical centroids), full Lloyd runs (the GPU
M-step order equals the reference with one thread per subspace run), cell
lists, permutations, scores and selected cell sets.  Attention: within
2e-2 abs / 1e-2 rel of the fp64 oracle (bf16 output, fp32 accumulation)."""
import math

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


# ------------------------------------------------------------- k-means ----

@pytest.mark.parametrize("T,k,parts,integer", [(3000, 64, 2, False), (1000, 16, 2, True), (2049, 32, 4, False),
                                                (777, 7, 2, False),
                                                (1000, 128, 2, False), (1500, 128, 2, True),    # configs[4]: k = 128
                                                (3000, 362, 2, False), (2000, 512, 2, True)])   # 2M / 4M adaptive k
def test_assign_bit_exact(ops, oracle, T, k, parts, integer):
    note(f"[assign] T={T} k={k} parts={parts} integer={integer}")
    H = 4
    keys, _ = _kv(H, T, seed=T, integer=integer)
    rng = np.random.default_rng(T)
    Dp = 128 // parts
    cent = rng.standard_normal((H, parts, k, Dp)).astype(np.float32) * 2
    if integer:
        cent = np.round(cent).astype(np.float32)
        cent[:, :, k // 2:] = cent[:, :, : k - k // 2]  # duplicated centroids: exact ties
    labels, mind = ops.kmeans_assign(keys.to(DEV), torch.from_numpy(cent).to(DEV), [k] * parts)
    labels = labels.cpu().numpy()
    mind = mind.cpu().numpy()
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        for p in range(parts):
            sub = np.ascontiguousarray(kf[h][:, p * Dp:(p + 1) * Dp])
            ref, rmind, _ = oracle.estep(sub, cent[h, p])
            assert np.array_equal(labels[h, p], ref), (h, p)
            assert np.array_equal(mind[h, p], rmind), (h, p)
    # labels only: lone screen candidates skip the exact distance
    lab2, none = ops.kmeans_assign(keys.to(DEV), torch.from_numpy(cent).to(DEV), [k] * parts, with_distance=False)
    assert none is None and np.array_equal(lab2.cpu().numpy(), labels)


@pytest.mark.parametrize("log2_scale", [40, 60, -60, -70])
def test_assign_bit_exact_extreme_magnitudes(ops, oracle, log2_scale):
    """Keys and centroids scaled by 2^s (exact in bf16 and fp32): 2^40 keeps
    the screen's bound finite; 2^60 puts |x|^2 + max |c|^2 past 1e37, where
    every centroid is a candidate; 2^-60 and 2^-70 make the matrix-core
    screen values and the halved |c|^2 subnormal, where the bound's absolute
    term takes over.  Labels and minimum distances equal the oracle's."""
    note(f"[assign-scale] 2^{log2_scale}")
    H, T, k, parts = 2, 2000, 64, 2
    keys, _ = _kv(H, T, seed=31)
    scale = 2.0 ** log2_scale
    keys = (keys.float() * scale).to(torch.bfloat16)
    rng = np.random.default_rng(31)
    Dp = 128 // parts
    cent = (rng.standard_normal((H, parts, k, Dp)) * 2 * scale).astype(np.float32)
    labels, mind = ops.kmeans_assign(keys.to(DEV), torch.from_numpy(cent).to(DEV), [k] * parts)
    labels, mind = labels.cpu().numpy(), mind.cpu().numpy()
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        for p in range(parts):
            sub = np.ascontiguousarray(kf[h][:, p * Dp:(p + 1) * Dp])
            ref, rmind, _ = oracle.estep(sub, cent[h, p])
            assert np.array_equal(labels[h, p], ref), (h, p)
            assert np.array_equal(mind[h, p].view(np.uint32), rmind.view(np.uint32)), (h, p)
    lab2, _ = ops.kmeans_assign(keys.to(DEV), torch.from_numpy(cent).to(DEV), [k] * parts, with_distance=False)
    assert np.array_equal(lab2.cpu().numpy(), labels)


@pytest.mark.parametrize("T,k,iters", [(4096, 64, 10), (2500, 32, 6), (300, 64, 4),
                                       (6000, 362, 3)])   # the 2-way adaptive k at 2M tokens
def test_kmeans_full_run_bit_exact(ops, oracle, T, k, iters):
    """First-k init, no early stop: labels AND centroids equal the oracle's
    Lloyd run with threads_per_phase = 1 (kmeans_core.cpp:190-314)."""
    note(f"[kmeans] T={T} k={k} iters={iters}")
    H, parts = 4, 2
    keys, _ = _kv(H, T, seed=7 + T)
    cent, labels, it = ops.kmeans(keys.to(DEV), [k, k], iters)
    cent, labels = cent.cpu().numpy(), labels.cpu().numpy()
    assert (it.cpu().numpy() == iters).all()
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        labs, cents, _ = oracle.kmeans_head(kf[h], [k, k], iters, init="first", mstep_threads=1)
        for p in range(parts):
            assert np.array_equal(labels[h, p], labs[p]), (h, p)
            assert np.array_equal(cent[h, p], cents[p]), (h, p)


@pytest.mark.parametrize("T,ks,iters", [(3000, (32, 32), 4), (2049, (16, 16, 16, 16), 3), (700, (64, 64), 2),
                                         (2500, (40, 24), 2), (1100, (1, 8), 1)])
def test_kmeans_plusplus_bit_exact(ops, oracle, T, ks, iters):
    """kmeans++ initialisation (kmeans_core.cpp:138-186, seeds 42 + subspace):
    the GPU picks the same rows as the oracle, which runs the reference's
    sequential double sums with std::mt19937_64, so centroids and labels
    after the Lloyd iterations are identical."""
    note(f"[kmeans++] T={T} ks={ks} iters={iters}")
    H = 3
    keys, _ = _kv(H, T, seed=21 + T)
    cent, labels, _ = ops.kmeans(keys.to(DEV), list(ks), iters, init="kmeans++")
    cent, labels = cent.cpu().numpy(), labels.cpu().numpy()
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        labs, cents, _ = oracle.kmeans_head(kf[h], list(ks), iters, init="kmeans++")
        for p in range(len(ks)):
            assert np.array_equal(cent[h, p, :ks[p]], cents[p]), (h, p)
            assert np.array_equal(labels[h, p], labs[p]), (h, p)


@pytest.mark.parametrize("init,log2_scale", [("first", 60), ("first", 62), ("first", -70),
                                              ("kmeans++", 60), ("kmeans++", 62), ("kmeans++", -70)])
def test_kmeans_extreme_magnitudes(ops, oracle, init, log2_scale):
    """Whole Lloyd runs on keys scaled by 2^s: at 2^60 and 2^62 squared
    norms and some distances overflow (the E-step's every-centroid path, the
    kmeans++ sums past the exact-integer test), at 2^-70 the distances are
    subnormal.  Labels and centroids equal the oracle's bit for bit."""
    note(f"[kmeans-scale] init={init} 2^{log2_scale}")
    H, T, k, iters = 2, 1500, 32, 3
    keys, _ = _kv(H, T, seed=41)
    keys = (keys.float() * 2.0 ** log2_scale).to(torch.bfloat16)
    cent, labels, _ = ops.kmeans(keys.to(DEV), [k, k], iters, init=init)
    cent, labels = cent.cpu().numpy(), labels.cpu().numpy()
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        labs, cents, _ = oracle.kmeans_head(kf[h], [k, k], iters, init=init, mstep_threads=1)
        for p in range(2):
            assert np.array_equal(labels[h, p], labs[p]), (h, p)
            assert np.array_equal(cent[h, p, :k].view(np.uint32), np.asarray(cents[p], np.float32).view(np.uint32)), (h, p)


def test_kmeans_plusplus_init_only_with_duplicates(ops, oracle):
    """Initial centroids alone (one Lloyd iteration is compared through its
    labels) on data with many duplicate rows, so min distances of 0 occur and
    picks can repeat."""
    note("[kmeans++] duplicates")
    H, T, k = 2, 1200, 32
    keys, _ = _kv(H, T, seed=5)
    keys[:, 600:] = keys[:, :600]
    cent, labels, _ = ops.kmeans(keys.to(DEV), [k, k], 1, init="kmeans++")
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        labs, cents, _ = oracle.kmeans_head(kf[h], [k, k], 1, init="kmeans++")
        for p in range(2):
            assert np.array_equal(labels.cpu().numpy()[h, p], labs[p]), (h, p)
            assert np.array_equal(cent.cpu().numpy()[h, p], cents[p]), (h, p)


def test_kmeans_plusplus_wide_range_sequential_path(ops, oracle):
    """Min distances spanning more than 53 bits (near-duplicate rows next
    to far outliers): the per-pick exactness test fails and the kernel
    replays the reference's sequential double sums; the picks still match."""
    note("[kmeans++] wide exponent range")
    H, T, k = 1, 2048, 16
    rng = np.random.default_rng(9)
    base = rng.integers(-4, 5, size=(T, 128)).astype(np.float32)
    base[1::2] = base[0::2]
    base[1::2, 0] += 1.0 / 64        # neighbours one small step apart
    base[::97] *= 256.0              # far outliers
    keys = torch.from_numpy(base).to(torch.bfloat16).unsqueeze(0).contiguous()
    cent, labels, _ = ops.kmeans(keys.to(DEV), [k, k], 2, init="kmeans++")
    kf = oracle.bf16_to_f32(bits(keys))
    labs, cents, _ = oracle.kmeans_head(kf[0], [k, k], 2, init="kmeans++")
    for p in range(2):
        assert np.array_equal(cent.cpu().numpy()[0, p], cents[p]), p
        assert np.array_equal(labels.cpu().numpy()[0, p], labs[p]), p


@pytest.mark.parametrize("T,sample,ks", [(24000, 6000, (32, 32)), (20001, 4096, (8, 8, 8, 8)),
                                         (60000, 16384, (128, 128))])   # configs[4]: 2 x 128 centroids
def test_kmeans_sampled_then_assign(ops, oracle, T, sample, ks):
    """The 1M-token build at reduced scale: k-means on every ceil(T/sample)-th
    key, then every key assigned to the final centroids -- bit-exact with the
    oracle's Lloyd run on the same sample and its E-step over all keys."""
    note(f"[kmeans] sampled T={T} sample={sample} ks={ks}")
    H = 2
    keys, _ = _kv(H, T, seed=17)
    cent, labels, _ = ops.kmeans_sampled(keys.to(DEV), list(ks), 4, sample)
    step = -(-T // sample)
    kf = oracle.bf16_to_f32(bits(keys))
    sl = oracle.subspace_slices(128, len(ks))
    for h in range(H):
        rl, rc, _ = oracle.kmeans_head(kf[h, ::step], list(ks), 4)
        for p in range(len(ks)):
            assert np.array_equal(cent[h, p, : ks[p]].cpu().numpy(), rc[p]), (h, p)
            lab, _, _ = oracle.estep(np.ascontiguousarray(kf[h][:, sl[p]]), rc[p])
            assert np.array_equal(labels[h, p].cpu().numpy(), lab), (h, p)


def test_kmeans_empty_cluster_reseed(ops, oracle):
    """Duplicate first rows make clusters empty in iteration 0; the GPU must
    re-seed them from the same mt19937 draws as the reference."""
    note("[kmeans] empty-cluster reseed")
    H, T, k = 2, 1500, 16
    keys, _ = _kv(H, T, seed=3)
    keys[:, 1:k] = keys[:, :1]      # first k rows identical -> k-1 empty clusters
    cent, labels, _ = ops.kmeans(keys.to(DEV), [k, k], 3)
    kf = oracle.bf16_to_f32(bits(keys))
    for h in range(H):
        labs, cents, _ = oracle.kmeans_head(kf[h], [k, k], 3, init="first")
        for p in range(2):
            assert np.array_equal(labels.cpu().numpy()[h, p], labs[p])
            assert np.array_equal(cent.cpu().numpy()[h, p], cents[p])


def _exact_cluster_keys(H, k=4, per=64, seed=0):
    """bf16 keys whose E-step distances and inertia are exact integers in any
    summation order: per 64-dim subspace, k clusters of `per` integer rows
    symmetric around integer centres (a power-of-two size, so the M-step
    mean is the exact centre), the first k rows off-centre members."""
    rng = np.random.default_rng(seed)
    out = np.zeros((H, k * per, 128), np.float32)
    for h in range(H):
        for p in range(2):
            centres = rng.integers(-7, 8, (k, 64)) * 16
            rows = []
            for c in range(k):
                half = rng.integers(-3, 4, (per // 2, 64))
                rows.append(np.concatenate([centres[c] + half, centres[c] - half]))
            x = np.concatenate(rows)
            firsts = np.array([c * per for c in range(k)])
            order = np.concatenate([firsts, np.setdiff1d(np.arange(k * per), firsts)])
            out[h, :, p * 64:(p + 1) * 64] = x[order]
    return torch.from_numpy(out).to(torch.bfloat16)


@pytest.mark.parametrize("min_iter,rel_tol,tol", [(1, 1e-6, 0.0), (2, 0.0, 0.0), (1, 0.9, 0.0), (5, 0.0, 0.0),
                                                  (7, 0.0, 0.0), (1, 0.0, 1e9)])
def test_kmeans_early_stop_matches_oracle(ops, oracle, min_iter, rel_tol, tol):
    """kmeans_core.cpp:244-262 on data whose inertia is exact in any order, so
    the GPU's summation order cannot move the stop: the iteration count, the
    labels and the centroids equal the oracle's.  The E-step skips the
    distances of lone screen candidates in the iterations before
    min_iter - 1, whose inertia no stop test reads (min_iter 5 and 7)."""
    note(f"[kmeans] early stop min_iter={min_iter} rel_tol={rel_tol} tol={tol}")
    H, k = 2, 4
    keys = _exact_cluster_keys(H, k)
    kf = oracle.bf16_to_f32(bits(keys))
    assert np.array_equal(kf, np.round(kf))
    cent, labels, it = ops.kmeans(keys.to(DEV), [k, k], 10, tol=tol, early_stop_min_iter=min_iter,
                                  early_stop_rel_tol=rel_tol)
    for h in range(H):
        labs, cents, iters = oracle.kmeans_head(kf[h], [k, k], 10, tol=tol, early_stop_min_iter=min_iter,
                                                early_stop_rel_tol=rel_tol)
        for p in range(2):
            assert int(it[h, p]) == iters[p], (h, p)
            assert np.array_equal(labels[h, p].cpu().numpy(), labs[p]), (h, p)
            assert np.array_equal(cent[h, p].cpu().numpy(), cents[p]), (h, p)


def test_kmeans_early_stop_semantics(ops, oracle):
    note("[kmeans] early stop")
    H, T, k = 2, 2000, 8
    keys, _ = _kv(H, T, seed=11)
    cent, labels, it = ops.kmeans(keys.to(DEV), [k, k], 30, tol=1e-2, early_stop_min_iter=2,
                                  early_stop_rel_tol=1e-3)
    it = it.cpu().numpy()
    assert (it < 30).all() and (it >= 2).all()
    # consistency: stopped runs hold labels == E-step of the final centroids
    lab2, _ = ops.kmeans_assign(keys.to(DEV), cent, [k, k])
    assert torch.equal(lab2, labels)


def test_mstep_reciprocal_over_cluster_sizes(ops, oracle):
    """The M-step's sum * (1.0f / size) (kmeans_core.cpp:280-290) on the GPU
    for 127 different cluster sizes and one of several thousand: every member
    of cluster c repeats the same row, so the sums are exact in any order
    and the centroids differ from those rows only through the rounding of
    1/size and of the product -- compared bit for bit with the oracle's host
    arithmetic after one Lloyd iteration from the rows themselves."""
    note("[mstep] 1/size over cluster sizes")
    k = 128
    sizes = np.arange(1, k + 1)
    sizes[-1] = 5000
    T = int(sizes.sum())
    rng = np.random.default_rng(12)
    rows = np.zeros((k, 128), np.float32)
    for c in range(k):   # distinct rows far apart (integers, exact in bf16)
        rows[c] = rng.integers(-40, 41, size=128) + 97 * (c % 3)
        rows[c, c % 128] += 200.0
    lab = np.repeat(np.arange(k), sizes)
    rng.shuffle(lab)
    keys = torch.from_numpy(rows[lab]).to(torch.bfloat16).unsqueeze(0).contiguous()
    init = torch.from_numpy(np.stack([rows[:, :64], rows[:, 64:]])[None]).contiguous()
    cent, labels, _ = ops.kmeans(keys.to(DEV), [k, k], 1, init_centroids=init.to(DEV))
    kf = oracle.bf16_to_f32(bits(keys))
    labs, cents, _ = oracle.kmeans_head(kf[0], [k, k], 1, init="given",
                                        init_centroids=[rows[:, :64], rows[:, 64:]])
    for p in range(2):
        assert np.array_equal(labels.cpu().numpy()[0, p], lab), p
        assert np.array_equal(labs[p], lab), p
        assert np.array_equal(cent.cpu().numpy()[0, p], cents[p]), p


# ---------------------------------------------------------- cell index ----

@pytest.mark.parametrize("T,ks", [(5000, (32, 32)), (4096, (64, 64)), (3001, (8, 4, 8, 4)), (20000, (512, 300))])
def test_build_index_bit_exact(ops, oracle, T, ks):
    note(f"[index] T={T} ks={ks}")
    H = 4
    parts = len(ks)
    keys, values = _kv(H, T, seed=T + 1)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 3)
    ncells = int(np.prod(ks))
    n_c = ncells + 1
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=n_c)
    lab = labels.cpu().numpy()
    centn = cent.cpu().numpy()
    kb, vb = bits(keys), bits(values)
    for h in range(H):
        r = oracle.compact_reorg([lab[h, p] for p in range(parts)], ks)
        perm = out["perm"][h].cpu().numpy()
        assert np.array_equal(perm, r["perm"]), h
        na = int(out["n_active"][h])
        assert na == r["n_active"]
        assert np.array_equal(out["compact_gid"][h, :na].cpu().numpy(), r["gids"])
        assert (out["compact_gid"][h, na:].cpu().numpy() == -1).all()
        assert np.array_equal(out["compact_offset"][h, : na + 1].cpu().numpy(), r["offsets"])
        assert (out["compact_offset"][h, na:].cpu().numpy() == T).all()
        assert np.array_equal(out["compact_size"][h, :na].cpu().numpy(), np.diff(r["offsets"]))
        assert out["compact_mask"][h, na:].all() and not out["compact_mask"][h, :na].any()
        merged = oracle.merged_centroids([centn[h, p, : ks[p]] for p in range(parts)], r["gids"], ks)
        assert np.array_equal(out["compact_centroids"][h, :na].cpu().numpy(), merged)
        # CSR over global cells
        cnt = out["cell_count"][h].cpu().numpy()
        off = out["cell_offset"][h].cpu().numpy()
        assert np.array_equal(np.flatnonzero(cnt), r["gids"])
        assert np.array_equal(off[r["gids"]], r["offsets"][:-1]) and off[-1] == T
        assert np.array_equal(bits(out["list_keys"][h]), kb[h][r["perm"]])
        assert np.array_equal(bits(out["list_values"][h]), vb[h][r["perm"]])


def test_build_index_strided_prefill_layout(ops, oracle):
    """Keys straight from the prefill layout [S, H, D] (no transpose copy)."""
    note("[index] strided")
    H, S = 8, 3000
    keys, values = _kv(H, S, seed=5)
    kt = keys.permute(1, 0, 2).contiguous().to(DEV)   # [S, H, D]
    vt = values.permute(1, 0, 2).contiguous().to(DEV)
    lo, hi = 32, S - 64
    kv = kt[lo:hi].transpose(0, 1)                     # [H, T, D] strided view
    vv = vt[lo:hi].transpose(0, 1)
    cent, labels, _ = ops.kmeans(kv, [32, 32], 4)
    cent2, labels2, _ = ops.kmeans(keys[:, lo:hi].contiguous().to(DEV), [32, 32], 4)
    assert torch.equal(cent, cent2) and torch.equal(labels, labels2)
    out = ops.build_index(kv, vv, cent, labels, [32, 32])
    ref = bits(keys[:, lo:hi])
    perm = out["perm"].cpu().numpy()
    for h in range(H):
        assert np.array_equal(bits(out["list_keys"][h]), ref[h][perm[h]])


# -------------------------------------------------------------- decode ----

def _index(ops, H, T, ks, seed, iters=4):
    keys, values = _kv(H, T, seed=seed)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), iters)
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=int(np.prod(ks)) + 1)
    out["labels"] = labels
    return keys, values, cent, out


def test_similarities_bit_exact(ops, oracle):
    note("[scores]")
    H, T, ks = 8, 4000, (32, 32)
    keys, _, cent, out = _index(ops, H, T, ks, 21)
    from adaptiveimi_amd import synthetic

    q = synthetic.make_queries(keys, 4, seed=2)[0]
    n_c = out["compact_centroids"].shape[1]
    s = ops.fused_query_group_similarities(q.to(DEV), out["compact_centroids"], mask=out["compact_mask"])
    ref = oracle.scores(bits(q), out["compact_centroids"].cpu().numpy())
    mask = out["compact_mask"].cpu().numpy()
    ref[mask] = -np.inf
    assert np.array_equal(s.cpu().numpy(), ref)
    assert s.shape == (H, n_c)


@pytest.mark.parametrize("T,ks,budget,G,seed", [
    (32768, (64, 64), 0.1, 4, 0),
    (8000, (32, 32), 0.1, 4, 1),
    (8000, (32, 32), 0.02, 7, 2),
    (20000, (45, 45), 0.05, 8, 3),
    (60000, (128, 128), 0.02, 4, 4),     # configs[4]'s 2 x 128 centroids: 16 cells per thread
    (30000, (100, 90), 0.05, 4, 5),
    (32768, (64, 64), 0.5, 4, 6),        # nprobe = buffer_pages = 2048: the one-kernel ranking capacity
    (60000, (256, 64), 0.05, 4, 7),      # k0 = 256: score + rank kernels
    (100000, (128, 128), 0.2, 4, 8),     # K' = 2500 pages > 2048: score + rank kernels
    (50000, (200, 80), 0.3, 8, 9),       # 16000 cells, K' = 4096 nprobe < 4688 pages
    (120000, (181, 181), 0.1, 4, 10),    # the 2-way adaptive k at 512k: 32761 cells
    (200000, (256, 256), 0.06, 4, 11),   # ... and at 1M: 65536 cells, K' = 1500 pages
    (150000, (128, 128), 0.45, 4, 12),   # K' = 7373 nprobe < 8438 pages: near the ranking capacity
    (300000, (362, 362), 0.02, 4, 13),   # the 2-way adaptive k at 2M tokens: 131044 cells
    (300000, (512, 512), 0.02, 4, 14),   # ... and at 4M: 262144 cells, the k cap
])
def test_select_bit_exact(ops, oracle, T, ks, budget, G, seed):
    note(f"[select] T={T} ks={ks} budget={budget} G={G}")
    H = 8
    keys, _, cent, out = _index(ops, H, T, ks, 100 + seed)
    from adaptiveimi_amd import synthetic

    sz = oracle.sizing(T, budget, k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    qs = synthetic.make_queries(keys, G, seed=seed, n_queries=3)
    n_c = sz["n_centroids"]
    sizes = out["compact_size"].cpu().numpy()
    mask = out["compact_mask"].cpu().numpy()
    gids = out["compact_gid"].cpu().numpy()
    merged = out["compact_centroids"].cpu().numpy()
    for qi in range(qs.shape[0]):
        q = qs[qi]
        sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud)
        sc = oracle.scores(bits(q), merged)
        rs, rm, rtok = oracle.select(sc, sizes, mask, bud.nprobe, bud.max_tokens, bud.buffer_pages)
        m = sel["n_selected"].cpu().numpy()
        assert np.array_equal(m, rm)
        cells = sel["sel_cell"].cpu().numpy()
        for h in range(H):
            assert np.array_equal(cells[h, : m[h]], gids[h][rs[h, : rm[h]]]), (qi, h)
        assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)
        assert n_c == sizes.shape[1]


@pytest.mark.parametrize("T,ks,budget,G,seed", [
    (20000, (8, 8, 8, 8), 0.1, 8, 0),
    (30000, (16, 16, 16, 16), 0.05, 4, 1),
    (12000, (5, 7, 6, 4), 0.2, 7, 2),
    (40000, (8, 8, 8, 8), 0.5, 4, 3),    # nprobe = 2048 < buffer_pages
    (120000, (16, 16, 16, 16), 0.25, 4, 4),   # K' = 3750 pages < nprobe 16384
])
def test_select_4way_bit_exact(ops, oracle, T, ks, budget, G, seed):
    """4-way IMI selection over the occupied cells (the reference scores the
    padded k^4 + 1 compact cells): same cells, rank order and row counts as
    the oracle."""
    note(f"[select4] T={T} ks={ks} budget={budget} G={G}")
    H = 4
    keys, values = _kv(H, T, seed=200 + seed)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 3)
    ncells = int(np.prod(ks))
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=ncells + 1)
    from adaptiveimi_amd import synthetic

    sz = oracle.sizing(T, budget, subspace_parts=4, k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    qs = synthetic.make_queries(keys, G, seed=seed, n_queries=2)
    sizes = out["compact_size"].cpu().numpy()
    mask = out["compact_mask"].cpu().numpy()
    gids = out["compact_gid"].cpu().numpy()
    merged = out["compact_centroids"].cpu().numpy()
    for qi in range(qs.shape[0]):
        q = qs[qi]
        sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud, compact=out)
        sc = oracle.scores(bits(q), merged)
        rs, rm, rtok = oracle.select(sc, sizes, mask, bud.nprobe, bud.max_tokens, bud.buffer_pages)
        m = sel["n_selected"].cpu().numpy()
        assert np.array_equal(m, rm), (qi, m, rm)
        cells = sel["sel_cell"].cpu().numpy()
        offs = sel["sel_offset"].cpu().numpy()
        coff = out["compact_offset"].cpu().numpy()
        for h in range(H):
            assert np.array_equal(cells[h, : m[h]], gids[h][rs[h, : rm[h]]]), (qi, h)
            assert np.array_equal(offs[h, : m[h]], coff[h][rs[h, : rm[h]]]), (qi, h)
        assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)


@pytest.mark.parametrize("qmode", ["zero", "three_dims"])
def test_select_4way_massive_ties(ops, oracle, qmode):
    """Integer data with few distinct scores.  qmode "zero": every occupied
    cell scores 0, so far more than 4096 cells share the threshold bucket and
    the exact radix-select path runs; "three_dims": scores depend on the first
    subspace only, a handful of values each shared by hundreds of cells.  Ties
    go to the lowest cell id either way."""
    note(f"[select4] massive ties {qmode}")
    H, T, ks = 2, 40000, (10, 10, 10, 10)
    keys, values = _kv(H, T, seed=11, integer=True)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 2)
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=10001)
    n_active = out["n_active"].cpu().numpy()
    q = torch.zeros((H, 4, 128), dtype=torch.bfloat16)
    if qmode == "three_dims":
        q[:, :, :3] = 1.0
    else:
        assert n_active.min() > 4096      # the zero query must overflow the candidate buffer
    bud = ops.Budget(3000, 30000, 2000)
    sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud, compact=out)
    sc = oracle.scores(bits(q), out["compact_centroids"].cpu().numpy())
    rs, rm, rtok = oracle.select(sc, out["compact_size"].cpu().numpy(), out["compact_mask"].cpu().numpy(),
                                 3000, 30000, 2000)
    gids = out["compact_gid"].cpu().numpy()
    m = sel["n_selected"].cpu().numpy()
    assert np.array_equal(m, rm)
    for h in range(H):
        assert np.array_equal(sel["sel_cell"].cpu().numpy()[h, : m[h]], gids[h][rs[h, : rm[h]]])
    assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)


def test_select_4way_workspace_reuse_across_shapes(ops, oracle):
    """ops.select shares one 4-way workspace between calls; calls of a
    different head count and compact width must not see each other's state."""
    note("[select4] workspace reuse across shapes")
    from adaptiveimi_amd import synthetic

    for H, T, ks in ((2, 9000, (8, 8, 8, 8)), (8, 12000, (6, 6, 6, 6)), (3, 20000, (10, 10, 10, 10)),
                     (2, 9000, (8, 8, 8, 8))):
        keys, values = _kv(H, T, seed=H + T)
        kd, vd = keys.to(DEV), values.to(DEV)
        cent, labels, _ = ops.kmeans(kd, list(ks), 2)
        ncells = int(np.prod(ks))
        out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=min(T, ncells) + 1)
        bud = ops.Budget(min(200, ncells), 1500, 60)
        q = synthetic.make_queries(keys, 4, seed=3)[0]
        sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud, compact=out)
        sc = oracle.scores(bits(q), out["compact_centroids"].cpu().numpy())
        rs, rm, rtok = oracle.select(sc, out["compact_size"].cpu().numpy(), out["compact_mask"].cpu().numpy(),
                                     bud.nprobe, bud.max_tokens, bud.buffer_pages)
        assert np.array_equal(sel["n_selected"].cpu().numpy(), rm), (H, T, ks)
        gids = out["compact_gid"].cpu().numpy()
        for h in range(H):
            assert np.array_equal(sel["sel_cell"].cpu().numpy()[h, : rm[h]], gids[h][rs[h, : rm[h]]]), (H, h)


@pytest.mark.parametrize("ks,pages", [((32, 32), 3), ((32, 32), 40), ((8, 8, 8, 8), 2)])
def test_select_tile_mode_bit_exact(ops, oracle, ks, pages):
    """Tile mode (IMI_MAX_TILES != 0): the kept cells are not cut by the
    running page total, and a head stops at its first cell that alone needs
    more than buffer_pages pages (retrieval.py:30-112).  Small page budgets
    make such cells common."""
    note(f"[select] tile mode ks={ks} pages={pages}")
    H, T, G = 8, 12000, 4
    keys, values = _kv(H, T, seed=61)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 3)
    ncells = int(np.prod(ks))
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=min(T, ncells) + 1 if len(ks) == 4 else None)
    bud = ops.Budget(min(300, ncells), 2500, pages, tile_mode=True)
    from adaptiveimi_amd import synthetic

    q = synthetic.make_queries(keys, G, seed=8)[0]
    sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud,
                     compact=out if len(ks) == 4 else None)
    sc = oracle.scores(bits(q), out["compact_centroids"].cpu().numpy())
    rs, rm, rtok = oracle.select_tiles(sc, out["compact_size"].cpu().numpy(), out["compact_mask"].cpu().numpy(),
                                       bud.nprobe, bud.max_tokens, bud.buffer_pages)
    gids = out["compact_gid"].cpu().numpy()
    m = sel["n_selected"].cpu().numpy()
    assert np.array_equal(m, rm), (m, rm)
    for h in range(H):
        assert np.array_equal(sel["sel_cell"].cpu().numpy()[h, : m[h]], gids[h][rs[h, : rm[h]]]), h
    assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)
    assert rm.max() > 0


def test_select_ties_integer_data(ops, oracle):
    """Integer keys/queries: many exactly tied scores; order must be by cell id."""
    note("[select] ties")
    H, T, ks = 4, 6000, (16, 16)
    keys, values = _kv(H, T, seed=9, integer=True)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 2)
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=257)
    q = torch.randint(-2, 3, (H, 4, 128), generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    bud = ops.Budget(60, 900, 200)
    sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud)
    sc = oracle.scores(bits(q), out["compact_centroids"].cpu().numpy())
    rs, rm, _ = oracle.select(sc, out["compact_size"].cpu().numpy(), out["compact_mask"].cpu().numpy(), 60, 900, 200)
    gids = out["compact_gid"].cpu().numpy()
    m = sel["n_selected"].cpu().numpy()
    assert np.array_equal(m, rm)
    for h in range(H):
        assert np.array_equal(sel["sel_cell"].cpu().numpy()[h, : m[h]], gids[h][rs[h, : rm[h]]])


def _check_attention(out, ref):
    out = out.float().cpu().numpy().reshape(ref.shape)
    err = np.abs(out - ref)
    assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), float(err.max())


@pytest.mark.parametrize("T,ks,G,static_len,tiles,budget", [
    (32768, (64, 64), 4, 96, False, 0.1), (9000, (32, 32), 7, 0, False, 0.1), (6000, (32, 32), 8, 200, False, 0.1),
    (20000, (32, 32), 4, 96, True, 0.1),
    (100000, (128, 128), 4, 96, False, 0.2),   # score + rank kernels; over 2048 selected cells per head
    (131072 - 96, (64, 64), 4, 97, False, 0.1),   # configs[1], the bench shape: nprobe 410, 1638 pages
    # GQA groups of other model shapes: Qwen2.5-14B / 32B (5), Qwen2-1.5B (6), Llama-3.1-405B (16), and 3
    (12000, (32, 32), 5, 96, False, 0.1), (8000, (32, 32), 6, 33, False, 0.1), (16000, (32, 32), 16, 96, False, 0.1),
    (7000, (32, 32), 3, 0, False, 0.1), (20000, (32, 32), 16, 96, True, 0.1),
])
def test_decode_step_matches_oracle(ops, oracle, T, ks, G, static_len, tiles, budget):
    note(f"[decode] T={T} ks={ks} G={G} static={static_len} tiles={tiles} budget={budget}")
    H = 8
    keys, values, cent, out = _index(ops, H, T, ks, 300 + G)
    from adaptiveimi_amd import synthetic

    sk, sv = synthetic.make_kv(H, max(static_len, 1) + 8, seed=77)
    sz = oracle.sizing(T, budget, k_override=ks)
    # tile mode: a small page budget, so that the tiles (and the oversized-cell stop) matter
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], 12 if tiles else sz["buffer_pages"], tile_mode=tiles)
    plan = ops.DecodePlan(cent, out["cell_count"], out["cell_offset"], ks, bud, out["list_keys"],
                          out["list_values"], sk.to(DEV), sv.to(DEV), G)
    plan.set_static_len(static_len)
    q = synthetic.make_queries(keys, G, seed=5)[0]
    plan.query.copy_(q.to(DEV))
    res = plan.step().clone()
    torch.cuda.synchronize()
    # oracle
    heads = []
    for h in range(H):
        na = int(out["n_active"][h])
        offs = out["compact_offset"][h, : na + 1].cpu().numpy()
        heads.append(dict(n_active=na, offsets=offs, merged=out["compact_centroids"][h, :na].cpu().numpy(),
                          list_keys=bits(out["list_keys"][h]), list_values=bits(out["list_values"][h])))
    ref, rs, rm, rrows = oracle.decode_step(bits(q), heads, bits(sk), bits(sv), static_len, sz["n_centroids"],
                                            bud.nprobe, bud.max_tokens, bud.buffer_pages, tile_mode=tiles)
    sel = plan.selection
    assert np.array_equal(sel["n_selected"].cpu().numpy(), rm)
    # the same cells in the same rank order (compact id -> global cell id) and row totals
    gids = out["compact_gid"].cpu().numpy()
    cells = sel["sel_cell"].cpu().numpy()
    nrows = sel["n_rows"].cpu().numpy()
    for h in range(H):
        assert np.array_equal(cells[h, : rm[h]], gids[h][rs[h, : rm[h]]]), h
        assert nrows[h] == len(rrows[h]), h
    if tiles:   # more rows than one page budget holds
        assert int(sel["n_rows"].max()) > bud.buffer_pages * bud.page_size
    if budget > 0.1:   # the attention prologue stages its selection in more than one round trip
        assert int(sel["n_selected"].max()) > 2048
    _check_attention(res, ref)


@pytest.mark.parametrize("log2_scale", [-40, 4, 12])
def test_decode_step_scaled_queries(ops, oracle, log2_scale):
    """Queries scaled by 2^s: tiny scores (2^-40), a sharp softmax (2^4)
    and one whose logits reach ~1e8 (2^12, a single dominant row per query):
    the selection stays bit-exact and the attention within tolerance."""
    note(f"[decode-scale] 2^{log2_scale}")
    from adaptiveimi_amd import synthetic

    H, T, ks, G, static_len = 4, 12000, (32, 32), 4, 96
    keys, values, cent, out = _index(ops, H, T, ks, 55)
    sk, sv = synthetic.make_kv(H, static_len + 8, seed=78)
    sz = oracle.sizing(T, 0.1, k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    plan = ops.DecodePlan(cent, out["cell_count"], out["cell_offset"], ks, bud, out["list_keys"],
                          out["list_values"], sk.to(DEV), sv.to(DEV), G)
    plan.set_static_len(static_len)
    q = (synthetic.make_queries(keys, G, seed=5)[0].float() * 2.0 ** log2_scale).to(torch.bfloat16)
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
                                            bud.nprobe, bud.max_tokens, bud.buffer_pages)
    sel = plan.selection
    assert np.array_equal(sel["n_selected"].cpu().numpy(), rm)
    gids = out["compact_gid"].cpu().numpy()
    cells = sel["sel_cell"].cpu().numpy()
    for h in range(H):
        assert np.array_equal(cells[h, : rm[h]], gids[h][rs[h, : rm[h]]]), h
    _check_attention(res, ref)


def test_config3_shape_decode_matches_oracle(ops, oracle):
    """configs[3] per sequence: 4-way IMI with 32 centroids per subspace (a
    1,048,576-cell space), 262,048 listed tokens per KV head (over 200k
    occupied cells each), G = 8, the fixed budget of 4096 tokens (nprobe
    16390, 512 pages).  Selection (cells in rank order, row totals) is
    bit-exact with the oracle; attention within the usual tolerance."""
    from adaptiveimi_amd import synthetic

    H, G, ks = 2, 8, (32, 32, 32, 32)
    T = 262144 - 96
    note(f"[config3] H={H} T={T} ks={ks} G={G}")
    keys, values = _kv(H, T, seed=333)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 3)
    ncells = int(np.prod(ks))
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=ncells + 1, merged=False)
    n_active = out["n_active"].cpu().numpy()
    assert (n_active > 200000).all(), n_active
    sz = oracle.sizing(T, 4096 / T, subspace_parts=4, k_override=ks)
    sz["max_tokens"] = 4096
    sz["buffer_pages"] = max(32, -(-4096 // sz["page_size"]))
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    assert (bud.nprobe, bud.buffer_pages) == (16390, 512)
    static_len = 97
    sk, sv = synthetic.make_kv(H, static_len + 8, seed=78)
    plan = ops.DecodePlan(cent, out["cell_count"], out["cell_offset"], ks, bud, out["list_keys"],
                          out["list_values"], sk.to(DEV), sv.to(DEV), G, compact=out)
    plan.set_static_len(static_len)
    q = synthetic.make_queries(keys, G, seed=6)[0]
    plan.query.copy_(q.to(DEV))
    res = plan.step().clone()
    torch.cuda.synchronize()
    cents = cent.cpu().numpy()
    heads = []
    gids = out["compact_gid"].cpu().numpy()
    for h in range(H):
        na = int(n_active[h])
        merged = oracle.merged_centroids([cents[h, p, : ks[p]] for p in range(4)], gids[h, :na], list(ks))
        heads.append(dict(n_active=na, offsets=out["compact_offset"][h, : na + 1].cpu().numpy(), merged=merged,
                          list_keys=bits(out["list_keys"][h]), list_values=bits(out["list_values"][h])))
    ref, rs, rm, rrows = oracle.decode_step(bits(q), heads, bits(sk), bits(sv), static_len, int(n_active.max()) + 1,
                                            bud.nprobe, bud.max_tokens, bud.buffer_pages)
    sel = plan.selection
    assert np.array_equal(sel["n_selected"].cpu().numpy(), rm)
    cells = sel["sel_cell"].cpu().numpy()
    nrows = sel["n_rows"].cpu().numpy()
    for h in range(H):
        assert np.array_equal(cells[h, : rm[h]], gids[h][rs[h, : rm[h]]]), h
        assert nrows[h] == len(rrows[h]), h
    _check_attention(res, ref)


def test_config4_build_and_decode_match_oracle(ops, oracle):
    """configs[4] per KV head at its own size: 1,048,480 listed tokens, IMI
    2 x 128 centroids, 20 Lloyd iterations on the evenly strided
    65,536-key sample, then every key assigned to the final centroids
    (kmeans_core.cpp:190-314 on the sample, the E-step 222-242 over all
    keys); the index (reorganize_core.cpp:18-311) and one decode step at
    budget 0.02 (runtime.py:31-63: nprobe 328, max_tokens 20969, 2622
    pages).  Centroids, the full 1M assignment, the CSR, the permutation,
    the list rows and the selected cells are bit-exact with the oracle;
    attention within 2e-2 abs + 1e-2 rel."""
    from adaptiveimi_amd import synthetic

    H, G, ks, iters, sample, budget = 2, 4, (128, 128), 20, 65536, 0.02
    T = 1048576 - 96
    note(f"[config4] H={H} T={T} ks={ks} iters={iters} sample={sample} budget={budget}")
    keys, values = _kv(H, T, seed=444)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans_sampled(kd, list(ks), iters, sample)
    ncells = ks[0] * ks[1]
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=ncells + 1)
    torch.cuda.synchronize()
    step = -(-T // sample)
    assert step == 16 and len(range(0, T, step)) == 65530
    kf = keys.float().numpy()   # exact bf16 widen
    kb, vb = bits(keys), bits(values)
    sl = oracle.subspace_slices(128, 2)
    cg, lg = cent.cpu().numpy(), labels.cpu().numpy()
    perm, cnt, off = out["perm"].cpu().numpy(), out["cell_count"].cpu().numpy(), out["cell_offset"].cpu().numpy()
    heads = []
    for h in range(H):
        _, rc, it = oracle.kmeans_head(kf[h, ::step], list(ks), iters)
        assert it == [iters, iters]
        labs = []
        for p in range(2):
            assert np.array_equal(cg[h, p, : ks[p]], rc[p]), (h, p)
            lab, _, _ = oracle.estep(np.ascontiguousarray(kf[h][:, sl[p]]), rc[p])
            assert np.array_equal(lg[h, p], lab), (h, p)
            labs.append(lab)
        r = oracle.compact_reorg(labs, list(ks))
        na = r["n_active"]
        assert int(out["n_active"][h]) == na
        assert np.array_equal(out["compact_gid"][h, :na].cpu().numpy(), r["gids"]), h
        assert np.array_equal(out["compact_offset"][h, : na + 1].cpu().numpy(), r["offsets"]), h
        assert np.array_equal(perm[h], r["perm"]), h
        full_cnt = np.zeros(ncells, np.int32)
        full_cnt[r["gids"]] = np.diff(r["offsets"])
        assert np.array_equal(cnt[h], full_cnt), h
        assert off[h, 0] == 0 and np.array_equal(np.diff(off[h]), full_cnt), h
        # list rows = the permuted keys / values, compared on the device
        ph = out["perm"][h].long()
        assert torch.equal(out["list_keys"][h], kd[h, ph]) and torch.equal(out["list_values"][h], vd[h, ph]), h
        heads.append(dict(n_active=na, offsets=r["offsets"], merged=oracle.merged_centroids(rc, r["gids"], list(ks)),
                          list_keys=kb[h][r["perm"]], list_values=vb[h][r["perm"]], gids=r["gids"]))
    del kf
    sz = oracle.sizing(T, budget, k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    assert (bud.nprobe, bud.max_tokens, bud.buffer_pages) == (328, 20969, 2622)
    static_len = 97
    sk, sv = synthetic.make_kv(H, static_len + 8, seed=79)
    plan = ops.DecodePlan(cent, out["cell_count"], out["cell_offset"], ks, bud, out["list_keys"],
                          out["list_values"], sk.to(DEV), sv.to(DEV), G)
    plan.set_static_len(static_len)
    q = synthetic.make_queries(keys, G, seed=7)[0]
    plan.query.copy_(q.to(DEV))
    res = plan.step().clone()
    torch.cuda.synchronize()
    ref, rs, rm, rrows = oracle.decode_step(bits(q), heads, bits(sk), bits(sv), static_len, sz["n_centroids"],
                                            bud.nprobe, bud.max_tokens, bud.buffer_pages)
    sel = plan.selection
    assert np.array_equal(sel["n_selected"].cpu().numpy(), rm)
    cells, nrows = sel["sel_cell"].cpu().numpy(), sel["n_rows"].cpu().numpy()
    for h in range(H):
        assert np.array_equal(cells[h, : rm[h]], heads[h]["gids"][rs[h, : rm[h]]]), h
        assert nrows[h] == len(rrows[h]), h
    note(f"[config4] selected cells {rm.tolist()}, rows {nrows.tolist()}")
    # nprobe binds (328 cells of ~53 rows stay under max_tokens and the pages)
    assert (rm == bud.nprobe).all() and (nrows < bud.max_tokens).all() and (nrows > 10000).all(), (rm, nrows)
    _check_attention(res, ref)


@pytest.mark.parametrize("ks,lens", [((32, 32), (3000, 6000, 9000, 12000)), ((6, 6, 6, 6), (3000, 6000, 9000, 12000)),
                                     ((32, 32), (2000, 12000)), ((32, 32), (3000, 4500, 6000, 9000, 12000)),
                                     # a 40:1 length ratio, and seven sequences of close lengths
                                     ((32, 32), (1500, 60000)), ((16, 16), (1200, 1300, 1400, 1500, 1600, 1700, 1800)),
                                     # configs[2] at its own lengths (32k-128k, 64 x 64, 16 KV heads, GQA 7)
                                     ((64, 64), (32768 - 96, 65536 - 96, 98304 - 96, 131072 - 96))])
def test_ragged_batch_decode_matches_oracle(ops, oracle, ks, lens):
    """Config 2 (reduced lengths, and its own 32k-128k): the KV heads of several sequences of
    different lengths (so different token and page budgets) share one
    selection and attention launch, their lists living in one
    [B*H, max_len, D] buffer.  Every sequence must match its own batch-1
    oracle step: same selected cells, attention within 2e-2 + 1e-2 |ref|.
    Two to four sequences take the attention's per-run split counts, five
    fall back to equal splits per head."""
    from adaptiveimi_amd import synthetic

    lens = list(lens)
    note(f"[ragged] lens={lens} ks={ks}")
    H, G, D, static_len = 4, 7, 128, 96
    B, cap = len(lens), max(lens)
    lk = torch.zeros((B * H, cap, D), dtype=torch.bfloat16, device=DEV)
    lv = torch.zeros_like(lk)
    sk, sv = synthetic.make_kv(B * H, static_len + 4, seed=91)
    cents, counts, offsets, compacts, buds, per_seq = [], [], [], [], [], []
    ncells = int(np.prod(ks))
    for s_, T in enumerate(lens):
        keys, values = synthetic.make_kv(H, T, seed=300 + s_)
        kd, vd = keys.to(DEV), values.to(DEV)
        cent, labels, _ = ops.kmeans(kd, list(ks), 3)
        out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=min(T, ncells) + 1 if len(ks) == 4 else None,
                              list_keys=lk[s_ * H:(s_ + 1) * H], list_values=lv[s_ * H:(s_ + 1) * H])
        cents.append(cent)
        counts.append(out["cell_count"])
        offsets.append(out["cell_offset"])
        compacts.append(out)
        sz = oracle.sizing(T, 0.1, k_override=ks)
        buds.append(ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"]))
        per_seq.append((keys, sz))
    bud = ops.Budget.ragged(buds, H)
    compact = None
    if len(ks) == 4:
        width = max(c["compact_gid"].shape[1] for c in compacts)

        def pad(name, extra=0):
            return torch.cat([torch.nn.functional.pad(c[name], (0, width + extra - c[name].shape[1])) for c in compacts])

        compact = dict(compact_gid=pad("compact_gid"), compact_size=pad("compact_size"),
                       compact_offset=pad("compact_offset", 1), n_active=torch.cat([c["n_active"] for c in compacts]))
    plan = ops.DecodePlan(torch.cat(cents), torch.cat(counts), torch.cat(offsets), ks, bud, lk, lv, sk.to(DEV),
                          sv.to(DEV), G, compact=compact)
    plan.set_static_len(static_len)
    q = torch.cat([synthetic.make_queries(per_seq[s_][0], G, seed=20 + s_)[0] for s_ in range(B)])
    plan.query.copy_(q.to(DEV))
    res = plan.step().clone().float().cpu().numpy().reshape(B * H, G, D)
    sel = plan.selection
    m_all = sel["n_selected"].cpu().numpy()
    cells_all = sel["sel_cell"].cpu().numpy()
    for s_ in range(B):
        out, (keys, sz) = compacts[s_], per_seq[s_]
        hs = slice(s_ * H, (s_ + 1) * H)
        heads = []
        for h in range(H):
            na = int(out["n_active"][h])
            heads.append(dict(n_active=na, offsets=out["compact_offset"][h, : na + 1].cpu().numpy(),
                              merged=out["compact_centroids"][h, :na].cpu().numpy(),
                              list_keys=bits(lk[s_ * H + h, : lens[s_]]), list_values=bits(lv[s_ * H + h, : lens[s_]])))
        ref, rs, rm, _ = oracle.decode_step(bits(q[hs]), heads, bits(sk[hs]), bits(sv[hs]), static_len,
                                            sz["n_centroids"], sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
        assert np.array_equal(m_all[hs], rm), (s_, m_all[hs], rm)
        gids = out["compact_gid"].cpu().numpy()
        for h in range(H):
            assert np.array_equal(cells_all[s_ * H + h, : rm[h]], gids[h][rs[h, : rm[h]]]), (s_, h)
        err = np.abs(res[hs] - ref)
        assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), (s_, float(err.max()))


@pytest.mark.parametrize("L,cap,span,holes", [(3000, 40, 50, False), (150000, 1400, 100, False),
                                              (150000, 6000, 20, False), (20000, 300, 50, True)])
def test_attention_standalone_and_lse(ops, oracle, L, cap, span, holes):
    """imi_sparse_attention with a caller-made selection, and the LSE output.
    The 1400-cell case gives heads of 35k-70k rows, i.e. 70-140 splits: the
    merge's first batch of partials, then chunks of 64 split weights.  The
    6000-cell case selects more cells than the prologue's first round trip
    stages (2048); holes: every third selected cell holds no rows."""
    note(f"[attention] standalone L={L} cap={cap} holes={holes}")
    H, G = 4, 4
    from adaptiveimi_amd import synthetic

    kl, vl = synthetic.make_kv(H, L, seed=31)
    q = synthetic.make_queries(kl, G, seed=4)[0]
    rng = np.random.default_rng(0)
    offs = np.zeros((H, cap), np.int32)
    cnts = np.zeros((H, cap), np.int32)
    pref = np.zeros((H, cap + 1), np.int32)
    nsel = np.zeros(H, np.int32)
    rows = []
    for h in range(H):
        m = int(rng.integers(0, cap)) if cap < 100 else int(rng.integers(cap // 2, cap))
        starts = np.sort(rng.choice(L // span, m, replace=False)) * span
        c = rng.integers(1, span, m)
        if holes:
            c[::3] = 0
        offs[h, :m], cnts[h, :m] = starts, c
        pref[h, 1 : m + 1] = np.cumsum(c)
        nsel[h] = m
        rows.append(np.concatenate([np.arange(s, s + n) for s, n in zip(starts, c)]) if m else np.zeros(0, np.int64))
    sel = dict(sel_cell=torch.zeros((H, cap), dtype=torch.int32, device=DEV),
               sel_offset=torch.from_numpy(offs).to(DEV), sel_count=torch.from_numpy(cnts).to(DEV),
               sel_prefix=torch.from_numpy(pref).to(DEV), n_selected=torch.from_numpy(nsel).to(DEV),
               n_rows=torch.from_numpy(pref[np.arange(H), nsel]).to(DEV))
    out, lse = ops.sparse_attention(q.to(DEV), None, None, 0, kl.to(DEV), vl.to(DEV), sel, max_rows=cap * span,
                                    return_lse=True)
    ref = oracle.attention(bits(q), bits(kl), bits(vl), rows)
    _check_attention(out, ref)
    # LSE (natural log) against fp64
    qf = oracle.bf16_to_f32(bits(q)).astype(np.float64)
    kf = oracle.bf16_to_f32(bits(kl)).astype(np.float64)
    lse = lse.cpu().numpy().reshape(H, G)
    for h in range(H):
        if len(rows[h]) == 0:
            assert np.all(np.isneginf(lse[h]))
            assert np.all(out.view(H, G, 128)[h].float().cpu().numpy() == 0)
            continue
        s = qf[h] @ kf[h, rows[h]].T / math.sqrt(128)
        ref_lse = np.log(np.exp(s - s.max(1, keepdims=True)).sum(1)) + s.max(1)
        assert np.allclose(lse[h], ref_lse, atol=1e-3, rtol=1e-4)


def test_decode_repeatable_and_graph_capture(ops, oracle):
    """The same step twice gives identical bytes; a captured HIP graph
    replayed several times matches eager results."""
    note("[decode] determinism + graph")
    H, T, ks, G = 8, 16384, (64, 64), 4
    keys, values, cent, out = _index(ops, H, T, ks, 55)
    from adaptiveimi_amd import synthetic

    sz = oracle.sizing(T, 0.1, k_override=ks)
    bud = ops.Budget(sz["nprobe"], sz["max_tokens"], sz["buffer_pages"])
    plan = ops.DecodePlan(cent, out["cell_count"], out["cell_offset"], ks, bud, out["list_keys"],
                          out["list_values"], None, None, G)
    qs = synthetic.make_queries(keys, G, seed=8, n_queries=3).to(DEV)
    eager = []
    for i in range(3):
        plan.query.copy_(qs[i])
        eager.append(plan.step().clone())
    plan.query.copy_(qs[0])
    again = plan.step().clone()
    assert torch.equal(again, eager[0])
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            plan.step()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        for i in range(3):
            plan.query.copy_(qs[i])
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(plan.out, eager[i]), (rep, i)
    # the step in parts: selection, split pass, merge (each reads what the
    # previous call left in the workspace) gives the same bytes
    for i in range(3):
        plan.query.copy_(qs[i])
        plan.out.zero_()
        for ph in (1, 4, 8):
            plan.step(phases=ph)
        torch.cuda.synchronize()
        assert torch.equal(plan.out, eager[i]), ("phases 1, 4, 8", i)


def test_full_size_properties_128k(ops):
    """BASELINE 128k shape: invariants that do not need the oracle."""
    note("[128k] properties")
    H, T, ks = 8, 131072 - 96, (64, 64)
    keys, values, cent, out = _index(ops, H, T, ks, 1234, iters=10)
    cnt = out["cell_count"]
    assert (cnt.sum(1) == T).all()
    off = out["cell_offset"]
    assert (off[:, 1:] >= off[:, :-1]).all() and (off[:, -1] == T).all()
    perm = out["perm"]
    assert torch.equal(torch.sort(perm, dim=1).values, torch.arange(T, device=DEV, dtype=torch.int32).expand(H, T))
    # CSR order = (cell, token): cells non-decreasing, tokens ascending inside a cell
    lab = out["labels"].long()
    g = lab[:, 0] * ks[1] + lab[:, 1]
    gs = torch.gather(g, 1, perm.long())
    assert (gs[:, 1:] >= gs[:, :-1]).all()
    same = gs[:, 1:] == gs[:, :-1]
    assert (perm[:, 1:][same] > perm[:, :-1][same]).all()
    assert torch.equal(torch.bincount(g[0], minlength=ks[0] * ks[1]).to(torch.int32), cnt[0])
    # the list holds the permuted rows
    kd = keys.to(DEV)
    for h in range(H):
        assert torch.equal(out["list_keys"][h], kd[h][perm[h].long()])


@pytest.mark.parametrize("case", ["outlier", "zero_query", "zero_query_4096", "near_ties", "huge_centroid",
                                  "zero_query_16384", "near_ties_16384", "huge_centroid_16384"])
def test_select_refinement_paths(ops, oracle, case):
    """Skewed scores (one subspace centroid blown up -> a few huge scores)
    force the bucket refinement; a zero query makes every score equal, so
    ranking falls back to cell ids alone.  Near ties: the second-subspace
    centroids differ by ~1e-6 relative, so the cells of one first-subspace
    centroid score within a few ulps of each other and their order is
    decided by the roundings of the chain.  A centroid of magnitude 1e33
    keeps every chain finite but puts the magnitude sums sum |q||c| past
    2^114.  The _16384 cases repeat them at 2 x 128 centroids (16 cells per
    thread, the layout of configs[4])."""
    note(f"[select] {case}")
    H, T = 4, 12000
    ks = (128, 128) if case.endswith("_16384") else ((64, 64) if case == "zero_query_4096" else (32, 32))
    case = case.replace("_16384", "").replace("_4096", "")
    keys, values = _kv(H, T, seed=17)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent, labels, _ = ops.kmeans(kd, list(ks), 3)
    if case == "outlier":
        cent[:, 1, 0] *= 300.0
    if case == "near_ties":
        g = torch.Generator().manual_seed(5)
        noise = torch.randn(cent[:, 1, : ks[1]].shape, generator=g).to(DEV)
        cent[:, 1, : ks[1]] = cent[:, 1, :1] * (1.0 + 1e-6 * noise)
    if case == "huge_centroid":
        cent[:, 0, 0] *= 1e33
    out = ops.build_index(kd, vd, cent, labels, list(ks), n_centroids=ks[0] * ks[1] + 1)
    from adaptiveimi_amd import synthetic

    q = synthetic.make_queries(keys, 4, seed=3)[0]
    if case == "zero_query":
        q.zero_()
    # the third budget ranks 3000 cells: the score + rank kernels
    for bud in (ops.Budget(102, 1200, 150), ops.Budget(400, 5000, 800), ops.Budget(3000, 11000, 3000)):
        sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud)
        sc = oracle.scores(bits(q), out["compact_centroids"].cpu().numpy())
        rs, rm, rtok = oracle.select(sc, out["compact_size"].cpu().numpy(), out["compact_mask"].cpu().numpy(),
                                     bud.nprobe, bud.max_tokens, bud.buffer_pages)
        gids = out["compact_gid"].cpu().numpy()
        m = sel["n_selected"].cpu().numpy()
        assert np.array_equal(m, rm)
        for h in range(H):
            assert np.array_equal(sel["sel_cell"].cpu().numpy()[h, : m[h]], gids[h][rs[h, : rm[h]]]), h
        assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok)


@pytest.mark.parametrize("ks", [(64, 64), (128, 128), (32, 32)])
def test_select_screen_across_offsets(ops, oracle, ks):
    """The selection screens cells by p1[l0] + q1[l1] with a rounding bound
    and computes exact chains for the candidates only, falling back to every
    cell's chain when the score range is narrow next to the bound.  A common
    offset added to every centroid grows the scores' magnitude (hence the
    bound) at a fixed spread, so the sweep crosses from the screened ranking
    into the fallback; 6 queries per offset, every selection bit-exact with
    the oracle's exhaustive ranking."""
    note(f"[select] screen across offsets ks={ks}")
    H, T = 4, 30000
    keys, values = _kv(H, T, seed=23)
    kd, vd = keys.to(DEV), values.to(DEV)
    cent0, labels, _ = ops.kmeans(kd, list(ks), 3)
    out = ops.build_index(kd, vd, cent0, labels, list(ks), n_centroids=ks[0] * ks[1] + 1)
    gids = out["compact_gid"].cpu().numpy()
    size, mask = out["compact_size"].cpu().numpy(), out["compact_mask"].cpu().numpy()
    na = out["n_active"].cpu().numpy()
    from adaptiveimi_amd import synthetic

    qs = synthetic.make_queries(keys, 4, seed=9, n_queries=6)
    u = torch.randn((2, 64), generator=torch.Generator().manual_seed(1)).to(DEV)
    bud = ops.Budget(round(ks[0] * ks[1] * 0.1), int(0.1 * T), -(-int(0.1 * T) // 8))
    for off in (0.0, 3.0, 30.0, 300.0, 3000.0, 3e4):
        cent = cent0.clone()
        cent[:, :, : max(ks)] += off * u[None, :, None, :]
        merged = np.zeros((H, ks[0] * ks[1] + 1, 128), np.float32)
        cc = cent.cpu().numpy()
        for h in range(H):
            merged[h, : na[h]] = oracle.merged_centroids([cc[h, 0, : ks[0]], cc[h, 1, : ks[1]]], gids[h, : na[h]],
                                                         list(ks))
        for n in range(qs.shape[0]):
            q = qs[n]
            sel = ops.select(q.to(DEV), cent, out["cell_count"], out["cell_offset"], ks, bud)
            sc = oracle.scores(bits(q), merged)
            rs, rm, rtok = oracle.select(sc, size, mask, bud.nprobe, bud.max_tokens, bud.buffer_pages)
            m = sel["n_selected"].cpu().numpy()
            assert np.array_equal(m, rm), (off, n)
            cells = sel["sel_cell"].cpu().numpy()
            for h in range(H):
                assert np.array_equal(cells[h, : m[h]], gids[h][rs[h, : rm[h]]]), (off, n, h)
            assert np.array_equal(sel["n_rows"].cpu().numpy(), rtok), (off, n)
