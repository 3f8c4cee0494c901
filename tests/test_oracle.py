"""Pins of the CPU oracle (oracle/) against closed forms, brute force and the
reference's own rules.  The reference ships no tests or golden vectors, so
every check here is derived from the mathematics or from the reference
source's literal rules (cited), never from the oracle itself."""
from fractions import Fraction
import math

import numpy as np
import pytest
import torch


def f32(x):
    return np.float32(x)


# ----------------------------------------------------------- bf16 widen ----

def test_bf16_roundtrip_exact(oracle):
    bits = np.arange(0, 1 << 16, dtype=np.uint16)
    f = oracle.bf16_to_f32(bits)
    finite = np.isfinite(f)
    back = oracle.f32_to_bf16(f[finite])
    assert np.array_equal(back, bits[finite])
    # the widen equals torch's bf16 -> fp32 conversion (a library routine)
    t = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(t[finite], f[finite])


# ------------------------------------------------------------- distance ----

def test_l2_integer_exact(oracle):
    rng = np.random.default_rng(0)
    for dim in (32, 64, 128):
        a = rng.integers(-50, 50, dim).astype(np.float32)
        b = rng.integers(-50, 50, dim).astype(np.float32)
        d = oracle.lib().orc_l2(a.ctypes.data_as(oracle._f32p), b.ctypes.data_as(oracle._f32p), dim)
        assert d == float(((a.astype(np.int64) - b.astype(np.int64)) ** 2).sum())


def test_l2_lane_order(oracle):
    """kmeans_core.cpp:22-44: lane j sums dims j, j+8, ... with FMA, then the
    lanes are added left to right.  2^24 + 1 rounds to 2^24 (ties to even), so
    two unit terms in the SAME lane (dims 1 and 9 -> lane 1 = 2) survive,
    whereas a plain sequential sum would drop both."""
    a = np.zeros(64, np.float32)
    b = np.zeros(64, np.float32)
    a[0] = 4096.0          # lane 0: 2^24
    a[1] = 1.0             # lane 1: 1
    a[9] = 1.0             # lane 1: 1 + 1 = 2
    d = oracle.lib().orc_l2(a.ctypes.data_as(oracle._f32p), b.ctypes.data_as(oracle._f32p), 64)
    assert d == 2.0 ** 24 + 2.0
    # the same two units in different lanes are each absorbed: 2^24 + 1 + 1
    a[9] = 0.0
    a[2] = 1.0
    d = oracle.lib().orc_l2(a.ctypes.data_as(oracle._f32p), b.ctypes.data_as(oracle._f32p), 64)
    assert d == 2.0 ** 24


def _exact_lane_l2(a, b):
    """Exact-rational evaluation of the documented order (fma = one rounding)."""
    lanes = [f32(0.0)] * 8
    for i in range(len(a)):
        d = f32(f32(a[i]) - f32(b[i]))
        j = i % 8
        lanes[j] = f32(float(Fraction(float(d)) * Fraction(float(d)) + Fraction(float(lanes[j]))))
    t = lanes[0]
    for j in range(1, 8):
        t = f32(t + lanes[j])
    return t


def test_l2_random_matches_exact_rational_order(oracle):
    rng = np.random.default_rng(1)
    for _ in range(200):
        a = (rng.standard_normal(64) * rng.lognormal(0, 1, 64)).astype(np.float32)
        b = (rng.standard_normal(64) * 2).astype(np.float32)
        d = oracle.lib().orc_l2(a.ctypes.data_as(oracle._f32p), b.ctypes.data_as(oracle._f32p), 64)
        assert np.float32(d) == _exact_lane_l2(a, b)


# ---------------------------------------------------------------- E-step ----

def test_estep_brute_force(oracle):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((500, 64)).astype(np.float32)
    c = rng.standard_normal((16, 64)).astype(np.float32)
    lab, mind, _ = oracle.estep(x, c)
    d64 = ((x[:, None, :].astype(np.float64) - c[None].astype(np.float64)) ** 2).sum(-1)
    ref = d64.argmin(1)
    diff = lab != ref
    # disagreements only at fp32-level near ties
    for i in np.nonzero(diff)[0]:
        assert abs(d64[i, lab[i]] - d64[i, ref[i]]) <= 1e-5 * d64[i].min()
    assert np.allclose(mind, d64.min(1), rtol=1e-5)


def test_estep_tie_lowest_index(oracle):
    """Strict '<' in kmeans_core.cpp:234: equal distances keep the lower id."""
    rng = np.random.default_rng(3)
    x = rng.integers(-3, 4, (300, 64)).astype(np.float32)
    c = rng.integers(-3, 4, (8, 64)).astype(np.float32)
    c = np.concatenate([c, c[::-1]])   # every centroid duplicated
    lab, _, _ = oracle.estep(x, c)
    d = ((x[:, None, :].astype(np.int64) - c[None].astype(np.int64)) ** 2).sum(-1)
    assert np.array_equal(lab, d.argmin(1))  # numpy argmin returns the first minimum
    assert (lab < 8).all()


# ---------------------------------------------------------------- M-step ----

def test_mstep_closed_form_mean(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((1000, 64)).astype(np.float32)
    lab = rng.integers(0, 10, 1000).astype(np.int32)
    for threads in (1, 3, 8):
        c = oracle.mstep(x, lab, 10, 0, nthreads=threads)
        for k in range(10):
            m = x[lab == k].astype(np.float64).mean(0)
            assert np.allclose(c[k], m, rtol=1e-5, atol=1e-6)


def test_mstep_integer_partition_invariant(oracle):
    """Integer members with power-of-two counts: every order gives the exact mean."""
    rng = np.random.default_rng(5)
    x = rng.integers(-100, 100, (512, 32)).astype(np.float32)
    lab = np.repeat(np.arange(8, dtype=np.int32), 64)
    rng.shuffle(lab)
    ref = np.stack([x[lab == k].astype(np.float64).mean(0) for k in range(8)])
    for threads in (1, 2, 5, 16):
        c = oracle.mstep(x, lab, 8, 3, nthreads=threads)
        assert np.array_equal(c.astype(np.float64), ref)


def test_mstep_sequential_order(oracle):
    """threads=1 sums members in ascending order: 2^24 + 1 + 1 stays 2^24 in
    fp32, while a pairwise order would give 2^24 + 2."""
    x = np.zeros((3, 8), np.float32)
    x[0, 0] = 2.0 ** 24
    x[1, 0] = 1.0
    x[2, 0] = 1.0
    c = oracle.mstep(x, np.zeros(3, np.int32), 1, 0, nthreads=1)
    assert c[0, 0] == np.float32(2.0 ** 24) * np.float32(1.0 / np.float32(3.0))
    # with two threads (chunks {0,1} and {2}) the partials are 2^24 and 1
    c2 = oracle.mstep(x, np.zeros(3, np.int32), 1, 0, nthreads=2)
    assert c2[0, 0] == np.float32(np.float32(2.0 ** 24) + np.float32(1.0)) * np.float32(1.0 / np.float32(3.0))


def test_mstep_empty_cluster_reseed(oracle):
    """kmeans_core.cpp:299-311: each empty cluster, in ascending order, copies
    the sample picked by the next draw of mt19937(iter + 12345)."""
    rng = np.random.default_rng(6)
    x = rng.standard_normal((100, 16)).astype(np.float32)
    lab = np.where(np.arange(100) % 2 == 0, 0, 3).astype(np.int32)  # clusters 1, 2 empty
    for it in (0, 7):
        c = oracle.mstep(x, lab, 4, it, nthreads=1)
        draws = oracle.reseed_draws(it, 100, 2)
        assert np.array_equal(c[1], x[draws[0]])
        assert np.array_equal(c[2], x[draws[1]])
        assert 0 <= draws.min() and draws.max() < 100
    # std::mt19937's 10000th output for the default seed is fixed by the C++
    # standard ([rand.predef]); with n = 2^32 the distribution is the identity
    # only if libstdc++ passes draws through unchanged, so check the engine
    # through a full-range request instead of the distribution
    assert oracle.reseed_draws(0, 1 << 30, 4).dtype == np.int32


def test_lloyd_labels_one_step_behind(oracle):
    """After a full run (no early stop) labels come from the last E-step and
    centroids from the M-step after it (kmeans_core.cpp:219-313)."""
    rng = np.random.default_rng(7)
    x = rng.standard_normal((400, 32)).astype(np.float32)
    c0 = x[:8].copy()
    c, lab, iters = oracle.lloyd(x, c0, 3)
    assert iters == 3
    # replay by hand
    cc = c0.copy()
    for it in range(3):
        ll, _, _ = oracle.estep(x, cc)
        cc = oracle.mstep(x, ll, 8, it)
    assert np.array_equal(lab, ll)
    assert np.array_equal(c, cc)


def test_lloyd_early_stop(oracle):
    """A converged run stops after the E-step without moving the centroids."""
    rng = np.random.default_rng(8)
    x = np.concatenate([rng.standard_normal((50, 16)) + 10 * i for i in range(4)]).astype(np.float32)
    c0 = x[[0, 50, 100, 150]].copy()
    c, lab, iters = oracle.lloyd(x, c0, 20, tol=1e-3, early_stop_min_iter=2, early_stop_rel_tol=1e-6)
    assert iters < 20
    ll, _, _ = oracle.estep(x, c)
    assert np.array_equal(ll, lab)


def test_kmeanspp_picks_data_rows(oracle):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((300, 16)).astype(np.float32)
    c = oracle.kmeanspp_init(x, 12, 42)
    rows = {tuple(r) for r in x}
    assert all(tuple(r) in rows for r in c)
    assert len({tuple(r) for r in c}) == 12   # D^2 sampling never re-picks a chosen row
    assert np.array_equal(c, oracle.kmeanspp_init(x, 12, 42))


# ------------------------------------------------------------ reorganize ----

def test_compact_reorg_invariants(oracle):
    rng = np.random.default_rng(10)
    T, ks = 2000, (16, 16)
    l0 = rng.integers(0, ks[0], T).astype(np.int32)
    l1 = rng.integers(0, ks[1], T).astype(np.int32)
    r = oracle.compact_reorg([l0, l1], ks)
    g = l0.astype(np.int64) * ks[1] + l1
    uniq = np.unique(g)
    assert r["n_active"] == len(uniq)
    assert np.array_equal(r["gids"], uniq)                          # compact id = rank of global id
    assert np.array_equal(r["final_labels"], np.searchsorted(uniq, g))
    assert r["offsets"][0] == 0 and r["offsets"][-1] == T
    assert (np.diff(r["offsets"]) > 0).all()                         # occupied cells only
    perm = r["perm"]
    assert np.array_equal(np.sort(perm), np.arange(T))
    # CSR order = (cell, token) lexicographic: a stable counting sort
    assert np.array_equal(perm, np.lexsort((np.arange(T), g)))


def test_compact_reorg_4way_mixed_radix(oracle):
    rng = np.random.default_rng(11)
    T, ks = 1000, (4, 3, 5, 2)
    labels = [rng.integers(0, k, T).astype(np.int32) for k in ks]
    r = oracle.compact_reorg(labels, ks)
    g = ((labels[0].astype(np.int64) * ks[1] + labels[1]) * ks[2] + labels[2]) * ks[3] + labels[3]
    assert np.array_equal(r["gids"], np.unique(g))
    assert np.array_equal(r["perm"], np.lexsort((np.arange(T), g)))
    cents = [rng.standard_normal((k, 8)).astype(np.float32) for k in ks]
    merged = oracle.merged_centroids(cents, r["gids"], ks)
    for c, gg in enumerate(r["gids"][:50]):
        rem, idx = int(gg), []
        for k in reversed(ks):
            idx.append(rem % k)
            rem //= k
        idx = idx[::-1]
        assert np.array_equal(merged[c], np.concatenate([cents[p][idx[p]] for p in range(4)]))


# -------------------------------------------------------------- scoring ----

def test_scores_integer_exact(oracle):
    rng = np.random.default_rng(12)
    q = rng.integers(-3, 4, (2, 4, 128)).astype(np.float32)
    c = rng.integers(-5, 6, (2, 50, 128)).astype(np.float32)
    s = oracle.scores(oracle.f32_to_bf16(q), c)
    ref = np.einsum("hd,hnd->hn", q.sum(1).astype(np.int64), c.astype(np.int64))
    assert np.array_equal(s, ref.astype(np.float32))


def test_scores_match_torch_fallback_within_rounding(oracle):
    """The reference's torch fallback (imi_adapter.py:102-103) is the same
    product up to summation order."""
    rng = np.random.default_rng(13)
    qb = oracle.f32_to_bf16(rng.standard_normal((2, 4, 128)).astype(np.float32))
    c = rng.standard_normal((2, 100, 128)).astype(np.float32)
    s = oracle.scores(qb, c)
    q = torch.from_numpy(oracle.bf16_to_f32(qb))
    ref = torch.einsum("hd,hnd->hn", q.double().sum(1), torch.from_numpy(c).double()).numpy()
    assert np.allclose(s, ref, rtol=1e-5, atol=1e-4)


# ------------------------------------------------------------ selection ----

def _select_literal(sc, sizes, mask, nprobe, max_tokens, buffer_pages, page=8):
    """retrieval.py:295-303 written with torch ops (stable sort for the tie
    contract), then the batch_access loop of wave_buffer_cpu_hotcold.cpp:320-368."""
    s = torch.from_numpy(sc).clone()
    s.masked_fill_(torch.from_numpy(mask), float("-inf"))
    order = torch.sort(s, dim=-1, descending=True, stable=True).indices[:, :nprobe]
    sz = torch.gather(torch.from_numpy(sizes), 1, order)
    valid = sz > 0
    cum = torch.cumsum(sz, dim=-1, dtype=torch.int32)
    keep = valid & ((cum - sz) < max_tokens)
    pad = -1
    selected = order.masked_fill(~keep, pad)
    out = []
    for h in range(sc.shape[0]):
        res, consider = [], 0
        for cid in selected[h].tolist():
            if cid == pad or sizes[h, cid] == 0:
                continue
            consider += (int(sizes[h, cid]) + page - 1) // page
            if consider > buffer_pages:
                break
            res.append(cid)
        out.append(res)
    return out


@pytest.mark.parametrize("seed", range(6))
def test_select_matches_literal_rules(oracle, seed):
    rng = np.random.default_rng(100 + seed)
    H, N = 3, 300
    sizes = rng.integers(1, 40, (H, N)).astype(np.int32)
    n_active = rng.integers(200, N, H)
    mask = np.zeros((H, N), bool)
    for h in range(H):
        sizes[h, n_active[h]:] = 0
        mask[h, n_active[h]:] = True
    sc = rng.standard_normal((H, N)).astype(np.float32)
    if seed % 2:  # many exact ties
        sc = np.round(sc * 2) / 2
    nprobe = int(rng.integers(5, 80))
    max_tokens = int(rng.integers(20, 1500))
    pages = int(rng.integers(3, 200))
    sel, m, tok = oracle.select(sc, sizes, mask, nprobe, max_tokens, pages)
    ref = _select_literal(sc, sizes, mask, nprobe, max_tokens, pages)
    for h in range(H):
        assert sel[h, : m[h]].tolist() == ref[h]
        assert tok[h] == sizes[h, ref[h]].sum()


# ------------------------------------------------------------ attention ----

def test_attention_closed_forms(oracle):
    rng = np.random.default_rng(14)
    H, G, D, L = 2, 4, 128, 40
    qb = oracle.f32_to_bf16(rng.standard_normal((H, G, D)).astype(np.float32))
    kb = oracle.f32_to_bf16(np.zeros((H, L, D), np.float32))       # equal scores -> mean of values
    vb = oracle.f32_to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
    rows = [np.arange(0, 30), np.arange(10, 40)]
    out = oracle.attention(qb, kb, vb, rows)
    v = oracle.bf16_to_f32(vb).astype(np.float64)
    assert np.allclose(out[0], v[0, :30].mean(0), atol=1e-12)
    assert np.allclose(out[1], v[1, 10:40].mean(0), atol=1e-12)
    # empty row set -> zeros
    out = oracle.attention(qb, kb, vb, [np.zeros(0, np.int64), np.arange(3)])
    assert np.all(out[0] == 0)


def test_attention_matches_torch_softmax(oracle):
    rng = np.random.default_rng(15)
    H, G, D, L = 2, 4, 128, 64
    qb = oracle.f32_to_bf16(rng.standard_normal((H, G, D)).astype(np.float32))
    kb = oracle.f32_to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
    vb = oracle.f32_to_bf16(rng.standard_normal((H, L, D)).astype(np.float32))
    rows = [np.arange(L), np.arange(0, L, 2)]
    out = oracle.attention(qb, kb, vb, rows)
    q = torch.from_numpy(oracle.bf16_to_f32(qb)).double()
    k = torch.from_numpy(oracle.bf16_to_f32(kb)).double()
    v = torch.from_numpy(oracle.bf16_to_f32(vb)).double()
    for h in range(H):
        r = torch.from_numpy(rows[h])
        ref = torch.softmax(q[h] @ k[h, r].T / math.sqrt(D), -1) @ v[h, r]
        assert np.allclose(out[h], ref.numpy(), atol=1e-10)


# --------------------------------------------------------------- sizing ----

def test_sizing_reference_formulas(oracle):
    # runtime.py:31-63 at list_capacity 32768, budget 0.1, 2-way
    s = oracle.sizing(32768, 0.1)
    assert s["n_centroids"] == 45 * 45 + 1          # k = max(int(sqrt(2048)), 32) = 45
    assert s["nprobe"] == round(2025 * 0.1) == 202  # Python banker's rounding of 202.5
    assert s["max_tokens"] == 3276                  # int(3276.8); BASELINE's 3277 is off by one
    assert s["buffer_pages"] == 410                 # max(32, ceil(3276 / 8))
    s = oracle.sizing(32768, 0.1, k_override=(64, 64))
    assert (s["n_centroids"], s["nprobe"]) == (4097, 410)
    s = oracle.sizing(131072 - 96, 0.1, k_override=(64, 64))
    assert (s["max_tokens"], s["buffer_pages"]) == (13097, 1638)
    s = oracle.sizing(1000, 0.1)
    assert s["n_centroids"] == 32 * 32 + 1 and s["buffer_pages"] == 32
    s = oracle.sizing(262144, 0.1, subspace_parts=4)
    assert s["n_centroids"] == 11 ** 4 + 1           # round((16384) ** 0.25) = round(11.31) = 11


def test_adaptive_k(oracle):
    # layer_pipeline.cpp:177-228
    assert oracle.adaptive_k(32768) == [45, 45]
    assert oracle.adaptive_k(1000) == [32, 32]
    assert oracle.adaptive_k(262144, subspace_parts=4) == [11] * 4
    assert oracle.adaptive_k(100, subspace_parts=0) == [6]           # round(6.25)
    assert oracle.adaptive_k(0) == [1, 1]


def test_reference_threads_per_phase(oracle):
    # cache.py:113-124 with kmeans_core.cpp:433-443: one thread per Lloyd run
    # below 32 cores, which is the M-step order the GPU reproduces
    assert [oracle.reference_threads_per_phase(c, 8, 2) for c in (8, 16, 31)] == [1, 1, 1]
    assert oracle.reference_threads_per_phase(32, 8, 2) == 2
    assert oracle.reference_threads_per_phase(96, 8, 2) == 6
