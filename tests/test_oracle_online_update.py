"""Pins of the online-update oracle (oracle.update_assign,
oracle.OnlineUpdateOracle) against the rules of the reference's async
update (cache_hub/adaptive_imi/async_update.py:20-162), closed forms and
brute force.  CPU only."""
import numpy as np


def _int_rows(rng, n, d, lo=-4, hi=5):
    return rng.integers(lo, hi, (n, d)).astype(np.float32)


def test_assign_integer_exact_and_lowest_row_on_ties(oracle):
    """Integer data: every fp32 dot product is exact, so the arg-max is the
    integer arg-max, and duplicated rows tie with the lower row winning
    (torch.argmax returns the first maximal index, async_update.py:127)."""
    rng = np.random.default_rng(1)
    rows = _int_rows(rng, 40, 128)
    rows[17] = rows[3]
    rows[30] = rows[3]
    keys = _int_rows(rng, 64, 128)
    keys[:8] = rows[3] * 2   # the duplicated row is (one of) the best for these
    got = oracle.update_assign(keys, rows)
    exact = keys.astype(np.int64) @ rows.astype(np.int64).T
    assert np.array_equal(got, np.argmax(exact, axis=1))
    assert np.all(got[:8] == 3)


def test_assign_zero_rows_and_signed_zero(oracle):
    """Padding slots of the shadow are zero rows with similarity 0: a key
    whose similarities to every occupied row are negative goes to the first
    zero row; a zero key ties everywhere (+0 and -0 alike) and goes to row 0."""
    d = 128
    rows = np.zeros((10, d), np.float32)
    rows[:6, 0] = np.arange(1, 7, dtype=np.float32)   # occupied rows: positive first dim
    key_neg = np.zeros((1, d), np.float32)
    key_neg[0, 0] = -1.0
    assert oracle.update_assign(key_neg, rows)[0] == 6
    zero = np.zeros((1, d), np.float32)
    rows_neg = -np.abs(rows)   # products -0.0 for the zero key
    assert oracle.update_assign(zero, rows_neg)[0] == 0
    neg_zero_key = np.full((1, d), -0.0, np.float32)
    assert oracle.update_assign(neg_zero_key, rows)[0] == 0


def test_assign_random_matches_fp64_away_from_ties(oracle):
    """Random data: the fp32 chain's arg-max equals the fp64 arg-max wherever
    the best two fp64 values differ by more than the chain's error bound."""
    rng = np.random.default_rng(2)
    rows = rng.standard_normal((300, 128)).astype(np.float32)
    keys = rng.standard_normal((200, 128)).astype(np.float32)
    got = oracle.update_assign(keys, rows)
    ref = keys.astype(np.float64) @ rows.astype(np.float64).T
    top2 = np.sort(ref, axis=1)[:, -2:]
    bound = 128 * 2.0 ** -23 * (np.abs(keys).astype(np.float64) @ np.abs(rows).astype(np.float64).T).max(axis=1)
    clear = (top2[:, 1] - top2[:, 0]) > 2 * bound
    assert clear.sum() > 150
    assert np.array_equal(got[clear], np.argmax(ref, axis=1)[clear])


def _state(oracle, n_rows=12, n_active=9, threshold=3, cap=16, seed=3):
    rng = np.random.default_rng(seed)
    shadow = np.zeros((1, n_rows, 128), np.float32)
    shadow[0, :n_active] = rng.integers(-3, 4, (n_active, 128)).astype(np.float32)
    sizes = np.zeros((1, n_rows), np.int32)
    sizes[0, :n_active] = rng.integers(1, 9, n_active)
    return oracle.OnlineUpdateOracle(shadow, sizes, n_rows - 1, threshold, cap), shadow, sizes


def _bits_of(oracle, x):
    return oracle.f32_to_bf16(np.asarray(x, np.float32))


def test_refresh_running_mean_closed_form(oracle):
    """(shadow * count + sum of new keys) / (count + new) on integer data whose
    result is exactly representable, for the rows whose delta count reached
    the threshold only; their delta state resets (async_update.py:135-143)."""
    upd, shadow, sizes = _state(oracle, threshold=3)
    c = 2
    # keys equal to row c (scaled) are assigned to it; 4 >= threshold of them
    base = shadow[0, c]
    keys = np.stack([base * 2, base * 2, base * 3, base * 1]).astype(np.float32)
    ids = upd.assign(_bits_of(oracle, keys)[None], [40, 41, 42, 43])
    assert np.all(ids[0] == c)
    assert upd.dc[0, c] == 4
    upd.refresh()
    n = int(sizes[0, c])
    want = (base * n + keys.sum(axis=0)) / (n + 4)
    np.testing.assert_allclose(upd.shadow[0, c], want, rtol=2 ** -23, atol=0)
    assert upd.cc[0, c] == n + 4 and upd.dc[0, c] == 0 and not upd.ds[0, c].any()
    assert upd.replaced[0] == [c]
    # rows below the threshold keep their centroid and accumulate
    before = upd.shadow.copy()
    upd.assign(_bits_of(oracle, keys[:2])[None], [44, 45])
    upd.refresh()
    assert upd.dc[0, c] == 2 and np.array_equal(upd.shadow, before)


def test_ring_order_and_delta_match_rules(oracle):
    """Ring entries in index order, saturating count, wrap-around; matches =
    kept cells, plus the padding id only when fewer than nprobe cells pass
    (the reference's `selected` then holds padding slots); truncation to the
    execution-buffer rows left (async_update.py:41-76)."""
    upd, shadow, _ = _state(oracle, n_rows=12, n_active=11, cap=5)
    pad = upd.padding_id   # 11: the first zero row is the padding id here
    neg = np.zeros((1, 128), np.float32)
    neg[0, 0] = -1.0
    shadow_pos = np.abs(upd.shadow)
    shadow_pos[0, :11, 0] += 1.0
    upd.shadow = shadow_pos
    keys = np.concatenate([shadow_pos[0, [1, 4]], neg, shadow_pos[0, [4]]]).astype(np.float32)
    ids = upd.assign(_bits_of(oracle, keys)[None], [10, 11, 12, 13])[0]
    assert list(ids) == [1, 4, pad, 4]
    assert upd.n[0] == 4 and upd.pos[0] == 4
    # kept {4}: entries 1 and 3; padding present when len(kept) < nprobe
    assert upd.delta_rows(0, [4], nprobe=1, exec_rows=100, rows_sel=0) == [11, 13]
    assert upd.delta_rows(0, [4], nprobe=2, exec_rows=100, rows_sel=0) == [11, 12, 13]
    assert upd.delta_rows(0, [4, 1], nprobe=3, exec_rows=100, rows_sel=0) == [10, 11, 12, 13]
    assert upd.delta_rows(0, [4, 1], nprobe=3, exec_rows=100, rows_sel=98) == [10, 11]
    assert upd.delta_rows(0, [4, 1], nprobe=3, exec_rows=100, rows_sel=120) == []
    # wrap: two more entries overwrite index 4 then 0; the count saturates
    upd.assign(_bits_of(oracle, keys[:2])[None], [20, 21])
    assert upd.n[0] == 5 and upd.pos[0] == 1
    assert list(upd.ring_row[0]) == [21, 11, 12, 13, 20]
    assert upd.delta_rows(0, [1], nprobe=1, exec_rows=100, rows_sel=0) == [20]
