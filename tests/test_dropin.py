"""The reference-named drop-in: adpimi_cache + imi_decode_attn.

CPU tests check the cache contract (sizes, errors, static_len rule, reuse
rules) against the reference formulas (cache.py:133-153, 380-395;
attn_hub/sparse_imi.py:1-10).  GPU tests run a small model-shaped prefill and
decode through the cache exactly as model_hub does (prefill_update_kv_cache
per layer, prepare_cache, decode_update_kv_cache + imi_decode_attn per layer)
and compare every layer with the oracle: selected cells bit-exact, output
within 2e-2 abs + 1e-2 rel of fp64 attention."""
import math

import numpy as np
import pytest
import torch

from conftest import gpu_available

DEV = "cuda:0"


def _cache(layer_mapping=None, **kw):
    from adaptiveimi_amd.cache_hub.adaptive_imi import adpimi_cache

    args = dict(valid_start=[0], layer_num=2, batch_size=1, max_length=6100, num_key_value_heads=8, num_heads=32,
                head_dim=128, dtype=torch.bfloat16, layer_mapping=layer_mapping or {"0": "cpu", "1": "cpu"},
                max_new_length=4, input_length=6096, static_pattern_start=32, static_pattern_end=64, core=4,
                pages_per_cluster=2, retrieval_budget=0.1, cache_ratio=0.05, buffer_cluster_num=32, prefill_bsz=1,
                num_gpus=1, model_size=8, subspace_parts=2,
                runtime_config={"kmeans": {"k1": 32, "k2": 32, "max_iters": 6, "early_stop_min_iter": 6,
                                            "init": "first"}})
    args.update(kw)
    return adpimi_cache(**args)


def test_cache_sizes_follow_reference():
    c = _cache()
    # cache.py:133-153 with input 6096, max_length 6100, max_new_length 4
    assert c.input_length == 6096 and c.capacity_input_length == 6096
    assert c.list_capacity == 6096 - 96 and c.list_stride == 6000
    assert c.static_capacity == 96 + 3 and c.static_stride == 99
    assert c.build_index_when_prefilling
    assert c.static_pattern_total == 96 and c.group_size == 4 and c.batch_groups == 8
    assert tuple(c.steady_zone_keys[0].shape) == (1, 8, 99, 128)
    assert c.attn_func == c.dense_attention


def test_cache_rejects_what_the_reference_rejects():
    with pytest.raises(ValueError, match="batch_size=1"):
        _cache(batch_size=2)
    with pytest.raises(ValueError, match="subspace_parts"):
        _cache(subspace_parts=3)
    with pytest.raises(ValueError, match="input length"):
        _cache(input_length=0)


def test_async_update_config():
    """cache.py:305-311: enabled, batch (16), threshold (16), delta_tokens (512)."""
    c = _cache(runtime_config={"async_update": {"enabled": True}})
    assert c.async_update_enabled and (c.async_update_batch, c.async_update_threshold,
                                       c.async_update_delta_tokens) == (16, 16, 512)
    c = _cache(runtime_config={"async_update": {"enabled": True, "batch": 4, "threshold": 0, "delta_tokens": 32}})
    assert (c.async_update_batch, c.async_update_threshold, c.async_update_delta_tokens) == (4, 1, 32)
    assert not _cache().async_update_enabled
    with pytest.raises(ValueError, match="batch"):
        _cache(runtime_config={"async_update": {"enabled": True, "batch": 100}})
    with pytest.raises(ValueError, match="delta_tokens"):
        _cache(runtime_config={"async_update": {"enabled": True, "delta_tokens": 4096}})


def test_static_len_rule():
    from adaptiveimi_amd.attn_hub.sparse_imi import imi_decode_attn

    class Stub:
        static_pattern_total = 100
        layer_num = 3

        def attn_func(self, q, layer_idx, static_len):
            return (layer_idx, static_len, q.is_contiguous())

    q = torch.zeros(1, 4, 1, 8).transpose(1, 2)   # non-contiguous [1, 1, 4, 8]
    assert imi_decode_attn(q, None, None, 0, Stub()) == (0, 101, True)
    assert imi_decode_attn(q, None, None, 2, Stub()) == (2, 100, True)


def test_reuse_rules():
    c = _cache()
    assert c.can_reuse_for_next_sequence([0], 4, 6096)
    assert not c.can_reuse_for_next_sequence([0], 4, 7000)       # list too long
    assert not c.can_reuse_for_next_sequence([0], 10, 6096)      # steady zone too short
    assert not c.can_reuse_for_next_sequence([0, 0], 4, 6096)
    c.reset_for_next_sequence([0], 3, 5000)
    assert c.context == 0 and c.list_stride == 5000 - 96 and c.attn_func == c.dense_attention
    with pytest.raises(ValueError, match="cannot reuse"):
        c.reset_for_next_sequence([0], 4, 9000)


def test_index_stats_before_build():
    s = _cache().get_index_stats()
    assert s["ready_layers"] == 0 and s["non_empty_clusters_total"] == 0
    assert s["total_heads"] == 16 and math.isclose(s["ideal_clusters_per_head"], 6000 / 16)


def test_ragged_budget_rules():
    """Per-head budgets of a ragged launch (sequence-major heads)."""
    from adaptiveimi_amd import ops as o

    b = o.Budget.ragged([o.Budget(102, 300, 38), o.Budget(102, 1200, 150)], 2)
    assert (b.max_tokens, b.buffer_pages, b.sel_cap) == (1200, 150, 102)
    assert b.head_max_tokens == [300, 300, 1200, 1200] and b.head_buffer_pages == [38, 38, 150, 150]
    with pytest.raises(ValueError, match="share nprobe"):
        o.Budget.ragged([o.Budget(102, 300, 38), o.Budget(50, 1200, 150)], 2)


# ----------------------------------------------------------------- GPU --

def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
@pytest.mark.parametrize("ks", [(32, 32), (6, 6, 6, 6), (8, 8, 8, 8), (375,)])   # (375,): IVF, k = round(6000 / 16)
def test_model_shaped_prefill_and_decode_match_oracle(ks):
    from adaptiveimi_amd import synthetic
    from adaptiveimi_amd.attn_hub.sparse_imi import imi_decode_attn
    from oracle import oracle as orc

    print(f"[dropin] 2 layers, S=6096, ks={ks}, 2 decode steps", flush=True)
    L, S, H, G, D = 2, 6096, 8, 4, 128
    kcfg = {f"k{i + 1}": k for i, k in enumerate(ks)}
    kcfg.update(max_iters=6, early_stop_min_iter=6, init="first")
    cache = _cache(layer_mapping={"0": DEV, "1": DEV}, subspace_parts=len(ks) if len(ks) > 1 else 0,
                   runtime_config={"kmeans": kcfg})
    kv = []
    for layer in range(L):
        k, v = synthetic.make_kv(H, S + 2, seed=40 + layer)
        kv.append((k, v))
        pk = k[:, :S].transpose(0, 1).unsqueeze(0).contiguous().to(DEV)   # [1, S, H, D]
        pv = v[:, :S].transpose(0, 1).unsqueeze(0).contiguous().to(DEV)
        rk, rv = cache.prefill_update_kv_cache(None, pk, pv, layer, 0)
        assert rk.shape == pk.shape
        cache.sync(layer, 0)
    assert cache.context == S and cache.attn_func == cache.sparse_attention
    cache.prepare_cache()
    ncells = int(np.prod(ks))
    assert cache.n_centroids == ncells + 1
    assert cache.nprobe == round(ncells * 0.1) and cache.max_retrieval_tokens == int(0.1 * 6000)

    # oracle index of each layer
    heads_by_layer = []
    for layer in range(L):
        k, v = kv[layer]
        mid_k, mid_v = _bits(k[:, 32:S - 64]), _bits(v[:, 32:S - 64])
        heads = []
        for h in range(H):
            labs, cents, _ = orc.kmeans_head(orc.bf16_to_f32(mid_k[h]), list(ks), 6, early_stop_min_iter=6)
            r = orc.compact_reorg(labs, list(ks))
            assert np.array_equal(cache.token_perm[layer][h].cpu().numpy(), r["perm"]), "cell order differs"
            heads.append(dict(n_active=r["n_active"], offsets=r["offsets"], gids=r["gids"],
                              merged=orc.merged_centroids(cents, r["gids"], list(ks)),
                              list_keys=mid_k[h][r["perm"]], list_values=mid_v[h][r["perm"]]))
        heads_by_layer.append(heads)

    for step in range(2):
        for layer in range(L):
            k, v = kv[layer]
            nk = k[:, S + step].reshape(1, 1, H, D).to(DEV)
            nv = v[:, S + step].reshape(1, 1, H, D).to(DEV)
            cache.decode_update_kv_cache(nk, nv, layer)
            q = synthetic.make_queries(k[:, :S], G, seed=10 * step + layer)[0]      # [H, G, D]
            qs = q.reshape(1, 1, H * G, D).to(DEV)
            out = imi_decode_attn(qs, nk, nv, layer, cache)
            assert tuple(out.shape) == (1, 1, H * G, D)
            static_len = cache.static_pattern_total + (1 if layer < L - 1 else 0)
            sk = _bits(cache.steady_zone_keys[layer][0])
            sv = _bits(cache.steady_zone_values[layer][0])
            ref, rs, rm, rrows = orc.decode_step(_bits(q), heads_by_layer[layer], sk, sv, static_len,
                                                 cache.n_centroids, cache.nprobe, cache.max_retrieval_tokens,
                                                 cache.buffer_size)
            plan = cache._plans[layer]
            assert np.array_equal(plan.selection["n_selected"].cpu().numpy(), rm), "selected cell counts differ"
            cells = plan.selection["sel_cell"].cpu().numpy()
            nrows = plan.selection["n_rows"].cpu().numpy()
            for h in range(H):   # same cells in rank order (compact id -> global id), same row totals
                gid = heads_by_layer[layer][h]["gids"]
                assert np.array_equal(cells[h, : rm[h]], gid[rs[h, : rm[h]]]), f"layer {layer} head {h}: cells"
                assert nrows[h] == len(rrows[h]), f"layer {layer} head {h}: rows"
            got = out.float().cpu().numpy().reshape(H, G, D)
            err = np.abs(got - ref)
            assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), f"layer {layer} step {step}: max err {err.max()}"
    assert cache.static_pattern_total == 96 + 2
    stats = cache.get_index_stats()
    assert stats["ready_layers"] == 2 and stats["non_empty_clusters_total"] > 0


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_dense_attention_before_index():
    """runtime.py:393-402: before the last layer's prefill the cache attends
    the steady zone only."""
    print("[dropin] dense attention over the steady zone", flush=True)
    from adaptiveimi_amd import synthetic
    from oracle import oracle as orc

    cache = _cache(layer_mapping={"0": DEV, "1": DEV})
    k, v = synthetic.make_kv(8, 99, seed=3)
    cache.steady_zone_keys[0][0].copy_(k.to(DEV))
    cache.steady_zone_values[0][0].copy_(v.to(DEV))
    q = synthetic.make_queries(k, 4, seed=1)[0]
    for static_len in (1, 57, 99):
        out = cache.attn_func(q.reshape(1, 1, 32, 128).to(DEV), 0, static_len)
        rows = [np.arange(static_len)] * 8
        ref = orc.attention(_bits(q), _bits(k), _bits(v), rows)
        got = out.float().cpu().numpy().reshape(8, 4, 128)
        err = np.abs(got - ref)
        assert np.all(err <= 2e-2 + 1e-2 * np.abs(ref)), f"static_len {static_len}: {err.max()}"


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_side_stream_build_matches_inline_build():
    """The index build on the side stream (the default, like the reference's
    background LayerPipeline) gives the same index and decode output as the
    build on the caller's stream, with the prefill tensors freed right after
    prefill_update_kv_cache returns."""
    from adaptiveimi_amd import synthetic
    from adaptiveimi_amd.attn_hub.sparse_imi import imi_decode_attn

    print("[dropin] side-stream build vs inline build", flush=True)
    L, S, H, G, D = 2, 6096, 8, 4, 128
    kv = [synthetic.make_kv(H, S + 1, seed=70 + layer) for layer in range(L)]
    outs = []
    for async_build in (False, True):
        cfg = {"kmeans": {"k1": 32, "k2": 32, "max_iters": 4, "early_stop_min_iter": 4, "init": "first"},
               "pipeline": {"async_build": async_build}}
        cache = _cache(layer_mapping={"0": DEV, "1": DEV}, runtime_config=cfg)
        assert cache.async_build == async_build
        for layer in range(L):
            k, v = kv[layer]
            pk = k[:, :S].transpose(0, 1).unsqueeze(0).contiguous().to(DEV)
            pv = v[:, :S].transpose(0, 1).unsqueeze(0).contiguous().to(DEV)
            cache.prefill_update_kv_cache(None, pk, pv, layer, 0)
            cache.sync(layer, 0)
            del pk, pv                      # the side stream still reads them
            torch.empty(8 << 20, dtype=torch.uint8, device=DEV).fill_(0xAB)   # reuse pressure
        cache.prepare_cache()
        res = []
        for layer in range(L):
            k, v = kv[layer]
            nk = k[:, S].reshape(1, 1, H, D).to(DEV)
            cache.decode_update_kv_cache(nk, v[:, S].reshape(1, 1, H, D).to(DEV), layer)
            q = synthetic.make_queries(k[:, :S], G, seed=layer)[0].reshape(1, 1, H * G, D).to(DEV)
            res.append(imi_decode_attn(q, nk, None, layer, cache).clone())
            res += [cache.token_perm[layer].clone(), cache.list_keys[layer].clone(), cache.centroids[layer].clone()]
        torch.cuda.synchronize()
        outs.append(res)
    for a, b in zip(*outs):
        assert torch.equal(a, b)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_host_tier_dropin_matches_oracle():
    """runtime_config["host_tier"]: lists in pinned host memory, the GPU block
    cache of round(n_centroids * cache_ratio) clusters x pages_per_cluster
    pages (runtime.py:48-53); same selection and attention as the oracle."""
    from adaptiveimi_amd import ops, synthetic
    from adaptiveimi_amd.attn_hub.sparse_imi import imi_decode_attn
    from oracle import oracle as orc

    print("[dropin host tier] 2 layers, S=6096, ks=(32, 32), 3 decode steps", flush=True)
    L, S, H, G, D, ks = 2, 6096, 8, 4, 128, (32, 32)
    cache = _cache(layer_mapping={"0": DEV, "1": DEV}, max_new_length=5, max_length=6101,
                   runtime_config={"kmeans": {"k1": 32, "k2": 32, "max_iters": 6, "early_stop_min_iter": 6,
                                              "init": "first"},
                                   "host_tier": {"enabled": True}})
    kv = []
    for layer in range(L):
        k, v = synthetic.make_kv(H, S + 3, seed=60 + layer)
        kv.append((k, v))
        pk = k[:, :S].transpose(0, 1).unsqueeze(0).contiguous().to(DEV)
        pv = v[:, :S].transpose(0, 1).unsqueeze(0).contiguous().to(DEV)
        cache.prefill_update_kv_cache(None, pk, pv, layer, 0)
        cache.sync(layer, 0)
    cache.prepare_cache()
    heads_by_layer = []
    for layer in range(L):
        k, v = kv[layer]
        mid_k, mid_v = _bits(k[:, 32:S - 64]), _bits(v[:, 32:S - 64])
        heads = []
        for h in range(H):
            labs, cents, _ = orc.kmeans_head(orc.bf16_to_f32(mid_k[h]), list(ks), 6, early_stop_min_iter=6)
            r = orc.compact_reorg(labs, list(ks))
            heads.append(dict(n_active=r["n_active"], offsets=r["offsets"], gids=r["gids"],
                              merged=orc.merged_centroids(cents, r["gids"], list(ks)),
                              list_keys=mid_k[h][r["perm"]], list_values=mid_v[h][r["perm"]]))
        heads_by_layer.append(heads)
    for step in range(3):
        for layer in range(L):
            k, v = kv[layer]
            nk = k[:, S + step].reshape(1, 1, H, D).to(DEV)
            nv = v[:, S + step].reshape(1, 1, H, D).to(DEV)
            cache.decode_update_kv_cache(nk, nv, layer)
            q = synthetic.make_queries(k[:, :S], G, seed=layer + 10 * (step % 2))[0]   # steps 0 and 2 repeat
            out = imi_decode_attn(q.reshape(1, 1, H * G, D).to(DEV), nk, nv, layer, cache)
            plan = cache._plans[layer]
            assert isinstance(plan, ops.HostTierPlan) and cache.list_keys[layer] is None
            static_len = cache.static_pattern_total + (1 if layer < L - 1 else 0)
            ref, rs, rm, rrows = orc.decode_step(_bits(q), heads_by_layer[layer], _bits(cache.steady_zone_keys[layer][0]),
                                                 _bits(cache.steady_zone_values[layer][0]), static_len,
                                                 cache.n_centroids, cache.nprobe, cache.max_retrieval_tokens,
                                                 cache.buffer_size)
            assert np.array_equal(plan.h_nsel.numpy(), rm)
            cells = plan.h_sel.numpy()
            for h in range(H):
                gid = heads_by_layer[layer][h]["gids"]
                assert np.array_equal(cells[h, : rm[h]], gid[rs[h, : rm[h]]]), (layer, h)
                assert int(plan.plan.selection["n_rows"][h]) == len(rrows[h]), (layer, h)
            got = out.float().cpu().numpy().reshape(H, G, D)
            assert np.all(np.abs(got - ref) <= 2e-2 + 1e-2 * np.abs(ref)), (layer, step)
    assert all(cache._plans[layer].hits > 0 for layer in range(L))   # the repeated step hit the cache


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")
def test_host_tier_keeps_lists_off_the_device():
    """With the host tier each layer's lists go to pinned host memory during
    its build (indexing.py:98-107 keeps them in host memory from the start),
    so after the prefill of every layer the device holds none of them: the
    allocated device memory grows by the per-layer metadata only, while the
    HBM-resident cache holds every layer's lists."""
    from adaptiveimi_amd import synthetic

    print("[dropin host tier] device memory after prefill, 3 layers", flush=True)
    L, S, H, D = 3, 6096, 8, 128
    kv = [synthetic.make_kv(H, S, seed=90 + layer) for layer in range(L)]
    list_bytes = 2 * H * (S - 96) * D * 2      # one layer's keys + values

    def prefill(host):
        cache = _cache(layer_mapping={str(i): DEV for i in range(L)}, layer_num=L,
                       runtime_config={"kmeans": {"k1": 32, "k2": 32, "max_iters": 3, "early_stop_min_iter": 3,
                                                  "init": "first"},
                                       "host_tier": {"enabled": host}})
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        for layer in range(L):
            k, v = kv[layer]
            pk = k.transpose(0, 1).unsqueeze(0).contiguous().to(DEV)
            pv = v.transpose(0, 1).unsqueeze(0).contiguous().to(DEV)
            cache.prefill_update_kv_cache(None, pk, pv, layer, 0)
            cache.sync(layer, 0)
            del pk, pv
        torch.cuda.synchronize()
        return cache, torch.cuda.memory_allocated() - before

    hbm, grown_hbm = prefill(False)      # also warms the shared k-means / index workspaces
    assert grown_hbm >= L * list_bytes
    del hbm
    host, grown_host = prefill(True)
    assert grown_host < list_bytes // 4, (grown_host, list_bytes)
    for layer in range(L):
        hk, hv = host.host_lists[layer]
        assert host.list_keys[layer] is None and hk.is_pinned() and hv.is_pinned()
        # the pinned lists hold the permuted rows of the middle keys
        k, v = kv[layer]
        perm = host.token_perm[layer].cpu().long()
        mid_k, mid_v = k[:, 32:S - 64], v[:, 32:S - 64]
        for h in (0, H - 1):
            assert torch.equal(hk[h], mid_k[h, perm[h]]) and torch.equal(hv[h], mid_v[h, perm[h]])
