"""Seeded random shapes through the GPU parity checks: 2-way decode steps,
4-way selections and drop-in runs with the online update, each against the
oracle as in the fixed-shape tests (selections bit-exact, attention within
2e-2 abs / 1e-2 rel).  The shapes are drawn once from fixed seeds, so every
run checks the same cases."""
import random

import pytest

from conftest import gpu_available

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a HIP device")]


@pytest.fixture(scope="module")
def ops():
    from adaptiveimi_amd import ops as o

    return o


def _decode_cases(n, seed):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        ks = (rng.choice([8, 16, 24, 32, 48, 64, 96, 128]), rng.choice([8, 16, 32, 64, 100, 128]))
        T = rng.choice([1500, 3000, 7000, 12000, 30000, 60000])
        budget = rng.choice([0.02, 0.05, 0.1])
        tiles = T * budget >= 600 and rng.random() < 0.25
        out.append((T, ks, rng.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]), rng.choice([0, 1, 33, 96, 200]), tiles, budget))
    return out


def _select4_cases(n, seed):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        kk = rng.choice([3, 4, 5, 6, 8, 10, 12, 16, 20, 24, 32])
        ks = tuple(max(2, kk + rng.choice([-1, 0, 0, 1])) for _ in range(4))
        out.append((rng.choice([3000, 9000, 20000, 50000, 120000]), ks, rng.choice([0.01, 0.02, 0.05, 0.1, 0.2, 0.4]),
                    rng.choice([1, 2, 4, 7, 8, 16]), rng.randrange(1000)))
    return out


def _online_cases(n, seed):
    rng = random.Random(seed)
    out = []
    for _ in range(n):
        kind = rng.choice(["2", "2", "4", "ivf"])
        ks = {"2": (rng.choice([8, 16, 32, 48]),) * 2, "4": (rng.choice([4, 6, 8]),) * 4,
              "ivf": (rng.choice([64, 200, 300]),)}[kind]
        batch = rng.choice([2, 4, 8])
        host = rng.random() < 0.25
        tiles = (not host) and rng.random() < 0.25
        # 24 steps: at least two updates land for every batch size drawn
        out.append((ks, 24, batch, rng.choice([1, 2, 3, 5]), rng.choice([24, 40, 64]), host, tiles))
    return out


@pytest.mark.parametrize("T,ks,G,static_len,tiles,budget", _decode_cases(12, 7))
def test_random_decode_steps(ops, oracle, T, ks, G, static_len, tiles, budget):
    import test_gpu_parity as p

    p.test_decode_step_matches_oracle(ops, oracle, T, ks, G, static_len, tiles, budget)


@pytest.mark.parametrize("T,ks,budget,G,seed", _select4_cases(10, 5))
def test_random_4way_selections(ops, oracle, T, ks, budget, G, seed):
    import test_gpu_parity as p

    p.test_select_4way_bit_exact(ops, oracle, T, ks, budget, G, seed)


@pytest.mark.parametrize("ks,steps,batch,thr,ring,host,tiles", _online_cases(6, 3))
def test_random_online_update_runs(ops, oracle, monkeypatch, ks, steps, batch, thr, ring, host, tiles):
    import test_gpu_online_update as u

    u.test_cache_with_async_update_matches_oracle(ops, oracle, monkeypatch, ks, steps, batch, thr, ring, host, tiles)
