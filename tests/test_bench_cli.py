"""bench.py's command line and bookkeeping, without a GPU: the one-GPU
refusal, the workload table and the traffic figure read from the committed
counter summary."""
import json
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))


def _parse(monkeypatch, argv):
    import bench

    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    return bench.parse()


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 2
    msg = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in msg["error"]


def test_default_workload_is_the_north_star(monkeypatch):
    a = _parse(monkeypatch, [])
    assert a.workload == "config1"
    assert (a.layers, a.context, a.kv_heads, a.groups, tuple(a.ks), a.iters, a.budget) == \
        (32, 131072, 8, 4, (64, 64), 10, 0.1)
    assert a.cpu_baseline == 1 and a.online_layers == 4
    # the legs on the other shapes ride in the default line, two layers each
    assert (a.config3_layers, a.config4_layers, a.host_tier_layers) == (2, 2, 2)
    # the end-to-end configs[1] leg: 32 layers, 131072-token prompt, 256 decode tokens
    assert (a.e2e_layers, a.e2e_context, a.e2e_decode) == (32, 131072, 256)
    import bench

    name = bench.workload_name(a, 32, 8, 4, tuple(a.ks))
    assert name.startswith("configs[1]") and "131072" in name and "budget 0.1" in name


def test_other_workloads_and_overrides(monkeypatch):
    a = _parse(monkeypatch, ["--workload", "config3"])
    assert (a.layers, a.context, a.batch, a.groups, tuple(a.ks), a.fixed_tokens, a.budget) == \
        (16, 262144, 2, 8, (32, 32, 32, 32), 4096, None)
    assert a.cpu_baseline == 0 and a.online_layers == 0 and a.e2e_layers == 0   # quoted on the default workload only
    assert a.config3_layers == 0 and a.config4_layers == 0 and a.host_tier_layers == 0
    a = _parse(monkeypatch, ["--workload", "config2"])
    assert (a.layers, a.kv_heads, a.groups, a.batch, tuple(a.contexts), tuple(a.ks), a.budget) == \
        (28, 4, 7, 4, (32768, 65536, 98304, 131072), (64, 64), 0.1)
    import bench

    assert "ragged batch of 4 sequences" in bench.workload_name(a, 28, 16, 7, (64, 64))
    a = _parse(monkeypatch, ["--workload", "config4", "--layers", "2", "--k", "96"])
    assert (a.layers, a.context, tuple(a.ks), a.sample, a.budget) == (2, 1048576, (96, 96), 65536, 0.02)


def test_traffic_comes_from_the_committed_summary_of_the_same_workload(monkeypatch):
    """roofline.traffic is the counter figure of the summary whose workload
    line names this exact workload, and null for any other workload."""
    import bench

    a = _parse(monkeypatch, [])
    name = bench.workload_name(a, 32, 8, 4, tuple(a.ks))
    f = ROOT / "profiles" / "fixed_attention_kernel_traffic_config1.md"
    assert bench.measured_traffic(name + " (other)") is None
    if not f.exists():
        assert bench.measured_traffic(name) is None
        return
    text = f.read_text()
    t = bench.measured_traffic(name)
    assert t is not None and f"traffic_bytes_per_launch: {t}" in text and f"workload: {name}" in text
    assert 40_000_000 < t < 60_000_000
    c3 = _parse(monkeypatch, ["--workload", "config3"])
    assert bench.measured_traffic(bench.workload_name(c3, 16, 16, 8, tuple(c3.ks))) is None


def test_build_roofline_fields(monkeypatch):
    import bench

    a = _parse(monkeypatch, [])
    r = bench.build_roofline(a, 8 * (131072 - 96), 131072 - 96, (64, 64), 3.0)   # listed tokens over the 8 heads
    # 2 T k D per iteration per head: 2 * 130976 * 64 * 128 * 8 * 10
    assert r["estep_gflop"] == round(2 * 130976 * 64 * 128 * 8 * 10 / 1e9, 2)
    assert r["bytes_min"] == 5 * 130976 * 128 * 2 * 8
    assert abs(r["hbm_frac"] - r["bytes_min"] / 3e-3 / 8e12) < 1e-4
