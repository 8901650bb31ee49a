"""bench.py's host-side pieces, without a GPU: the per-configuration CPU
oracle sample, the traffic file and the whole-call traffic figure."""
import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402
from cast_amd import scenarios as SC  # noqa: E402


def test_every_named_workload_exists():
    for name in bench.ATTN_WORKLOADS:
        base = name[:-5] if name.endswith(("-fp32", "-fp16")) else name
        assert base in SC.CONFIGS, name
    assert set(bench.CPU_SAMPLED) <= set(bench.ATTN_WORKLOADS)


def test_traffic_file_entries():
    entries = json.loads(bench.TRAFFIC_FILE.read_text())
    assert "qwen3-8b-b8-ctx8k-p128" in entries
    for name, e in entries.items():
        base = name[:-5] if name.endswith(("-fp32", "-fp16")) else name
        assert base in SC.CONFIGS, name
        assert e["hbm_bytes_per_launch"] == pytest.approx(e["read_bytes"] + e["write_bytes"], abs=2)
        if "combine_bytes" in e:
            assert e["combine_bytes"] == pytest.approx(e["combine_read_bytes"] + e["combine_write_bytes"], abs=2)


def test_whole_call_traffic_adds_the_combine():
    wl = SC.qwen3_headline()
    e = {"hbm_bytes_per_launch": 300, "combine_bytes": 50}
    w = bench.whole_call_traffic(wl, e)
    assert w["bytes"] == 350 and w["combine_bytes"] == 50
    assert w["ratio"] == round(350 / wl.algorithmic_bytes(), 3)
    assert bench.whole_call_traffic(wl, None) is None
    stress = bench.whole_call_traffic(SC.stress_mixed(), bench.traffic_of("qwen3-8b-stress-b32"))
    assert stress["combine_bytes"] == 0 and 0.9 < stress["ratio"] < 1.2


def test_cpu_sample_scales_by_score_count():
    wl = SC.cpu_plumbing()
    r = bench.cpu_baseline_sample(wl, budget_s=0.2)
    assert r["unit"] == "us/call" and r["kind"] == "port" and r["value"] > 0
    assert "requests 0-0 of 1" in r["sample"]
    rg = SC.random_parent_batch(seed=3, B=4, Hq=4, Hkv=2, D=64, s_lo=32, s_hi=96, p_lo=4, p_hi=16)
    r = bench.cpu_baseline_sample(rg, budget_s=0.2)
    assert r["value"] > 0 and "of 4" in r["sample"]


def test_a_failing_secondary_workload_is_recorded_not_fatal(monkeypatch):
    # every secondary workload replaced by a fake (no device work); one raises
    def fake_attn(dev, name, steps, warmup, cpu=False):
        if name == "qwen3-8b-ragged":
            raise RuntimeError("planted failure")
        return dict(us_per_call=1.0, steps=steps, warmup=warmup)

    monkeypatch.setattr(bench, "attn_workload", fake_attn)
    for fn in ("store_layout", "kv_append", "cache_gather", "draft_trees", "graph_replay", "verify_round"):
        monkeypatch.setattr(bench, fn, lambda dev, n, w: dict(ok=1))
    monkeypatch.setattr(bench, "bitmask_lines", lambda dev, n, w: {"tree_bitmask": dict(us_per_call=1.0)})
    res = bench.secondary(None, 50, 20, cpu=False)
    assert res["qwen3-8b-ragged"] == {"error": "RuntimeError: planted failure"}
    assert res["qwen3-8b-single"]["us_per_call"] == 1.0
    assert res["verify_round"] == {"ok": 1, "steps": 50, "warmup": 20}
    assert res["tree_bitmask"]["steps"] == 50
