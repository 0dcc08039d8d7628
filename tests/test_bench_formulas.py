"""The bench line's accounting on the CPU: algorithmic bytes per decode token,
prefill FLOPs, workload names and the committed-traffic lookup, against the
closed forms of the workloads (1.5B: 28 layers of 46,797,824 bf16 weights,
the final norm, the tied 151936 x 1536 head and one embedding row per token;
KV 28 x 2 x 2 x 128 values per position)."""
import importlib.util
import json
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(ROOT, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_decode_bytes_per_token(bench):
    s = bench.myos.preset(bench.myos.SHAPE_QWEN25_1_5B)
    per_layer = 46_797_824  # q/k/v/o/gate/up/down + biases + two norms, in weights
    assert bench.weight_bytes(s) == 2 * (28 * per_layer + 1536 + 151936 * 1536 + 1536)
    assert bench.weight_bytes(s) == 3_087_431_680
    # 14,336 values per cached position (28 layers x K and V x 2 kv heads x 128),
    # 4 bytes each in an f32 cache and 2 in bf16
    assert bench.kv_bytes_per_token(s, 1, 4) == 14_336 * 4
    assert bench.kv_bytes_per_token(s, 256, 2) == 256 * 14_336 * 2


def test_s1_launch_bytes_match_the_profile(bench):
    # the S1 launch: 128 steps at cache lengths 129..256, f32 cache
    s = bench.myos.preset(bench.myos.SHAPE_QWEN25_1_5B)
    total = sum(bench.weight_bytes(s) + bench.kv_bytes_per_token(s, q, 4) for q in range(129, 257))
    assert total == 396_604_211_200
    # the long-context launch: 256 steps at 2049..2304, bf16 cache
    total = sum(bench.weight_bytes(s) + bench.kv_bytes_per_token(s, q, 2) for q in range(2049, 2305))
    assert total == 806_358_089_728


def test_prefill_flops(bench):
    s = bench.myos.preset(bench.myos.SHAPE_QWEN25_1_5B)
    linear = 1_310_195_712  # weights per row: every projection of every layer
    for n in (128, 2048):
        attn = 4 * 128 * 12 * 28 * n * (n + 1) / 2
        assert bench.prefill_flops(s, n) == pytest.approx(2 * n * linear + attn + 2 * 151936 * 1536)
    assert bench.prefill_flops(s, 128) == pytest.approx(337.3e9, rel=1e-3)
    assert bench.prefill_flops(s, 2048) == pytest.approx(5.728e12, rel=1e-3)


def test_workload_names(bench):
    assert bench.workload_name(False, 128, 128, "f32").startswith("Qwen2.5-1.5B-shape S1:")
    assert bench.workload_name(False, 2048, 256, "bf16").startswith("Qwen2.5-1.5B-shape long-context:")
    assert bench.workload_name(True, 128, 128, "f32").startswith("Qwen2.5-7B-shape S1:")
    assert "S1" not in bench.workload_name(False, 64, 32, "f32")


def _entries(name):
    with open(os.path.join(ROOT, "profiles", name)) as f:
        return {k: v for k, v in json.load(f).items() if isinstance(v, dict) and "fetch_kib" in v}


def test_committed_traffic_is_the_scaled_counters():
    # traffic = FETCH_SIZE KiB x 1024 x fetch factor + WRITE_SIZE KiB x 1024 x
    # write factor; the stored figure was summed from unrounded per-dispatch
    # counters, the KiB means and factors are printed to 0.1 KiB / 1e-6
    n = 0
    for name in ("decode_traffic_qwen25_1_5b.json", "decode_traffic_qwen25_7b.json"):
        for key, e in _entries(name).items():
            scaled = e["fetch_kib"] * 1024 * e["fetch_factor"] + e["write_kib"] * 1024 * e["write_factor"]
            assert e["traffic_bytes"] == pytest.approx(scaled, rel=2e-6), key
            assert 1.0 < e["fetch_factor"] < 2.5 and e["write_factor"] == pytest.approx(1.0, abs=0.05)
            n += 1
    assert n >= 3


def test_committed_traffic_lookup(bench):
    e15 = _entries("decode_traffic_qwen25_1_5b.json")
    e7 = _entries("decode_traffic_qwen25_7b.json")
    t, src = bench.committed_traffic(False, "persistent", 128, 128, "f32")
    assert t == e15["persistent_launch"]["traffic_bytes"]
    assert src.endswith("decode_persistent_qwen25_1_5b_s1.md")
    # the S1 launch moves at least its algorithmic bytes and at most 1.2x them
    assert 396_604_211_200 < t < 1.2 * 396_604_211_200
    t, src = bench.committed_traffic(False, "persistent", 2048, 256, "bf16")
    assert t == e15["persistent_launch_long_bf16"]["traffic_bytes"]
    assert src.endswith("decode_persistent_qwen25_1_5b_long_bf16.md")
    assert 806_358_089_728 < t < 1.2 * 806_358_089_728
    t, _ = bench.committed_traffic(True, "streamed", 128, 128, "f32")
    assert t == e7["streamed_launch"]["traffic_bytes"]
    # no figure for a workload that was not profiled, or for another cache dtype
    assert bench.committed_traffic(False, "persistent", 2048, 256, "f32") == (None, None)
    assert bench.committed_traffic(False, "persistent", 64, 8, "f32") == (None, None)
    for _, src in (bench.committed_traffic(False, "persistent", 128, 128, "f32"),
                   bench.committed_traffic(False, "persistent", 2048, 256, "bf16")):
        assert os.path.exists(os.path.join(ROOT, src))
