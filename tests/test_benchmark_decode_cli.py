"""The decode benchmark CLI (kotflash_amd.benchmark_decode) on the CPU: the
SDPA candidates run, are checked and timed; the HIP ones are reported as
failures (no GPU); the argument checks follow the reference's
(benchmarks/benchmark_decode.py:85-112)."""
import json

import pytest

from kotflash_amd import benchmark_decode


def test_cpu_report_structure(capsys, tmp_path):
    out = tmp_path / "r.json"
    benchmark_decode.main(["--device", "cpu", "--batch", "1", "--q-heads", "4", "--kv-heads", "2",
                           "--head-dim", "16", "--kv-seq", "1024", "--warmup", "1",
                           "--iterations", "2", "--repeats", "3", "--output", str(out)])
    report = json.loads(capsys.readouterr().out)
    assert json.loads(out.read_text()) == report
    assert report["shape"] == {"batch": 1, "q_heads": 4, "kv_heads": 2, "query_length": 1,
                               "visible_kv_length": 1024, "head_dim": 16}
    assert report["preallocated_cache_capacity"] == 2048
    assert set(report["results"]) == {"auto", "pytorch_expanded_sdpa", "preallocated_auto"}
    assert set(report["backend_failures"]) == {"hip", "preallocated_hip_separate_append",
                                               "preallocated_fused_append"}
    for name, r in report["results"].items():
        for metric in ("attention_only", "append_plus_attention"):
            m = r[metric]
            assert len(m["wall_per_repeat_ms"]) == 3
            assert m["wall_min_ms"] <= m["wall_median_ms"] <= m["wall_max_ms"]
            assert m["incremental_peak_allocated_bytes"] is None
            assert report["correctness"][name][metric]["within_tolerance"]
        assert r["append_plus_attention"]["batch_tokens_per_second"] > 0
    base = report["results"]["pytorch_expanded_sdpa"]["attention_only"]
    assert base["wall_speedup_vs_expanded_sdpa"] == 1.0
    assert report["cache_append_only"]["wall_median_ms"] > 0


@pytest.mark.parametrize("argv, message", [
    (["--q-heads", "6", "--kv-heads", "4"], "divisible"),
    (["--repeats", "2"], "repeats >= 3"),
    (["--batch", "0"], "must be positive"),
    (["--kv-seq", "512"], "--kv-seq >= 1024"),
    (["--head-dim", "12"], "multiple of 8"),
    (["--append-backend", "nope"], "invalid choice"),
])
def test_argument_checks(argv, message, capsys):
    with pytest.raises(SystemExit):
        benchmark_decode.parse_args(["--device", "cpu"] + argv)
    assert message in capsys.readouterr().err
