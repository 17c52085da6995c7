"""The decode benchmark CLI on the GPU: every candidate, including the fused
append + decode, runs, passes the expanded-SDPA check for attention alone
and append + attention, and is timed."""
import json

import pytest

from kotflash_amd import benchmark_decode

pytestmark = pytest.mark.gpu


def test_gpu_report_all_candidates(capsys):
    print("benchmark_decode B=2 Hq=8 Hkv=2 D=64 Sk=2048", flush=True)
    capsys.readouterr()  # drop the case label: the report must be the only output
    benchmark_decode.main(["--kv-seq", "2048", "--warmup", "2", "--iterations", "3",
                           "--repeats", "3"])
    report = json.loads(capsys.readouterr().out)
    assert report["backend_failures"] == {}
    assert set(report["results"]) == {"hip", "auto", "pytorch_expanded_sdpa",
                                      "preallocated_hip_separate_append", "preallocated_auto",
                                      "preallocated_fused_append"}
    for name, checks in report["correctness"].items():
        for metric in ("attention_only", "append_plus_attention"):
            assert checks[metric]["within_tolerance"], (name, metric)
    fused = report["results"]["preallocated_fused_append"]["append_plus_attention"]
    assert fused["gpu_median_ms"] > 0 and fused["incremental_peak_allocated_bytes"] >= 0
