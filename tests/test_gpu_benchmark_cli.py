"""The interleaved benchmark CLI on the GPU: the HIP backend is timed next
to both SDPA baselines, agrees with them, and gets speedup entries."""
import json

import pytest

from kotflash_amd import benchmark

pytestmark = pytest.mark.gpu


def test_gpu_report_includes_hip(capsys):
    benchmark.main(["--device", "cuda", "--batch", "1", "--q-heads", "4", "--kv-heads", "2",
                    "--seq", "256", "--head-dim", "64", "--causal", "--warmup", "2",
                    "--iterations", "3", "--repeats", "3"])
    report = json.loads(capsys.readouterr().out)
    assert "backend_failures" not in report, report.get("backend_failures")
    assert report["environment"]["arch"].split(":")[0] == "gfx950"
    for name in ("hip", "auto", "pytorch_sdpa_native_gqa", "pytorch_sdpa_expanded_kv"):
        r = report[name]
        assert r["max_abs_error_vs_expanded_sdpa"] < 5e-3, (name, r["max_abs_error_vs_expanded_sdpa"])
        assert r["forward_backward_incremental_peak_allocated_bytes"] is not None
    assert report["hip_forward_backward_speedup_vs_pytorch_sdpa_expanded_kv"] > 0
