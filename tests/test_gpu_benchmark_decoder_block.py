"""The decoder-block training benchmark on the GPU: every backend trains,
stays finite, and the HIP block matches the expanded-SDPA block."""
import json

import pytest

from kotflash_amd import benchmark_decoder_block as bdb

pytestmark = pytest.mark.gpu


def test_decoder_block_report(capsys):
    bdb.main(["--batch", "1", "--seq", "256", "--q-heads", "4", "--kv-heads", "2",
              "--head-dim", "64", "--warmup", "1", "--iterations", "3"])
    report = json.loads(capsys.readouterr().out)
    assert "hip_forward" not in report, report.get("hip_forward")
    assert report["max_abs_output_error_vs_expanded_sdpa"] < 2e-2
    for name in bdb.BACKENDS:
        r = report[name]
        assert r["loss_finite"] and r["parameters_finite_after_update"], name
    assert report["hip_speedup_vs_sdpa_expanded_kv"] > 0
