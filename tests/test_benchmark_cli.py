"""The interleaved benchmark CLI (kotflash_amd.benchmark) on the CPU: the
SDPA baselines run and are timed, the HIP backend is reported as a failure
(no GPU), and the argument checks match the reference's."""
import json

import pytest

from kotflash_amd import benchmark


def test_cpu_report_structure(capsys):
    benchmark.main(["--device", "cpu", "--batch", "1", "--q-heads", "4", "--kv-heads", "2",
                    "--seq", "32", "--head-dim", "16", "--causal", "--warmup", "1",
                    "--iterations", "2", "--repeats", "3", "--seed", "7"])
    report = json.loads(capsys.readouterr().out)
    assert report["shape"] == {"B": 1, "Hq": 4, "Hkv": 2, "Sq": 32, "Sk": 32, "D": 16}
    assert len(report["measurement_order_by_round"]) == 3
    for name in ("pytorch_sdpa_native_gqa", "pytorch_sdpa_expanded_kv", "auto"):
        r = report[name]
        assert len(r["forward_ms"]["per_round"]) == 3
        assert r["forward_ms"]["min"] <= r["forward_ms"]["median"] <= r["forward_ms"]["max"]
        assert r["max_abs_error_vs_expanded_sdpa"] < 1e-5
        assert r["forward_incremental_peak_allocated_bytes"] is None
    assert "hip" in report["backend_failures"]
    assert "auto_forward_speedup_vs_pytorch_sdpa_native_gqa" in report
    # Every round measured every timed backend exactly once.
    for order in report["measurement_order_by_round"]:
        assert sorted(order) == sorted(["pytorch_sdpa_native_gqa", "pytorch_sdpa_expanded_kv",
                                        "auto"])


@pytest.mark.parametrize("argv, message", [
    (["--q-heads", "6", "--kv-heads", "4"], "divisible"),
    (["--repeats", "2"], "repeats at least 3"),
    (["--seq", "0"], "must be positive"),
    (["--kv-seq", "-1"], "--kv-seq must be positive"),
])
def test_argument_checks(argv, message, capsys):
    with pytest.raises(SystemExit):
        benchmark.parse_args(["--device", "cpu"] + argv)
    assert message in capsys.readouterr().err
