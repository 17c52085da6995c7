"""The measurement-probe library (libkotflash_probe.so, not part of the
attention ABI; bench.py --decode-floor and --issue-rates load it): it loads,
exports its entry points, and kfp_issue_rate rejects bad arguments before any
launch. No kernel is launched here."""
import ctypes
import re
import subprocess

import pytest

from kotflash_amd import build

PROBES = ("kfp_stream", "kfp_merge_like", "kfp_empty", "kfp_issue_rate", "kfp_issue_rounds")


@pytest.fixture(scope="module")
def probe_lib():
    if not build.PROBE_LIB_PATH.is_file():
        pytest.skip("probe library not built (__graft_entry__.build() builds it)")
    return ctypes.CDLL(str(build.PROBE_LIB_PATH))


def test_probe_library_exports(probe_lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(build.PROBE_LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (kfp_[a-z_0-9]+)$", out, re.M))
    assert set(PROBES) <= exported
    for name in PROBES:
        assert hasattr(probe_lib, name), name


def test_issue_rate_probe_rejects_bad_arguments(probe_lib):
    f = probe_lib.kfp_issue_rate
    f.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                  ctypes.c_void_p]
    f.restype = ctypes.c_int
    hip_error_invalid_value = 1
    sink = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation first
    # no workgroups, or missing buffers
    assert f(0, 0, 0, sink, sink, None) == hip_error_invalid_value
    assert f(0, 0, 1024, None, sink, None) == hip_error_invalid_value
    assert f(0, 0, 1024, sink, None, None) == hip_error_invalid_value
    # an unknown kind, or an instruction count the probe is not built for
    assert f(10, 0, 1024, sink, sink, None) == hip_error_invalid_value
    assert f(-1, 0, 1024, sink, sink, None) == hip_error_invalid_value
    assert f(0, 7, 1024, sink, sink, None) == hip_error_invalid_value
    assert f(3, 1, 1024, sink, sink, None) == hip_error_invalid_value
    probe_lib.kfp_issue_rounds.restype = ctypes.c_int
    assert probe_lib.kfp_issue_rounds() == 512
