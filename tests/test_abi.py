"""The C-ABI library: it loads, exports every entry point the header declares,
the ctypes signatures cover exactly those, and argument validation (which runs
before any GPU work) reports errors through kf_last_error. No kernel is
launched here."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from kotflash_amd import _hip

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kotflash_amd.h"


def header_functions():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\*?\s+\*?(kf_[a-z_0-9]+)\(", text, re.M)))


def test_header_declares_the_expected_entry_points():
    assert header_functions() == sorted(_hip.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _hip.lib()
    for name in header_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(_hip.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r" T (kf_[a-z_0-9]+)$", out, re.M))
    assert set(header_functions()) <= exported


def test_abi_version():
    assert _hip.lib().kf_abi_version() == _hip.ABI_VERSION


def test_library_has_gfx950_code_object_only():
    out = subprocess.run(["strings", str(_hip.LIB_PATH)], capture_output=True, text=True).stdout
    assert "gfx950" in out
    assert "sm_" not in re.findall(r"amdgcn-amd-amdhsa--(\w+)", out)


def _arr(*vals):
    return ctypes.cast((ctypes.c_int64 * len(vals))(*vals), _hip._I64P)


@pytest.mark.parametrize("kwargs,match", [
    (dict(B=0), "positive"),
    (dict(Hq=3, Hkv=2), "divisible"),
    (dict(D=72 + 4), "multiple of 8"),
    (dict(D=136), "multiple of 8"),
    (dict(dtype=7), "dtype"),
    (dict(q=None), "q is null"),
    (dict(q=0x1008), "aligned"),
    (dict(scale=float("inf")), "finite"),
])
def test_fwd_argument_validation(kwargs, match):
    a = dict(q=0x1000, k=0x2000, v=0x3000, o=0x4000, lse=0x5000, B=1, Hq=2, Hkv=1, Sq=4, Sk=4,
             D=64, dtype=0, scale=0.125)
    a.update(kwargs)
    s = _arr(512, 256, 64)
    rc = _hip.lib().kf_attn_fwd(a["q"], a["k"], a["v"], a["o"], a["lse"], a["B"], a["Hq"], a["Hkv"],
                                a["Sq"], a["Sk"], a["D"], s, s, s, s, a["scale"], 0, a["dtype"], None)
    assert rc != 0
    assert match in _hip.lib().kf_last_error().decode()


def test_bad_strides_rejected():
    s_ok = _arr(512, 256, 64)
    s_bad = _arr(512, 256, 63)
    rc = _hip.lib().kf_attn_fwd(0x1000, 0x2000, 0x3000, 0x4000, 0x5000, 1, 2, 1, 4, 4, 64,
                                s_bad, s_ok, s_ok, s_ok, 0.1, 0, 0, None)
    assert rc == 1 and "strides" in _hip.lib().kf_last_error().decode()


def test_bwd_requires_workspace():
    s = _arr(512, 256, 64)
    rc = _hip.lib().kf_attn_bwd(*([0x1000] * 9), 1, 2, 1, 4, 4, 64, *([s] * 8), 0.1, 1, 0, None, 0, None)
    assert rc == 1 and "workspace" in _hip.lib().kf_last_error().decode()
    assert _hip.lib().kf_attn_bwd_workspace_bytes(2, 16, 4, 4096, 4096, 128, 1) >= 2 * 16 * 4096 * 4


def test_decode_planner_and_workspace():
    lib = _hip.lib()
    for sk in (2048, 4096, 8192, 16384, 1537, 8193, 100000):
        ns = lib.kf_decode_num_splits(2, 8, 2, 1, sk, 64)
        chunk = ((-(-sk // ns)) + 127) // 128 * 128  # whole 128-key granules
        assert ns >= 1 and -(-sk // chunk) == ns
    assert lib.kf_decode_num_splits(2, 8, 2, 1, 16384, 64) == 64
    assert lib.kf_decode_workspace_bytes(2, 8, 2, 1, 64, 1) == 0
    assert lib.kf_decode_workspace_bytes(2, 8, 2, 1, 64, 128) >= 128 * 16 * 65 * 4
    s = _arr(512, 64, 64)
    rc = lib.kf_attn_decode(0x1000, 0x2000, 0x3000, 0x4000, None, None, 2, 8, 2, 1, 16384, 64,
                            s, s, s, s, 0.125, 127, 0, None, 0, None)
    assert rc == 1 and "partition" in lib.kf_last_error().decode()
    rc = lib.kf_attn_decode(0x1000, 0x2000, 0x3000, 0x4000, None, None, 2, 8, 2, 1, 16384, 64,
                            s, s, s, s, 0.125, 64, 0, None, 0, None)
    assert rc == 1 and "workspace" in lib.kf_last_error().decode()


def test_append_argument_validation():
    lib = _hip.lib()
    s3 = _arr(64 * 8, 64 * 8, 8)
    s4 = _arr(2 * 8, 8, 8, 1)
    rc = lib.kf_kv_append(0x1000, 0x2000, 0x3000, 0x4000, None, 62, 1, 1, 3, 8, 64, s3, s3, s4, s4, 0, None)
    assert rc == 1 and "capacity" in lib.kf_last_error().decode()
    rc = lib.kf_kv_append(None, 0x2000, 0x3000, 0x4000, None, 0, 1, 1, 3, 8, 64, s3, s3, s4, s4, 0, None)
    assert rc == 1 and "null" in lib.kf_last_error().decode()


@pytest.mark.parametrize("bound,snew", [
    (62, 3),    # the last token would land one past the end (kv_append_cuda.cu:72-73)
    (64, 1),
    (-1, 1),
])
def test_append_device_starts_are_bounded_on_the_host(bound, snew):
    """With per-sequence device starts, `start` is the host-side bound on
    them and an append that would not fit is rejected before anything is
    launched (the start array, a fake address here, is never read)."""
    lib = _hip.lib()
    s3 = _arr(64 * 8, 64 * 8, 8)
    s4 = _arr(2 * 8, 8, 8, 1)
    rc = lib.kf_kv_append(0x1000, 0x2000, 0x3000, 0x4000, 0x5000, bound, 1, 1, snew, 8, 64,
                          s3, s3, s4, s4, 0, None)
    msg = lib.kf_last_error().decode()
    assert rc == 1 and "capacity" in msg and "max start" in msg


def test_ragged_decode_planner():
    """The ragged planner's count partitions max(lengths) into whole 128-key
    granules, sizes the chunk from the total visible keys (about 384
    non-empty workgroups), and degrades to one split for empty batches."""
    lib = _hip.lib()

    def plan(lengths, b=None, hq=32, hkv=8, sq=1, d=64):
        return _hip.decode_num_splits_ragged(b or len(lengths), hq, hkv, sq, lengths, d)

    for lengths in ([4096, 28000, 129, 7777], [1, 1, 1], [16384] * 2, [65536], [300, 20000]):
        ns = plan(lengths)
        mx = max(lengths)
        chunk = ((-(-mx // ns)) + 127) // 128 * 128
        assert ns >= 1 and -(-mx // chunk) == ns
    # Config 5 shape: total visible keys x kv heads / 384 workgroups.
    lengths = [4096, 28000, 16000, 9000, 22000, 5000, 12000, 27000]
    ns = plan(lengths)
    chunk = ((-(-28000 // ns)) + 127) // 128 * 128
    nonempty = sum(8 * -(-x // chunk) for x in lengths)
    assert 250 <= nonempty <= 560
    assert plan([0, 0]) == 1
    assert lib.kf_decode_num_splits_ragged(2, 8, 2, 1, None, 64) == 1


def _append_decode(lib, **kw):
    a = dict(q=0x1000, kc=0x2000, vc=0x3000, nk=0x4000, nv=0x5000, o=0x6000, lengths=None, past=100,
             B=1, Hq=4, Hkv=1, Sq=1, Snew=1, max_length=100, capacity=128, D=64, scale=0.125,
             splits=1, ws=0x7000, ws_bytes=1 << 20)
    a.update(kw)
    s = _arr(128 * 64, 128 * 64, 64)
    return lib.kf_attn_append_decode(a["q"], a["kc"], a["vc"], a["nk"], a["nv"], a["o"], None,
                                     a["lengths"], a["past"], a["B"], a["Hq"], a["Hkv"], a["Sq"],
                                     a["Snew"], a["max_length"], a["capacity"], a["D"],
                                     s, s, s, s, s, s, a["scale"], a["splits"], 0, a["ws"],
                                     a["ws_bytes"], None)


@pytest.mark.parametrize("kwargs,match", [
    (dict(past=128, max_length=128), "capacity"),          # no room for the new token
    # Device lengths: max_length is the host-side bound on them and must leave
    # room for every new token (kv_append_cuda.cu:72-73).
    (dict(lengths=0x8000, max_length=120, Snew=9), "exceeds cache capacity"),
    (dict(lengths=0x8000, max_length=128, Snew=1), "exceeds cache capacity"),
    (dict(past=99), "past_length"),                        # scalar position != max_length
    (dict(max_length=129), "max_length <= capacity"),
    (dict(Snew=0), "Snew"),
    (dict(nk=None), "new_k is null"),
    (dict(kc=0x2008), "aligned"),
    (dict(ws=None), "workspace"),
    (dict(ws_bytes=16), "workspace"),
    (dict(splits=2, max_length=100, past=100), "partition"),
    (dict(D=76), "multiple of 8"),
])
def test_append_decode_argument_validation(kwargs, match):
    lib = _hip.lib()
    rc = _append_decode(lib, **kwargs)
    assert rc == 1 or rc == 2
    assert match in lib.kf_last_error().decode()


def test_append_decode_workspace_has_one_extra_split():
    lib = _hip.lib()
    ns = lib.kf_decode_num_splits(8, 32, 8, 16, 28000, 64)
    assert (lib.kf_decode_workspace_bytes(8, 32, 8, 16, 64, ns + 1)
            > lib.kf_decode_workspace_bytes(8, 32, 8, 16, 64, ns))
    # Zero cache keys: one (empty) cache split plus the new tokens' split.
    assert lib.kf_decode_num_splits(1, 4, 1, 1, 0, 64) == 1


def test_decode_noalloc_rejects_problems_beyond_its_scratch():
    """kf_attn_decode_noalloc refuses a problem whose split partials exceed
    its static scratch, before touching the device (no kernel launch)."""
    lib = _hip.lib()
    b, hq, hkv, sq, d, splits = 64, 64, 8, 16, 128, 64
    need = lib.kf_decode_workspace_bytes(b, hq, hkv, sq, d, splits)
    assert need > _hip.NOALLOC_SCRATCH_BYTES
    s = _arr(1 << 20, 1 << 16, 128)
    rc = lib.kf_attn_decode_noalloc(0x1000, 0x2000, 0x3000, 0x4000, None, None, b, hq, hkv, sq,
                                    4096, d, s, s, s, s, 0.1, splits, 0, None)
    assert rc == 1
    assert "static scratch" in lib.kf_last_error().decode()
    assert lib.kf_decode_workspace_bytes(2, 8, 2, 1, 64, 64) <= _hip.NOALLOC_SCRATCH_BYTES


@pytest.mark.parametrize("kwargs,match", [
    (dict(ns=0), "positive"),
    (dict(D=130), "multiple of 4"),
    (dict(D=6), "multiple of 4"),
    (dict(dtype=3), "dtype"),
    (dict(part_o=None), "non-null"),
    (dict(part_o=0x1008), "aligned"),
    (dict(o=0x3004), "aligned"),
])
def test_lse_merge_argument_validation(kwargs, match):
    a = dict(part_o=0x1000, part_lse=0x2000, o=0x3000, ns=4, D=64, dtype=0)
    a.update(kwargs)
    s = _arr(2 * 8 * 64, 8 * 64, 64)
    rc = _hip.lib().kf_lse_merge(a["part_o"], a["part_lse"], a["o"], None, a["ns"], 2, 2, 8,
                                 a["D"], s, a["dtype"], None)
    assert rc != 0
    assert match in _hip.lib().kf_last_error().decode()
