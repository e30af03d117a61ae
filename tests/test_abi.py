"""The C-ABI library loads, exports every symbol declared in include/oscar_hip.h and
rejects invalid arguments on the host (no GPU needed: nothing is launched)."""

import ctypes
import re
from pathlib import Path

import pytest

from oscar_new_amd import _ext

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "oscar_hip.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*)\s+(oscar_\w+)\s*\(", text,
                                 re.M)))


def test_header_and_binding_agree():
    assert declared_symbols() == _ext.exported_symbols()


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_ext.LIBRARY_PATH))
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert _ext.library().oscar_abi_version() == 1


def test_host_side_argument_errors():
    lib = _ext.library()
    assert lib.oscar_rotate(None, 4, 1, 128, 0, 0, 1, None, 0, 0, None, None) == -5
    assert lib.oscar_rotate(None, 4, 1, 256, 0, 0, 1, None, 0, 0, None, None) == -1
    assert lib.oscar_rotate(None, 0, 1, 256, 0, 0, 1, None, 0, 0, None, None) == 0
    bad = _ext.OscarLayout(256, 1, 768, 100, 160, 68, 4, 128, 132, 0, 393216)
    clip = _ext.OscarClip(0, 0.96, 0.92, 1.0, 1.0)
    assert lib.oscar_store_int2(None, None, 4, None, 0, None, None, bad, clip, None) == -3
    good = _ext.OscarLayout(256, 1, 768, 128, 160, 68, 4, 128, 132, 0, 393216)
    assert lib.oscar_store_int2(None, None, 4, None, 0, None, None, good, clip, None) == -1
    # n * H must stay below 2^31 (the kernel divides 32-bit row indices); fake, aligned,
    # never dereferenced addresses.
    a = 1 << 20
    assert lib.oscar_store_int2(a, a, 1 << 31, a, 1 << 24, a, a, good, clip, None) == -2
    assert lib.oscar_merge_splits(None, None, None, 3, 6, 4, 128, None, None, None) == -5
    assert lib.oscar_unpack(None, 0, None, 5000, good, None, None, None) == -2
    with pytest.raises(ValueError):
        _ext.check(-2, "probe")


def test_history_post_host_side_errors():
    # Fake, aligned, never dereferenced addresses: every call below returns before a launch.
    lib = _ext.library()
    good = _ext.OscarLayout(256, 1, 768, 128, 160, 68, 4, 128, 132, 0, 393216)
    a = 1 << 20

    def call(mql=1, splits=8, counters=a, slots=64, programs=8):
        return lib.oscar_history_post(
            a, 1536, 256, 1, a, 1 << 24, a, a, a, 64, 64, a, a, a, 8, 6, programs, splits, 32, 4,
            mql, 1 / 16, 0, good, a, a, counters, slots, a, a, a, a, None, a, 256, 256, a, 256,
            256, a, 1 << 20, 8, None)

    assert call(mql=4) == -5  # 24 query rows per task: the two-launch form covers it
    assert call(splits=17) == -5  # above the one-round split merge
    assert call(counters=None) == -1
    assert call(counters=a + 2) == -4
    assert call(slots=7) == -2  # fewer counters than programs x kv heads


def test_rotate_store_host_side_errors():
    # Fake, never dereferenced addresses: every call below returns before a launch.
    lib = _ext.library()
    good = _ext.OscarLayout(256, 1, 768, 128, 160, 68, 4, 128, 132, 0, 393216)
    clip = _ext.OscarClip(2, 0.96, 0.92, 1.0, 1.0)
    a = 1 << 20

    def call(key=a, k_s0=256, n=4, rk_t=a, history=a, clip=clip):
        return lib.oscar_rotate_store_int2(key, k_s0, 256, a, 256, 256, n, rk_t, a, history,
                                           1 << 24, a, a, good, clip, None)

    assert call(n=0) == 0
    assert call(n=-1) == -2
    assert call(rk_t=None) == -1
    assert call(key=a + 8) == -4  # rows must be 16-byte aligned
    assert call(k_s0=260) == -4
    assert call(history=a + 2) == -4
    assert call(clip=_ext.OscarClip(9, 0.96, 0.92, 1.0, 1.0)) == -2


def test_status_strings():
    lib = _ext.library()
    assert lib.oscar_status_string(0) == b"ok"
    assert b"layout" in lib.oscar_status_string(-3)
