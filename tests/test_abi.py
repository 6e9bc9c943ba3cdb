"""The C-ABI library builds, loads and exports every symbol ``include/lngram_hip.h`` declares (CPU).

No compute call is made: only entry points that fail argument validation before
touching the GPU, and the version / error-string accessors.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "lngram_hip.h"


def declared() -> list:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lng_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from lngram_hip import _lib

    if not _lib.LIB_PATH.exists():
        import importlib.util

        spec = importlib.util.spec_from_file_location("lngram_build", ROOT / "lngram-decode_amd" / "build.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build(verbose=False)
    return _lib.load()


def test_header_declares_the_hot_path(lib):
    names = declared()
    for must in ("lng_router_codes", "lng_ngram_address", "lng_ngram_rows", "lng_route_tokens",
                 "lng_memory_readout_fused", "lng_ssm_scan", "lng_tree_accept", "lng_sink_attention"):
        assert must in names


def test_every_declared_symbol_is_exported_and_bound(lib):
    from lngram_hip._lib import SIGNATURES

    names = declared()
    assert set(names) == set(SIGNATURES), set(names) ^ set(SIGNATURES)
    for n in names:
        assert hasattr(lib, n), n


def test_version_and_argument_errors(lib):
    assert lib.lng_abi_version() == 2
    # rejected before any GPU work: negative M
    rc = lib.lng_linear(None, None, 0, -1, 4, 4, None, None)
    assert rc == -1
    assert b"linear" in lib.lng_last_error()
    rc = lib.lng_pack_route_codes(None, 4, 7, 4, None, 3, None)  # C not divisible by bits
    assert rc == -1
    rc = lib.lng_ngram_rows(None, 9, 1, 1, 1, 0, 1, (ctypes.c_int32 * 1)(2), 1, 4, None, None, None, 4, None)
    assert rc == -2  # bad codes dtype
    # int32 rows past the int32 range are refused: 130 routes x 2^(8*3) rows
    rc = lib.lng_ngram_rows(None, 3, 1, 1, 130, 0, 130, (ctypes.c_int32 * 1)(3), 1, 8, None, None, None, 4, None)
    assert rc == -4 and b"int32" in lib.lng_last_error()
    rc = lib.lng_rmsnorm(None, None, 0, 1, 8, 1e-5, 7, None, None)
    assert rc == -1 and b"rounding" in lib.lng_last_error()
    rc = lib.lng_online_mix(None, None, 4, None, None, 1, 2, 2, None, 10, 0.0, None, None, None)
    assert rc == -1 and b"kappa" in lib.lng_last_error()
    rc = lib.lng_route_tokens(None, 3, 1, 4, 2, 0, 2, (ctypes.c_int32 * 1)(2), 1, 4, None, 1, 8, None, None, 9,
                              None, None)
    assert rc == -1 and b"target_length" in lib.lng_last_error()
    # the fused readout's 32-bit buffer offsets bound a launch to 2^21 tokens
    rc = lib.lng_memory_readout_fused(None, None, 0.0, None, 2, (1 << 20) + 1, 184, None, None, None, None, 1e-6,
                                      0.125, 0.0, None, None)
    assert rc == -1 and b"2^21 tokens" in lib.lng_last_error()


def test_error_message_is_thread_local(lib):
    import threading

    lib.lng_linear(None, None, 0, -1, 4, 4, None, None)
    seen = {}

    def other():
        seen["msg"] = lib.lng_last_error()

    th = threading.Thread(target=other)
    th.start()
    th.join()
    assert seen["msg"] == b""
    assert b"linear" in lib.lng_last_error()
