"""The C-ABI library: it loads, exports every entry point include/vortex_hip.h
declares, and rejects bad arguments on the host (these calls return before
any device work, so they run without a GPU)."""
import ctypes
import os
import re

import pytest

from vortex_torch import _hip

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "vortex_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(vtx_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _hip.load_library()
    declared = _declared()
    assert len(declared) >= 8
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in vortex_hip.h but not exported"
    assert set(declared) == set(_hip.EXPORTED_SYMBOLS)
    assert lib.vtx_version().startswith(b"vortex-mi355x")


def test_host_side_argument_errors():
    lib = _hip.load_library()
    rc = lib.vtx_plan_decode(None, -1, None, None, 0, None, None, 0, None, None, 0, 0, None, None, None, None,
                             0, None, None, 16, 8, 30, 1, 1, 64, 16, None, 0, 0, None)
    assert rc == -1 and b"batch_size" in lib.vtx_last_error()
    rc = lib.vtx_topk_select(None, 0, None, None, None, 0, None, 0, 1, 5000, 1, 1, 512, None)
    assert rc == -1 and b"exceeds" in lib.vtx_last_error()
    rc = lib.vtx_page_reduce(None, 0, 16, 128, None, 0, 0, None, 5, 8, 16, 3, 0, None)
    assert rc == -1 and b"dim" in lib.vtx_last_error()
    rc = lib.vtx_indexer_fused(None, 0, 2, None, None, None, 0, None, 0, None, None, None, 0, None, 0,
                               4, 30, 1, 1, 512, 100, None, 0, 0, None, 0, None)
    assert rc == -1 and b"head_dim" in lib.vtx_last_error()
    # well-formed (never dereferenced) addresses: the layout checks fail before any device work
    fake = [0x10000 * (i + 1) for i in range(9)]
    args = [fake[0], 4, 2, None, fake[1], fake[2], 100, fake[3], 100, fake[4], fake[5], fake[6], 100,
            fake[7], 100, 4, 30, 1, 1, 512, 128]
    rc = lib.vtx_indexer_fused(*args, None, 0, 7, None, 0, None)
    assert rc == -1 and b"unknown mode" in lib.vtx_last_error()
    rc = lib.vtx_indexer_fused(*args, fake[8], 3, _hip.FUSED_SPLIT, None, 0, None)
    assert rc == -1 and b"segment counters" in lib.vtx_last_error()
    assert lib.vtx_indexer_fused_supported(128) == 1 and lib.vtx_indexer_fused_supported(100) == 0


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        _hip.load_library(tmp_path / "nope.so")
