"""The C-ABI library: builds, loads, exports what include/wkv_hip.h declares,
and rejects bad arguments on the host (no GPU work is launched here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "wkv_hip.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\**\s*(\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from spikegpt_myelin_amd import _lib

    if not _lib.LIB_PATH.exists():
        from spikegpt_myelin_amd.build import build

        build(verbose=False)
    return _lib.load()


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for n in ("wkv4_forward", "wkv4_backward", "wkv4_backward_workspace_bytes", "wkv4_decode_step",
              "wkv7_forward", "wkv_last_error_string", "wkv_version"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    from spikegpt_myelin_amd import _lib

    for name in _declared_functions():
        assert hasattr(lib, name), name
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
    assert lib.wkv_version().decode().startswith("wkv_hip")


def test_host_side_argument_errors(lib):
    # Rejected before any launch: unknown dtype, negative size, null pointers.
    rc = lib.wkv4_forward(None, None, None, None, None, 1, 1, 1, 7, None)
    assert rc == 1 and b"dtype" in lib.wkv_last_error_string()
    rc = lib.wkv4_forward(None, None, None, None, None, -1, 1, 1, 0, None)
    assert rc == 1 and b"sizes" in lib.wkv_last_error_string()
    rc = lib.wkv4_forward(None, None, None, None, None, 1, 1, 1, 1, None)
    assert rc == 1 and b"null" in lib.wkv_last_error_string()
    rc = lib.wkv7_forward(None, None, None, None, None, None, None, None, None, 1, 1, 1, 32, 0, None)
    assert rc == 1 and b"64" in lib.wkv_last_error_string()
    # Empty problems are a no-op success.
    assert lib.wkv4_forward(None, None, None, None, None, 0, 5, 8, 0, None) == 0


def test_checkpoint_size_matches_python_layout(lib):
    from spikegpt_myelin_amd.wkv import checkpoint_shape
    for b, t, c in [(64, 1024, 512), (3, 7, 96), (1, 1, 1), (24, 3072, 512), (2, 65, 4100)]:
        f, bb, nblk, cc = checkpoint_shape(b, t, c)
        assert (f, bb, nblk, cc) == (3, b, (t + 63) // 64, c)
        assert lib.wkv4_checkpoint_bytes(b, t, c) == 4 * f * bb * nblk * cc


def test_backward_workspace_size_and_check(lib):
    n = lib.wkv4_backward_workspace_bytes(64, 1024, 512, 1)
    # per-segment checkpoints (3 floats per channel per segment) + [B, C] partials
    assert 2 * 64 * 512 * 4 < n < 64 * 1024 * 512 * 4
    buf = ctypes.create_string_buffer(16)
    addr = ctypes.addressof(buf)
    rc = lib.wkv4_backward(addr, addr, addr, addr, addr, addr, addr, addr, addr, addr, 16,
                           2, 8, 8, 1, None)
    assert rc == 3 and b"workspace" in lib.wkv_last_error_string()
