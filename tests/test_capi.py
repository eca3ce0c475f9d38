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
    rc = lib.wkv4_forward(None, None, None, None, None, None, 0, 1, 1, 1, 7, None)
    assert rc == 1 and b"dtype" in lib.wkv_last_error_string()
    rc = lib.wkv4_forward(None, None, None, None, None, None, 0, -1, 1, 1, 0, None)
    assert rc == 1 and b"sizes" in lib.wkv_last_error_string()
    rc = lib.wkv4_forward(None, None, None, None, None, None, 0, 1, 1, 1, 1, None)
    assert rc == 1 and b"null" in lib.wkv_last_error_string()
    rc = lib.wkv7_forward(None, None, None, None, None, None, None, None, None, 1, 1, 1, 32, 0, None)
    assert rc == 1 and b"64" in lib.wkv_last_error_string()
    # Empty problems are a no-op success.
    assert lib.wkv4_forward(None, None, None, None, None, None, 0, 0, 5, 8, 0, None) == 0


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


def test_lif_forward_workspace_sizes(lib, monkeypatch):
    # Empty and one-block sequences are never split (no workspace); the 41M
    # activation shape splits into eight segments: the start and end
    # membranes of the seven inner boundaries, fp32.  Forced segment counts are capped
    # by the number of 32-step blocks.
    for b, t, c in [(0, 5, 8), (2, 0, 8), (2, 5, 0), (3, 1, 96), (4, 32, 64), (1, 1, 1)]:
        assert lib.lif_forward_workspace_bytes(b, t, c) == 0, (b, t, c)
    assert lib.lif_forward_workspace_bytes(64, 1024, 512) == 2 * 7 * 64 * 512 * 4
    assert lib.lif_forward_workspace_bytes(16, 1024, 768) == 2 * 7 * 16 * 768 * 4
    monkeypatch.setenv("WKV_LIF_SEGS", "16")
    assert lib.lif_forward_workspace_bytes(2, 100, 70) == 2 * 3 * 2 * 70 * 4  # 4 blocks
    assert lib.lif_forward_workspace_bytes(2, 0, 70) == 0
    monkeypatch.setenv("WKV_LIF_SEGS", "1")
    assert lib.lif_forward_workspace_bytes(64, 1024, 512) == 0
    monkeypatch.delenv("WKV_LIF_SEGS")
    # the residual forward splits only below 384 rows (eight segments at
    # B=16, C=768, as the plain one), so the query's maximum is the plain one
    assert lib.lif_forward_workspace_bytes(16, 1024, 768) == 2 * 7 * 16 * 768 * 4
    # the backward: segments of at least eight blocks, ~2048 waves (plain) or
    # ~1024 (residual); the query covers the larger
    assert lib.lif_backward_workspace_bytes(64, 1024, 512) == 2 * 3 * 64 * 512 * 4
    assert lib.lif_backward_workspace_bytes(16, 1024, 768) == 2 * 3 * 16 * 768 * 4
    assert lib.lif_backward_workspace_bytes(2, 200, 64) == 0  # 7 blocks
    assert lib.lif_backward_workspace_bytes(2, 0, 64) == 0


def test_token_shift_mix_workspace_sizes(lib):
    # One fp32 partial row of grad_mu per (mixing vector, batch row, chunk of
    # steps); chunks are the longest power of two (64 down to 8) that still
    # gives 2048 waves of 256 channels.
    assert lib.token_shift_mix_workspace_bytes(3, 64, 1024, 512) == 3 * 64 * 16 * 512 * 4  # 64
    assert lib.token_shift_mix_workspace_bytes(3, 128, 1024, 8) == 3 * 128 * 16 * 8 * 4  # 64
    assert lib.token_shift_mix_workspace_bytes(2, 64, 1003, 16) == 2 * 64 * 32 * 16 * 4  # 32
    assert lib.token_shift_mix_workspace_bytes(2, 4, 257, 512) == 2 * 4 * 33 * 512 * 4  # 8
    assert lib.token_shift_mix_workspace_bytes(3, 0, 5, 8) == 0
    assert lib.token_shift_mix_workspace_bytes(3, 2, 0, 8) == 0


def test_step_row_args_layout_matches_header(tmp_path):
    # The ctypes mirror of wkv_step_row_args has the C struct's size and field
    # offsets (compiled with the host C compiler from the header).
    import shutil
    import subprocess

    from spikegpt_myelin_amd import _lib

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    fields = [f for f, _ in _lib.StepRowArgs._fields_]
    src = tmp_path / "layout.c"
    body = "".join(f'  printf("%zu\\n", offsetof(wkv_step_row_args, {f}));\n' for f in fields)
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "wkv_hip.h"\n'
                   "int main(void) {\n" + body +
                   '  printf("%zu\\n", sizeof(wkv_step_row_args));\n  return 0;\n}\n')
    exe = tmp_path / "layout"
    subprocess.run([cc, "-I", str(ROOT / "include"), str(src), "-o", str(exe)], check=True)
    got = [int(v) for v in subprocess.run([str(exe)], check=True, capture_output=True,
                                          text=True).stdout.split()]
    want = [getattr(_lib.StepRowArgs, f).offset for f in fields] + [ctypes.sizeof(_lib.StepRowArgs)]
    assert got == want


def test_block_step_argument_errors(lib):
    from spikegpt_myelin_amd import _lib

    a = _lib.StepRowArgs()
    a.batch, a.channels = 2, 8
    assert lib.block_step_row(0, ctypes.byref(a), None) == 1  # null residual
    a.residual = 16
    a.channels = 5000
    assert lib.block_step_row(1, ctypes.byref(a), None) == 1
    assert b"4096" in lib.wkv_last_error_string()
    a.channels, a.n_mix = 8, 1
    assert lib.block_step_row(1, ctypes.byref(a), None) == 1
    assert b"n_mix" in lib.wkv_last_error_string()
    a.n_mix = 2  # token shift without a layer norm
    assert lib.block_step_row(1, ctypes.byref(a), None) == 1
    assert lib.block_step_row(9, ctypes.byref(a), None) == 1
    a.batch = 0
    a.n_mix = 0
    assert lib.block_step_row(1, ctypes.byref(a), None) == 0  # empty batch: no-op
    assert lib.block_step_wkv(*([None] * 12), 2, 8, None) == 1
    assert lib.block_step_wkv(*([None] * 12), 0, 8, None) == 0


def test_noalloc_backward_rejects_sizes_beyond_its_scratch(lib):
    # Rejected on the host before any pointer is read: 3 fp32 records per
    # channel per 64 steps at B=64, T=4096, C=512 are 25 MB > 16 MiB.
    rc = lib.wkv4_backward_noalloc(None, None, None, None, None, None, None, None, None,
                                   64, 4096, 512, 1, None)
    assert rc == 3
    msg = lib.wkv_last_error_string()
    assert b"scratch" in msg and str(16 << 20).encode() in msg
    # Within the maximum, the null pointers are what is rejected.
    rc = lib.wkv4_backward_noalloc(None, None, None, None, None, None, None, None, None,
                                   64, 1024, 512, 1, None)
    assert rc == 1 and b"null" in lib.wkv_last_error_string()
    assert lib.wkv4_backward_workspace_bytes(64, 1024, 512, 1) <= 16 << 20
