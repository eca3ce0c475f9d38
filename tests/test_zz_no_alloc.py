"""``wkv4_backward_noalloc`` (the WKV-4 backward with a fixed device scratch
array instead of a workspace) against ``wkv4_backward`` through the C ABI.

Both run the same kernels on the same inputs, so the outputs must be equal
bit for bit.  The calls come in a row with the second one smaller, so stale
records and partials left in the shared scratch by the first call must not
reach the second.
"""

from __future__ import annotations

import pytest
import torch

from oracle import wkv4 as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _lib():
    from spikegpt_myelin_amd import _lib

    return _lib, _lib.load()


def _inputs(b, t, c, dtype, seed):
    k, v, td, tf, gy = O.make_inputs(b, t, c, seed=seed, dtype=dtype)
    k, v, gy = (x.to(DEV) for x in (k, v, gy))
    w = (-torch.exp(td.double())).float().to(DEV)
    u = tf.float().to(DEV)
    return gy, w, u, k, v


def _outputs(k, c):
    return (torch.empty_like(k), torch.empty_like(k),
            torch.empty(c, dtype=torch.float32, device=DEV),
            torch.empty(c, dtype=torch.float32, device=DEV))


def _with_workspace(L, lib, gy, w, u, k, v):
    b, t, c = k.shape
    code = L.dtype_code(k.dtype)
    gk, gv, gtd, gtf = _outputs(k, c)
    nbytes = lib.wkv4_backward_workspace_bytes(b, t, c, code)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.wkv4_backward(gy.data_ptr(), w.data_ptr(), u.data_ptr(), k.data_ptr(), v.data_ptr(),
                           gk.data_ptr(), gv.data_ptr(), gtd.data_ptr(), gtf.data_ptr(),
                           ws.data_ptr(), nbytes, b, t, c, code, stream)
    L.check(rc, "wkv4_backward")
    return gk, gv, gtd, gtf


def _no_alloc(L, lib, gy, w, u, k, v):
    b, t, c = k.shape
    code = L.dtype_code(k.dtype)
    gk, gv, gtd, gtf = _outputs(k, c)
    # Poison the outputs so that an output the call fails to write shows up.
    for x in (gk, gv, gtd, gtf):
        x.fill_(float("nan"))
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.wkv4_backward_noalloc(gy.data_ptr(), w.data_ptr(), u.data_ptr(), k.data_ptr(),
                                   v.data_ptr(), gk.data_ptr(), gv.data_ptr(), gtd.data_ptr(),
                                   gtf.data_ptr(), b, t, c, code, stream)
    L.check(rc, "wkv4_backward_noalloc")
    return gk, gv, gtd, gtf


def _check_pair(shape, dtype, seed):
    L, lib = _lib()
    b, t, c = shape
    print(f"no-alloc backward: B={b} T={t} C={c} {dtype} seed={seed}", flush=True)
    args = _inputs(b, t, c, dtype, seed)
    got = _no_alloc(L, lib, *args)
    exp = _with_workspace(L, lib, *args)
    torch.cuda.synchronize()
    for g, e, name in zip(got, exp, ("grad_k", "grad_v", "grad_time_decay", "grad_time_first")):
        assert torch.equal(g, e), f"{name} differs from wkv4_backward at {shape} {dtype}"


def test_no_alloc_backward_matches_workspace_backward_twice_in_a_row():
    # Headline channel count first, then a smaller ragged shape (C not a
    # multiple of 128, T not a multiple of 64) on the same scratch.
    _check_pair((16, 1024, 512), torch.bfloat16, seed=1)
    _check_pair((3, 70, 96), torch.bfloat16, seed=2)


def test_no_alloc_backward_fp32_and_fp16():
    _check_pair((4, 200, 256), torch.float32, seed=3)
    _check_pair((2, 33, 70), torch.float16, seed=4)


def test_no_alloc_backward_largest_headline_size():
    # B=64, T=1024, C=512 (the 41M training shape) needs 6.6 MB of the 16 MiB.
    _check_pair((64, 1024, 512), torch.bfloat16, seed=5)
    _check_pair((8, 128, 512), torch.bfloat16, seed=6)


def test_no_alloc_backward_empty_and_oversized():
    L, lib = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    # T = 0: the parameter gradients are zeroed, nothing else is touched.
    c = 64
    gtd = torch.full((c,), 5.0, device=DEV)
    gtf = torch.full((c,), 5.0, device=DEV)
    rc = lib.wkv4_backward_noalloc(None, None, None, None, None, None, None, gtd.data_ptr(),
                                   gtf.data_ptr(), 2, 0, c, 1, stream)
    L.check(rc, "wkv4_backward_noalloc")
    torch.cuda.synchronize()
    assert torch.count_nonzero(gtd) == 0 and torch.count_nonzero(gtf) == 0
    # Beyond the fixed scratch: rejected with the workspace status, no launch.
    rc = lib.wkv4_backward_noalloc(None, None, None, None, None, None, None, gtd.data_ptr(),
                                   gtf.data_ptr(), 64, 4096, 512, 1, stream)
    assert rc == 3 and b"scratch" in lib.wkv_last_error_string()
