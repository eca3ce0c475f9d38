"""RWKV-7 DPLR recurrence op (``myelin::wkv7_forward``), forward only.

Per (batch, head), head size N = 64, state ``S`` [N_v, N_k] float32::

    S_t = S_{t-1} (diag(w_t) + a_t b_t^T) + v_t k_t^T
    y_t = S_t r_t

``r, w, k, v, a, b`` are ``[B, T, H, 64]`` (float32, bfloat16 or float16),
``w`` is the per-step decay in (0, 1) (callers pass ``exp(-exp(x))``), and
the optional ``state`` is ``[B, H, 64, 64]`` float32 (zeros when omitted).
Returns ``(y [B, T, H, 64] in r's dtype, final state [B, H, 64, 64] fp32)``.

The reference's RWKV-7 code (``wkv7_compile.py``, ``wkv7_fla_op.py``) was
deleted from its tree (``benchmarks/results/optimizer_wkv_experiments_5090.md:3``)
and its numerics came from the external ``fla`` package, which is not pinned
anywhere in the reference; the op signature and the output convention
(post-update state, scale 1) are this library's own.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

HEAD_SIZE = 64


@torch.library.custom_op("myelin::wkv7_forward", mutates_args=())
def _wkv7_forward_op(
    r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, state: Tensor | None
) -> tuple[Tensor, Tensor]:
    tensors = [r, w, k, v, a, b]
    _lib.require_gpu(*tensors)
    if r.ndim != 4 or r.shape[-1] != HEAD_SIZE:
        raise ValueError(f"r, w, k, v, a, b must have shape [B, T, H, {HEAD_SIZE}]; got {tuple(r.shape)}")
    for x in tensors[1:]:
        if x.shape != r.shape:
            raise ValueError(f"r, w, k, v, a, b must share one shape; got {tuple(r.shape)} and {tuple(x.shape)}")
    bsz, steps, heads, n = r.shape
    dt = r.dtype if all(x.dtype == r.dtype for x in tensors) and r.dtype in (
        torch.float32, torch.bfloat16, torch.float16) else torch.float32
    xs = [_lib.aligned(x.to(dt)) for x in tensors]
    s0 = None
    if state is not None:
        if state.shape != (bsz, heads, n, n):
            raise ValueError(f"state must have shape {(bsz, heads, n, n)}; got {tuple(state.shape)}")
        _lib.require_gpu(r, state)
        s0 = _lib.aligned(state.float())
    y = torch.empty_like(xs[0])
    s_out = torch.empty((bsz, heads, n, n), dtype=torch.float32, device=r.device)
    lib = _lib.load()
    rc = lib.wkv7_forward(
        *[x.data_ptr() for x in xs], _lib.ptr(s0), y.data_ptr(), s_out.data_ptr(),
        bsz, steps, heads, n, _lib.dtype_code(dt), _lib.stream_of(r),
    )
    _lib.check(rc, "wkv7_forward")
    if y.dtype != r.dtype:
        y = y.to(r.dtype)
    return y, s_out


@_wkv7_forward_op.register_fake
def _(r, w, k, v, a, b, state):
    bsz, _, heads, n = r.shape
    return torch.empty_like(r), torch.empty((bsz, heads, n, n), dtype=torch.float32, device=r.device)


def wkv7_forward(r, w, k, v, a, b, state=None):
    """RWKV-7 DPLR forward; returns ``(y, final_state)``."""
    return torch.ops.myelin.wkv7_forward(r, w, k, v, a, b, state)
