"""The ``myelin::`` WKV custom ops, served by hand-written gfx950 HIP kernels.

Drop-in for the reference's Triton-backed ops (same op names, schemas, dtype
rules, fake impls and autograd formulas):

* ``myelin::wkv_forward(Tensor key, Tensor value, Tensor time_decay,
  Tensor time_first) -> Tensor`` -- ``src/spikegpt/wkv_triton.py:147-162``.
  fp32 recurrence; output in ``key.dtype``.
* ``myelin::wkv_backward(Tensor grad_y, Tensor w, Tensor u, Tensor k,
  Tensor v) -> Tensor[]`` -- ``wkv_triton.py:164-198``.  ``w`` is
  ``-exp(time_decay)``; returns ``[gk, gv, g_time_decay, g_time_first]`` with
  the ``* w`` chain rule applied and the parameter grads summed over B.
* ``myelin::wkv_forward_bf16io`` / ``myelin::wkv_backward_bf16io`` --
  ``src/spikegpt/wkv_bf16.py:143-215``: native 16-bit I/O, fp32 state.
* autograd: ``setup_context`` saves ``(key, value, time_decay, time_first)``
  and the backward recomputes ``w, u`` (``wkv_triton.py:200-218``,
  ``wkv_bf16.py:197-215``).

Python API (``wkv_triton.py:221-228``, ``wkv_bf16.py:218-231``):
:func:`weighted_key_value_hip` and :func:`weighted_key_value_hip_bf16io`, also
exported under the reference's names ``weighted_key_value_triton`` and
``weighted_key_value_triton_bf16io`` so that callers switch by import only.

The ops run on HIP devices only and raise on CPU tensors: there is no
non-GPU implementation behind them.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

_NATIVE = (torch.float32, torch.bfloat16, torch.float16)


def _launch_forward(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """y = WKV(key, value) with fp32 state; y has ``key.dtype`` when that is
    float32/bfloat16/float16 (same dtype as ``value``), else float32."""
    _lib.require_gpu(key, value, time_decay, time_first)
    b, t, c = key.shape
    if key.dtype == value.dtype and key.dtype in _NATIVE:
        k = _lib.aligned(key)
        v = _lib.aligned(value)
    else:  # mixed or wider dtypes: exact fp32 path (the reference's .float())
        k = _lib.aligned(key.float())
        v = _lib.aligned(value.float())
    td = _lib.aligned(time_decay.float())
    tf = _lib.aligned(time_first.float())
    y = torch.empty_like(k)
    lib = _lib.load()
    rc = _lib.timed("wkv4_forward", k.device, lambda: lib.wkv4_forward(
        k.data_ptr(), v.data_ptr(), td.data_ptr(), tf.data_ptr(), y.data_ptr(),
        b, t, c, _lib.dtype_code(k.dtype), _lib.stream_of(k),
    ))
    _lib.check(rc, "wkv4_forward")
    return y


def _launch_backward(grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor) -> list[Tensor]:
    """[gk, gv (k's dtype), g_time_decay, g_time_first (fp32 [C])]."""
    _lib.require_gpu(grad_y, w, u, k, v)
    b, t, c = k.shape
    out_dtype = k.dtype
    if grad_y.dtype == k.dtype == v.dtype and k.dtype in _NATIVE:
        gy_, k_, v_ = _lib.aligned(grad_y), _lib.aligned(k), _lib.aligned(v)
    else:
        gy_, k_, v_ = _lib.aligned(grad_y.float()), _lib.aligned(k.float()), _lib.aligned(v.float())
    w_ = _lib.aligned(w.float())
    u_ = _lib.aligned(u.float())
    gk = torch.empty_like(k_)
    gv = torch.empty_like(k_)
    gtd = torch.empty(c, dtype=torch.float32, device=k.device)
    gtf = torch.empty(c, dtype=torch.float32, device=k.device)
    code = _lib.dtype_code(k_.dtype)
    lib = _lib.load()
    nbytes = lib.wkv4_backward_workspace_bytes(b, t, c, code)
    ws = torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=k.device)
    rc = _lib.timed("wkv4_backward", k.device, lambda: lib.wkv4_backward(
        gy_.data_ptr(), w_.data_ptr(), u_.data_ptr(), k_.data_ptr(), v_.data_ptr(),
        gk.data_ptr(), gv.data_ptr(), gtd.data_ptr(), gtf.data_ptr(),
        ws.data_ptr(), ws.numel(), b, t, c, code, _lib.stream_of(k_),
    ))
    _lib.check(rc, "wkv4_backward")
    if gk.dtype != out_dtype:
        gk, gv = gk.to(out_dtype), gv.to(out_dtype)
    return [gk, gv, gtd, gtf]


# ------------------------------------------------------------- fp32-I/O op --
@torch.library.custom_op("myelin::wkv_forward", mutates_args=())
def _wkv_forward_op(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    # fp32 recurrence on the exactly widened inputs; y cast back to key.dtype
    # (wkv_triton.py:151-158).  bf16/fp16 inputs are widened in registers,
    # which gives the same values as the reference's .float() copies.
    y = _launch_forward(key, value, time_decay, time_first)
    return y if y.dtype == key.dtype else y.to(key.dtype)


@_wkv_forward_op.register_fake
def _(key, value, time_decay, time_first):
    return torch.empty_like(key)


@torch.library.custom_op("myelin::wkv_backward", mutates_args=())
def _wkv_backward_op(grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor) -> list[Tensor]:
    return _launch_backward(grad_y, w, u, k, v)


@_wkv_backward_op.register_fake
def _(grad_y, w, u, k, v):
    return [torch.empty_like(k), torch.empty_like(k), torch.empty_like(w), torch.empty_like(u)]


def _setup_context(ctx, inputs, output):
    key, value, time_decay, time_first = inputs
    ctx.save_for_backward(key, value, time_decay, time_first)


def _backward(ctx, grad_y):
    key, value, time_decay, time_first = ctx.saved_tensors
    w = _lib.aligned(-torch.exp(time_decay.float()))
    u = _lib.aligned(time_first.float())
    gk, gv, gtd, gtf = torch.ops.myelin.wkv_backward(
        _lib.aligned(grad_y.float()), w, u, _lib.aligned(key.float()), _lib.aligned(value.float())
    )
    return gk.to(key.dtype), gv.to(value.dtype), gtd.to(time_decay.dtype), gtf.to(time_first.dtype)


_wkv_forward_op.register_autograd(_backward, setup_context=_setup_context)


# ------------------------------------------------------------ 16-bit-I/O op --
@torch.library.custom_op("myelin::wkv_forward_bf16io", mutates_args=())
def _wkv_forward_bf16io_op(
    key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor
) -> Tensor:
    # Native-dtype k/v/y (wkv_bf16.py:147-154); fp32 state in registers.
    y = _launch_forward(key, value, time_decay, time_first)
    return y if y.dtype == key.dtype else y.to(key.dtype)


@_wkv_forward_bf16io_op.register_fake
def _(key, value, time_decay, time_first):
    return torch.empty_like(key)


@torch.library.custom_op("myelin::wkv_backward_bf16io", mutates_args=())
def _wkv_backward_bf16io_op(
    grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor
) -> list[Tensor]:
    return _launch_backward(grad_y, w, u, k, v)


@_wkv_backward_bf16io_op.register_fake
def _(grad_y, w, u, k, v):
    return [torch.empty_like(k), torch.empty_like(k), torch.empty_like(w), torch.empty_like(u)]


def _backward_bf16io(ctx, grad_y):
    key, value, time_decay, time_first = ctx.saved_tensors
    w = _lib.aligned(-torch.exp(time_decay.float()))
    u = _lib.aligned(time_first.float())
    gk, gv, gtd, gtf = torch.ops.myelin.wkv_backward_bf16io(
        _lib.aligned(grad_y), w, u, _lib.aligned(key), _lib.aligned(value)
    )
    return gk.to(key.dtype), gv.to(value.dtype), gtd.to(time_decay.dtype), gtf.to(time_first.dtype)


_wkv_forward_bf16io_op.register_autograd(_backward_bf16io, setup_context=_setup_context)


# ------------------------------------------------------------- Python API --
def weighted_key_value_hip(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """RWKV WKV recurrence via the fused HIP custom op (``myelin::wkv_forward``)."""
    return torch.ops.myelin.wkv_forward(key, value, time_decay, time_first)


def weighted_key_value_hip_bf16io(
    key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor
) -> Tensor:
    """RWKV WKV via the 16-bit-I/O HIP custom op (``myelin::wkv_forward_bf16io``).

    Same values as :func:`weighted_key_value_hip` for bf16/fp16 inputs (the
    widening to fp32 is exact and the output rounding is the same), without
    the fp32 copies of k and v.
    """
    return torch.ops.myelin.wkv_forward_bf16io(key, value, time_decay, time_first)


# The reference's public names for the same two entry points.
weighted_key_value_triton = weighted_key_value_hip
weighted_key_value_triton_bf16io = weighted_key_value_hip_bf16io
