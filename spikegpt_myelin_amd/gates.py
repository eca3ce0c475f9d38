"""Fused element-wise activations of the SpikeGPT blocks (gfx950 HIP kernels).

* ``myelin::relu_square(Tensor x) -> Tensor`` -- ``relu(x)**2`` of the
  channel mix (``src/spikegpt/language.py:1192``), computed in fp32 and
  rounded once to ``x.dtype``: the values the eager expression gives under
  autocast (square in fp32, cast at the next projection), in one pass and
  without the fp32 ``[B, T, 4C]`` temporaries;
* ``myelin::sigmoid_gate(Tensor r, Tensor x) -> Tensor`` -- ``sigmoid(r) * x``
  of the receptance gates (``language.py:1035, 1194``), with the eager 16-bit
  path's two roundings.

Both are differentiable (one-pass backward kernels).  Tensors whose element
count is not a multiple of 16 bytes take the eager expression instead.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

_NATIVE = (torch.float32, torch.bfloat16, torch.float16)


def _vec_ok(t: Tensor) -> bool:
    return t.dtype in _NATIVE and t.numel() % (16 // t.element_size()) == 0


@torch.library.custom_op("myelin::relu_square", mutates_args=())
def _relu_square(x: Tensor) -> Tensor:
    _lib.require_gpu(x)
    xs = _lib.aligned(x)
    y = torch.empty_like(xs)
    lib = _lib.load()
    rc = _lib.timed("relu_square", x.device, lambda: lib.relu_square_forward(
        xs.data_ptr(), y.data_ptr(), xs.numel(), _lib.dtype_code(xs.dtype), _lib.stream_of(xs)))
    _lib.check(rc, "relu_square_forward")
    return y


@_relu_square.register_fake
def _(x):
    return torch.empty_like(x)


@torch.library.custom_op("myelin::relu_square_backward", mutates_args=())
def _relu_square_backward(grad: Tensor, x: Tensor) -> Tensor:
    _lib.require_gpu(grad, x)
    xs = _lib.aligned(x)
    g = _lib.aligned(grad.to(xs.dtype))
    gx = torch.empty_like(xs)
    lib = _lib.load()
    rc = _lib.timed("relu_square_backward", x.device, lambda: lib.relu_square_backward(
        xs.data_ptr(), g.data_ptr(), gx.data_ptr(), xs.numel(), _lib.dtype_code(xs.dtype),
        _lib.stream_of(xs)))
    _lib.check(rc, "relu_square_backward")
    return gx


@_relu_square_backward.register_fake
def _(grad, x):
    return torch.empty_like(x)


def _rs_setup(ctx, inputs, output):
    (x,) = inputs
    ctx.save_for_backward(x)


def _rs_backward(ctx, grad):
    (x,) = ctx.saved_tensors
    return torch.ops.myelin.relu_square_backward(grad, x)


_relu_square.register_autograd(_rs_backward, setup_context=_rs_setup)


@torch.library.custom_op("myelin::sigmoid_gate", mutates_args=())
def _sigmoid_gate(r: Tensor, x: Tensor) -> Tensor:
    _lib.require_gpu(r, x)
    if r.shape != x.shape or r.dtype != x.dtype:
        raise ValueError(f"r and x must match; got {r.shape}/{r.dtype} and {x.shape}/{x.dtype}")
    rs, xs = _lib.aligned(r), _lib.aligned(x)
    y = torch.empty_like(xs)
    lib = _lib.load()
    rc = _lib.timed("sigmoid_gate", x.device, lambda: lib.sigmoid_gate_forward(
        rs.data_ptr(), xs.data_ptr(), y.data_ptr(), xs.numel(), _lib.dtype_code(xs.dtype),
        _lib.stream_of(xs)))
    _lib.check(rc, "sigmoid_gate_forward")
    return y


@_sigmoid_gate.register_fake
def _(r, x):
    return torch.empty_like(x)


@torch.library.custom_op("myelin::sigmoid_gate_backward", mutates_args=())
def _sigmoid_gate_backward(grad: Tensor, r: Tensor, x: Tensor) -> tuple[Tensor, Tensor]:
    _lib.require_gpu(grad, r, x)
    rs, xs = _lib.aligned(r), _lib.aligned(x)
    g = _lib.aligned(grad.to(xs.dtype))
    gr, gx = torch.empty_like(rs), torch.empty_like(xs)
    lib = _lib.load()
    rc = _lib.timed("sigmoid_gate_backward", x.device, lambda: lib.sigmoid_gate_backward(
        rs.data_ptr(), xs.data_ptr(), g.data_ptr(), gr.data_ptr(), gx.data_ptr(), xs.numel(),
        _lib.dtype_code(xs.dtype), _lib.stream_of(xs)))
    _lib.check(rc, "sigmoid_gate_backward")
    return gr, gx


@_sigmoid_gate_backward.register_fake
def _(grad, r, x):
    return torch.empty_like(r), torch.empty_like(x)


def _sg_setup(ctx, inputs, output):
    r, x = inputs
    ctx.save_for_backward(r, x)


def _sg_backward(ctx, grad):
    r, x = ctx.saved_tensors
    return torch.ops.myelin.sigmoid_gate_backward(grad, r, x)


_sigmoid_gate.register_autograd(_sg_backward, setup_context=_sg_setup)


def relu_square(x: Tensor) -> Tensor:
    """``torch.relu(x).square()`` (autocast values), fused on the GPU."""
    if x.is_cuda and _vec_ok(x):
        return torch.ops.myelin.relu_square(x)
    return torch.relu(x).square()


def sigmoid_gate(r: Tensor, x: Tensor) -> Tensor:
    """``torch.sigmoid(r) * x``, fused on the GPU when both share a dtype."""
    if r.is_cuda and r.dtype == x.dtype and r.shape == x.shape and _vec_ok(x):
        return torch.ops.myelin.sigmoid_gate(r, x)
    return torch.sigmoid(r) * x
