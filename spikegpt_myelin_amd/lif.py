"""Sequence LIF activation as custom ops served by the gfx950 HIP kernels.

The reference's ``SpikingSequenceLIF.forward`` (``src/spikegpt/language.py:848-918``)
runs the leaky integrate-and-fire recurrence over ``[B, T, C]`` through the
external ``myelin`` package's Triton kernels (``surrogate_lif_bf16io`` for
16-bit inputs, a store-all fp32 function otherwise) after moving time to the
front (``[T, B, C]`` copies), or through an eager per-step loop
(``language.py:813-840``).  Here one HIP kernel walks ``[B, T, C]`` in place:

``myelin::lif_sequence_forward(Tensor x, float decay, float threshold,
float reset, float slope) -> (Tensor spikes, Tensor checkpoint)`` -- spikes in
``x.dtype`` (exact 0/1), fp32 membrane, plus the membrane at every 32-step
block start for the backward;

``myelin::lif_sequence_backward(Tensor grad_spikes, Tensor x, Tensor
checkpoint, float decay, float threshold, float reset, float slope) -> Tensor``
-- ``dL/dx`` with the arctan surrogate derivative
``slope * 0.5 / (1 + (pi/2 * slope * (h - threshold))^2)`` and the reset path
differentiated, as autograd does through the reference's eager step.

The surrogate's exact definition lives in ``myelin`` (not part of the
reference tree and not installed); the form used here is SpikingJelly's ATan
surrogate with ``alpha = surrogate_slope``.  Spikes and membranes do not
depend on it; input gradients do.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

from . import _lib

CKPT_BLOCK = 32  # steps per membrane checkpoint
_NATIVE = (torch.float32, torch.bfloat16, torch.float16)


def checkpoint_shape(b: int, t: int, c: int) -> tuple[int, int, int]:
    return (b, (t + CKPT_BLOCK - 1) // CKPT_BLOCK, c)


def _forward_workspace(lib, b: int, t: int, c: int, device) -> tuple[Tensor | None, int]:
    """Workspace of the forward's split over time (boundary membranes), or
    (None, 0) for sizes that run as one pass."""
    nbytes = int(lib.lif_forward_workspace_bytes(b, t, c))
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


def _backward_workspace(lib, b: int, t: int, c: int, device) -> tuple[Tensor | None, int]:
    """Workspace of the backward's split over time (boundary carries), or
    (None, 0) for sizes that run as one pass."""
    nbytes = int(lib.lif_backward_workspace_bytes(b, t, c))
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


def _native(x: Tensor) -> Tensor:
    return _lib.aligned(x if x.dtype in _NATIVE else x.float())


@torch.library.custom_op("myelin::lif_sequence_forward", mutates_args=())
def _lif_forward(
    x: Tensor, decay: float, threshold: float, reset: float, slope: float
) -> tuple[Tensor, Tensor]:
    _lib.require_gpu(x)
    if x.ndim != 3:
        raise ValueError(f"inputs must have shape [B, T, C]; got {x.shape}")
    b, t, c = x.shape
    xs = _native(x)
    spikes = torch.empty_like(xs)
    ck = torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    ws, nbytes = _forward_workspace(lib, b, t, c, x.device)
    rc = _lib.timed("lif_forward", x.device, lambda: lib.lif_forward(
        xs.data_ptr(), spikes.data_ptr(), ck.data_ptr(), _lib.ptr(ws), nbytes, b, t, c, decay,
        threshold, reset, slope, _lib.dtype_code(xs.dtype), _lib.stream_of(xs),
    ))
    _lib.check(rc, "lif_forward")
    return spikes, ck


@_lif_forward.register_fake
def _(x, decay, threshold, reset, slope):
    b, t, c = x.shape
    dt = x.dtype if x.dtype in _NATIVE else torch.float32
    return (
        torch.empty(x.shape, dtype=dt, device=x.device),
        torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=x.device),
    )


@torch.library.custom_op("myelin::lif_sequence_backward", mutates_args=())
def _lif_backward(
    grad_spikes: Tensor, x: Tensor, checkpoint: Tensor, decay: float, threshold: float,
    reset: float, slope: float,
) -> Tensor:
    _lib.require_gpu(grad_spikes, x, checkpoint)
    b, t, c = x.shape
    xs = _native(x)
    gs = _lib.aligned(grad_spikes.to(xs.dtype))
    ck = _lib.aligned(checkpoint)
    gx = torch.empty_like(xs)
    lib = _lib.load()
    ws, nbytes = _backward_workspace(lib, b, t, c, x.device)
    rc = _lib.timed("lif_backward", x.device, lambda: lib.lif_backward(
        xs.data_ptr(), gs.data_ptr(), ck.data_ptr(), gx.data_ptr(), _lib.ptr(ws), nbytes, b, t, c,
        decay, threshold, reset, slope, _lib.dtype_code(xs.dtype), _lib.stream_of(xs),
    ))
    _lib.check(rc, "lif_backward")
    return gx


@_lif_backward.register_fake
def _(grad_spikes, x, checkpoint, decay, threshold, reset, slope):
    dt = x.dtype if x.dtype in _NATIVE else torch.float32
    return torch.empty(x.shape, dtype=dt, device=x.device)


def _setup_context(ctx, inputs, output):
    x, decay, threshold, reset, slope = inputs
    _, ck = output
    ctx.save_for_backward(x, ck)
    ctx.params = (decay, threshold, reset, slope)
    ctx.mark_non_differentiable(ck)
    ctx.set_materialize_grads(False)


def _backward(ctx, grad_spikes, _grad_ck):
    x, ck = ctx.saved_tensors
    if grad_spikes is None:
        return None, None, None, None, None
    gx = torch.ops.myelin.lif_sequence_backward(grad_spikes, x, ck, *ctx.params)
    return gx.to(x.dtype), None, None, None, None


_lif_forward.register_autograd(_backward, setup_context=_setup_context)


def atan_surrogate(x: Tensor) -> Tensor:
    """The smooth arctan spike ``atan(pi/2 * x) / pi + 1/2`` (``x`` already
    scaled by the slope).  Its derivative ``0.5 / (1 + (pi/2 * x)^2)`` is the
    surrogate gradient the LIF kernels apply.  It stands in for the default
    ``surrogate`` of ``SpikingSequenceLIF`` (``language.py:775``), which the
    external ``myelin`` package defines under the same name."""
    return torch.atan((math.pi / 2.0) * x) / math.pi + 0.5


def serves_surrogate(surrogate, hard_forward: bool = True) -> bool:
    """True when the LIF kernels compute what ``SpikingSequenceLIF`` with this
    ``surrogate`` and ``hard_forward`` computes: a Heaviside forward
    (``hard_forward=True``, ``language.py:835-836``) with the arctan
    surrogate's derivative.  The arctan surrogate is this module's
    :func:`atan_surrogate` or ``myelin``'s function of that name (recognised
    by module and name; ``myelin`` is not imported).  Any other surrogate, or
    the smooth forward ``spike = surrogate(c)`` (``:838``), is not served."""
    if not hard_forward:
        return False
    if surrogate is atan_surrogate:
        return True
    module = getattr(surrogate, "__module__", None) or ""
    return module.split(".")[0] == "myelin" and getattr(surrogate, "__name__", "") == \
        "atan_surrogate"


def lif_sequence(
    x: Tensor, *, tau: float = 2.0, threshold: float = 1.0, reset: float = 0.0,
    surrogate_slope: float = 2.0,
) -> Tensor:
    """Spikes of the LIF recurrence over ``[B, T, C]`` (``x.dtype``), differentiable."""
    spikes, _ = torch.ops.myelin.lif_sequence_forward(
        x, 1.0 - 1.0 / tau, float(threshold), float(reset), float(surrogate_slope)
    )
    return spikes if spikes.dtype == x.dtype else spikes.to(x.dtype)


# ------------------------------------------------------ fused residual add --
# myelin::lif_residual_forward(Tensor x, Tensor residual, float decay,
#     float threshold, float reset, float slope) -> (Tensor out, Tensor ck)
# out = residual + spikes(x) in fp32: the block's `residual + lif(...)`
# (language.py:1326-1330) with the spikes added as they are produced, so the
# spikes tensor, the separate add and, in the backward, the cast of the fp32
# residual gradient to x's dtype disappear.


def _residual_ok(x: Tensor, residual: Tensor) -> bool:
    if x.ndim != 3 or residual.shape != x.shape or residual.dtype != torch.float32:
        return False
    b, t, c = x.shape
    return x.dtype in _NATIVE and c % 8 == 0 and t * c * 4 < (1 << 31)


@torch.library.custom_op("myelin::lif_residual_forward", mutates_args=())
def _lif_res_forward(x: Tensor, residual: Tensor, decay: float, threshold: float, reset: float,
                     slope: float) -> tuple[Tensor, Tensor]:
    _lib.require_gpu(x, residual)
    if not _residual_ok(x, residual):
        raise ValueError("lif_residual_forward: x [B, T, C] (C % 8 == 0) and an fp32 residual "
                         f"of the same shape; got {x.shape}/{x.dtype}, {residual.shape}/"
                         f"{residual.dtype}")
    b, t, c = x.shape
    xs = _native(x)
    rs = _lib.aligned(residual)
    out = torch.empty_like(rs)
    ck = torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    ws, nbytes = _forward_workspace(lib, b, t, c, x.device)
    rc = _lib.timed("lif_residual_forward", x.device, lambda: lib.lif_residual_forward(
        xs.data_ptr(), rs.data_ptr(), out.data_ptr(), ck.data_ptr(), _lib.ptr(ws), nbytes, b, t, c,
        decay, threshold, reset, slope, _lib.dtype_code(xs.dtype), _lib.stream_of(xs)))
    _lib.check(rc, "lif_residual_forward")
    return out, ck


@_lif_res_forward.register_fake
def _(x, residual, decay, threshold, reset, slope):
    b, t, c = x.shape
    return (torch.empty(x.shape, dtype=torch.float32, device=x.device),
            torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=x.device))


@torch.library.custom_op("myelin::lif_residual_backward", mutates_args=())
def _lif_res_backward(grad_out: Tensor, x: Tensor, checkpoint: Tensor, decay: float,
                      threshold: float, reset: float, slope: float) -> Tensor:
    _lib.require_gpu(grad_out, x, checkpoint)
    b, t, c = x.shape
    xs = _native(x)
    g = _lib.aligned(grad_out.float())
    gx = torch.empty_like(xs)
    lib = _lib.load()
    ws, nbytes = _backward_workspace(lib, b, t, c, x.device)
    rc = _lib.timed("lif_residual_backward", x.device, lambda: lib.lif_residual_backward(
        xs.data_ptr(), g.data_ptr(), checkpoint.data_ptr(), gx.data_ptr(), _lib.ptr(ws), nbytes,
        b, t, c, decay, threshold, reset, slope, _lib.dtype_code(xs.dtype), _lib.stream_of(xs)))
    _lib.check(rc, "lif_residual_backward")
    return gx


@_lif_res_backward.register_fake
def _(grad_out, x, checkpoint, decay, threshold, reset, slope):
    dt = x.dtype if x.dtype in _NATIVE else torch.float32
    return torch.empty(x.shape, dtype=dt, device=x.device)


def _res_setup_context(ctx, inputs, output):
    x, _residual, decay, threshold, reset, slope = inputs
    _, ck = output
    ctx.save_for_backward(x, ck)
    ctx.params = (decay, threshold, reset, slope)
    ctx.mark_non_differentiable(ck)
    ctx.set_materialize_grads(False)


def _res_backward(ctx, grad_out, _grad_ck):
    if grad_out is None:
        return None, None, None, None, None, None
    x, ck = ctx.saved_tensors
    gx = torch.ops.myelin.lif_residual_backward(grad_out, x, ck, *ctx.params)
    return gx.to(x.dtype), grad_out, None, None, None, None


_lif_res_forward.register_autograd(_res_backward, setup_context=_res_setup_context)


def lif_residual(residual: Tensor, x: Tensor, *, tau: float = 2.0, threshold: float = 1.0,
                 reset: float = 0.0, surrogate_slope: float = 2.0) -> Tensor:
    """``residual + lif_sequence(x, ...)`` (fp32), fused into the LIF kernels
    for an fp32 residual on the GPU with C a multiple of 8; otherwise the two
    operations."""
    if x.is_cuda and residual.is_cuda and _residual_ok(x, residual):
        out, _ = torch.ops.myelin.lif_residual_forward(
            x, residual, 1.0 - 1.0 / tau, float(threshold), float(reset), float(surrogate_slope))
        return out
    return residual + lif_sequence(x, tau=tau, threshold=threshold, reset=reset,
                                   surrogate_slope=surrogate_slope)
