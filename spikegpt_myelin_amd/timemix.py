"""Fused token-shift mixing as custom ops served by a gfx950 HIP kernel.

The reference forms every projection input of the time mix and the channel
mix with the eager expression ``x * mix + shift(x) * (1 - mix)``
(``src/spikegpt/language.py:344-353``; three mixing vectors at :1016-1018,
two at :1190-1191), each a handful of full passes over ``[B, T, C]`` in fp32
plus autocast's cast to bf16 for the projection.  Here:

``myelin::token_shift_mix(Tensor x, Tensor mix, ScalarType out_dtype) ->
Tensor[]`` -- one pass: reads ``x`` once and writes the ``n = mix.shape[0]``
mixed tensors, rounded once to ``out_dtype``, with the
reference's fp32 arithmetic and operation order, so the values equal the
eager expression followed by the cast.

``myelin::token_shift_mix_backward(Tensor[] grads, Tensor x, Tensor mix) ->
(Tensor grad_x, Tensor grad_mix)`` -- one pass for ``grad_x`` plus a fixed-
order reduction for ``grad_mix`` ``[n, C]``.

:func:`token_shift_mix` picks ``out_dtype`` from the active CUDA autocast
dtype, as the projections would cast their inputs.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import _lib

_NATIVE = (torch.float32, torch.bfloat16, torch.float16)


def _check(x: Tensor, mix: Tensor) -> None:
    if x.ndim != 3:
        raise ValueError(f"inputs must have shape [B, T, C]; got {x.shape}")
    if mix.ndim != 2 or mix.shape[1] != x.shape[2] or not 1 <= mix.shape[0] <= 3:
        raise ValueError(f"mix must have shape [n, {x.shape[2]}] with 1 <= n <= 3; got {mix.shape}")


@torch.library.custom_op("myelin::token_shift_mix", mutates_args=())
def _shift_mix(x: Tensor, mix: Tensor, out_dtype: torch.dtype) -> list[Tensor]:
    _lib.require_gpu(x, mix)
    _check(x, mix)
    xs = _lib.aligned(x if x.dtype in _NATIVE else x.float())
    od = out_dtype
    mx = _lib.aligned(mix.float())
    n = mx.shape[0]
    b, t, c = xs.shape
    outs = [torch.empty(xs.shape, dtype=od, device=x.device) for _ in range(n)]
    ptrs = [o.data_ptr() for o in outs] + [None] * (3 - n)
    lib = _lib.load()
    rc = _lib.timed("token_shift_mix", x.device, lambda: lib.token_shift_mix_forward(
        xs.data_ptr(), _lib.dtype_code(xs.dtype), mx.data_ptr(), n, *ptrs, _lib.dtype_code(od),
        b, t, c, _lib.stream_of(xs),
    ))
    _lib.check(rc, "token_shift_mix_forward")
    return outs


@_shift_mix.register_fake
def _(x, mix, out_dtype):
    return [torch.empty(x.shape, dtype=out_dtype, device=x.device) for _ in range(mix.shape[0])]


@torch.library.custom_op("myelin::token_shift_mix_backward", mutates_args=())
def _shift_mix_backward(grads: list[Tensor], x: Tensor, mix: Tensor) -> tuple[Tensor, Tensor]:
    _lib.require_gpu(x, mix, *grads)
    xs = _lib.aligned(x if x.dtype in _NATIVE else x.float())
    mx = _lib.aligned(mix.float())
    n = mx.shape[0]
    b, t, c = xs.shape
    gdt = grads[0].dtype if grads[0].dtype in _NATIVE else torch.float32
    if gdt != xs.dtype and xs.dtype != torch.float32:
        gdt = xs.dtype
    gs = [_lib.aligned(g.to(gdt)) for g in grads]
    gx = torch.empty_like(xs)
    gmix = torch.empty((n, c), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    ws = torch.empty(max(int(lib.token_shift_mix_workspace_bytes(n, b, t, c)), 16),
                     dtype=torch.uint8, device=x.device)
    ptrs = [g.data_ptr() for g in gs] + [None] * (3 - n)
    rc = _lib.timed("token_shift_mix_backward", x.device, lambda: lib.token_shift_mix_backward(
        xs.data_ptr(), _lib.dtype_code(xs.dtype), mx.data_ptr(), n, *ptrs, _lib.dtype_code(gdt),
        gx.data_ptr(), gmix.data_ptr(), ws.data_ptr(), ws.numel(), b, t, c, _lib.stream_of(xs),
    ))
    _lib.check(rc, "token_shift_mix_backward")
    return gx, gmix


@_shift_mix_backward.register_fake
def _(grads, x, mix):
    dt = x.dtype if x.dtype in _NATIVE else torch.float32
    return (torch.empty(x.shape, dtype=dt, device=x.device),
            torch.empty(mix.shape, dtype=torch.float32, device=x.device))


def _setup_context(ctx, inputs, output):
    x, mix, _ = inputs
    ctx.save_for_backward(x, mix)


def _backward(ctx, grads):
    x, mix = ctx.saved_tensors
    grads = [torch.zeros_like(x) if g is None else g for g in grads]
    gx, gmix = torch.ops.myelin.token_shift_mix_backward(grads, x, mix)
    return gx.to(x.dtype), gmix.to(mix.dtype), None


_shift_mix.register_autograd(_backward, setup_context=_setup_context)


def token_shift_mix(x: Tensor, mix: Tensor) -> list[Tensor]:
    """``[x * mix[j] + shift(x) * (1 - mix[j]) for j]`` in the autocast dtype
    when CUDA autocast is on (the projections' input type), else in
    ``x.dtype``."""
    if torch.is_autocast_enabled("cuda"):
        out_dtype = torch.get_autocast_dtype("cuda")
    else:
        out_dtype = x.dtype if x.dtype in _NATIVE else torch.float32
    return torch.ops.myelin.token_shift_mix(x, mix, out_dtype)


# ------------------------------------------------ layer norm + token shift --
# myelin::layer_norm_shift_mix(Tensor x, Tensor weight, Tensor bias, Tensor mix,
#     float eps, ScalarType out_dtype) -> Tensor[]
# returns the n mixed tensors followed by the per-row mean and rstd [B*T]
# (saved for the backward): a block half's F.layer_norm and token-shift mixes
# (language.py:1341-1356, 344-353) in one pass over x.
LN_MIX_CHANNELS = (256, 512)


@torch.library.custom_op("myelin::layer_norm_shift_mix", mutates_args=())
def _ln_shift_mix(x: Tensor, weight: Tensor, bias: Tensor, mix: Tensor, eps: float,
                  out_dtype: torch.dtype) -> list[Tensor]:
    _lib.require_gpu(x, weight, bias, mix)
    _check(x, mix)
    b, t, c = x.shape
    if x.dtype != torch.float32 or c not in LN_MIX_CHANNELS or mix.shape[0] < 2:
        raise ValueError("layer_norm_shift_mix takes fp32 x with C in (256, 512) and 2-3 mixes")
    xs = _lib.aligned(x)
    w, bb = _lib.aligned(weight.float()), _lib.aligned(bias.float())
    mx = _lib.aligned(mix.float())
    n = mx.shape[0]
    outs = [torch.empty(xs.shape, dtype=out_dtype, device=x.device) for _ in range(n)]
    mean = torch.empty(b * t, dtype=torch.float32, device=x.device)
    rstd = torch.empty_like(mean)
    ptrs = [o.data_ptr() for o in outs] + [None] * (3 - n)
    lib = _lib.load()
    rc = _lib.timed("layer_norm_shift_mix", x.device, lambda: lib.layer_norm_shift_mix_forward(
        xs.data_ptr(), w.data_ptr(), bb.data_ptr(), eps, mx.data_ptr(), n, *ptrs,
        _lib.dtype_code(out_dtype), mean.data_ptr(), rstd.data_ptr(), b, t, c,
        _lib.stream_of(xs)))
    _lib.check(rc, "layer_norm_shift_mix_forward")
    return outs + [mean, rstd]


@_ln_shift_mix.register_fake
def _(x, weight, bias, mix, eps, out_dtype):
    b, t, _ = x.shape
    return ([torch.empty(x.shape, dtype=out_dtype, device=x.device) for _ in range(mix.shape[0])]
            + [x.new_empty(b * t, dtype=torch.float32), x.new_empty(b * t, dtype=torch.float32)])


@torch.library.custom_op("myelin::layer_norm_shift_mix_backward", mutates_args=())
def _ln_shift_mix_backward(grads: list[Tensor], x: Tensor, weight: Tensor, bias: Tensor,
                           mix: Tensor, mean: Tensor, rstd: Tensor,
                           grad_x_add: Optional[Tensor] = None) -> tuple[Tensor, Tensor]:
    """Returns ``grad_x`` [B, T, C] fp32 (plus ``grad_x_add`` when given) and
    ``[n + 2, C]`` fp32 parameter gradients (the n mixing vectors, the
    weight, the bias)."""
    _lib.require_gpu(x, weight, bias, mix, mean, rstd, *grads)
    if grad_x_add is not None:
        _lib.require_gpu(grad_x_add)
        if grad_x_add.shape != x.shape:
            raise ValueError("layer_norm_shift_mix_backward: grad_x_add must have the shape of x")
        gadd = _lib.aligned(grad_x_add.float().contiguous())
    b, t, c = x.shape
    n = mix.shape[0]
    gdt = grads[0].dtype if grads[0].dtype in _NATIVE else torch.float32
    gs = [_lib.aligned(g.to(gdt)) for g in grads]
    xs = _lib.aligned(x)
    w, bb, mx = (_lib.aligned(p.float()) for p in (weight, bias, mix))
    gx = torch.empty_like(xs)
    gp = torch.empty((n + 2, c), dtype=torch.float32, device=x.device)  # every entry written
    lib = _lib.load()
    ws = torch.empty(max(int(lib.layer_norm_shift_mix_workspace_bytes(n, b, t, c)), 16),
                     dtype=torch.uint8, device=x.device)
    ptrs = [g.data_ptr() for g in gs] + [None] * (3 - n)
    rc = _lib.timed("layer_norm_shift_mix_backward", x.device,
                    lambda: lib.layer_norm_shift_mix_backward(
                        xs.data_ptr(), w.data_ptr(), bb.data_ptr(), mx.data_ptr(), n,
                        mean.data_ptr(), rstd.data_ptr(), *ptrs, _lib.dtype_code(gdt),
                        gx.data_ptr(), None if grad_x_add is None else gadd.data_ptr(),
                        gp.data_ptr(), ws.data_ptr(), ws.numel(), b, t, c,
                        _lib.stream_of(xs)))
    _lib.check(rc, "layer_norm_shift_mix_backward")
    return gx, gp


@_ln_shift_mix_backward.register_fake
def _(grads, x, weight, bias, mix, mean, rstd, grad_x_add=None):
    return (torch.empty(x.shape, dtype=torch.float32, device=x.device),
            x.new_empty((mix.shape[0] + 2, x.shape[2]), dtype=torch.float32))


def _ln_setup_context(ctx, inputs, output):
    x, weight, bias, mix, _, _ = inputs
    mean, rstd = output[-2], output[-1]
    ctx.save_for_backward(x, weight, bias, mix, mean, rstd)


def _ln_backward(ctx, grads):
    x, weight, bias, mix, mean, rstd = ctx.saved_tensors
    n = mix.shape[0]
    gouts = [torch.zeros(x.shape, dtype=torch.float32, device=x.device) if g is None else g
             for g in grads[:n]]
    gx, gp = torch.ops.myelin.layer_norm_shift_mix_backward(gouts, x, weight, bias, mix, mean,
                                                           rstd)
    return (gx, gp[n].to(weight.dtype), gp[n + 1].to(bias.dtype), gp[:n].to(mix.dtype), None,
            None)


_ln_shift_mix.register_autograd(_ln_backward, setup_context=_ln_setup_context)


class _LnShiftMixFork(torch.autograd.Function):
    """``myelin::layer_norm_shift_mix`` that also hands back its input ``x``
    (the residual stream, ``language.py:1326-1356``).  The gradient that
    reaches ``x`` through that second use arrives here and is added to
    ``grad_x`` inside the backward kernel, in place of autograd's separate
    fp32 add of the two gradients (same values: one fp32 add either way)."""

    @staticmethod
    def forward(ctx, x, weight, bias, mix, eps, out_dtype):  # noqa: D102
        outs = torch.ops.myelin.layer_norm_shift_mix(x, weight, bias, mix, eps, out_dtype)
        ctx.save_for_backward(x, weight, bias, mix, outs[-2], outs[-1])
        return (*outs[:-2], x)

    @staticmethod
    def backward(ctx, *grads):  # noqa: D102
        x, weight, bias, mix, mean, rstd = ctx.saved_tensors
        n = mix.shape[0]
        gouts = [torch.zeros(x.shape, dtype=torch.float32, device=x.device) if g is None else g
                 for g in grads[:n]]
        gx, gp = torch.ops.myelin.layer_norm_shift_mix_backward(gouts, x, weight, bias, mix,
                                                               mean, rstd, grads[n])
        return (gx, gp[n].to(weight.dtype), gp[n + 1].to(bias.dtype), gp[:n].to(mix.dtype),
                None, None)


def _ln_fusable(x: Tensor, norm: torch.nn.LayerNorm, mix: Tensor) -> bool:
    c = x.shape[-1]
    return (x.is_cuda and x.dtype == torch.float32 and x.ndim == 3 and c in LN_MIX_CHANNELS
            and mix.ndim == 2 and 2 <= mix.shape[0] <= 3 and norm.weight is not None
            and norm.bias is not None and tuple(norm.normalized_shape) == (c,))


def _ln_out_dtype() -> torch.dtype:
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return torch.float32


def layer_norm_shift_mix(x: Tensor, norm: torch.nn.LayerNorm, mix: Tensor) -> list[Tensor]:
    """``token_shift_mix(norm(x), mix)`` (values of the eager layer norm and
    mixes, in the autocast dtype when CUDA autocast is on), fused into one
    kernel pair when ``x`` is fp32 on the GPU with C in (256, 512) and 2-3
    mixing vectors; otherwise the layer norm and :func:`token_shift_mix`."""
    if not _ln_fusable(x, norm, mix):
        return token_shift_mix(norm(x), mix)
    outs = torch.ops.myelin.layer_norm_shift_mix(x, norm.weight, norm.bias, mix, float(norm.eps),
                                                _ln_out_dtype())
    return list(outs[:-2])


def layer_norm_shift_mix_fork(x: Tensor, norm: torch.nn.LayerNorm, mix: Tensor) -> list[Tensor]:
    """:func:`layer_norm_shift_mix` followed by ``x`` itself, for a block half
    whose residual stream ``x`` is also added to the half's output: use the
    returned ``x`` for that add, and the gradient it receives joins
    ``grad_x`` inside the fused backward kernel (same values as autograd's
    own sum of the two gradients)."""
    if not _ln_fusable(x, norm, mix):
        return [*token_shift_mix(norm(x), mix), x]
    return list(_LnShiftMixFork.apply(x, norm.weight, norm.bias, mix, float(norm.eps),
                                      _ln_out_dtype()))
