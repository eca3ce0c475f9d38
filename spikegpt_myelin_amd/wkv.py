"""The ``myelin::`` WKV custom ops, served by hand-written gfx950 HIP kernels.

Drop-in for the reference's Triton-backed ops (same op names, schemas, dtype
rules and results):

* ``myelin::wkv_forward(Tensor key, Tensor value, Tensor time_decay,
  Tensor time_first) -> Tensor`` -- ``src/spikegpt/wkv_triton.py:147-162``.
  fp32 recurrence; output in ``key.dtype``.
* ``myelin::wkv_backward(Tensor grad_y, Tensor w, Tensor u, Tensor k,
  Tensor v) -> Tensor[]`` -- ``wkv_triton.py:164-198``.  ``w`` is
  ``-exp(time_decay)``; returns ``[gk, gv, g_time_decay, g_time_first]`` with
  the ``* w`` chain rule applied and the parameter grads summed over B.
* ``myelin::wkv_forward_bf16io`` / ``myelin::wkv_backward_bf16io`` --
  ``src/spikegpt/wkv_bf16.py:143-215``: native 16-bit I/O, fp32 state.

Autograd.  The public forward ops are registered as the reference registers
them: opaque custom ops whose autograd saves the four inputs and calls the
public backward op, which computes the forward-state records from the inputs
before its reverse sweep (the reference's backward kernel replays the whole
forward, ``wkv_triton.py:85-115``).  The Python API
(:func:`weighted_key_value_hip` and the reference's names) runs the private
op ``myelin::wkv4_forward_train`` instead (or, in eager mode, a plain
``autograd.Function`` over the same launchers), which returns ``y`` together
with small forward-state checkpoint records (``[3, B, ceil(T/64), C]`` fp32,
~0.19 B per element) that autograd saves; its backward
(``myelin::wkv4_backward_train``) reads the sequence once from them.  Values
and gradients are the same on both routes.

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
CKPT_BLOCK = 64  # steps per checkpoint record
CKPT_FIELDS = 3


def _compute_inputs(key: Tensor, value: Tensor) -> tuple[Tensor, Tensor]:
    """k, v as the kernels read them: native when both share a float32 /
    bfloat16 / float16 dtype, else exactly widened to float32 (the
    reference's ``.float()``)."""
    if key.dtype == value.dtype and key.dtype in _NATIVE:
        return _lib.aligned(key), _lib.aligned(value)
    return _lib.aligned(key.float()), _lib.aligned(value.float())


def checkpoint_shape(b: int, t: int, c: int) -> tuple[int, int, int, int]:
    return (CKPT_FIELDS, b, (t + CKPT_BLOCK - 1) // CKPT_BLOCK, c)


def _forward_workspace(lib, b: int, t: int, c: int, device) -> tuple[Tensor | None, int]:
    """Workspace of the split-over-time forward (few rows), or (None, 0)
    when the one-row kernel runs; the library fills it itself."""
    nbytes = int(lib.wkv4_forward_workspace_bytes(b, t, c))
    if nbytes == 0:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


def _backward_workspace(lib, b: int, t: int, c: int, device) -> Tensor:
    """Workspace of a backward from records: [2, B, C] partials, or the split
    kernel's per-segment partials and carries for few rows."""
    nbytes = int(lib.wkv4_backward_checkpointed_workspace_bytes(b, t, c))
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _launch_forward(key, value, time_decay, time_first, *, with_checkpoint: bool):
    """y (compute dtype) and, optionally, the checkpoint records."""
    _lib.require_gpu(key, value, time_decay, time_first)
    b, t, c = key.shape
    k, v = _compute_inputs(key, value)
    td = _lib.aligned(time_decay.float())
    tf = _lib.aligned(time_first.float())
    y = torch.empty_like(k)
    lib = _lib.load()
    code = _lib.dtype_code(k.dtype)
    ws, nbytes = _forward_workspace(lib, b, t, c, k.device)
    if with_checkpoint:
        ck = torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=k.device)
        rc = _lib.timed("wkv4_forward", k.device, lambda: lib.wkv4_forward_checkpointed(
            k.data_ptr(), v.data_ptr(), td.data_ptr(), tf.data_ptr(), y.data_ptr(), ck.data_ptr(),
            _lib.ptr(ws), nbytes, b, t, c, code, _lib.stream_of(k),
        ))
        _lib.check(rc, "wkv4_forward_checkpointed")
        return y, ck
    rc = _lib.timed("wkv4_forward", k.device, lambda: lib.wkv4_forward(
        k.data_ptr(), v.data_ptr(), td.data_ptr(), tf.data_ptr(), y.data_ptr(),
        _lib.ptr(ws), nbytes, b, t, c, code, _lib.stream_of(k),
    ))
    _lib.check(rc, "wkv4_forward")
    return y, None


def _grad_inputs(grad_y: Tensor, k: Tensor, v: Tensor) -> tuple[Tensor, Tensor, Tensor]:
    if grad_y.dtype == k.dtype == v.dtype and k.dtype in _NATIVE:
        return _lib.aligned(grad_y), _lib.aligned(k), _lib.aligned(v)
    return _lib.aligned(grad_y.float()), _lib.aligned(k.float()), _lib.aligned(v.float())


def _launch_backward(grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor) -> list[Tensor]:
    """Standalone backward: [gk, gv (k's dtype), g_time_decay, g_time_first]."""
    _lib.require_gpu(grad_y, w, u, k, v)
    b, t, c = k.shape
    out_dtype = k.dtype
    gy_, k_, v_ = _grad_inputs(grad_y, k, v)
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


# ------------------------------------------------ private training ops ------
@torch.library.custom_op("myelin::wkv4_forward_train", mutates_args=())
def _wkv4_forward_train(
    key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor
) -> tuple[Tensor, Tensor]:
    y, ck = _launch_forward(key, value, time_decay, time_first, with_checkpoint=True)
    return y, ck


@_wkv4_forward_train.register_fake
def _(key, value, time_decay, time_first):
    b, t, c = key.shape
    dt = key.dtype if key.dtype == value.dtype and key.dtype in _NATIVE else torch.float32
    return (
        torch.empty(key.shape, dtype=dt, device=key.device),
        torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=key.device),
    )


def _launch_backward_train(grad_y: Tensor, key: Tensor, value: Tensor, time_decay: Tensor,
                           time_first: Tensor, checkpoint: Tensor) -> list[Tensor]:
    """[gk, gv (k's compute dtype), g_time_decay, g_time_first] from the
    forward's checkpoint records."""
    _lib.require_gpu(grad_y, key, value, time_decay, time_first, checkpoint)
    b, t, c = key.shape
    k, v = _compute_inputs(key, value)
    gy = _lib.aligned(grad_y.to(k.dtype))
    td = _lib.aligned(time_decay.float())
    tf = _lib.aligned(time_first.float())
    ck = _lib.aligned(checkpoint)
    gk = torch.empty_like(k)
    gv = torch.empty_like(k)
    gtd = torch.empty(c, dtype=torch.float32, device=k.device)
    gtf = torch.empty(c, dtype=torch.float32, device=k.device)
    lib = _lib.load()
    ws = _backward_workspace(lib, b, t, c, k.device)
    rc = _lib.timed("wkv4_backward", k.device, lambda: lib.wkv4_backward_checkpointed(
        gy.data_ptr(), td.data_ptr(), tf.data_ptr(), k.data_ptr(), v.data_ptr(), ck.data_ptr(),
        gk.data_ptr(), gv.data_ptr(), gtd.data_ptr(), gtf.data_ptr(), ws.data_ptr(),
        ws.numel(), b, t, c, _lib.dtype_code(k.dtype), _lib.stream_of(k),
    ))
    _lib.check(rc, "wkv4_backward_checkpointed")
    return [gk, gv, gtd, gtf]


@torch.library.custom_op("myelin::wkv4_backward_train", mutates_args=())
def _wkv4_backward_train(
    grad_y: Tensor, key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor,
    checkpoint: Tensor,
) -> list[Tensor]:
    return _launch_backward_train(grad_y, key, value, time_decay, time_first, checkpoint)


@_wkv4_backward_train.register_fake
def _(grad_y, key, value, time_decay, time_first, checkpoint):
    dt = key.dtype if key.dtype == value.dtype and key.dtype in _NATIVE else torch.float32
    c = key.shape[-1]
    f32 = {"dtype": torch.float32, "device": key.device}
    return [
        torch.empty(key.shape, dtype=dt, device=key.device),
        torch.empty(key.shape, dtype=dt, device=key.device),
        torch.empty(c, **f32),
        torch.empty(c, **f32),
    ]


def _train_setup_context(ctx, inputs, output):
    key, value, time_decay, time_first = inputs
    _, ck = output
    ctx.save_for_backward(key, value, time_decay, time_first, ck)
    ctx.mark_non_differentiable(ck)
    # The records never receive a gradient: do not materialise zeros for it.
    ctx.set_materialize_grads(False)


def _train_backward(ctx, grad_y, _grad_ck):
    key, value, time_decay, time_first, ck = ctx.saved_tensors
    gk, gv, gtd, gtf = torch.ops.myelin.wkv4_backward_train(grad_y, key, value, time_decay, time_first, ck)
    return gk.to(key.dtype), gv.to(value.dtype), gtd.to(time_decay.dtype), gtf.to(time_first.dtype)


_wkv4_forward_train.register_autograd(_train_backward, setup_context=_train_setup_context)


# ------------------------------------------- gated training ops (time mix) --
# y = sigmoid(receptance) * wkv(key, value), the time mix's gate
# (language.py:1028-1035) folded into the WKV kernels; values equal
# myelin::wkv_forward_bf16io followed by myelin::sigmoid_gate, bit for bit.
def _launch_gated_forward(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor,
                         receptance: Tensor) -> tuple[Tensor, Tensor]:
    """y = sigmoid(receptance) * wkv and the checkpoint records."""
    _lib.require_gpu(key, value, time_decay, time_first, receptance)
    if not (key.dtype == value.dtype == receptance.dtype and key.dtype in _NATIVE
            and receptance.shape == key.shape):
        raise ValueError("wkv4_gated_forward_train: key, value, receptance of one shape and dtype")
    b, t, c = key.shape
    k, v, r = _lib.aligned(key), _lib.aligned(value), _lib.aligned(receptance)
    td = _lib.aligned(time_decay.float())
    tf = _lib.aligned(time_first.float())
    y = torch.empty_like(k)
    ck = torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=k.device)
    lib = _lib.load()
    ws, nbytes = _forward_workspace(lib, b, t, c, k.device)
    rc = _lib.timed("wkv4_forward_gated", k.device, lambda: lib.wkv4_forward_gated_checkpointed(
        k.data_ptr(), v.data_ptr(), td.data_ptr(), tf.data_ptr(), r.data_ptr(), y.data_ptr(),
        ck.data_ptr(), _lib.ptr(ws), nbytes, b, t, c, _lib.dtype_code(k.dtype), _lib.stream_of(k)))
    _lib.check(rc, "wkv4_forward_gated_checkpointed")
    return y, ck


@torch.library.custom_op("myelin::wkv4_gated_forward_train", mutates_args=())
def _wkv4_gated_forward_train(
    key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor, receptance: Tensor
) -> tuple[Tensor, Tensor]:
    return _launch_gated_forward(key, value, time_decay, time_first, receptance)


@_wkv4_gated_forward_train.register_fake
def _(key, value, time_decay, time_first, receptance):
    b, t, c = key.shape
    return (torch.empty_like(key),
            torch.empty(checkpoint_shape(b, t, c), dtype=torch.float32, device=key.device))


def _launch_gated_backward(grad_y: Tensor, key: Tensor, value: Tensor, time_decay: Tensor,
                          time_first: Tensor, receptance: Tensor,
                          checkpoint: Tensor) -> list[Tensor]:
    """[grad_key, grad_value, grad_receptance, grad_time_decay, grad_time_first]."""
    _lib.require_gpu(grad_y, key, value, time_decay, time_first, receptance, checkpoint)
    b, t, c = key.shape
    k, v, r = _lib.aligned(key), _lib.aligned(value), _lib.aligned(receptance)
    gy = _lib.aligned(grad_y.to(k.dtype))
    td = _lib.aligned(time_decay.float())
    tf = _lib.aligned(time_first.float())
    ck = _lib.aligned(checkpoint)
    gk, gv, gr = torch.empty_like(k), torch.empty_like(k), torch.empty_like(k)
    gtd = torch.empty(c, dtype=torch.float32, device=k.device)
    gtf = torch.empty(c, dtype=torch.float32, device=k.device)
    lib = _lib.load()
    ws = _backward_workspace(lib, b, t, c, k.device)
    rc = _lib.timed("wkv4_backward_gated", k.device, lambda: lib.wkv4_backward_gated_checkpointed(
        gy.data_ptr(), td.data_ptr(), tf.data_ptr(), k.data_ptr(), v.data_ptr(), r.data_ptr(),
        ck.data_ptr(), gk.data_ptr(), gv.data_ptr(), gr.data_ptr(), gtd.data_ptr(), gtf.data_ptr(),
        ws.data_ptr(), ws.numel(), b, t, c, _lib.dtype_code(k.dtype), _lib.stream_of(k)))
    _lib.check(rc, "wkv4_backward_gated_checkpointed")
    return [gk, gv, gr, gtd, gtf]


@torch.library.custom_op("myelin::wkv4_gated_backward_train", mutates_args=())
def _wkv4_gated_backward_train(
    grad_y: Tensor, key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor,
    receptance: Tensor, checkpoint: Tensor,
) -> list[Tensor]:
    return _launch_gated_backward(grad_y, key, value, time_decay, time_first, receptance,
                                  checkpoint)


@_wkv4_gated_backward_train.register_fake
def _(grad_y, key, value, time_decay, time_first, receptance, checkpoint):
    c = key.shape[-1]
    f32 = {"dtype": torch.float32, "device": key.device}
    return [torch.empty_like(key), torch.empty_like(key), torch.empty_like(key),
            torch.empty(c, **f32), torch.empty(c, **f32)]


def _gated_setup_context(ctx, inputs, output):
    ctx.save_for_backward(*inputs, output[1])
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)


def _gated_backward(ctx, grad_y, _grad_ck):
    key, value, time_decay, time_first, receptance, ck = ctx.saved_tensors
    gk, gv, gr, gtd, gtf = torch.ops.myelin.wkv4_gated_backward_train(
        grad_y, key, value, time_decay, time_first, receptance, ck)
    return gk, gv, gtd.to(time_decay.dtype), gtf.to(time_first.dtype), gr


_wkv4_gated_forward_train.register_autograd(_gated_backward, setup_context=_gated_setup_context)


# ------------------------------------------------------ eager fast path -----
# The private ops above carry torch.compile / fake-tensor / functorch support,
# and their Python layers (autograd wrapper, default filling, redispatch)
# cost more host time per call than the kernels take at training shapes.
# Plain eager calls on real GPU tensors go through these two Functions
# instead: the same launchers, the same saved tensors and results.
def _eager(t: Tensor) -> bool:
    """Real GPU tensor, outside tracing, transforms and dispatch modes."""
    return (t.is_cuda and not torch.compiler.is_compiling()
            and not torch._C._are_functorch_transforms_active()
            and torch._C._len_torch_dispatch_stack() == 0
            and not _subclass_or_fake(t))


def _subclass_or_fake(t: Tensor) -> bool:
    from torch._subclasses.fake_tensor import is_fake

    # Tensor subclasses (functional, fake, wrapper tensors) keep the op path.
    if type(t) is not Tensor and not isinstance(t, torch.nn.Parameter):
        return True
    return is_fake(t)


class _Wkv4TrainFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, key, value, time_decay, time_first):
        y, ck = _launch_forward(key, value, time_decay, time_first, with_checkpoint=True)
        ctx.save_for_backward(key, value, time_decay, time_first, ck)
        return y

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_y):
        key, value, time_decay, time_first, ck = ctx.saved_tensors
        gk, gv, gtd, gtf = _launch_backward_train(grad_y, key, value, time_decay, time_first, ck)
        return (gk.to(key.dtype), gv.to(value.dtype), gtd.to(time_decay.dtype),
                gtf.to(time_first.dtype))


class _Wkv4GatedTrainFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, key, value, time_decay, time_first, receptance):
        y, ck = _launch_gated_forward(key, value, time_decay, time_first, receptance)
        ctx.save_for_backward(key, value, time_decay, time_first, receptance, ck)
        return y

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, grad_y):
        key, value, time_decay, time_first, receptance, ck = ctx.saved_tensors
        gk, gv, gr, gtd, gtf = _launch_gated_backward(grad_y, key, value, time_decay, time_first,
                                                      receptance, ck)
        return gk, gv, gtd.to(time_decay.dtype), gtf.to(time_first.dtype), gr


# Whether the model's time mix runs sigmoid(r) * wkv through the fused gated
# kernel pair (True) or through the WKV ops followed by the separate
# sigmoid_gate kernels (False).  Both give the same values bit for bit; the
# choice is the faster of the two in a same-box measurement at B=64, T=1024,
# C=512 bf16 (bench.py --workload gated).
GATED_TIME_MIX = True


def weighted_key_value_gated(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor,
                             receptance: Tensor) -> Tensor:
    """``sigmoid(receptance) * weighted_key_value(key, value, ...)`` (the time
    mix's output before its projection, ``language.py:1028-1035``).  One
    fused kernel pair when key, value and receptance share a shape and a
    float32/bfloat16/float16 dtype on the GPU (values equal the two separate
    ops bit for bit); otherwise the two ops."""
    if (key.is_cuda and key.dtype == value.dtype == receptance.dtype and key.dtype in _NATIVE
            and key.shape == value.shape == receptance.shape and key.ndim == 3):
        if _eager(key):
            return _Wkv4GatedTrainFn.apply(key, value, time_decay, time_first, receptance)
        y, _ = torch.ops.myelin.wkv4_gated_forward_train(key, value, time_decay, time_first,
                                                         receptance)
        return y
    from .gates import sigmoid_gate
    from .language import weighted_key_value

    return sigmoid_gate(receptance, weighted_key_value(key, value, time_decay, time_first))


# ------------------------------------------------------------ public ops ----
# myelin::wkv_forward / myelin::wkv_forward_bf16io as the reference registers
# them (wkv_triton.py:147-162, 200-218; wkv_bf16.py:143-158, 197-215):
# opaque custom ops with a fake implementation, whose autograd saves the four
# inputs and calls the public backward op (which computes the forward-state
# records from the inputs before its reverse sweep, as the reference's
# backward kernel replays the forward).  The Python API below takes the
# record-saving route instead; values are identical.
@torch.library.custom_op("myelin::wkv_forward", mutates_args=())
def _wkv_forward_op(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    # fp32 recurrence on the exactly widened inputs; y in key.dtype.
    y, _ = _launch_forward(key, value, time_decay, time_first, with_checkpoint=False)
    return y if y.dtype == key.dtype else y.to(key.dtype)


@_wkv_forward_op.register_fake
def _(key, value, time_decay, time_first):
    return torch.empty_like(key)


@torch.library.custom_op("myelin::wkv_forward_bf16io", mutates_args=())
def _wkv_forward_bf16io_op(
    key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor
) -> Tensor:
    # Native 16-bit I/O, fp32 recurrence in registers.
    y, _ = _launch_forward(key, value, time_decay, time_first, with_checkpoint=False)
    return y if y.dtype == key.dtype else y.to(key.dtype)


@_wkv_forward_bf16io_op.register_fake
def _(key, value, time_decay, time_first):
    return torch.empty_like(key)


def _public_setup_context(ctx, inputs, output):
    key, value, time_decay, time_first = inputs
    ctx.save_for_backward(key, value, time_decay, time_first)


def _public_backward(ctx, grad_y):
    # wkv_triton.py:204-216: fp32 copies of every input.
    key, value, time_decay, time_first = ctx.saved_tensors
    w = (-torch.exp(time_decay.float())).contiguous()
    u = time_first.float().contiguous()
    gk, gv, gtd, gtf = torch.ops.myelin.wkv_backward(
        grad_y.float().contiguous(), w, u, key.float().contiguous(), value.float().contiguous())
    return gk.to(key.dtype), gv.to(value.dtype), gtd.to(time_decay.dtype), gtf.to(time_first.dtype)


def _public_backward_bf16io(ctx, grad_y):
    # wkv_bf16.py:201-213: k, v and the gradient in their native dtype.
    key, value, time_decay, time_first = ctx.saved_tensors
    w = (-torch.exp(time_decay.float())).contiguous()
    u = time_first.float().contiguous()
    gk, gv, gtd, gtf = torch.ops.myelin.wkv_backward_bf16io(
        grad_y.contiguous(), w, u, key.contiguous(), value.contiguous())
    return gk.to(key.dtype), gv.to(value.dtype), gtd.to(time_decay.dtype), gtf.to(time_first.dtype)


_wkv_forward_op.register_autograd(_public_backward, setup_context=_public_setup_context)
_wkv_forward_bf16io_op.register_autograd(_public_backward_bf16io,
                                         setup_context=_public_setup_context)


@torch.library.custom_op("myelin::wkv_backward", mutates_args=())
def _wkv_backward_op(grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor) -> list[Tensor]:
    return _launch_backward(grad_y, w, u, k, v)


@_wkv_backward_op.register_fake
def _(grad_y, w, u, k, v):
    return [torch.empty_like(k), torch.empty_like(k), torch.empty_like(w), torch.empty_like(u)]


@torch.library.custom_op("myelin::wkv_backward_bf16io", mutates_args=())
def _wkv_backward_bf16io_op(
    grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor
) -> list[Tensor]:
    return _launch_backward(grad_y, w, u, k, v)


@_wkv_backward_bf16io_op.register_fake
def _(grad_y, w, u, k, v):
    return [torch.empty_like(k), torch.empty_like(k), torch.empty_like(w), torch.empty_like(u)]


def wkv_forward_no_checkpoint(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """Forward only (no autograd, no checkpoint records): the inference path."""
    y, _ = _launch_forward(key, value, time_decay, time_first, with_checkpoint=False)
    return y if y.dtype == key.dtype else y.to(key.dtype)


# ------------------------------------------------------------- Python API --
def _train_forward(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """y in key.dtype with autograd saving the checkpoint records: eager calls
    on GPU tensors run ``_Wkv4TrainFn``; calls under tracing, fake tensors,
    functorch transforms or a dispatch mode run the private custom op
    ``myelin::wkv4_forward_train``.  Tensors off the GPU raise."""
    if _eager(key):
        y = _Wkv4TrainFn.apply(key, value, time_decay, time_first)
    else:
        y, _ = torch.ops.myelin.wkv4_forward_train(key, value, time_decay, time_first)
    return y if y.dtype == key.dtype else y.to(key.dtype)


def weighted_key_value_hip(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """RWKV WKV recurrence (``wkv_triton.py:221-228``): the values of
    ``myelin::wkv_forward`` (fp32 recurrence, y in ``key.dtype``), with the
    backward reading the forward's checkpoint records instead of replaying
    the forward."""
    return _train_forward(key, value, time_decay, time_first)


def weighted_key_value_hip_bf16io(
    key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor
) -> Tensor:
    """RWKV WKV with native 16-bit I/O (``wkv_bf16.py:218-231``): the values of
    ``myelin::wkv_forward_bf16io``, the same as :func:`weighted_key_value_hip`
    for bf16/fp16 inputs (the widening to fp32 is exact and the output
    rounding is the same), without fp32 copies of k and v."""
    return _train_forward(key, value, time_decay, time_first)


# The reference's public names for the same two entry points.
weighted_key_value_triton = weighted_key_value_hip
weighted_key_value_triton_bf16io = weighted_key_value_hip_bf16io
