"""RWKV-7 DPLR recurrence ops (``myelin::wkv7_forward``, ``myelin::wkv7_backward``).

Per (batch, head), head size N = 64, state ``S`` [N_v, N_k] float32::

    S_t = S_{t-1} (diag(w_t) + a_t b_t^T) + v_t k_t^T
    y_t = S_t r_t

``r, w, k, v, a, b`` are ``[B, T, H, 64]`` (float32, bfloat16 or float16),
``w`` is the per-step decay in (0, 1) (callers pass ``exp(-exp(x))``), and
the optional ``state`` is ``[B, H, 64, 64]`` float32 (zeros when omitted).
``myelin::wkv7_forward`` returns ``(y [B, T, H, 64] in r's dtype, final
state [B, H, 64, 64] fp32)`` and is differentiable in every input and in the
initial state; ``myelin::wkv7_backward`` is the standalone backward (gradients
of ``y`` and of the final state in, ``[dr, dw, dk, dv, da, db, d_state]``
out).

Autograd.  The public forward is a composite of the private op
``myelin::wkv7_forward_train``, which also returns the 64x64 state at the
start of every 8-step block; its registered backward
(``myelin::wkv7_backward_train``) recomputes each block from its checkpoint
instead of replaying the sequence.

The reference's RWKV-7 code (``wkv7_compile.py``, ``wkv7_fla_op.py``) was
deleted from its tree (``benchmarks/results/optimizer_wkv_experiments_5090.md:3``)
and its numerics came from the external ``fla`` package, which is not pinned
anywhere in the reference; the op signatures and the output convention
(post-update state, scale 1) are this library's own.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib

HEAD_SIZE = 64
CKPT_STEPS = 8  # steps per state checkpoint
_NATIVE = (torch.float32, torch.bfloat16, torch.float16)


def _compute_dtype(tensors) -> torch.dtype:
    dt = tensors[0].dtype
    if dt in _NATIVE and all(x.dtype == dt for x in tensors):
        return dt
    return torch.float32


def _check_shapes(r: Tensor, others, state: Tensor | None) -> None:
    if r.ndim != 4 or r.shape[-1] != HEAD_SIZE:
        raise ValueError(f"r, w, k, v, a, b must have shape [B, T, H, {HEAD_SIZE}]; got {tuple(r.shape)}")
    for x in others:
        if x.shape != r.shape:
            raise ValueError(f"r, w, k, v, a, b must share one shape; got {tuple(r.shape)} and {tuple(x.shape)}")
    bsz, _, heads, n = r.shape
    if state is not None and state.shape != (bsz, heads, n, n):
        raise ValueError(f"state must have shape {(bsz, heads, n, n)}; got {tuple(state.shape)}")


def checkpoint_shape(b: int, t: int, h: int) -> tuple[int, int, int, int, int]:
    """Records of the training forward, one per CKPT_STEPS steps: rows
    0..HEAD_SIZE-1 hold the state at the record's first step, row
    HEAD_SIZE + s holds S_{t-1} a_t of its step s (read by the backward)."""
    return (b, h, (t + CKPT_STEPS - 1) // CKPT_STEPS, HEAD_SIZE + CKPT_STEPS, HEAD_SIZE)


def _launch_forward(r, w, k, v, a, b, state, *, with_checkpoint: bool):
    tensors = [r, w, k, v, a, b]
    _lib.require_gpu(*tensors, *([state] if state is not None else []))
    _check_shapes(r, tensors[1:], state)
    bsz, steps, heads, n = r.shape
    dt = _compute_dtype(tensors)
    xs = [_lib.aligned(x.to(dt)) for x in tensors]
    s0 = _lib.aligned(state.float()) if state is not None else None
    y = torch.empty_like(xs[0])
    s_out = torch.empty((bsz, heads, n, n), dtype=torch.float32, device=r.device)
    lib = _lib.load()
    code = _lib.dtype_code(dt)
    if with_checkpoint:
        ck = torch.empty(checkpoint_shape(bsz, steps, heads), dtype=torch.float32, device=r.device)
        rc = _lib.timed("wkv7_forward", r.device, lambda: lib.wkv7_forward_checkpointed(
            *[x.data_ptr() for x in xs], _lib.ptr(s0), y.data_ptr(), s_out.data_ptr(),
            ck.data_ptr(), bsz, steps, heads, n, code, _lib.stream_of(r),
        ))
        _lib.check(rc, "wkv7_forward_checkpointed")
    else:
        ck = None
        rc = _lib.timed("wkv7_forward", r.device, lambda: lib.wkv7_forward(
            *[x.data_ptr() for x in xs], _lib.ptr(s0), y.data_ptr(), s_out.data_ptr(),
            bsz, steps, heads, n, code, _lib.stream_of(r),
        ))
        _lib.check(rc, "wkv7_forward")
    return y, s_out, ck


def _launch_backward(r, w, k, v, a, b, state, checkpoint, grad_y, grad_state, want_state_grad):
    """[dr, dw, dk, dv, da, db] in the compute dtype and d_state (fp32, or None
    unless ``want_state_grad``).  ``checkpoint`` None: the backward computes
    the checkpoints itself from ``state`` (standalone op); otherwise the
    checkpoints already hold the initial state and ``state`` is unused."""
    tensors = [r, w, k, v, a, b]
    extra = [x for x in (state, checkpoint, grad_state) if x is not None]
    _lib.require_gpu(*tensors, grad_y, *extra)
    _check_shapes(r, [*tensors[1:], grad_y], state)
    bsz, steps, heads, n = r.shape
    dt = _compute_dtype(tensors)
    xs = [_lib.aligned(x.to(dt)) for x in tensors]
    gy = _lib.aligned(grad_y.to(dt))
    gs = _lib.aligned(grad_state.float()) if grad_state is not None else None
    if gs is not None and gs.shape != (bsz, heads, n, n):
        raise ValueError(f"grad of the final state must have shape {(bsz, heads, n, n)}; got {tuple(gs.shape)}")
    grads = [torch.empty_like(xs[0]) for _ in range(6)]
    ds0 = (torch.empty((bsz, heads, n, n), dtype=torch.float32, device=r.device)
           if want_state_grad else None)
    lib = _lib.load()
    code = _lib.dtype_code(dt)
    if checkpoint is None:
        s0 = _lib.aligned(state.float()) if state is not None else None
        nbytes = int(lib.wkv7_backward_workspace_bytes(bsz, steps, heads, n))
        ws = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=r.device)
        rc = _lib.timed("wkv7_backward", r.device, lambda: lib.wkv7_backward(
            *[x.data_ptr() for x in xs], _lib.ptr(s0), gy.data_ptr(), _lib.ptr(gs),
            *[g.data_ptr() for g in grads], _lib.ptr(ds0), ws.data_ptr(), ws.numel(),
            bsz, steps, heads, n, code, _lib.stream_of(r),
        ))
        _lib.check(rc, "wkv7_backward")
    else:
        ck = _lib.aligned(checkpoint)
        rc = _lib.timed("wkv7_backward", r.device, lambda: lib.wkv7_backward_checkpointed(
            *[x.data_ptr() for x in xs], ck.data_ptr(), gy.data_ptr(), _lib.ptr(gs),
            *[g.data_ptr() for g in grads], _lib.ptr(ds0), bsz, steps, heads, n, code,
            _lib.stream_of(r),
        ))
        _lib.check(rc, "wkv7_backward_checkpointed")
    return grads, ds0


# ------------------------------------------------ private training ops ------
@torch.library.custom_op("myelin::wkv7_forward_train", mutates_args=())
def _wkv7_forward_train(
    r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, state: Tensor | None
) -> tuple[Tensor, Tensor, Tensor]:
    y, s_out, ck = _launch_forward(r, w, k, v, a, b, state, with_checkpoint=True)
    return y, s_out, ck


@_wkv7_forward_train.register_fake
def _(r, w, k, v, a, b, state):
    bsz, steps, heads, n = r.shape
    dt = _compute_dtype([r, w, k, v, a, b])
    f32 = {"dtype": torch.float32, "device": r.device}
    return (
        torch.empty(r.shape, dtype=dt, device=r.device),
        torch.empty((bsz, heads, n, n), **f32),
        torch.empty(checkpoint_shape(bsz, steps, heads), **f32),
    )


@torch.library.custom_op("myelin::wkv7_backward_train", mutates_args=())
def _wkv7_backward_train(
    r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, checkpoint: Tensor,
    grad_y: Tensor, grad_state: Tensor | None, with_state_grad: bool,
) -> list[Tensor]:
    # The checkpoints already hold the initial state.
    grads, ds0 = _launch_backward(r, w, k, v, a, b, None, checkpoint, grad_y, grad_state,
                                  with_state_grad)
    return [*grads, ds0] if ds0 is not None else grads


@_wkv7_backward_train.register_fake
def _(r, w, k, v, a, b, checkpoint, grad_y, grad_state, with_state_grad):
    bsz, _, heads, n = r.shape
    dt = _compute_dtype([r, w, k, v, a, b])
    out = [torch.empty(r.shape, dtype=dt, device=r.device) for _ in range(6)]
    if with_state_grad:
        out.append(torch.empty((bsz, heads, n, n), dtype=torch.float32, device=r.device))
    return out


def _train_setup_context(ctx, inputs, output):
    r, w, k, v, a, b, state = inputs
    _, _, ck = output
    ctx.save_for_backward(r, w, k, v, a, b, ck)
    ctx.state_meta = None if state is None else state.dtype
    ctx.mark_non_differentiable(ck)
    ctx.set_materialize_grads(False)


def _train_backward(ctx, grad_y, grad_state, _grad_ck):
    r, w, k, v, a, b, ck = ctx.saved_tensors
    if grad_y is None:
        grad_y = torch.zeros_like(r)
    with_state = ctx.state_meta is not None
    out = torch.ops.myelin.wkv7_backward_train(r, w, k, v, a, b, ck, grad_y, grad_state, with_state)
    grads = [g.to(x.dtype) for g, x in zip(out[:6], (r, w, k, v, a, b))]
    ds0 = out[6].to(ctx.state_meta) if with_state else None
    return (*grads, ds0)


_wkv7_forward_train.register_autograd(_train_backward, setup_context=_train_setup_context)


# ------------------------------------------------------------ public ops ----
_LIB = torch.library.Library("myelin", "FRAGMENT")
_LIB.define(
    "wkv7_forward(Tensor r, Tensor w, Tensor k, Tensor v, Tensor a, Tensor b, Tensor? state) "
    "-> (Tensor, Tensor)"
)


def _wkv7_forward_composite(r, w, k, v, a, b, state):
    y, s_out, _ = torch.ops.myelin.wkv7_forward_train(r, w, k, v, a, b, state)
    return (y if y.dtype == r.dtype else y.to(r.dtype)), s_out


_LIB.impl("wkv7_forward", _wkv7_forward_composite, "CompositeImplicitAutograd")


@torch.library.custom_op("myelin::wkv7_backward", mutates_args=())
def _wkv7_backward_op(
    r: Tensor, w: Tensor, k: Tensor, v: Tensor, a: Tensor, b: Tensor, state: Tensor | None,
    grad_y: Tensor, grad_state: Tensor | None,
) -> list[Tensor]:
    grads, ds0 = _launch_backward(r, w, k, v, a, b, state, None, grad_y, grad_state,
                                  state is not None)
    grads = [g.to(x.dtype) for g, x in zip(grads, (r, w, k, v, a, b))]
    return [*grads, ds0] if ds0 is not None else grads


@_wkv7_backward_op.register_fake
def _(r, w, k, v, a, b, state, grad_y, grad_state):
    out = [torch.empty_like(x) for x in (r, w, k, v, a, b)]
    if state is not None:
        bsz, _, heads, n = r.shape
        out.append(torch.empty((bsz, heads, n, n), dtype=torch.float32, device=r.device))
    return out


def wkv7_forward_no_checkpoint(r, w, k, v, a, b, state=None):
    """Forward only (no autograd, no checkpoints): the inference path."""
    y, s_out, _ = _launch_forward(r, w, k, v, a, b, state, with_checkpoint=False)
    return (y if y.dtype == r.dtype else y.to(r.dtype)), s_out


def wkv7_forward(r, w, k, v, a, b, state=None):
    """RWKV-7 DPLR forward; returns ``(y, final_state)`` (differentiable)."""
    return torch.ops.myelin.wkv7_forward(r, w, k, v, a, b, state)


def wkv7_backward(r, w, k, v, a, b, grad_y, state=None, grad_state=None):
    """Standalone backward: ``[dr, dw, dk, dv, da, db]`` (+ ``d_state`` when
    ``state`` is given)."""
    return torch.ops.myelin.wkv7_backward(r, w, k, v, a, b, state, grad_y, grad_state)
