"""CPU oracle for the RWKV-4 / SpikeGPT WKV recurrence (test infrastructure).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of ``bench.py``; never by the product package.

Notation (the reference's, ``src/spikegpt/language.py:399-449``): for one
(batch, channel) lane with ``w = -exp(time_decay)``, ``u = time_first``::

    y_t = (sum_{i<t} e^{(t-1-i)w + k_i} v_i + e^{u+k_t} v_t)
          / (sum_{i<t} e^{(t-1-i)w + k_i}     + e^{u+k_t})

evaluated by the log-sum-exp stabilised recurrence on the state
``(numerator, denominator, log_scale)`` (= the Triton kernel's ``(p, q, o)``).

Functions and what pins each one (tests in ``tests/test_oracle_wkv4.py``):

* :func:`wkv_loop` -- restates ``language.py:399-449``.  Pinned against the
  brute-force closed form :func:`wkv_closed_form` in float64, against the
  special cases T=1 (y=v), w->0 with k=u=0 (running mean) and w->-inf (only
  tokens t-1 and t contribute), and the convexity bound min v <= y <= max v.
* :func:`wkv_closed_form` -- the closed form above, written from the
  mathematics (``docs/neuromorphic_deployment.md:31-32``,
  ``src/spikegpt/benchmarks/spikegpt_wkv_compare.py:41-104``) as a masked
  softmax; pinned by the special cases and by agreement with the loop (two
  independent formulations).
* :func:`wkv_monoid_scan` -- restates ``language.py:452-527`` (upcast rule and
  the log-space monoid ``(acc_decay, log_scale, num, den)``).  Pinned against
  the loop in float64 and by associativity checked on random triples.
* :func:`reference_backward` -- restates the reference backward kernel
  ``src/spikegpt/wkv_triton.py:60-142`` plus the wrapper's batch sum
  (``:194``).  Pinned against torch autograd through the float64 loop, which
  is itself pinned by central finite differences, and by the invariants
  ``sum_t gk = 0`` and ``sum_t gv = sum_t gy`` per lane.
* :func:`wkv_forward_op` / :func:`wkv_backward_op` and the ``_bf16io``
  variants -- the dtype contracts of ``wkv_triton.py:147-218`` and
  ``wkv_bf16.py:143-215`` applied to the math above.
* :func:`decode_step` -- restates ``SpikeTimeMix.step`` ``language.py:977-1013``
  (WKV part only).  Pinned by: iterating it over T equals :func:`wkv_loop`
  at every t (``tests/test_language.py:437-459`` in the reference).
"""

from __future__ import annotations

import torch
from torch import Tensor

__all__ = [
    "validate_wkv_inputs",
    "wkv_loop",
    "wkv_loop_with_state",
    "wkv_closed_form",
    "wkv_monoid_scan",
    "monoid_combine",
    "reference_forward",
    "reference_backward",
    "autograd_grads",
    "wkv_forward_op",
    "wkv_forward_bf16io_op",
    "wkv_backward_op",
    "wkv_backward_bf16io_op",
    "initial_decode_state",
    "decode_step",
    "make_inputs",
]

# Initial log-scale of the reference Triton kernels (wkv_triton.py:43,90,123).
KERNEL_LOG_SCALE_INIT = -1e38


def validate_wkv_inputs(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> None:
    """Shape checks of ``language.py:379-396`` (same messages, ``ValueError``)."""
    if key.shape != value.shape:
        raise ValueError(f"key and value must have the same shape; got {key.shape} and {value.shape}")
    if key.ndim != 3:
        raise ValueError(f"key and value must have shape [B, T, C]; got {key.shape}")
    if time_decay.shape != (key.shape[-1],):
        raise ValueError(f"time_decay must have shape [{key.shape[-1]}]; got {time_decay.shape}")
    if time_first.shape != (key.shape[-1],):
        raise ValueError(f"time_first must have shape [{key.shape[-1]}]; got {time_first.shape}")


def wkv_loop_with_state(
    key: Tensor,
    value: Tensor,
    time_decay: Tensor,
    time_first: Tensor,
    state: tuple[Tensor, Tensor, Tensor] | None = None,
) -> tuple[Tensor, tuple[Tensor, Tensor, Tensor]]:
    """Sequential WKV in the input dtype (no upcast), ``language.py:399-449``.

    Returns ``y`` [B,T,C] and the final ``(numerator, denominator, log_scale)``.
    ``state`` defaults to the reference's initial state: zeros and
    ``finfo(dtype).min`` (``language.py:421-427``).
    """
    validate_wkv_inputs(key, value, time_decay, time_first)
    batch, steps, channels = key.shape
    dtype, device = key.dtype, key.device
    decay = -torch.exp(time_decay.to(device=device, dtype=dtype))
    first = time_first.to(device=device, dtype=dtype)
    if state is None:
        num = torch.zeros((batch, channels), dtype=dtype, device=device)
        den = torch.zeros((batch, channels), dtype=dtype, device=device)
        log_scale = torch.full((batch, channels), torch.finfo(dtype).min, dtype=dtype, device=device)
    else:
        num, den, log_scale = (s.to(dtype) for s in state)
    outs = []
    for t in range(steps):
        k_t = key[:, t]
        v_t = value[:, t]
        nxt = torch.maximum(log_scale, first + k_t)
        old = torch.exp(log_scale - nxt)
        new = torch.exp(first + k_t - nxt)
        outs.append((old * num + new * v_t) / (old * den + new))
        decayed = log_scale + decay
        nxt = torch.maximum(decayed, k_t)
        old = torch.exp(decayed - nxt)
        new = torch.exp(k_t - nxt)
        num = old * num + new * v_t
        den = old * den + new
        log_scale = nxt
    if steps == 0:
        y = key.new_empty((batch, 0, channels))
    else:
        y = torch.stack(outs, dim=1)
    return y, (num, den, log_scale)


def wkv_loop(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """``weighted_key_value_loop`` (``language.py:399-449``): the reference's oracle."""
    return wkv_loop_with_state(key, value, time_decay, time_first)[0]


def wkv_closed_form(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """Brute-force O(T^2) closed form, evaluated in float64 as a masked softmax.

    ``y_t = softmax_i(x_{t,i}) . v`` over ``i <= t`` with
    ``x_{t,i} = (t-1-i) w + k_i`` for ``i < t`` and ``x_{t,t} = u + k_t``.
    Independent of the recurrence (no carried state), so it pins it.
    """
    validate_wkv_inputs(key, value, time_decay, time_first)
    k = key.double()
    v = value.double()
    w = -torch.exp(time_decay.double())
    u = time_first.double()
    steps = k.shape[1]
    t_idx = torch.arange(steps, dtype=torch.float64)
    lag = t_idx[:, None] - 1.0 - t_idx[None, :]  # [t, i] = t-1-i
    # x[b, c, t, i]
    x = lag[None, None] * w[None, :, None, None] + k.permute(0, 2, 1)[:, :, None, :]
    diag = (u[None, :, None] + k.permute(0, 2, 1))  # [b, c, t]
    eye = torch.eye(steps, dtype=torch.bool)
    x = torch.where(eye[None, None], diag[..., None].expand_as(x), x)
    causal = t_idx[None, :] <= t_idx[:, None]
    x = x.masked_fill(~causal[None, None], float("-inf"))
    weights = torch.softmax(x, dim=-1)
    y = torch.einsum("bcti,bci->bct", weights, v.permute(0, 2, 1))
    return y.permute(0, 2, 1).contiguous()


def monoid_combine(left, right):
    """The associative combine of ``language.py:498-508``.

    Elements are ``(acc_decay, log_scale, num, den)``; the earlier (left)
    segment decays by the later segment's total decay before merging.
    """
    decay_l, scale_l, num_l, den_l = left
    decay_r, scale_r, num_r, den_r = right
    merged = torch.maximum(scale_l + decay_r, scale_r)
    weight_l = torch.exp(scale_l + decay_r - merged)
    weight_r = torch.exp(scale_r - merged)
    return (
        decay_l + decay_r,
        merged,
        weight_l * num_l + weight_r * num_r,
        weight_l * den_l + weight_r * den_r,
    )


def _monoid_operands(key, value, time_decay, time_first):
    """Inputs of the monoid form of ``language.py:482-494``: the compute dtype
    (bf16/fp16 upcast to float32, float32/float64 kept), ``decay = -exp(td)``,
    ``first``, and the per-token elements ``(acc_decay, log_scale=k, num=v,
    den=1)`` on ``[T, B, C]``."""
    orig = key.dtype
    dtype = torch.float32 if orig in (torch.float16, torch.bfloat16) else orig
    batch, steps, channels = key.shape
    decay = -torch.exp(time_decay.to(dtype))
    first = time_first.to(dtype)
    keys = key.movedim(1, 0).contiguous().to(dtype)
    values = value.movedim(1, 0).contiguous().to(dtype)
    acc_decay = decay[None, None, :].expand(steps, batch, channels).contiguous()
    return orig, dtype, first, (acc_decay, keys, values, torch.ones_like(keys))


def _monoid_output(scale_inc, num_inc, den_inc, keys, values, first, dtype, orig):
    """Exclusive prefix (shift by one token, ``language.py:514-519``) merged
    with the ``time_first`` bonus of the current token (``:521-526``)."""
    neg = torch.full_like(scale_inc[:1], torch.finfo(dtype).min)
    zeros = torch.zeros_like(num_inc[:1])
    scale_ex = torch.cat([neg, scale_inc[:-1]])
    num_ex = torch.cat([zeros, num_inc[:-1]])
    den_ex = torch.cat([zeros, den_inc[:-1]])
    bonus = first[None, None, :] + keys
    merged = torch.maximum(scale_ex, bonus)
    wp = torch.exp(scale_ex - merged)
    wb = torch.exp(bonus - merged)
    out = (wp * num_ex + wb * values) / (wp * den_ex + wb)
    return out.movedim(0, 1).to(orig)


def wkv_monoid_scan(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """The reference's CPU path ``weighted_key_value`` (``language.py:452-527``)
    with its inclusive prefix taken as a sequential left fold of the monoid.

    Upcasts bf16/fp16 to float32 and keeps float32/float64 (``:483-485``).
    :func:`wkv_associative_scan` hands the same combine to
    ``associative_scan`` as the reference does; associativity makes the two
    equal up to rounding.
    """
    validate_wkv_inputs(key, value, time_decay, time_first)
    if key.shape[1] == 0:
        return key.new_empty(key.shape)
    orig, dtype, first, elems = _monoid_operands(key, value, time_decay, time_first)
    acc = None
    scales, nums, dens = [], [], []
    for t in range(key.shape[1]):
        elem = tuple(x[t] for x in elems)
        acc = elem if acc is None else monoid_combine(acc, elem)
        scales.append(acc[1])
        nums.append(acc[2])
        dens.append(acc[3])
    return _monoid_output(torch.stack(scales), torch.stack(nums), torch.stack(dens), elems[1],
                          elems[2], first, dtype, orig)


def wkv_associative_scan(key: Tensor, value: Tensor, time_decay: Tensor,
                         time_first: Tensor) -> Tensor:
    """``weighted_key_value`` (``language.py:452-527``) as the reference runs
    it: the inclusive prefix of the monoid by
    ``torch._higher_order_ops.associative_scan(combine, ..., dim=0,
    combine_mode="generic")`` (``:496-512``), a tree of O(log T) combine
    levels, so its rounding differs from the left fold's.  Forward only here:
    the reference notes that its autograd needs torch >= 2.13 (this image has
    torch 2.10)."""
    from torch._higher_order_ops.associative_scan import associative_scan

    validate_wkv_inputs(key, value, time_decay, time_first)
    if key.shape[1] == 0:
        return key.new_empty(key.shape)
    orig, dtype, first, elems = _monoid_operands(key, value, time_decay, time_first)
    _, scale_inc, num_inc, den_inc = associative_scan(monoid_combine, elems, dim=0,
                                                      combine_mode="generic")
    return _monoid_output(scale_inc, num_inc, den_inc, elems[1], elems[2], first, dtype, orig)


def reference_forward(k: Tensor, v: Tensor, w: Tensor, u: Tensor) -> Tensor:
    """The forward kernel ``wkv_triton.py:34-58`` in the dtype of ``k``.

    ``w`` is the already-transformed decay ``-exp(time_decay)``.  Initial
    ``o = -1e38`` as in the kernel.
    """
    batch, steps, channels = k.shape
    p = torch.zeros((batch, channels), dtype=k.dtype)
    q = torch.zeros_like(p)
    o = torch.full_like(p, KERNEL_LOG_SCALE_INIT)
    y = torch.empty_like(k)
    for t in range(steps):
        kt, vt = k[:, t], v[:, t]
        no = torch.maximum(o, u + kt)
        a = torch.exp(o - no)
        b = torch.exp(u + kt - no)
        y[:, t] = (a * p + b * vt) / (a * q + b)
        no = torch.maximum(w + o, kt)
        a = torch.exp(w + o - no)
        b = torch.exp(kt - no)
        p = a * p + b * vt
        q = a * q + b
        o = no
    return y


def reference_backward(grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor) -> list[Tensor]:
    """The backward kernel ``wkv_triton.py:60-142`` and its op's batch sum (``:194``).

    Computes in the dtype of ``k``.  ``w`` is ``-exp(time_decay)``; the
    returned time-decay gradient already includes the ``* w`` chain rule
    (``:117``) and both parameter gradients are summed over the batch.
    Returns ``[gk, gv, g_time_decay [C], g_time_first [C]]``.
    """
    dt = k.dtype
    gy = grad_y.to(dt)
    w = w.to(dt)
    u = u.to(dt)
    batch, steps, channels = k.shape
    zero = torch.zeros((batch, channels), dtype=dt)
    p, q, dpdw, dqdw, gw, gu = (zero.clone() for _ in range(6))
    o = torch.full_like(zero, KERNEL_LOG_SCALE_INIT)
    ys = torch.empty_like(k)
    zs = torch.empty_like(k)
    zexps = torch.empty_like(k)
    for t in range(steps):  # pass 1: forward replay (:93-115)
        kt, vt, gyt = k[:, t], v[:, t], gy[:, t]
        no = torch.maximum(o, kt + u)
        a = torch.exp(o - no)
        b = torch.exp(kt + u - no)
        iden = 1.0 / (a * q + b)
        y = (a * p + b * vt) * iden
        ys[:, t], zs[:, t], zexps[:, t] = y, iden, kt + u - no
        gw = gw + gyt * (dpdw - dqdw * y) * iden * a
        gu = gu + gyt * (vt - y) * b * iden
        no = torch.maximum(w + o, kt)
        a = torch.exp(w + o - no)
        b = torch.exp(kt - no)
        dpdw = a * (p + dpdw)
        dqdw = a * (q + dqdw)
        p = a * p + b * vt
        q = a * q + b
        o = no
    gw = gw * w
    gk = torch.empty_like(k)
    gv = torch.empty_like(k)
    gp, gq = zero.clone(), zero.clone()
    o = torch.full_like(zero, KERNEL_LOG_SCALE_INIT)
    for t in reversed(range(steps)):  # pass 2: reverse (:124-142)
        kt, vt, gyt = k[:, t], v[:, t], gy[:, t]
        y, z, zx = ys[:, t], zs[:, t], zexps[:, t]
        a = gyt * z * torch.exp(zx)
        b = torch.exp(kt + o)
        gk[:, t] = a * (vt - y) + b * (gp * vt + gq)
        gv[:, t] = a + b * gp
        no = torch.maximum(w + o, zx - kt - u)
        a = torch.exp(w + o - no)
        b = gyt * z * torch.exp(zx - kt - u - no)
        gp = a * gp + b
        gq = a * gq - b * y
        o = no
    return [gk, gv, gw.sum(0), gu.sum(0)]


def autograd_grads(
    key: Tensor,
    value: Tensor,
    time_decay: Tensor,
    time_first: Tensor,
    grad_y: Tensor,
    dtype: torch.dtype = torch.float64,
) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor]:
    """Exact gradients by torch autograd through :func:`wkv_loop` in ``dtype``.

    Returns ``(y, gk, gv, g_time_decay, g_time_first)``; an input that does not
    influence the output (``time_decay`` at T=1) gets a zero gradient, as in
    ``tests/test_wkv_triton.py:29-30`` of the reference.
    """
    leaves = [x.detach().to(dtype).clone().requires_grad_(True) for x in (key, value, time_decay, time_first)]
    y = wkv_loop(*leaves)
    y.backward(grad_y.to(dtype))
    grads = [torch.zeros_like(x) if x.grad is None else x.grad for x in leaves]
    return (y.detach(), *grads)


def wkv_forward_op(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """Contract of ``myelin::wkv_forward`` (``wkv_triton.py:147-158``).

    fp32 recurrence on ``key.float()``/``value.float()``, ``w = -exp(td)``;
    the result is cast back to ``key.dtype``.
    """
    w = -torch.exp(time_decay.float())
    u = time_first.float()
    y = reference_forward(key.float(), value.float(), w, u)
    return y.to(key.dtype)


def wkv_forward_bf16io_op(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """Contract of ``myelin::wkv_forward_bf16io`` (``wkv_bf16.py:143-154``).

    Native-dtype loads widened exactly to fp32, fp32 recurrence, the store
    rounds to the native dtype -- the same values as :func:`wkv_forward_op`.
    """
    return wkv_forward_op(key, value, time_decay, time_first)


def wkv_backward_op(grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor) -> list[Tensor]:
    """Contract of ``myelin::wkv_backward`` (``wkv_triton.py:164-194``).

    ``w``/``u`` are fp32 and already transformed; gk/gv come back in ``k``'s
    dtype (fp32 on the autograd path), the parameter grads in fp32 [C].
    """
    gk, gv, gtd, gtf = reference_backward(grad_y.float(), w.float(), u.float(), k.float(), v.float())
    return [gk.to(k.dtype), gv.to(k.dtype), gtd, gtf]


def wkv_backward_bf16io_op(grad_y: Tensor, w: Tensor, u: Tensor, k: Tensor, v: Tensor) -> list[Tensor]:
    """Contract of ``myelin::wkv_backward_bf16io`` (``wkv_bf16.py:160-191``)."""
    return wkv_backward_op(grad_y, w, u, k, v)


def initial_decode_state(batch: int, channels: int, dtype: torch.dtype = torch.float32):
    """``SpikeTimeMix.initial_state`` WKV part (``language.py:957-975``)."""
    zeros = torch.zeros((batch, channels), dtype=dtype)
    return zeros, zeros.clone(), torch.full((batch, channels), torch.finfo(dtype).min, dtype=dtype)


def decode_step(
    key: Tensor,
    value: Tensor,
    time_decay: Tensor,
    time_first: Tensor,
    numerator: Tensor,
    denominator: Tensor,
    log_scale: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    """One token of ``SpikeTimeMix.step`` (``language.py:989-1012``), WKV part.

    ``key``/``value`` are [B,C]; returns ``(y, numerator, denominator, log_scale)``.
    """
    dtype = key.dtype
    decay = -torch.exp(time_decay.to(dtype))
    first = time_first.to(dtype)
    nxt = torch.maximum(log_scale, first + key)
    old = torch.exp(log_scale - nxt)
    new = torch.exp(first + key - nxt)
    mixed = (old * numerator + new * value) / (old * denominator + new)
    decayed = log_scale + decay
    rec = torch.maximum(decayed, key)
    old = torch.exp(decayed - rec)
    new = torch.exp(key - rec)
    return mixed, old * numerator + new * value, old * denominator + new, rec


def make_inputs(
    batch: int,
    steps: int,
    channels: int,
    *,
    seed: int,
    dtype: torch.dtype = torch.float32,
    with_grad: bool = True,
):
    """Seeded synthetic inputs with the benchmark distributions.

    ``time_decay ~ U(-5, 1)``, ``time_first ~ N(0, 0.5)`` (0.5 is the std),
    ``k, v ~ N(0, 1)`` with ``k`` clamped to +-30, ``dy ~ N(0, 1)``; all drawn
    on the CPU from ``torch.Generator().manual_seed(seed)`` in that order, then
    ``k, v, dy`` are rounded to ``dtype``.  Returns ``(k, v, td, tf, dy)``.
    """
    g = torch.Generator().manual_seed(seed)
    td = -5.0 + 6.0 * torch.rand(channels, generator=g)
    tf = 0.5 * torch.randn(channels, generator=g)
    k = torch.randn(batch, steps, channels, generator=g).clamp_(-30.0, 30.0)
    v = torch.randn(batch, steps, channels, generator=g)
    dy = torch.randn(batch, steps, channels, generator=g) if with_grad else None
    k, v = k.to(dtype), v.to(dtype)
    if dy is not None:
        dy = dy.to(dtype)
    return k, v, td, tf, dy
