"""CPU oracle for SpikeGPT's sequence LIF activation (test infrastructure).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` and ``bench.py``'s CPU leg;
never by the product package.

The reference (``src/spikegpt/language.py:766-918``) runs, per (batch,
channel) lane with membrane ``m_0 = 0`` and ``decay = 1 - 1/tau``::

    h_t = m_{t-1} * decay + x_t                      (language.py:833)
    c_t = slope * (h_t - threshold)                  (language.py:834)
    s_t = hard_surrogate_spike(c_t, atan_surrogate)  (language.py:836)
    m_t = h_t * (1 - s_t) + reset * s_t              (language.py:839)

``hard_surrogate_spike`` and ``atan_surrogate`` come from the external
``myelin`` package, which is neither in the reference tree nor installed.
They are restated here as a Heaviside forward (``c >= 0``) with the arctan
surrogate derivative of SpikingJelly's ATan (``alpha`` = the slope already
applied to ``c``): ``ds/dc = 0.5 / (1 + (pi/2 c)^2)``.  The spikes and
membranes follow from the reference's own lines; the surrogate derivative
(hence input gradients) is **parity unpinned** against the reference.

Functions and what pins each one (``tests/test_oracle_lif.py``):

* :func:`lif_loop` -- restates the step (``language.py:813-840``) and the time
  loop (``:908-918``) with autograd through :class:`HardSurrogateSpike`.
  Forward pinned by closed forms: with no spike the membrane is the decayed
  sum ``sum_i decay^(t-i) x_i``; a constant input ``x`` with ``decay = 0.5``
  and ``threshold = 1`` spikes with the period computed by hand; spikes are
  exactly 0/1.
* :func:`lif_reverse` -- the backward written independently as an explicit
  reverse recurrence.  It and autograd through :func:`lif_loop` agree on random
  inputs (two formulations; dropping the reset-path term or the decay carry
  fails it), and the surrogate derivative matches central differences of the
  smooth surrogate ``atan(pi/2 c)/pi + 1/2``.
* :func:`lif_membranes` -- the forward replay in a chosen dtype.  Pinned at a
  constructed exact float32 threshold tie (``h == fp32(theta)``): its float32
  spikes equal :func:`lif_loop`'s, and :func:`lif_reverse` built on it equals
  autograd through the float32 :func:`lif_loop`; a float64 replay of the same
  float32 inputs misses that spike, which the test also asserts.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

__all__ = ["HardSurrogateSpike", "lif_loop", "lif_reverse", "lif_membranes", "surrogate_grad"]

HALF_PI = math.pi / 2.0


def surrogate_grad(c: Tensor) -> Tensor:
    """d/dc of the arctan surrogate ``atan(pi/2 c)/pi + 1/2``."""
    return 0.5 / (1.0 + (HALF_PI * c) ** 2)


class HardSurrogateSpike(torch.autograd.Function):
    """Heaviside forward (``c >= 0``), arctan surrogate backward."""

    @staticmethod
    def forward(ctx, c: Tensor) -> Tensor:  # noqa: D102
        ctx.save_for_backward(c)
        return (c >= 0).to(c.dtype)

    @staticmethod
    def backward(ctx, grad: Tensor) -> Tensor:  # noqa: D102
        (c,) = ctx.saved_tensors
        return grad * surrogate_grad(c)


def lif_loop(x: Tensor, tau: float = 2.0, threshold: float = 1.0, reset: float = 0.0,
             slope: float = 2.0) -> Tensor:
    """Spikes ``[B, T, C]`` of the reference eager loop (differentiable).

    16-bit inputs are widened to float32 and the spikes cast back, as the
    reference's non-fused path does (``language.py:891-893, 918``)."""
    if x.ndim != 3:
        raise ValueError(f"inputs must have shape [B, T, C]; got {x.shape}")
    orig = x.dtype
    if orig in (torch.float16, torch.bfloat16):
        x = x.float()
    decay = 1.0 - 1.0 / tau
    m = torch.zeros(x.shape[0], x.shape[2], dtype=x.dtype, device=x.device)
    out = []
    for t in range(x.shape[1]):
        h = m * decay + x[:, t]
        s = HardSurrogateSpike.apply(slope * (h - threshold))
        m = h * (1.0 - s) + reset * s
        out.append(s)
    return torch.stack(out, dim=1).to(orig)


def lif_membranes(x: Tensor, tau: float = 2.0, threshold: float = 1.0, reset: float = 0.0,
                  slope: float = 2.0, dtype: torch.dtype = torch.float64) -> tuple[Tensor, Tensor]:
    """Pre-spike membranes ``h`` and spikes ``s`` of the loop evaluated in
    ``dtype`` (float64 by default; float32 replays the kernels' arithmetic),
    no autograd.

    Every step stays in ``dtype``: the spike is cast to ``dtype`` before the
    reset line, so a float32 replay fires at exactly the steps where
    :func:`lif_loop` fires in float32, exact threshold ties included."""
    x = x.to(dtype)
    decay = 1.0 - 1.0 / tau
    m = torch.zeros(x.shape[0], x.shape[2], dtype=x.dtype)
    hs, ss = [], []
    for t in range(x.shape[1]):
        h = m * decay + x[:, t]
        s = (slope * (h - threshold) >= 0).to(dtype)
        m = h * (1.0 - s) + reset * s
        hs.append(h)
        ss.append(s)
    return torch.stack(hs, dim=1), torch.stack(ss, dim=1)


def lif_reverse(x: Tensor, grad_spikes: Tensor, tau: float = 2.0, threshold: float = 1.0,
                reset: float = 0.0, slope: float = 2.0,
                forward_dtype: torch.dtype = torch.float64) -> Tensor:
    """``dL/dx`` by the explicit reverse recurrence (float64 arithmetic)::

        dh_t = g_t s'_t + gm_t ((1 - s_t) + (reset - h_t) s'_t),
        s'_t = slope * surrogate_grad(slope (h_t - threshold)),
        gm_{t-1} = decay * dh_t,   dx_t = dh_t.

    ``forward_dtype`` is the precision of the forward replay that fixes
    ``h`` and the spike pattern (float32 to match a float32 forward)."""
    h, s = lif_membranes(x, tau, threshold, reset, slope, dtype=forward_dtype)
    h, s = h.double(), s.double()
    g = grad_spikes.double()
    decay = 1.0 - 1.0 / tau
    gm = torch.zeros_like(h[:, 0])
    out = torch.empty_like(h)
    for t in range(h.shape[1] - 1, -1, -1):
        ds = slope * surrogate_grad(slope * (h[:, t] - threshold))
        dh = g[:, t] * ds + gm * ((1.0 - s[:, t]) + (reset - h[:, t]) * ds)
        out[:, t] = dh
        gm = decay * dh
    return out
