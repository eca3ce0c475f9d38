"""Pins the sequence-LIF oracle (oracle/lif.py) by closed forms and by two
independent formulations of its backward (CPU only)."""

from __future__ import annotations

import math

import pytest
import torch

from oracle import lif as L


def test_subthreshold_membrane_is_the_decayed_sum():
    # Inputs too small to ever reach the threshold: no spikes, and the
    # membrane is sum_i decay^(t-i) x_i (language.py:833 without reset).
    g = torch.Generator().manual_seed(0)
    x = torch.rand(2, 40, 5, generator=g, dtype=torch.float64) * 0.2
    tau = 3.0
    decay = 1.0 - 1.0 / tau
    h, s = L.lif_membranes(x, tau=tau, threshold=1.0)
    assert float(s.sum()) == 0.0
    assert torch.equal(L.lif_loop(x, tau=tau), torch.zeros_like(x))
    T = x.shape[1]
    w = torch.tensor([[decay ** (t - i) if i <= t else 0.0 for i in range(T)] for t in range(T)],
                     dtype=torch.float64)
    closed = torch.einsum("ti,bic->btc", w, x)
    assert torch.allclose(h, closed, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("xc,period", [(0.6, 3), (0.75, 2), (1.0, 1), (0.55, 4)])
def test_constant_input_spikes_periodically(xc, period):
    # decay 0.5, threshold 1, reset 0: membranes x, 1.5x, 1.75x, ... spike
    # at the first n with x (2 - 2^(1-n)) >= 1, then restart from zero.
    n = next(n for n in range(1, 20) if xc * (2.0 - 2.0 ** (1 - n)) >= 1.0)
    assert n == period
    x = torch.full((1, 24, 1), xc, dtype=torch.float64)
    s = L.lif_loop(x, tau=2.0, threshold=1.0, reset=0.0)
    expect = torch.tensor([1.0 if (t + 1) % period == 0 else 0.0 for t in range(24)],
                          dtype=torch.float64)
    assert torch.equal(s[0, :, 0], expect)


def test_spikes_are_exactly_binary_and_keep_dtype():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(3, 17, 6, generator=g) * 2).to(torch.bfloat16)
    s = L.lif_loop(x)
    assert s.dtype == torch.bfloat16
    assert set(s.float().unique().tolist()) <= {0.0, 1.0}


def test_surrogate_matches_the_derivative_of_the_smooth_arctan():
    c = torch.linspace(-3, 3, 41, dtype=torch.float64)
    f = lambda z: torch.atan(math.pi / 2 * z) / math.pi + 0.5  # noqa: E731
    eps = 1e-6
    fd = (f(c + eps) - f(c - eps)) / (2 * eps)
    assert torch.allclose(L.surrogate_grad(c), fd, rtol=1e-8, atol=1e-10)
    assert float(L.surrogate_grad(torch.tensor(0.0))) == 0.5


@pytest.mark.parametrize("reset", [0.0, -0.3])
def test_reverse_recurrence_equals_autograd_of_the_loop(reset):
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(2, 33, 7, generator=g, dtype=torch.float64) * 1.5).requires_grad_(True)
    gs = torch.randn(2, 33, 7, generator=g, dtype=torch.float64)
    s = L.lif_loop(x, tau=2.5, threshold=0.8, reset=reset, slope=2.0)
    (gx,) = torch.autograd.grad(s, x, gs)
    ref = L.lif_reverse(x.detach(), gs, tau=2.5, threshold=0.8, reset=reset, slope=2.0)
    assert torch.allclose(gx, ref, rtol=1e-12, atol=1e-12)


def test_dropping_the_reset_term_is_detected():
    # A planted mistake in the reverse recurrence (reset path not
    # differentiated) must disagree with autograd through the loop.
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(1, 20, 4, generator=g, dtype=torch.float64) * 1.5).requires_grad_(True)
    gs = torch.randn(1, 20, 4, generator=g, dtype=torch.float64)
    (gx,) = torch.autograd.grad(L.lif_loop(x), x, gs)
    h, s = L.lif_membranes(x.detach())
    gm = torch.zeros_like(h[:, 0])
    wrong = torch.empty_like(h)
    for t in range(h.shape[1] - 1, -1, -1):
        ds = 2.0 * L.surrogate_grad(2.0 * (h[:, t] - 1.0))
        dh = gs[:, t] * ds + gm * (1.0 - s[:, t])
        wrong[:, t] = dh
        gm = 0.5 * dh
    assert not torch.allclose(gx, wrong, rtol=1e-6, atol=1e-6)


def _tie_inputs():
    # x = [0, fp32(1.3), 0, 0] with tau 2, threshold 1.3: at t = 1 the float32
    # membrane is exactly fp32(1.3), so h - threshold == 0 in float32 and the
    # step fires (language.py:833-839 evaluated in float32).
    x = torch.tensor([0.0, 1.3, 0.0, 0.0], dtype=torch.float32).view(1, 4, 1)
    return x, dict(tau=2.0, threshold=1.3, reset=0.0, slope=1.5)


def test_float32_replay_fires_at_an_exact_threshold_tie():
    x, kw = _tie_inputs()
    s_loop = L.lif_loop(x, **kw)
    assert s_loop[0, :, 0].tolist() == [0.0, 1.0, 0.0, 0.0]
    h, s = L.lif_membranes(x, **kw, dtype=torch.float32)
    assert h.dtype == torch.float32 and s.dtype == torch.float32
    assert torch.equal(s, s_loop)
    assert float(h[0, 1, 0]) == float(torch.tensor(1.3, dtype=torch.float32))
    # The same float32 inputs replayed in float64 sit just below 1.3 and miss
    # the spike: the replay's dtype matters exactly at such ties.
    _, s64 = L.lif_membranes(x, **kw, dtype=torch.float64)
    assert s64[0, :, 0].tolist() == [0.0, 0.0, 0.0, 0.0]


def test_float32_reverse_equals_autograd_through_the_float32_loop_at_a_tie():
    x, kw = _tie_inputs()
    g = torch.Generator().manual_seed(5)
    gs = torch.randn(1, 4, 1, generator=g, dtype=torch.float32)
    xr = x.clone().requires_grad_(True)
    (gx,) = torch.autograd.grad(L.lif_loop(xr, **kw), xr, gs)
    ref = L.lif_reverse(x, gs, **kw, forward_dtype=torch.float32)
    assert torch.allclose(gx.double(), ref, rtol=1e-6, atol=1e-6)
    # A float64 replay (spike missed) gives a different gradient.
    wrong = L.lif_reverse(x, gs, **kw, forward_dtype=torch.float64)
    assert not torch.allclose(gx.double(), wrong, rtol=1e-3, atol=1e-3)


@pytest.mark.parametrize("dtype,tau,thr", [(torch.float32, 2.0, 1.3), (torch.bfloat16, 3.0, 1.0)])
def test_float32_replay_spikes_equal_the_loop_on_tie_rich_inputs(dtype, tau, thr):
    # bf16 inputs put exact ties everywhere (after a reset h = x, and 1.0 is a
    # bf16 value); the float32 replay must reproduce every spike of the loop.
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 33, 64, generator=g).to(dtype)
    if dtype == torch.float32:
        x[:, ::5] = thr  # plant exact fp32 ties after resets
    s_loop = L.lif_loop(x, tau=tau, threshold=thr, slope=1.5).float()
    _, s = L.lif_membranes(x.float(), tau=tau, threshold=thr, slope=1.5, dtype=torch.float32)
    assert torch.equal(s, s_loop)
