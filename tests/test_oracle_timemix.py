"""Pins the token-shift-mix oracle (oracle/timemix.py) on the CPU."""

from __future__ import annotations

import torch

from oracle import timemix as M


def test_mix_one_is_identity_and_mix_zero_is_the_shift():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(2, 9, 5, generator=g)
    ones, zeros = torch.ones(1, 5), torch.zeros(1, 5)
    assert torch.equal(M.shift_mix(x, ones)[0], x)
    shifted = M.shift_mix(x, zeros)[0]
    assert torch.equal(shifted[:, 0], torch.zeros(2, 5))
    assert torch.equal(shifted[:, 1:], x[:, :-1])


def test_hand_computed_example():
    x = torch.tensor([[[1.0, 2.0], [3.0, 4.0], [5.0, 6.0]]])
    mu = torch.tensor([[0.25, 0.5]])
    out = M.shift_mix(x, mu)[0]
    expect = torch.tensor([[[0.25, 1.0], [0.25 * 3 + 0.75 * 1, 0.5 * 4 + 0.5 * 2],
                            [0.25 * 5 + 0.75 * 3, 0.5 * 6 + 0.5 * 4]]])
    assert torch.allclose(out, expect, rtol=0, atol=1e-7)


def test_linear_in_x():
    g = torch.Generator().manual_seed(1)
    x, y = torch.randn(2, 2, 7, 4, generator=g, dtype=torch.float64)
    mu = torch.rand(3, 4, generator=g, dtype=torch.float64)
    for a, b, c in zip(M.shift_mix(2.0 * x - 3.0 * y, mu), M.shift_mix(x, mu), M.shift_mix(y, mu)):
        assert torch.allclose(a, 2.0 * b - 3.0 * c, rtol=1e-12, atol=1e-12)
