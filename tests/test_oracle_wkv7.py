"""Pins the RWKV-7 oracle by mathematics (the reference has no RWKV-7 code)."""

from __future__ import annotations

import numpy as np
import torch

from oracle import wkv7 as O7

F64 = torch.float64


def test_zero_low_rank_is_decayed_linear_attention():
    r, w, k, v, a, b = O7.make_inputs(2, 10, 2, 8, seed=0, dtype=F64)
    zero = torch.zeros_like(a)
    y, _ = O7.wkv7_loop(r, w, k, v, zero, zero)
    assert torch.allclose(y, O7.linear_attention(r, w, k, v), atol=1e-12, rtol=1e-10)


def test_unit_decay_zero_low_rank_is_causal_linear_attention():
    r, w, k, v, a, b = O7.make_inputs(1, 7, 1, 4, seed=1, dtype=F64)
    ones = torch.ones_like(w)
    zero = torch.zeros_like(a)
    y, _ = O7.wkv7_loop(r, ones, k, v, zero, zero)
    # y_t = sum_{s<=t} v_s (k_s . r_t): a masked matrix product
    scores = torch.einsum("bthj,bshj->bhts", r, k).tril()
    expect = torch.einsum("bhts,bshi->bthi", scores, v)
    assert torch.allclose(y, expect, atol=1e-12)


def test_state_carry_reproduces_unsplit_run():
    xs = O7.make_inputs(2, 9, 2, 8, seed=2, dtype=F64)
    y, s = O7.wkv7_loop(*xs)
    y1, s1 = O7.wkv7_loop(*(x[:, :4] for x in xs))
    y2, s2 = O7.wkv7_loop(*(x[:, 4:] for x in xs), state=s1)
    assert torch.allclose(torch.cat([y1, y2], 1), y, atol=1e-12)
    assert torch.allclose(s2, s, atol=1e-12)


def test_low_rank_term_matters_and_matches_finite_differences():
    xs = [x.clone().requires_grad_(True) for x in O7.make_inputs(1, 5, 1, 4, seed=3, dtype=F64)]
    y, _ = O7.wkv7_loop(*xs)
    gy = torch.randn_like(y)
    (y * gy).sum().backward()
    eps = 1e-6
    base = [x.detach() for x in xs]
    for idx in (4, 5):  # a and b
        fd = torch.zeros_like(base[idx])
        for j in range(fd.numel()):
            p = [x.clone() for x in base]
            mm = [x.clone() for x in base]
            p[idx].reshape(-1)[j] += eps
            mm[idx].reshape(-1)[j] -= eps
            fd.reshape(-1)[j] = ((O7.wkv7_loop(*p)[0] - O7.wkv7_loop(*mm)[0]) * gy).sum() / (2 * eps)
        assert torch.allclose(xs[idx].grad, fd, atol=1e-7, rtol=1e-6)
        assert float(fd.abs().max()) > 1e-3


def test_golden_fixture_reproduces():
    from pathlib import Path

    data = np.load(Path(__file__).parent / "golden" / "wkv7_small.npz", allow_pickle=False)
    g = {n.split("__")[1]: torch.from_numpy(data[n]) for n in data.files}
    y, s = O7.wkv7_loop(*(g[n] for n in ("r", "w", "k", "v", "a", "b")))
    assert torch.allclose(y, g["y"], atol=1e-12) and torch.allclose(s, g["s"], atol=1e-12)
    grads = O7.wkv7_backward_loop(*(g[n] for n in ("r", "w", "k", "v", "a", "b")), None, g["gy"])
    for name, got in zip(("dr", "dw", "dk", "dv", "da", "db"), grads):
        assert torch.allclose(got, g[name], atol=1e-11), name


def _grad_case(seed, t=9, n=8):
    xs = O7.make_inputs(2, t, 2, n, seed=seed, dtype=F64)
    g = torch.Generator().manual_seed(100 + seed)
    s0 = torch.randn(2, 2, n, n, generator=g, dtype=F64)
    gy = torch.randn(2, t, 2, n, generator=g, dtype=F64)
    gs = torch.randn(2, 2, n, n, generator=g, dtype=F64)
    return xs, s0, gy, gs


def test_explicit_reverse_recurrence_equals_autograd():
    for seed in (5, 6):
        xs, s0, gy, gs = _grad_case(seed)
        auto = O7.wkv7_autograd_grads(*xs, s0, gy, gs)[2:]
        loop = O7.wkv7_backward_loop(*xs, s0, gy, gs)
        for name, x, y in zip(("dr", "dw", "dk", "dv", "da", "db", "ds0"), auto, loop):
            assert torch.allclose(x, y, atol=1e-12, rtol=1e-12), name
    # without an initial state or final-state gradient
    xs, _, gy, _ = _grad_case(7)
    auto = O7.wkv7_autograd_grads(*xs, None, gy)[2:8]
    loop = O7.wkv7_backward_loop(*xs, None, gy)[:6]
    for x, y in zip(auto, loop):
        assert torch.allclose(x, y, atol=1e-12, rtol=1e-12)


def test_autograd_of_every_input_matches_finite_differences():
    xs, s0, gy, gs = _grad_case(8, t=4, n=4)
    auto = O7.wkv7_autograd_grads(*xs, s0, gy, gs)[2:]

    def loss(inputs, state):
        y, s = O7.wkv7_loop(*inputs, state=state)
        return float((y * gy).sum() + (s * gs).sum())

    eps = 1e-6
    for idx in range(7):
        base = xs[idx] if idx < 6 else s0
        fd = torch.zeros_like(base)
        for j in range(base.numel()):
            vals = []
            for sgn in (1.0, -1.0):
                pert = base.clone()
                pert.reshape(-1)[j] += sgn * eps
                ins = [pert if i == idx else x for i, x in enumerate(xs)]
                vals.append(loss(ins, pert if idx == 6 else s0))
            fd.reshape(-1)[j] = (vals[0] - vals[1]) / (2 * eps)
        assert torch.allclose(auto[idx], fd, atol=1e-6, rtol=1e-5), idx


def test_planted_transpose_in_the_reverse_recurrence_is_detected():
    # Feeding the reverse recurrence a transposed G (the [value, key] vs
    # [key, value] mix-up a kernel could make) must fail the comparison with
    # autograd: the check has the power to see it.
    xs, s0, gy, gs = _grad_case(9)
    auto_dk = O7.wkv7_autograd_grads(*xs, s0, gy, gs)[4]
    r, w, k, v, a, b = xs
    _, _, dk, _, _, _, _ = O7.wkv7_backward_loop(r, w, k, v, a, b, s0, gy, gs)
    assert torch.allclose(dk, auto_dk, atol=1e-12)
    wrong = O7.wkv7_backward_loop(r, w, k, v, a, b, s0, gy, gs.transpose(-1, -2))[2]
    assert not torch.allclose(wrong, auto_dk, atol=1e-6)
