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
