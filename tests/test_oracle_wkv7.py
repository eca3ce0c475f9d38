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


# ---------------------------------------------------------------------------
# The low-rank term, pinned by checks that share no code with the loop.


def _mutant_loop(r, w, k, v, a, b, state=None, *, kind):
    """The oracle loop with one planted mistake (CPU only, to show that the
    checks below have the power to see it)."""
    bsz, steps, heads, n = r.shape
    s = torch.zeros((bsz, heads, n, n), dtype=r.dtype) if state is None else state.clone()
    ys = []
    for t in range(steps):
        rt, wt, kt, vt, at, bt = (x[:, t] for x in (r, w, k, v, a, b))
        if kind == "sb_at":  # (S b) a^T instead of (S a) b^T
            sb = torch.einsum("bhij,bhj->bhi", s, bt)
            low = sb[..., :, None] * at[:, :, None, :]
        else:
            sa = torch.einsum("bhij,bhj->bhi", s, at)
            low = sa[..., :, None] * bt[:, :, None, :]
        dec = wt[..., :, None] if kind == "decay_on_rows" else wt[:, :, None, :]
        new = s * dec + low + vt[..., :, None] * kt[:, :, None, :]
        ys.append(torch.einsum("bhij,bhj->bhi", s if kind == "pre_update_output" else new, rt))
        s = new
    return torch.stack(ys, dim=1), s


def _one_hot_case(n=8, i=2, j=5, m=1):
    """S_0 = e_i e_j^T, a = e_j, b = e_m, w = 0, v = k = 0, r = ones."""
    z = torch.zeros(1, 1, 1, n, dtype=F64)
    a, b, w, k, v = z.clone(), z.clone(), z.clone(), z.clone(), z.clone()
    a[..., j] = 1.0
    b[..., m] = 1.0
    r = torch.arange(1, n + 1, dtype=F64).reshape(1, 1, 1, n)
    s0 = torch.zeros(1, 1, n, n, dtype=F64)
    s0[0, 0, i, j] = 1.0
    expect_s = torch.zeros(1, 1, n, n, dtype=F64)
    expect_s[0, 0, i, m] = 1.0  # e_i e_j^T (e_j e_m^T) = e_i e_m^T
    expect_y = torch.zeros(1, 1, 1, n, dtype=F64)
    expect_y[..., i] = float(m + 1)  # S_1 r = e_i r_m
    return (r, w, k, v, a, b), s0, expect_s, expect_y


def test_one_hot_low_rank_step_is_hand_computed():
    xs, s0, expect_s, expect_y = _one_hot_case()
    y, s = O7.wkv7_loop(*xs, state=s0)
    assert torch.equal(s, expect_s) and torch.equal(y, expect_y)


def test_delta_rule_identity():
    # w = 1, a = -kappa, b = kappa, r = kappa with |kappa| = 1:
    # S_t kappa = S_{t-1}(I - kappa kappa^T) kappa + v (k . kappa) = v (k . kappa)
    # from any state, so y_t = v_t (k_t . kappa_t).
    r, w, k, v, a, b = O7.make_inputs(2, 6, 3, 8, seed=30, dtype=F64)
    kappa = a / a.norm(dim=-1, keepdim=True)  # unit in float64, not only in float32
    s0 = torch.randn(2, 3, 8, 8, generator=torch.Generator().manual_seed(31), dtype=F64)
    y, _ = O7.wkv7_loop(kappa, torch.ones_like(w), k, v, -kappa, kappa, state=s0)
    expect = v * (k * kappa).sum(-1, keepdim=True)
    assert torch.allclose(y, expect, atol=1e-12, rtol=1e-12)


def test_matrix_form_agrees_for_independent_a_and_b():
    xs = O7.make_general_inputs(2, 11, 2, 8, seed=32, dtype=F64)
    s0 = torch.randn(2, 2, 8, 8, generator=torch.Generator().manual_seed(33), dtype=F64)
    y, s = O7.wkv7_loop(*xs, state=s0)
    ym, sm = O7.wkv7_matrix_form(*xs, state=s0)
    assert np.allclose(y.numpy(), ym, atol=1e-12, rtol=1e-12)
    assert np.allclose(s.numpy(), sm, atol=1e-12, rtol=1e-12)
    # on these inputs a b^T is far from symmetric, so the order of the
    # low-rank product is visible
    a, b = xs[4], xs[5]
    cos = ((a * b).sum(-1) / (a.norm(dim=-1) * b.norm(dim=-1))).abs()
    assert float(cos.max()) < 0.9


def test_matrix_form_at_head_size_64():
    xs = O7.make_general_inputs(1, 5, 1, 64, seed=34, dtype=F64)
    y, s = O7.wkv7_loop(*xs)
    ym, sm = O7.wkv7_matrix_form(*xs)
    assert np.allclose(y.numpy(), ym, atol=1e-11) and np.allclose(s.numpy(), sm, atol=1e-11)


def test_planted_mistakes_fail_the_independent_checks():
    # (S b) a^T: fails the one-hot step and the matrix form with general a, b
    # (with a parallel to b, as in make_inputs and the delta rule, a b^T is
    # symmetric and this mistake is invisible, hence make_general_inputs).
    xs, s0, expect_s, _ = _one_hot_case()
    _, s = _mutant_loop(*xs, state=s0, kind="sb_at")
    assert not torch.equal(s, expect_s)
    gen = O7.make_general_inputs(1, 7, 2, 8, seed=35, dtype=F64)
    ym, _ = O7.wkv7_matrix_form(*gen)
    y_bad, _ = _mutant_loop(*gen, kind="sb_at")
    assert not np.allclose(y_bad.numpy(), ym, atol=1e-6)
    # output taken before the update: fails the delta-rule identity
    r, w, k, v, a, b = O7.make_inputs(1, 5, 2, 8, seed=36, dtype=F64)
    kappa = a / a.norm(dim=-1, keepdim=True)
    y_bad, _ = _mutant_loop(kappa, torch.ones_like(w), k, v, -kappa, kappa, kind="pre_update_output")
    assert not torch.allclose(y_bad, v * (k * kappa).sum(-1, keepdim=True), atol=1e-6)
    # decay applied along the value index: fails the matrix form
    y_bad, _ = _mutant_loop(*gen, kind="decay_on_rows")
    assert not np.allclose(y_bad.numpy(), ym, atol=1e-6)
    # the unmutated copy passes all three (the harness itself is sound)
    y_ok, s_ok = _mutant_loop(*xs, state=s0, kind="none")
    assert torch.equal(s_ok, expect_s)
    assert np.allclose(_mutant_loop(*gen, kind="none")[0].numpy(), ym, atol=1e-12)


def test_general_inputs_gradients_match_finite_differences():
    # autograd through the loop for independent a, b (the GPU tests' second
    # input family), against central differences of the matrix form.
    xs = O7.make_general_inputs(1, 4, 1, 4, seed=37, dtype=F64)
    gy = torch.randn(1, 4, 1, 4, generator=torch.Generator().manual_seed(38), dtype=F64)
    auto = O7.wkv7_autograd_grads(*xs, None, gy)[2:8]
    eps = 1e-6
    gy_np = gy.numpy()
    for idx in range(6):
        base = xs[idx]
        fd = np.zeros(base.numel())
        for j in range(base.numel()):
            vals = []
            for sgn in (1.0, -1.0):
                pert = base.clone()
                pert.reshape(-1)[j] += sgn * eps
                ins = [pert if i == idx else x for i, x in enumerate(xs)]
                vals.append(float((O7.wkv7_matrix_form(*ins)[0] * gy_np).sum()))
            fd[j] = (vals[0] - vals[1]) / (2 * eps)
        assert np.allclose(auto[idx].numpy().reshape(-1), fd, atol=1e-6, rtol=1e-5), idx
