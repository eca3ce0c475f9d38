"""Pins the RWKV-4 CPU oracle before anything is compared against it.

Each oracle function is checked against something that does not share its
code path: the brute-force closed form (a masked softmax, no carried state),
special cases with known answers, torch autograd, central finite
differences, and invariants of the gradients.  Mutated copies of the loop
(plausible mistakes) must fail the same checks, showing they have power.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import wkv4 as O

F64 = torch.float64


def _inputs(batch, steps, channels, *, seed=0, dtype=F64):
    """The reference test's generator (tests/test_wkv_variants.py:24-30)."""
    g = torch.Generator().manual_seed(seed)
    key = torch.randn(batch, steps, channels, generator=g, dtype=dtype)
    value = torch.randn(batch, steps, channels, generator=g, dtype=dtype)
    time_decay = torch.randn(channels, generator=g, dtype=dtype)
    time_first = torch.randn(channels, generator=g, dtype=dtype)
    return key, value, time_decay, time_first


@pytest.mark.parametrize("steps", [1, 4, 16, 17, 40])
def test_loop_matches_closed_form(steps):
    k, v, td, tf = _inputs(3, steps, 8)
    ref = O.wkv_closed_form(k, v, td, tf)
    got = O.wkv_loop(k, v, td, tf)
    assert got.shape == ref.shape
    assert torch.allclose(got, ref, atol=1e-12, rtol=1e-10)


def test_single_step_returns_value():
    k, v, td, tf = _inputs(2, 1, 5)
    assert torch.equal(O.wkv_loop(k, v, td, tf), v)
    assert torch.allclose(O.wkv_closed_form(k, v, td, tf), v, atol=1e-15)


def test_vanishing_decay_with_zero_keys_is_running_mean():
    # time_decay -> -inf gives w = -exp(td) -> 0-: no forgetting; with k = u = 0
    # every token has weight 1, so y_t is the mean of v_0..v_t.
    steps = 12
    g = torch.Generator().manual_seed(3)
    v = torch.randn(2, steps, 4, generator=g, dtype=F64)
    k = torch.zeros_like(v)
    td = torch.full((4,), -60.0, dtype=F64)
    tf = torch.zeros(4, dtype=F64)
    expect = torch.cumsum(v, dim=1) / torch.arange(1, steps + 1, dtype=F64)[None, :, None]
    assert torch.allclose(O.wkv_loop(k, v, td, tf), expect, atol=1e-12)
    assert torch.allclose(O.wkv_closed_form(k, v, td, tf), expect, atol=1e-12)


def test_huge_decay_keeps_only_previous_and_current_token():
    k, v, td, tf = _inputs(2, 10, 6, seed=4)
    td = torch.full_like(td, 6.0)  # w = -exp(6) ~ -403: older tokens vanish
    y = O.wkv_loop(k, v, td, tf)
    ea = torch.exp(k[:, :-1])
    eb = torch.exp(tf + k[:, 1:])
    expect = (ea * v[:, :-1] + eb * v[:, 1:]) / (ea + eb)
    assert torch.allclose(y[:, 1:], expect, atol=1e-12)
    assert torch.allclose(y[:, 0], v[:, 0])


def test_output_is_convex_combination_of_values_so_far():
    k, v, td, tf = _inputs(4, 30, 16, seed=5)
    y = O.wkv_loop(k, v, td, tf)
    lo = torch.cummin(v, dim=1).values
    hi = torch.cummax(v, dim=1).values
    assert bool(((y >= lo - 1e-12) & (y <= hi + 1e-12)).all())


def test_monoid_scan_matches_loop_and_is_associative():
    k, v, td, tf = _inputs(3, 23, 8, seed=6)
    assert torch.allclose(O.wkv_monoid_scan(k, v, td, tf), O.wkv_loop(k, v, td, tf), atol=1e-12, rtol=1e-10)
    g = torch.Generator().manual_seed(7)

    def elem():
        return (
            -torch.rand(5, generator=g, dtype=F64) * 3,
            torch.randn(5, generator=g, dtype=F64) * 4,
            torch.randn(5, generator=g, dtype=F64),
            torch.rand(5, generator=g, dtype=F64) + 0.1,
        )

    a, b, c = elem(), elem(), elem()
    left = O.monoid_combine(O.monoid_combine(a, b), c)
    right = O.monoid_combine(a, O.monoid_combine(b, c))
    # Compare the represented values exp(log_scale) * (num, den) and the decay.
    for x, y in ((left, right),):
        assert torch.allclose(x[0], y[0], atol=1e-12)
        assert torch.allclose(torch.exp(x[1]) * x[2], torch.exp(y[1]) * y[2], rtol=1e-10)
        assert torch.allclose(torch.exp(x[1]) * x[3], torch.exp(y[1]) * y[3], rtol=1e-10)


def test_monoid_scan_upcasts_bf16_like_the_reference():
    k, v, td, tf = _inputs(2, 9, 4, seed=8, dtype=torch.float32)
    kb, vb = k.bfloat16(), v.bfloat16()
    out = O.wkv_monoid_scan(kb, vb, td, tf)
    assert out.dtype == torch.bfloat16
    ref = O.wkv_loop(kb.double(), vb.double(), td.double(), tf.double())
    assert torch.allclose(out.double(), ref, atol=1e-2, rtol=1e-2)


def test_kernel_forward_restatement_matches_loop():
    k, v, td, tf = _inputs(3, 33, 8, seed=9)
    w = -torch.exp(td)
    assert torch.allclose(O.reference_forward(k, v, w, tf), O.wkv_loop(k, v, td, tf), atol=1e-12, rtol=1e-10)


def test_autograd_of_loop_matches_finite_differences():
    k, v, td, tf = _inputs(1, 6, 3, seed=10)
    gy = torch.randn(1, 6, 3, generator=torch.Generator().manual_seed(11), dtype=F64)
    _, gk, gv, gtd, gtf = O.autograd_grads(k, v, td, tf, gy)
    eps = 1e-6

    def loss(kk, vv, dd, ff):
        return float((O.wkv_loop(kk, vv, dd, ff) * gy).sum())

    args = [k, v, td, tf]
    for idx, grad in enumerate((gk, gv, gtd, gtf)):
        base = args[idx]
        fd = torch.zeros_like(base)
        flat = base.reshape(-1)
        for j in range(flat.numel()):
            plus = [a.clone() for a in args]
            minus = [a.clone() for a in args]
            plus[idx].reshape(-1)[j] += eps
            minus[idx].reshape(-1)[j] -= eps
            fd.reshape(-1)[j] = (loss(*plus) - loss(*minus)) / (2 * eps)
        assert torch.allclose(grad, fd, atol=1e-7, rtol=1e-6), idx


@pytest.mark.parametrize("steps", [1, 7, 24])
def test_kernel_backward_restatement_matches_autograd(steps):
    k, v, td, tf = _inputs(2, steps, 8, seed=12)
    gy = torch.randn(2, steps, 8, generator=torch.Generator().manual_seed(13), dtype=F64)
    _, gk, gv, gtd, gtf = O.autograd_grads(k, v, td, tf, gy)
    rk, rv, rtd, rtf = O.reference_backward(gy, -torch.exp(td), tf, k, v)
    for got, ref in ((rk, gk), (rv, gv), (rtd, gtd), (rtf, gtf)):
        assert torch.allclose(got, ref, atol=1e-9, rtol=1e-6)


def test_gradient_invariants():
    k, v, td, tf = _inputs(3, 40, 8, seed=14)
    gy = torch.randn(3, 40, 8, generator=torch.Generator().manual_seed(15), dtype=F64)
    gk, gv, _, _ = O.reference_backward(gy, -torch.exp(td), tf, k, v)
    # y is invariant to adding one constant to every key: sum_t dL/dk_t = 0.
    assert torch.allclose(gk.sum(1), torch.zeros_like(gk[:, 0]), atol=1e-10)
    # the weights of each y_t sum to one: sum_t dL/dv_t = sum_t gy_t.
    assert torch.allclose(gv.sum(1), gy.sum(1), atol=1e-10)


def test_single_step_gradients():
    k, v, td, tf = _inputs(2, 1, 5, seed=16)
    gy = torch.randn(2, 1, 5, dtype=F64)
    gk, gv, gtd, gtf = O.reference_backward(gy, -torch.exp(td), tf, k, v)
    assert torch.allclose(gk, torch.zeros_like(gk), atol=1e-15)
    assert torch.allclose(gv, gy)
    assert torch.allclose(gtd, torch.zeros_like(gtd), atol=1e-15)
    assert torch.allclose(gtf, torch.zeros_like(gtf), atol=1e-15)


def test_iterated_decode_step_equals_sequence_forward():
    # tests/test_language.py:437-459 of the reference: step-by-step == full.
    k, v, td, tf = _inputs(2, 20, 6, seed=17, dtype=torch.float32)
    full = O.wkv_loop(k, v, td, tf)
    num, den, ls = O.initial_decode_state(2, 6)
    for t in range(20):
        y, num, den, ls = O.decode_step(k[:, t], v[:, t], td, tf, num, den, ls)
        assert torch.allclose(y, full[:, t], atol=1e-6)
    _, (n2, d2, l2) = O.wkv_loop_with_state(k, v, td, tf)
    assert torch.allclose(num, n2) and torch.allclose(den, d2) and torch.allclose(ls, l2)


def test_op_contracts_cast_like_the_reference():
    k, v, td, tf = _inputs(2, 10, 8, seed=18, dtype=torch.float32)
    kb, vb = k.bfloat16(), v.bfloat16()
    y32 = O.wkv_forward_op(kb.float(), vb.float(), td, tf)
    yb = O.wkv_forward_bf16io_op(kb, vb, td, tf)
    assert yb.dtype == torch.bfloat16
    assert torch.equal(yb, y32.to(torch.bfloat16))
    gy = torch.randn(2, 10, 8)
    gk, gv, gtd, gtf = O.wkv_backward_op(gy, -torch.exp(td), tf, k, v)
    assert gk.dtype == gv.dtype == torch.float32 and gtd.shape == (8,) and gtf.shape == (8,)


def test_validation_messages():
    with pytest.raises(ValueError, match="same shape"):
        O.wkv_loop(torch.randn(2, 4, 3), torch.randn(2, 4, 2), torch.zeros(3), torch.zeros(3))
    with pytest.raises(ValueError, match=r"\[B, T, C\]"):
        O.wkv_loop(torch.randn(4, 3), torch.randn(4, 3), torch.zeros(3), torch.zeros(3))
    with pytest.raises(ValueError, match="time_decay"):
        O.wkv_loop(torch.randn(2, 4, 3), torch.randn(2, 4, 3), torch.zeros(2), torch.zeros(3))


# ---------------------------------------------------------------- power ----
def _mutant_loop(key, value, time_decay, time_first, mistake):
    dtype = key.dtype
    decay = -torch.exp(time_decay.to(dtype))
    if mistake == "decay_sign":
        decay = -decay
    first = time_first.to(dtype)
    if mistake == "no_bonus":
        first = torch.zeros_like(first)
    b, steps, c = key.shape
    num = torch.zeros(b, c, dtype=dtype)
    den = torch.zeros(b, c, dtype=dtype)
    ls = torch.full((b, c), torch.finfo(dtype).min, dtype=dtype)
    outs = []
    for t in range(steps):
        kt, vt = key[:, t], value[:, t]
        if mistake == "value_lag" and t > 0:
            vt = value[:, t - 1]
        nxt = torch.maximum(ls, first + kt)
        a, bb = torch.exp(ls - nxt), torch.exp(first + kt - nxt)
        outs.append((a * num + bb * vt) / (a * den + bb))
        dec = ls + (decay if mistake != "decay_after" else 0.0)
        nxt = torch.maximum(dec, kt)
        a, bb = torch.exp(dec - nxt), torch.exp(kt - nxt)
        num, den, ls = a * num + bb * value[:, t], a * den + bb, nxt
    return torch.stack(outs, 1)


@pytest.mark.parametrize("mistake", ["decay_sign", "no_bonus", "value_lag", "decay_after"])
def test_closed_form_catches_plausible_mistakes(mistake):
    k, v, td, tf = _inputs(2, 12, 5, seed=19)
    ref = O.wkv_closed_form(k, v, td, tf)
    bad = _mutant_loop(k, v, td, tf, mistake)
    assert not torch.allclose(bad, ref, atol=1e-6, rtol=1e-4)
    assert torch.allclose(_mutant_loop(k, v, td, tf, "none"), ref, atol=1e-12, rtol=1e-10)


# -------------------------------------------------------------- fixtures ----
def test_golden_fixtures_reproduce():
    from pathlib import Path

    path = Path(__file__).parent / "golden" / "wkv4_small.npz"
    data = np.load(path, allow_pickle=False)
    for case in sorted({name.split("__")[0] for name in data.files}):
        g = {n.split("__")[1]: torch.from_numpy(data[n]) for n in data.files if n.startswith(case + "__")}
        y, gk, gv, gtd, gtf = O.autograd_grads(g["k"], g["v"], g["td"], g["tf"], g["gy"])
        assert torch.allclose(y, g["y"], atol=1e-12, rtol=1e-10), case
        for got, name in ((gk, "gk"), (gv, "gv"), (gtd, "gtd"), (gtf, "gtf")):
            assert torch.allclose(got, g[name], atol=1e-10, rtol=1e-9), (case, name)


def test_associative_scan_matches_the_loop_in_float64():
    # language.py:452-527 as the reference runs it (associative_scan, generic
    # combine mode): equal to the independently pinned loop in fp64, at T
    # values that are and are not powers of two (the scan's tree shape).
    for steps in (1, 2, 7, 16, 33):
        k, v, td, tf = _inputs(2, steps, 6, seed=40 + steps)
        y = O.wkv_associative_scan(k, v, td, tf)
        assert torch.allclose(y, O.wkv_loop(k, v, td, tf), atol=1e-12, rtol=1e-10), steps
    # T = 1 gives y = v (tests/test_language.py:42 of the reference)
    k, v, td, tf = _inputs(3, 1, 5, seed=47)
    assert torch.allclose(O.wkv_associative_scan(k, v, td, tf), v, atol=1e-14)


def test_associative_scan_float32_and_bf16_upcast():
    # Config-0 distributions in fp32 (C0: B=2, T=128, C=512): the tree-ordered
    # scan, the left fold and the fp64 loop agree to fp32 rounding; bf16
    # inputs are upcast to fp32 and the result cast back (language.py:483-485).
    k, v, td, tf, _ = O.make_inputs(2, 128, 512, seed=0)
    y = O.wkv_associative_scan(k, v, td, tf)
    assert y.dtype == torch.float32
    ref = O.wkv_loop(k.double(), v.double(), td.double(), tf.double())
    assert torch.allclose(y.double(), ref, rtol=1e-5, atol=1e-5 * float(ref.abs().max()))
    assert torch.allclose(y, O.wkv_monoid_scan(k, v, td, tf), rtol=1e-5, atol=1e-5)
    kb, vb = k.bfloat16(), v.bfloat16()
    yb = O.wkv_associative_scan(kb, vb, td, tf)
    assert yb.dtype == torch.bfloat16
    assert torch.equal(yb, O.wkv_associative_scan(kb.float(), vb.float(), td, tf).bfloat16())
