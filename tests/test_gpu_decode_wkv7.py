"""GPU parity of the decode step and the RWKV-7 DPLR op against the oracle."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import wkv4 as O4
from oracle import wkv7 as O7

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ops():
    import spikegpt_myelin_amd  # noqa: F401

    return torch.ops.myelin


def test_decode_step_matches_oracle_step():
    ops = _ops()
    b, c = 256, 768
    k, v, td, tf, _ = O4.make_inputs(b, 3, c, seed=0, with_grad=False)
    num, den, ls = O4.initial_decode_state(b, c)
    state = tuple(x.to(DEV) for x in (num, den, ls))
    for t in range(3):
        y_ref, num, den, ls = O4.decode_step(k[:, t].double(), v[:, t].double(), td.double(), tf.double(),
                                             num.double(), den.double(), ls.double())
        y, *state = ops.wkv_decode_step(k[:, t].to(DEV), v[:, t].to(DEV), td.to(DEV), tf.to(DEV), *state)
        assert torch.allclose(y.double().cpu(), y_ref, atol=1e-6, rtol=1e-5)
        assert torch.allclose(state[0].double().cpu(), num, rtol=1e-5, atol=1e-6)
        assert torch.allclose(state[1].double().cpu(), den, rtol=1e-5, atol=1e-6)
        assert torch.allclose(state[2].double().cpu(), ls, rtol=1e-6, atol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_iterated_decode_equals_sequence_forward(dtype):
    # tests/test_language.py:437-459 of the reference (cached step == full).
    ops = _ops()
    b, t, c = 4, 40, 96
    k, v, td, tf, _ = O4.make_inputs(b, t, c, seed=1, dtype=dtype, with_grad=False)
    kd, vd, tdd, tfd = (x.to(DEV) for x in (k, v, td, tf))
    full = ops.wkv_forward(kd, vd, tdd, tfd).float()
    state = tuple(x.to(DEV) for x in O4.initial_decode_state(b, c))
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    for step in range(t):
        y, *state = ops.wkv_decode_step(kd[:, step], vd[:, step], tdd, tfd, *state)
        assert y.dtype == dtype
        assert torch.allclose(y.float(), full[:, step], atol=tol, rtol=tol), step


def test_decode_channels_not_multiple_of_four():
    ops = _ops()
    b, c = 3, 37
    k, v, td, tf, _ = O4.make_inputs(b, 1, c, seed=2, with_grad=False)
    st = O4.initial_decode_state(b, c)
    y_ref, *_ = O4.decode_step(k[:, 0], v[:, 0], td, tf, *st)
    y, *_ = ops.wkv_decode_step(k[:, 0].to(DEV), v[:, 0].to(DEV), td.to(DEV), tf.to(DEV),
                                *(x.to(DEV) for x in st))
    assert torch.allclose(y.cpu(), y_ref, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_wkv7_forward_matches_oracle(dtype):
    ops = _ops()
    r, w, k, v, a, b = O7.make_inputs(2, 48, 3, 64, seed=3, dtype=dtype)
    y, s = ops.wkv7_forward(*(x.to(DEV) for x in (r, w, k, v, a, b)), None)
    y_ref, s_ref = O7.wkv7_loop(*(x.double() for x in (r, w, k, v, a, b)))
    assert y.dtype == dtype and s.dtype == torch.float32
    # y: the 16-bit bar (2e-2 relative, 1e-2 absolute) or, for fp32, 1e-5
    # relative with a floor of 1e-5 * max|ref|; the fp32 state: the latter.
    y_ref_scale = float(y_ref.abs().max())
    if dtype == torch.float32:
        assert torch.allclose(y.double().cpu(), y_ref, rtol=1e-5, atol=1e-5 * y_ref_scale)
    else:
        assert torch.allclose(y.double().cpu(), y_ref, rtol=2e-2, atol=1e-2)
    assert torch.allclose(s.double().cpu(), s_ref, rtol=1e-5, atol=1e-5 * float(s_ref.abs().max()))


def test_wkv7_state_carry_and_golden_fixture():
    ops = _ops()
    from pathlib import Path

    data = np.load(Path(__file__).parent / "golden" / "wkv7_small.npz", allow_pickle=False)
    g = {n.split("__")[1]: torch.from_numpy(data[n]) for n in data.files}
    xs = [g[n].float().to(DEV) for n in ("r", "w", "k", "v", "a", "b")]
    y, s = ops.wkv7_forward(*xs, None)
    assert torch.allclose(y.double().cpu(), g["y"], rtol=1e-5, atol=1e-5 * float(g["y"].abs().max()))
    # split the sequence: run the first half, carry the state into the second
    y1, s1 = ops.wkv7_forward(*(x[:, :5] for x in xs), None)
    y2, s2 = ops.wkv7_forward(*(x[:, 5:] for x in xs), s1)
    assert torch.allclose(torch.cat([y1, y2], 1), y, rtol=1e-5, atol=1e-5)
    assert torch.allclose(s2, s, rtol=1e-5, atol=1e-5)
