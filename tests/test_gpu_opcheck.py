"""torch.library.opcheck over the library's custom ops beyond the RWKV-4 ones
(which tests/test_gpu_wkv4.py and test_gpu_wkv4_gated.py check): schema,
fake (meta) implementation, autograd registration and AOT dispatch with
dynamic shapes -- what torch.compile relies on when it traces a model that
calls them.  Small inputs; where an op has an autograd formula, one sample
carries inputs that require grad so that the registration is exercised.
"""

from __future__ import annotations

import pytest
import torch

from oracle import wkv4 as O4
from oracle import wkv7 as O7

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ops():
    import spikegpt_myelin_amd  # noqa: F401

    return torch.ops.myelin


def _opcheck(op, args, kwargs=None):
    torch.library.opcheck(op, args, kwargs or {})


def _grad(*xs):
    return tuple(x.detach().clone().requires_grad_(True) for x in xs)


def _wkv7_inputs(dtype=torch.bfloat16):
    xs = [x.to(DEV) for x in O7.make_inputs(2, 19, 2, 64, seed=41, dtype=dtype)]
    g = torch.Generator().manual_seed(42)
    s0 = (0.5 * torch.randn(2, 2, 64, 64, generator=g)).to(DEV)
    gy = torch.randn(2, 19, 2, 64, generator=g).to(dtype).to(DEV)
    gs = torch.randn(2, 2, 64, 64, generator=g).to(DEV)
    return xs, s0, gy, gs


def test_wkv7_training_forward():
    ops = _ops()
    xs, s0, _, _ = _wkv7_inputs()
    op = ops.wkv7_forward_train.default
    _opcheck(op, (*xs, s0))
    _opcheck(op, (*xs, None))
    _opcheck(op, (*_grad(*xs), s0.clone().requires_grad_(True)))


def test_wkv7_training_backward_and_public_backward():
    ops = _ops()
    xs, s0, gy, gs = _wkv7_inputs()
    _, _, ck = ops.wkv7_forward_train(*xs, s0)
    _opcheck(ops.wkv7_backward_train.default, (*xs, ck, gy, gs, True))
    _opcheck(ops.wkv7_backward_train.default, (*xs, ck, gy, None, False))
    _opcheck(ops.wkv7_backward.default, (*xs, s0, gy, gs))
    _opcheck(ops.wkv7_backward.default, (*xs, None, gy, None))


def test_wkv_decode_step():
    ops = _ops()
    k, v, td, tf, _ = O4.make_inputs(4, 1, 96, seed=43, with_grad=False)
    num, den, ls = O4.initial_decode_state(4, 96)
    args = tuple(x.to(DEV) for x in (k[:, 0], v[:, 0], td, tf, num, den, ls))
    _opcheck(ops.wkv_decode_step.default, args)


def test_gates():
    ops = _ops()
    g = torch.Generator().manual_seed(44)
    x, r, gy = (torch.randn(2, 8, 64, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3))
    _opcheck(ops.relu_square.default, (x,))
    _opcheck(ops.relu_square.default, _grad(x))
    _opcheck(ops.relu_square_backward.default, (gy, x))
    _opcheck(ops.sigmoid_gate.default, (r, x))
    _opcheck(ops.sigmoid_gate.default, _grad(r, x))
    _opcheck(ops.sigmoid_gate_backward.default, (gy, r, x))


LIF_ARGS = (0.5, 0.3, 0.0, 4.0)  # decay, threshold, reset, slope


def test_lif_sequence():
    ops = _ops()
    g = torch.Generator().manual_seed(45)
    x = torch.randn(2, 70, 64, generator=g).to(torch.bfloat16).to(DEV)
    gsp = torch.randn(2, 70, 64, generator=g).to(torch.bfloat16).to(DEV)
    _opcheck(ops.lif_sequence_forward.default, (x, *LIF_ARGS))
    _opcheck(ops.lif_sequence_forward.default, (*_grad(x), *LIF_ARGS))
    _, ck = ops.lif_sequence_forward(x, *LIF_ARGS)
    _opcheck(ops.lif_sequence_backward.default, (gsp, x, ck, *LIF_ARGS))


def test_lif_residual():
    ops = _ops()
    g = torch.Generator().manual_seed(46)
    x = torch.randn(2, 70, 64, generator=g).to(torch.bfloat16).to(DEV)
    res = torch.randn(2, 70, 64, generator=g).to(DEV)
    gout = torch.randn(2, 70, 64, generator=g).to(DEV)
    _opcheck(ops.lif_residual_forward.default, (x, res, *LIF_ARGS))
    _opcheck(ops.lif_residual_forward.default, (*_grad(x, res), *LIF_ARGS))
    _, ck = ops.lif_residual_forward(x, res, *LIF_ARGS)
    _opcheck(ops.lif_residual_backward.default, (gout, x, ck, *LIF_ARGS))


def test_split_k_sum():
    ops = _ops()
    g = torch.Generator().manual_seed(47)
    _opcheck(ops.split_k_sum.default, (torch.randn(4, 64, 64, generator=g).to(DEV),))


def test_token_shift_mix():
    ops = _ops()
    g = torch.Generator().manual_seed(48)
    x = torch.randn(2, 70, 128, generator=g).to(DEV)
    mix = torch.rand(3, 128, generator=g).to(DEV)
    _opcheck(ops.token_shift_mix.default, (x, mix, torch.bfloat16))
    _opcheck(ops.token_shift_mix.default, (*_grad(x, mix), torch.bfloat16))
    grads = [torch.randn(2, 70, 128, generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    _opcheck(ops.token_shift_mix_backward.default, (grads, x, mix))


def test_layer_norm_shift_mix_forward():
    ops = _ops()
    g = torch.Generator().manual_seed(49)
    x = torch.randn(2, 40, 256, generator=g).to(DEV)
    w = (1 + 0.1 * torch.randn(256, generator=g)).to(DEV)
    b = (0.1 * torch.randn(256, generator=g)).to(DEV)
    mix = torch.rand(3, 256, generator=g).to(DEV)
    _opcheck(ops.layer_norm_shift_mix.default, (x, w, b, mix, 1e-5, torch.bfloat16))
    _opcheck(ops.layer_norm_shift_mix.default, (*_grad(x, w, b, mix), 1e-5, torch.bfloat16))
