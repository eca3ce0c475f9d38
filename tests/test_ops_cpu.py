"""Op boundary on the CPU: schemas, fake (meta) impls, validation, and that
the ops refuse to run without a GPU (there is no CPU implementation)."""

from __future__ import annotations

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

import spikegpt_myelin_amd as m

REFERENCE_SCHEMAS = {
    # inferred by torch.library.custom_op from the reference's signatures
    # (src/spikegpt/wkv_triton.py:147-167, src/spikegpt/wkv_bf16.py:143-163)
    "wkv_forward": "myelin::wkv_forward(Tensor key, Tensor value, Tensor time_decay, Tensor time_first) -> Tensor",
    "wkv_backward": "myelin::wkv_backward(Tensor grad_y, Tensor w, Tensor u, Tensor k, Tensor v) -> Tensor[]",
    "wkv_forward_bf16io": "myelin::wkv_forward_bf16io(Tensor key, Tensor value, Tensor time_decay, Tensor time_first) -> Tensor",
    "wkv_backward_bf16io": "myelin::wkv_backward_bf16io(Tensor grad_y, Tensor w, Tensor u, Tensor k, Tensor v) -> Tensor[]",
}


@pytest.mark.parametrize("name", sorted(REFERENCE_SCHEMAS))
def test_schema_matches_reference(name):
    assert str(getattr(torch.ops.myelin, name).default._schema) == REFERENCE_SCHEMAS[name]


def test_fake_impls_give_reference_shapes_and_dtypes():
    with FakeTensorMode():
        k = torch.empty(2, 5, 8, dtype=torch.bfloat16)
        td = torch.empty(8)
        y = torch.ops.myelin.wkv_forward_bf16io(k, k, td, td)
        assert y.shape == k.shape and y.dtype == torch.bfloat16
        y32 = torch.ops.myelin.wkv_forward(k.float(), k.float(), td, td)
        assert y32.dtype == torch.float32
        gk, gv, gtd, gtf = torch.ops.myelin.wkv_backward_bf16io(k, td, td, k, k)
        assert gk.dtype == gv.dtype == torch.bfloat16 and gtd.shape == (8,) and gtf.dtype == torch.float32
        y, n, d, s = torch.ops.myelin.wkv_decode_step(k[:, 0], k[:, 0], td, td, td.expand(2, 8), td.expand(2, 8),
                                                      td.expand(2, 8))
        assert y.dtype == torch.bfloat16 and n.dtype == torch.float32 and s.shape == (2, 8)
        r = torch.empty(1, 4, 2, 64, dtype=torch.bfloat16)
        y7, s7 = torch.ops.myelin.wkv7_forward(r, r, r, r, r, r, None)
        assert y7.shape == r.shape and s7.shape == (1, 2, 64, 64) and s7.dtype == torch.float32


def test_validation_errors_match_reference_messages():
    with pytest.raises(ValueError, match="same shape"):
        m.weighted_key_value(torch.randn(2, 4, 3), torch.randn(2, 4, 2), torch.zeros(3), torch.zeros(3))
    with pytest.raises(ValueError, match=r"shape \[B, T, C\]"):
        m.weighted_key_value(torch.randn(4, 3), torch.randn(4, 3), torch.zeros(3), torch.zeros(3))
    with pytest.raises(ValueError, match=r"time_first must have shape \[3\]"):
        m.weighted_key_value(torch.randn(2, 4, 3), torch.randn(2, 4, 3), torch.zeros(3), torch.zeros(2))


def test_ops_refuse_cpu_tensors():
    k = torch.randn(2, 4, 8)
    with pytest.raises(RuntimeError, match="GPU"):
        torch.ops.myelin.wkv_forward(k, k, torch.zeros(8), torch.zeros(8))
    with pytest.raises(RuntimeError, match="GPU"):
        torch.ops.myelin.wkv_backward_bf16io(k, torch.zeros(8), torch.zeros(8), k, k)


def test_reference_api_names_are_exported():
    assert m.weighted_key_value_triton is m.weighted_key_value_hip
    assert m.weighted_key_value_triton_bf16io is m.weighted_key_value_hip_bf16io


def test_lif_module_takes_the_reference_options_and_refuses_what_it_cannot_serve():
    # SpikingSequenceLIF(tau, threshold, reset, surrogate, surrogate_slope,
    # hard_forward, fused, recompute) -- language.py:769-781.  The kernels
    # serve the arctan surrogate with a Heaviside forward; fused/recompute do
    # not change the values.  Anything else is refused at construction, so it
    # can never reach the kernels.
    import math
    import types

    from spikegpt_myelin_amd import atan_surrogate
    from spikegpt_myelin_amd.model import SpikingSequenceLIF

    for kw in (dict(), dict(fused=False), dict(recompute=True), dict(surrogate=atan_surrogate)):
        m = SpikingSequenceLIF(**kw)
        assert m.hard_forward is True and m.surrogate is atan_surrogate
    with pytest.raises(NotImplementedError, match="surrogate"):
        SpikingSequenceLIF(surrogate=lambda c: torch.sigmoid(4.0 * c))
    with pytest.raises(NotImplementedError, match="hard_forward=False"):
        SpikingSequenceLIF(hard_forward=False)
    # myelin's own arctan surrogate is recognised by module and name.
    fake = types.FunctionType(atan_surrogate.__code__, atan_surrogate.__globals__,
                              "atan_surrogate")
    fake.__module__ = "myelin.surrogates"
    assert SpikingSequenceLIF(surrogate=fake).surrogate is fake
    other = types.FunctionType(atan_surrogate.__code__, atan_surrogate.__globals__,
                               "sigmoid_surrogate")
    other.__module__ = "myelin.surrogates"
    with pytest.raises(NotImplementedError):
        SpikingSequenceLIF(surrogate=other)
    # The surrogate's derivative is the one the kernels apply (the oracle's).
    from oracle import lif as L

    c = torch.linspace(-3, 3, 61, dtype=torch.float64).requires_grad_(True)
    (d,) = torch.autograd.grad(atan_surrogate(c).sum(), c)
    assert torch.allclose(d, L.surrogate_grad(c.detach()), rtol=1e-12, atol=1e-14)
    assert float(atan_surrogate(torch.tensor(0.0))) == 0.5
    assert math.isclose(float(atan_surrogate(torch.tensor(1e9, dtype=torch.float64))), 1.0,
                        abs_tol=1e-9)
