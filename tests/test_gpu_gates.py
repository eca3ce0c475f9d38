"""GPU parity of the fused squared ReLU and receptance gate.

Bars: forward of ``relu_square`` bit-exact against ``relu(x).square()`` in
fp32 rounded once (the autocast values); ``sigmoid_gate`` forward within one
unit in the last place of the element type of torch's own two-kernel result
and equal on at least 99.9 % of elements, also over every 16-bit input, where
bf16 is equal on every input (fp32 gates evaluate torch's expression; 16-bit
gates a short exp2/reciprocal form whose rounded value is what counts);
backward against float64 autograd with ``rtol=1e-5`` (fp32) or
``rtol=2e-2, atol=1e-2`` (16-bit).
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _ops():
    import spikegpt_myelin_amd  # noqa: F401

    return torch.ops.myelin


def _tol(dt):
    return dict(rtol=1e-5, atol=1e-6) if dt == torch.float32 else dict(rtol=2e-2, atol=1e-2)


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", [(8,), (3, 7, 64), (64, 1024, 128)])
def test_relu_square(dt, shape):
    g = torch.Generator().manual_seed(1)
    x = (torch.randn(shape, generator=g) * 3).to(dt)
    gy = torch.randn(shape, generator=g).to(dt)
    y = _ops().relu_square(x.to(DEV))
    ref = (torch.relu(x.float()) ** 2).to(dt)
    assert torch.equal(y.cpu(), ref)
    gx = _ops().relu_square_backward(gy.to(DEV), x.to(DEV))
    xr = x.double().requires_grad_(True)
    (rg,) = torch.autograd.grad(torch.relu(xr) ** 2, xr, gy.double())
    assert torch.allclose(gx.double().cpu(), rg, **_tol(dt))


@pytest.mark.parametrize("dt", DTYPES)
@pytest.mark.parametrize("shape", [(16,), (5, 33, 96), (64, 1024, 64)])
def test_sigmoid_gate(dt, shape):
    g = torch.Generator().manual_seed(2)
    r = (torch.randn(shape, generator=g) * 4).to(dt)
    x = torch.randn(shape, generator=g).to(dt)
    gy = torch.randn(shape, generator=g).to(dt)
    rd, xd = r.to(DEV), x.to(DEV)
    y = _ops().sigmoid_gate(rd, xd)
    eager = torch.sigmoid(rd) * xd
    diff = (y.float() - eager.float()).abs()
    ulp = torch.finfo(dt).eps * eager.float().abs().clamp_min(torch.finfo(dt).tiny)
    assert bool((diff <= ulp).all()), float(diff.max())
    assert float((y == eager).float().mean()) >= 0.999
    gr, gx = _ops().sigmoid_gate_backward(gy.to(DEV), rd, xd)
    rr = r.double().requires_grad_(True)
    xr = x.double().requires_grad_(True)
    grr, gxr = torch.autograd.grad(torch.sigmoid(rr) * xr, [rr, xr], gy.double())
    assert torch.allclose(gr.double().cpu(), grr, **_tol(dt))
    assert torch.allclose(gx.double().cpu(), gxr, **_tol(dt))


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float16])
def test_sigmoid_gate_every_16bit_input(dt):
    # Every finite value of the type as r, x = 1: the gate is then the
    # rounded sigmoid itself.  Against torch's sigmoid of the same inputs:
    # bf16 equal everywhere (65,280 inputs, the denormal and overflow ends
    # included); fp16 within one unit in the last place everywhere and equal
    # on >= 99.9 % (its 10-bit mantissa puts more values near a rounding
    # midpoint than the short sigmoid's few-ulp fp32 error can resolve).
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16)
    r = bits.view(dt)
    r = r[torch.isfinite(r.float())].to(DEV)
    y = _ops().sigmoid_gate(r, torch.ones_like(r))
    ref = torch.sigmoid(r)
    diff = (y.float() - ref.float()).abs()
    ulp = torch.finfo(dt).eps * ref.float().abs().clamp_min(torch.finfo(dt).tiny)
    equal = float((y == ref).float().mean())
    print(f"{dt}: {r.numel()} inputs, equal {equal:.6f}, max diff / ulp "
          f"{float((diff / ulp).max()):.3f}")
    assert bool((diff <= ulp).all()), float((diff / ulp).max())
    assert equal >= 0.999
    if dt == torch.bfloat16:
        assert torch.equal(y, ref)


def test_module_functions_route_and_differentiate():
    from spikegpt_myelin_amd import relu_square, sigmoid_gate

    x = torch.randn(4, 32, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    r = torch.randn(4, 32, 64, device=DEV, dtype=torch.bfloat16, requires_grad=True)
    (sigmoid_gate(r, relu_square(x)).float().sum()).backward()
    assert x.grad is not None and r.grad is not None
    # odd sizes take the eager expression
    z = torch.randn(3, 5, device=DEV, dtype=torch.bfloat16)
    assert torch.equal(relu_square(z), torch.relu(z).square())
