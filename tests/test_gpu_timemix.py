"""GPU parity of the fused token-shift mix against the CPU oracle.

Bars (written per test):
* forward: bit-exact against the eager expression of language.py:344-353 in
  fp32 followed by the cast to the output type (same fp32 operations, one
  rounding);
* grad_x: ``rtol=1e-5, atol=1e-5 * max|ref|`` against float64 autograd of the
  oracle for fp32 gradients; ``rtol=2e-2, atol=1e-2 * max|ref|`` when x is
  16-bit;
* grad_mix (a sum over B*T terms): ``|err| <= 1e-5 * sum|terms|`` per channel
  for fp32 x (the fp32 accumulation error bound), 2e-2 for 16-bit x.
"""

from __future__ import annotations

import pytest
import torch

from oracle import timemix as M

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ops():
    import spikegpt_myelin_amd  # noqa: F401

    return torch.ops.myelin


def _inputs(b, t, c, n, xdt, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(b, t, c, generator=g).to(xdt)
    mix = torch.rand(n, c, generator=g)
    return x, mix


CASES = [  # (B, T, C, n, x dtype, out dtype)
    (2, 64, 128, 3, torch.float32, torch.bfloat16),
    (3, 100, 96, 3, torch.float32, torch.float32),
    (2, 7, 70, 2, torch.float32, torch.bfloat16),
    (1, 1, 8, 1, torch.float32, torch.float16),
    (2, 130, 256, 2, torch.bfloat16, torch.bfloat16),
    (2, 65, 64, 3, torch.float16, torch.float16),
    (4, 257, 512, 2, torch.float32, torch.bfloat16),
    # Enough (batch, channel-group) rows that the host picks 64-step chunks
    # (128 x 16 = 2048 waves), then 32-step chunks with a 3-step tail after the
    # last 8-step block (T = 1003).
    (128, 1024, 8, 3, torch.float32, torch.bfloat16),
    (64, 1003, 16, 2, torch.float32, torch.float32),
]


@pytest.mark.parametrize("b,t,c,n,xdt,odt", CASES)
def test_forward_bit_exact(b, t, c, n, xdt, odt):
    x, mix = _inputs(b, t, c, n, xdt, seed=b + t + c + n)
    outs = _ops().token_shift_mix(x.to(DEV), mix.to(DEV), odt)
    torch.cuda.synchronize()
    ref = M.shift_mix(x.float(), mix, odt)
    assert len(outs) == n
    for j, (o, r) in enumerate(zip(outs, ref)):
        assert o.dtype == odt
        assert torch.equal(o.cpu(), r), f"out {j} differs"


@pytest.mark.parametrize("b,t,c,n,xdt,odt", CASES)
def test_backward_matches_autograd(b, t, c, n, xdt, odt):
    x, mix = _inputs(b, t, c, n, xdt, seed=7 * b + t + c)
    g = torch.Generator().manual_seed(99)
    grads = [torch.randn(b, t, c, generator=g).to(odt) for _ in range(n)]
    gx, gmix = _ops().token_shift_mix_backward([q.to(DEV) for q in grads], x.to(DEV), mix.to(DEV))
    torch.cuda.synchronize()
    xr = x.double().requires_grad_(True)
    mr = mix.double().requires_grad_(True)
    outs = M.shift_mix(xr, mr)
    rgx, rgm = torch.autograd.grad(outs, [xr, mr], [q.double() for q in grads])
    rtol, asc = (1e-5, 1e-5) if xdt == torch.float32 else (2e-2, 1e-2)
    atol = asc * max(float(rgx.abs().max()), 1.0)
    err = float((gx.double().cpu() - rgx).abs().max())
    assert gx.dtype == xdt
    assert torch.allclose(gx.double().cpu(), rgx, rtol=rtol, atol=atol), f"grad_x err {err:.3e}"
    # grad_mix: sum over b, t of g * (x - shift(x)); bound by the magnitude sum.
    xs = x.double()
    diff = xs - M.time_shift(xs)
    mag = torch.stack([(q.double() * diff).abs().sum(dim=(0, 1)) for q in grads])
    bound = (1e-5 if xdt == torch.float32 else 2e-2) * mag + 1e-6
    assert torch.all((gmix.double().cpu() - rgm).abs() <= bound), "grad_mix out of bound"


def test_autograd_through_token_shift_mix_under_autocast():
    from spikegpt_myelin_amd.timemix import token_shift_mix

    x, mix = _inputs(2, 96, 128, 3, torch.float32, seed=5)
    xd = x.to(DEV).requires_grad_(True)
    md = mix.to(DEV).requires_grad_(True)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        outs = token_shift_mix(xd, md)
    assert all(o.dtype == torch.bfloat16 for o in outs)
    loss = sum((o.float() * (j + 1)).sum() for j, o in enumerate(outs))
    loss.backward()
    xr = x.double().requires_grad_(True)
    mr = mix.double().requires_grad_(True)
    rl = sum((o * (j + 1)).sum() for j, o in enumerate(M.shift_mix(xr, mr)))
    rgx, rgm = torch.autograd.grad(rl, [xr, mr])
    assert torch.allclose(xd.grad.double().cpu(), rgx, rtol=1e-5, atol=1e-5)
    assert torch.allclose(md.grad.double().cpu(), rgm, rtol=1e-4, atol=1e-3)


def test_bad_mix_shape_raises():
    with pytest.raises(ValueError, match="mix must have shape"):
        _ops().token_shift_mix(torch.zeros(1, 4, 8, device=DEV), torch.zeros(4, 8, device=DEV), torch.float32)
