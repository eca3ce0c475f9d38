"""Layer norm fused into the token-shift mix (myelin::layer_norm_shift_mix):
forward and backward against F.layer_norm followed by the oracle's shift mix,
with autograd of that composition (fp64 on the CPU) for the gradients."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import spikegpt_myelin_amd  # noqa: F401  (registers the ops)
from oracle import timemix as TM
from spikegpt_myelin_amd.timemix import layer_norm_shift_mix

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _inputs(B, T, C, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, C, generator=g) * 2 + 0.5
    w = 1 + 0.3 * torch.randn(C, generator=g)
    b = 0.2 * torch.randn(C, generator=g)
    mix = torch.rand(n, C, generator=g)
    return x, w, b, mix


def _reference(x, w, b, mix, eps=1e-5):
    y = F.layer_norm(x, (x.shape[-1],), w, b, eps)
    return [TM.mix_with_previous(y, mix[j]) for j in range(mix.shape[0])]


@pytest.mark.parametrize("B,T,C,n", [(2, 70, 256, 3), (3, 33, 512, 2), (1, 1, 512, 3),
                                     (5, 64, 512, 3)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_forward_matches_layer_norm_then_mix(B, T, C, n, out_dtype):
    x, w, b, mix = _inputs(B, T, C, n, seed=B * 100 + T)
    print(f"ln_mix fwd B={B} T={T} C={C} n={n} {out_dtype}", flush=True)
    outs = torch.ops.myelin.layer_norm_shift_mix(x.to(DEV), w.to(DEV), b.to(DEV), mix.to(DEV),
                                                 1e-5, out_dtype)
    ref = _reference(x.double(), w.double(), b.double(), mix.double())
    tol = dict(atol=2e-5, rtol=2e-5) if out_dtype == torch.float32 else dict(atol=1e-2, rtol=1e-2)
    for j in range(n):
        torch.testing.assert_close(outs[j].cpu().double(), ref[j].to(out_dtype).double(), **tol)
    mean = x.double().mean(-1).reshape(-1)
    rstd = (x.double().var(-1, unbiased=False) + 1e-5).rsqrt().reshape(-1)
    torch.testing.assert_close(outs[n].cpu().double(), mean, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(outs[n + 1].cpu().double(), rstd, atol=1e-5, rtol=1e-5)


@pytest.mark.parametrize("B,T,C,n", [(2, 70, 256, 3), (3, 33, 512, 2), (1, 1, 256, 2),
                                     (5, 130, 512, 3)])
@pytest.mark.parametrize("g_dtype", [torch.float32, torch.bfloat16])
def test_backward_matches_autograd(B, T, C, n, g_dtype):
    x, w, b, mix = _inputs(B, T, C, n, seed=7 + T)
    gen = torch.Generator().manual_seed(11)
    grads = [torch.randn(B, T, C, generator=gen).to(g_dtype) for _ in range(n)]
    print(f"ln_mix bwd B={B} T={T} C={C} n={n} {g_dtype}", flush=True)
    xd, wd, bd, md = (t.double().requires_grad_() for t in (x, w, b, mix))
    ref = _reference(xd, wd, bd, md)
    torch.autograd.backward(ref, [g.double() for g in grads])
    xg, wg, bg, mg = (t.to(DEV).requires_grad_() for t in (x, w, b, mix))
    outs = torch.ops.myelin.layer_norm_shift_mix(xg, wg, bg, mg, 1e-5, g_dtype)
    torch.autograd.backward(list(outs[:n]), [g.to(DEV) for g in grads])

    def close(got, want, what):
        scale = want.abs().max().item() + 1e-12
        err = (got.cpu().double() - want).abs().max().item() / scale
        assert err < 2e-5, f"{what}: max error {err:.2e} of max |ref| {scale:.3g}"

    close(xg.grad, xd.grad, "grad_x")
    close(wg.grad, wd.grad, "grad_weight")
    close(bg.grad, bd.grad, "grad_bias")
    close(mg.grad, md.grad, "grad_mix")


def test_full_size_matches_unfused_kernels():
    # B=64, T=1024, C=512 under bf16 autocast: the fused op against torch's
    # layer norm followed by the (separately pinned) token_shift_mix kernel.
    from spikegpt_myelin_amd.timemix import token_shift_mix

    torch.manual_seed(0)
    B, T, C = 64, 1024, 512
    x = (torch.randn(B, T, C, device=DEV) * 1.5).requires_grad_()
    norm = torch.nn.LayerNorm(C).to(DEV)
    with torch.no_grad():
        norm.weight.add_(0.1 * torch.randn(C, device=DEV))
        norm.bias.add_(0.1 * torch.randn(C, device=DEV))
    mix = torch.rand(3, C, device=DEV, requires_grad=True)
    grads = [torch.randn(B, T, C, device=DEV).to(torch.bfloat16) for _ in range(3)]
    with torch.autocast("cuda", dtype=torch.bfloat16):
        fused = layer_norm_shift_mix(x, norm, mix)
    torch.autograd.backward(fused, grads)
    got = (x.grad.clone(), norm.weight.grad.clone(), norm.bias.grad.clone(), mix.grad.clone())
    for t in (x, norm.weight, norm.bias, mix):
        t.grad = None
    with torch.autocast("cuda", dtype=torch.bfloat16):
        plain = token_shift_mix(norm(x), mix)
    torch.autograd.backward(plain, grads)
    want = (x.grad, norm.weight.grad, norm.bias.grad, mix.grad)
    for a, b in zip(fused, plain):
        assert a.dtype == torch.bfloat16
        # Both round the same fp32 values to bf16; layer-norm statistics may
        # differ in the last fp32 bit, so allow one bf16 step.
        torch.testing.assert_close(a.float(), b.float(), atol=1e-2, rtol=8e-3)
        assert (a != b).float().mean().item() < 1e-3
    for g, w_, name in zip(got, want, ("x", "weight", "bias", "mix")):
        scale = w_.abs().max().item()
        err = (g - w_).abs().max().item() / scale
        assert err < 1e-4, f"grad {name}: {err:.2e}"


@pytest.mark.parametrize("B,T,C,n", [(2, 70, 256, 3), (3, 33, 512, 2)])
@pytest.mark.parametrize("residual_grad", [True, False])
def test_fork_adds_the_residual_gradient(B, T, C, n, residual_grad):
    # layer_norm_shift_mix_fork returns x again; the gradient of that second
    # use is added inside the backward kernel.  It must equal the plain op
    # with autograd summing the two gradients of x (one fp32 add either way).
    from spikegpt_myelin_amd.timemix import layer_norm_shift_mix_fork

    x, w, b, mix = _inputs(B, T, C, n, seed=40 + T)
    gen = torch.Generator().manual_seed(41)
    grads = [torch.randn(B, T, C, generator=gen).to(torch.bfloat16).to(DEV) for _ in range(n)]
    g_res = torch.randn(B, T, C, generator=gen).to(DEV)
    print(f"ln_mix fork B={B} T={T} C={C} n={n} residual_grad={residual_grad}", flush=True)

    def norm_module():
        m = torch.nn.LayerNorm(C).to(DEV)
        with torch.no_grad():
            m.weight.copy_(w)
            m.bias.copy_(b)
        return m

    n1, n2 = norm_module(), norm_module()
    x1, x2 = (x.to(DEV).requires_grad_() for _ in range(2))
    m1, m2 = (mix.to(DEV).requires_grad_() for _ in range(2))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        *outs1, xr = layer_norm_shift_mix_fork(x1, n1, m1)
        outs2 = layer_norm_shift_mix(x2, n2, m2)
    assert xr.data_ptr() == x1.data_ptr() and xr.requires_grad
    if residual_grad:
        torch.autograd.backward([*outs1, xr], [*grads, g_res])
        torch.autograd.backward([*outs2, x2], [*grads, g_res])
    else:
        torch.autograd.backward(outs1, grads)
        torch.autograd.backward(outs2, grads)
    for a, c in zip(outs1, outs2):
        assert torch.equal(a, c)
    assert torch.equal(x1.grad, x2.grad)
    assert torch.equal(m1.grad, m2.grad)
    assert torch.equal(n1.weight.grad, n2.weight.grad)
    assert torch.equal(n1.bias.grad, n2.bias.grad)


def test_backward_op_opcheck_with_added_gradient():
    x, w, b, mix = (t.to(DEV) for t in _inputs(2, 9, 256, 2, seed=3))
    outs = torch.ops.myelin.layer_norm_shift_mix(x, w, b, mix, 1e-5, torch.bfloat16)
    grads = [torch.randn_like(o, dtype=torch.float32).to(torch.bfloat16) for o in outs[:2]]
    gadd = torch.randn_like(x)
    args = (grads, x, w, b, mix, outs[2], outs[3])
    torch.library.opcheck(torch.ops.myelin.layer_norm_shift_mix_backward, args,
                          {"grad_x_add": gadd})
    torch.library.opcheck(torch.ops.myelin.layer_norm_shift_mix_backward, args)
    gx_add, gp_add = torch.ops.myelin.layer_norm_shift_mix_backward(*args, grad_x_add=gadd)
    gx, gp = torch.ops.myelin.layer_norm_shift_mix_backward(*args)
    assert torch.equal(gx_add, gx + gadd)
    assert torch.equal(gp_add, gp)
