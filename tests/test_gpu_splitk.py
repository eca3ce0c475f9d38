"""myelin::split_k_sum (the fixed-order fp32 sum ending the model's split-K
weight gradients) against the same sum done step by step in fp32 by torch,
and the split-K projection's weight gradient against nn.Linear's."""

from __future__ import annotations

import pytest
import torch

import spikegpt_myelin_amd  # noqa: F401
from spikegpt_myelin_amd.splitk import split_k_sum

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


@pytest.mark.parametrize("shape", [(16, 512, 512), (16, 2048, 512), (3, 4), (1, 8, 4),
                                   (7, 1000, 36)])
def test_matches_sequential_fp32_sum(shape):
    print(f"split_k_sum {shape}", flush=True)
    g = torch.Generator().manual_seed(sum(shape))
    partial = torch.randn(*shape, generator=g).to(DEV)
    got = split_k_sum(partial)
    want = partial[0].clone()
    for s in range(1, shape[0]):
        want = want + partial[s]
    assert got.shape == shape[1:] and got.dtype == torch.float32
    assert torch.equal(got, want)


def test_odd_trailing_size_and_cpu():
    partial = torch.randn(5, 3, 3, device=DEV)   # 9 elements: torch's sum
    torch.testing.assert_close(split_k_sum(partial), partial.sum(0))
    with pytest.raises(Exception):
        torch.ops.myelin.split_k_sum(torch.randn(4, 8))


def test_split_k_linear_weight_gradient():
    # Under bf16 autocast the projection multiplies bf16-rounded operands; the
    # split-K weight gradient accumulates and sums in fp32, so it must match
    # the fp32 product of those rounded operands (nn.Linear's own gradient is
    # the same product rounded to bf16, off by up to 2^-9 relative).
    from spikegpt_myelin_amd.model import SplitKLinear

    torch.manual_seed(3)
    lin = SplitKLinear(512, 512, bias=False).to(DEV)
    x = torch.randn(16 * 2048, 512, device=DEV)
    gy = torch.randn(16 * 2048, 512, device=DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = lin(x)
    torch.autograd.backward(y, gy.to(y.dtype))
    want_y = x.bfloat16().float() @ lin.weight.detach().bfloat16().float().t()
    torch.testing.assert_close(y.float(), want_y, atol=2e-2, rtol=8e-3)
    want = gy.bfloat16().float().t() @ x.bfloat16().float()
    scale = want.abs().max().item()
    err = (lin.weight.grad - want).abs().max().item() / scale
    assert err < 1e-5, f"weight grad rel err {err:.2e}"


def test_opcheck():
    # Schema, fake (meta) implementation and dispatch registration.
    partial = torch.randn(4, 16, 8, device=DEV)
    torch.library.opcheck(torch.ops.myelin.split_k_sum, (partial,))
