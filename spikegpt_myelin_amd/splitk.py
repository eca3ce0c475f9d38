"""``myelin::split_k_sum``: the fixed-order fp32 sum that ends a split-K
weight gradient (``out = partial.sum(0)`` for ``partial`` [S, ...] fp32,
added in the order s = 0, 1, ..., S-1), one HIP kernel with 16-byte loads.

The model's projections (``SplitKLinear``) compute their weight gradient as S
GEMMs over slices of the B*T rows; the reference's ``nn.Linear`` projections
(``src/spikegpt/language.py:952-955, 1155-1157``) use one GEMM over all rows.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib


@torch.library.custom_op("myelin::split_k_sum", mutates_args=())
def _split_k_sum(partial: Tensor) -> Tensor:
    _lib.require_gpu(partial)
    if partial.dtype != torch.float32 or partial.ndim < 2:
        raise ValueError("split_k_sum takes fp32 [S, ...] partials")
    src = _lib.aligned(partial.contiguous())
    out = torch.empty(partial.shape[1:], dtype=torch.float32, device=partial.device)
    s, n = src.shape[0], out.numel()
    lib = _lib.load()
    rc = _lib.timed("split_k_sum", partial.device,
                    lambda: lib.split_k_sum(src.data_ptr(), out.data_ptr(), s, n,
                                            _lib.stream_of(src)))
    _lib.check(rc, "split_k_sum")
    return out


@_split_k_sum.register_fake
def _(partial):
    return partial.new_empty(partial.shape[1:])


def split_k_sum(partial: Tensor) -> Tensor:
    """``partial.sum(0)`` of fp32 GPU partials, summed in index order.  The
    kernel reads 4 elements per thread; a trailing size that is not a
    multiple of 4 takes torch's (GPU) sum."""
    if partial.ndim >= 2 and partial[0].numel() % 4 != 0:
        return partial.sum(0)
    return torch.ops.myelin.split_k_sum(partial)
