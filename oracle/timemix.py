"""CPU oracle for SpikeGPT's token-shift mixing (test infrastructure).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``; never by the product
package.

Restates ``_time_shift`` and ``_mix_with_previous`` of
``src/spikegpt/language.py:344-353``::

    shift(x)[:, t] = x[:, t-1]  (zeros at t = 0)
    mix(x, mu)     = x * mu + shift(x) * (1 - mu)

and the cast that autocast applies when the result feeds a projection.

Pinned (``tests/test_oracle_timemix.py``) by: ``mu = 1`` gives ``x`` and
``mu = 0`` gives the shifted sequence exactly; a hand-computed example; and
linearity in ``x``.  Gradients come from torch autograd through these lines.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor

__all__ = ["time_shift", "mix_with_previous", "shift_mix"]


def time_shift(x: Tensor) -> Tensor:
    """``language.py:344-345``."""
    return F.pad(x[:, :-1], (0, 0, 1, 0))


def mix_with_previous(x: Tensor, mix: Tensor) -> Tensor:
    """``language.py:348-353``."""
    return x * mix + time_shift(x) * (1.0 - mix)


def shift_mix(x: Tensor, mixes: Tensor, out_dtype: torch.dtype | None = None) -> list[Tensor]:
    """Every row of ``mixes`` ``[n, C]`` applied to ``x`` ``[B, T, C]``, each
    result cast to ``out_dtype`` (the projection's input type)."""
    out = [mix_with_previous(x, m.view(1, 1, -1)) for m in mixes]
    return out if out_dtype is None else [o.to(out_dtype) for o in out]
