"""Caller-side WKV entry point, mirroring ``src/spikegpt/language.py``.

``weighted_key_value`` keeps the reference's validation (``language.py:379-396``,
same ``ValueError`` messages) and the dispatch of ``SpikeTimeMix.forward``
(``language.py:1028-1032``): bfloat16/float16 inputs go to the 16-bit-I/O
entry point (``weighted_key_value_triton_bf16io``), everything else to the
fp32 one.  The reference's third branch -- an eager
``associative_scan`` on CPU (``language.py:1033-1034``) -- has no counterpart
here: the ops run on the GPU only and raise on CPU tensors.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .wkv import weighted_key_value_hip, weighted_key_value_hip_bf16io


def validate_wkv_inputs(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> None:
    """``_validate_wkv_inputs`` of ``language.py:379-396``."""
    if key.shape != value.shape:
        raise ValueError(f"key and value must have the same shape; got {key.shape} and {value.shape}")
    if key.ndim != 3:
        raise ValueError(f"key and value must have shape [B, T, C]; got {key.shape}")
    if time_decay.shape != (key.shape[-1],):
        raise ValueError(f"time_decay must have shape [{key.shape[-1]}]; got {time_decay.shape}")
    if time_first.shape != (key.shape[-1],):
        raise ValueError(f"time_first must have shape [{key.shape[-1]}]; got {time_first.shape}")


def weighted_key_value(key: Tensor, value: Tensor, time_decay: Tensor, time_first: Tensor) -> Tensor:
    """RWKV WKV recurrence on ``[B, T, C]`` inputs (validated), HIP only."""
    validate_wkv_inputs(key, value, time_decay, time_first)
    if key.dtype in (torch.bfloat16, torch.float16):
        return weighted_key_value_hip_bf16io(key, value, time_decay, time_first)
    return weighted_key_value_hip(key, value, time_decay, time_first)
