"""Single-token WKV decode step as a custom op (``myelin::wkv_decode_step``).

The reference advances the WKV state of ``SpikeTimeMix.step``
(``src/spikegpt/language.py:977-1013``) with ~20 eager element-wise torch
launches per layer and has no op for it.  This op does the same arithmetic
(``language.py:989-1012``) in one HIP launch:

``myelin::wkv_decode_step(Tensor key, Tensor value, Tensor time_decay,
Tensor time_first, Tensor numerator, Tensor denominator, Tensor log_scale)
-> (Tensor y, Tensor numerator, Tensor denominator, Tensor log_scale)``

``key``/``value`` are ``[B, C]`` (float32, bfloat16 or float16); the state is
float32 ``[B, C]`` in the reference's natural-log units (``SpikeTimeMixState``,
``language.py:182-189``; initial state: zeros and ``finfo(float32).min``,
``language.py:957-975``).  Functional: returns a new state.
"""

from __future__ import annotations

import torch
from torch import Tensor

from . import _lib


@torch.library.custom_op("myelin::wkv_decode_step", mutates_args=())
def _wkv_decode_step_op(
    key: Tensor,
    value: Tensor,
    time_decay: Tensor,
    time_first: Tensor,
    numerator: Tensor,
    denominator: Tensor,
    log_scale: Tensor,
) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    _lib.require_gpu(key, value, time_decay, time_first, numerator, denominator, log_scale)
    if key.ndim != 2 or key.shape != value.shape:
        raise ValueError(f"key and value must have the same shape [B, C]; got {key.shape} and {value.shape}")
    b, c = key.shape
    for name, s in (("numerator", numerator), ("denominator", denominator), ("log_scale", log_scale)):
        if s.shape != key.shape:
            raise ValueError(f"{name} must have shape {tuple(key.shape)}; got {tuple(s.shape)}")
    if time_decay.shape != (c,) or time_first.shape != (c,):
        raise ValueError(f"time_decay and time_first must have shape [{c}]")
    if key.dtype == value.dtype and key.dtype in (torch.float32, torch.bfloat16, torch.float16):
        k, v = _lib.aligned(key), _lib.aligned(value)
    else:
        k, v = _lib.aligned(key.float()), _lib.aligned(value.float())
    td = _lib.aligned(time_decay.float())
    tf = _lib.aligned(time_first.float())
    num = _lib.aligned(numerator.float())
    den = _lib.aligned(denominator.float())
    ls = _lib.aligned(log_scale.float())
    y = torch.empty_like(k)
    num_o = torch.empty_like(num)
    den_o = torch.empty_like(den)
    ls_o = torch.empty_like(ls)
    lib = _lib.load()
    rc = lib.wkv4_decode_step(
        k.data_ptr(), v.data_ptr(), td.data_ptr(), tf.data_ptr(),
        num.data_ptr(), den.data_ptr(), ls.data_ptr(), y.data_ptr(),
        num_o.data_ptr(), den_o.data_ptr(), ls_o.data_ptr(), b, c,
        _lib.dtype_code(k.dtype), _lib.stream_of(k),
    )
    _lib.check(rc, "wkv4_decode_step")
    if y.dtype != key.dtype:
        y = y.to(key.dtype)
    return y, num_o, den_o, ls_o


@_wkv_decode_step_op.register_fake
def _(key, value, time_decay, time_first, numerator, denominator, log_scale):
    f32 = {"dtype": torch.float32, "device": key.device}
    return (
        torch.empty_like(key),
        torch.empty(key.shape, **f32),
        torch.empty(key.shape, **f32),
        torch.empty(key.shape, **f32),
    )


def wkv_decode_step(key, value, time_decay, time_first, numerator, denominator, log_scale):
    """One decode step; returns ``(y, numerator, denominator, log_scale)``."""
    return torch.ops.myelin.wkv_decode_step(
        key, value, time_decay, time_first, numerator, denominator, log_scale
    )


def initial_wkv_state(batch: int, channels: int, device) -> tuple[Tensor, Tensor, Tensor]:
    """Empty WKV state (``language.py:957-975``): zeros, zeros, ``finfo.min``."""
    z = torch.zeros((batch, channels), dtype=torch.float32, device=device)
    return z, z.clone(), torch.full_like(z, torch.finfo(torch.float32).min)
