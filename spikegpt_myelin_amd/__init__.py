"""MI355X (gfx950) WKV time-mixing recurrence for SpikeGPT.

Importing the package registers the ``myelin::`` custom ops backed by the HIP
library ``libwkv_hip.so`` (built in-tree by ``python -m
spikegpt_myelin_amd.build``):

* ``myelin::wkv_forward`` / ``myelin::wkv_backward`` (fp32 I/O) and
  ``myelin::wkv_forward_bf16io`` / ``myelin::wkv_backward_bf16io`` (16-bit
  I/O) -- the reference's op names and schemas;
* ``myelin::wkv_decode_step`` -- one-token WKV state update for generation;
* ``myelin::wkv7_forward`` / ``myelin::wkv7_backward`` -- RWKV-7 DPLR
  recurrence (the forward is differentiable);
* ``myelin::lif_sequence_forward`` / ``myelin::lif_sequence_backward`` -- the
  sequence LIF spiking activation (differentiable);
* ``myelin::token_shift_mix`` / ``myelin::token_shift_mix_backward`` -- the
  fused token-shift mixing that feeds the block projections (differentiable).

:mod:`spikegpt_myelin_amd.model` holds the SpikeGPT model built on them;
:mod:`spikegpt_myelin_amd.generation` its recurrent one-token step (the fused
block-step kernels, optionally captured in a HIP graph) and
:mod:`spikegpt_myelin_amd.checkpoint` the reference's checkpoint format
(``myelin.spike_language_checkpoint.v1``) and vocabularies.
"""

from .decode import initial_wkv_state, wkv_decode_step
from .language import validate_wkv_inputs, weighted_key_value
from .gates import relu_square, sigmoid_gate
from .lif import atan_surrogate, lif_sequence
from .splitk import split_k_sum
from .timemix import token_shift_mix
from .wkv import (
    weighted_key_value_gated,
    weighted_key_value_hip,
    weighted_key_value_hip_bf16io,
    weighted_key_value_triton,
    weighted_key_value_triton_bf16io,
)
from .wkv7 import wkv7_backward, wkv7_forward

__all__ = [
    "atan_surrogate",
    "initial_wkv_state",
    "lif_sequence",
    "relu_square",
    "sigmoid_gate",
    "split_k_sum",
    "token_shift_mix",
    "validate_wkv_inputs",
    "weighted_key_value",
    "weighted_key_value_gated",
    "weighted_key_value_hip",
    "weighted_key_value_hip_bf16io",
    "weighted_key_value_triton",
    "weighted_key_value_triton_bf16io",
    "wkv7_backward",
    "wkv7_forward",
    "wkv_decode_step",
]
