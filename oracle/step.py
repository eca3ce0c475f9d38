"""CPU oracle for SpikeGPT's recurrent one-token step (test infrastructure).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` (never by the product
package).  Restates, in eager fp32 PyTorch on the CPU, over a model's
``state_dict`` (the reference's parameter names):

* :func:`lif_step` -- ``SpikingSequenceLIF.step`` (``src/spikegpt/language.py:813-840``);
* :func:`time_mix_step` -- ``SpikeTimeMix.step`` (``:989-1012``), its WKV part
  being :func:`oracle.wkv4.decode_step`;
* :func:`channel_mix_step` -- ``SpikeChannelMix.step`` (``:1174-1188``);
* :func:`block_step` -- ``SpikeGPTBlock.step`` (``:1301-1335``);
* :func:`model_forward_step` -- ``SpikeLanguageModel.forward_step`` (``:1434-1453``);
* :func:`model_sequence_logits` -- ``SpikeLanguageModel.forward`` (``:1455-1467``)
  with ``SpikeGPTBlock.forward`` (``:1337-1360``), the WKV of
  :func:`oracle.wkv4.wkv_loop` and the LIF of :func:`oracle.lif.lif_loop`.

Pinning (``tests/test_oracle_step.py``): the reference's own check
(``tests/test_language.py:437-459``) -- stepping a model token by token gives
the logits of the sequence forward at every position, with the LIF threshold
at 0 so that spikes occur -- relates the step functions to the sequence forward,
whose recurrences are pinned independently (``tests/test_oracle_wkv4.py``,
``tests/test_oracle_lif.py``).  A dropped state update, a wrong mixing order
or a missing reset fails it.  The spiking embedding's hard spike is
``[slope * e >= 0]`` (``:1386-1394``), as in :mod:`oracle.lif`.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import Tensor

from . import lif as L
from . import timemix as TM
from . import wkv4 as W

__all__ = ["StepConfig", "lif_step", "time_mix_step", "channel_mix_step", "block_step",
           "initial_state", "model_forward_step", "model_sequence_logits"]


@dataclass(frozen=True)
class StepConfig:
    """The ``SpikeGPTConfig`` fields the step reads (``language.py:234-256``)."""

    n_layer: int
    n_embd: int
    lif_tau: float = 2.0
    lif_threshold: float = 1.0
    lif_reset: float = 0.0
    surrogate_slope: float = 2.0
    spike_embedding: bool = True
    spiking: bool = True

    @classmethod
    def of(cls, config) -> "StepConfig":
        return cls(**{k: getattr(config, k) for k in cls.__dataclass_fields__})


def _ln(sd: dict, name: str, x: Tensor) -> Tensor:
    return F.layer_norm(x, (x.shape[-1],), sd[f"{name}.weight"], sd[f"{name}.bias"], 1e-5)


def _linear(sd: dict, name: str, x: Tensor) -> Tensor:
    return x @ sd[f"{name}.weight"].t()


def lif_step(x: Tensor, membrane: Tensor, cfg: StepConfig) -> tuple[Tensor, Tensor]:
    """``language.py:830-840`` (identity when ``spiking`` is off, ``:1219-1222``)."""
    if not cfg.spiking:
        return x, membrane
    decay = 1.0 - 1.0 / cfg.lif_tau
    membrane = membrane * decay + x
    spike = (cfg.surrogate_slope * (membrane - cfg.lif_threshold) >= 0).to(x.dtype)
    membrane = membrane * (1.0 - spike) + cfg.lif_reset * spike
    return spike, membrane


def time_mix_step(sd: dict, p: str, x: Tensor, st: dict) -> Tensor:
    """``language.py:989-1012``; updates ``st`` (previous, num, den, log_scale)."""
    prev = st["time_previous"]
    mixed = {}
    for n in ("k", "v", "r"):
        mu = sd[f"{p}.time_mix_{n}"][0, 0]
        mixed[n] = x * mu + prev * (1.0 - mu)
    key = _linear(sd, f"{p}.key", mixed["k"])
    value = _linear(sd, f"{p}.value", mixed["v"])
    receptance = torch.sigmoid(_linear(sd, f"{p}.receptance", mixed["r"]))
    y, st["numerator"], st["denominator"], st["log_scale"] = W.decode_step(
        key, value, sd[f"{p}.time_decay"], sd[f"{p}.time_first"], st["numerator"],
        st["denominator"], st["log_scale"])
    st["time_previous"] = x
    return _linear(sd, f"{p}.output", receptance * y)


def channel_mix_step(sd: dict, p: str, x: Tensor, st: dict) -> Tensor:
    """``language.py:1174-1188``; updates ``st["channel_previous"]``."""
    prev = st["channel_previous"]
    mu_k, mu_r = sd[f"{p}.time_mix_k"][0, 0], sd[f"{p}.time_mix_r"][0, 0]
    key = torch.relu(_linear(sd, f"{p}.key", x * mu_k + prev * (1.0 - mu_k))).square()
    value = _linear(sd, f"{p}.value", key)
    receptance = torch.sigmoid(_linear(sd, f"{p}.receptance", x * mu_r + prev * (1.0 - mu_r)))
    st["channel_previous"] = x
    return receptance * value


def block_step(sd: dict, cfg: StepConfig, layer: int, x: Tensor, st: dict) -> Tensor:
    """``language.py:1301-1335`` (``rwkv`` time mix, eval: no dropout)."""
    p = f"blocks.{layer}"
    residual = _ln(sd, f"{p}.ln0", x) if layer == 0 else x
    mixed = time_mix_step(sd, f"{p}.att", _ln(sd, f"{p}.ln1", residual), st)
    spike1, st["lif1_membrane"] = lif_step(mixed, st["lif1_membrane"], cfg)
    residual = residual + spike1
    channel = channel_mix_step(sd, f"{p}.ffn", _ln(sd, f"{p}.ln2", residual), st)
    spike2, st["lif2_membrane"] = lif_step(channel, st["lif2_membrane"], cfg)
    return residual + spike2


def initial_state(cfg: StepConfig, batch: int) -> list[dict]:
    """Per-layer state (``language.py:957-975, 1160-1171, 797-811``)."""
    out = []
    for _ in range(cfg.n_layer):
        z = lambda: torch.zeros(batch, cfg.n_embd)  # noqa: E731
        num, den, ls = W.initial_decode_state(batch, cfg.n_embd)
        out.append({"time_previous": z(), "numerator": num, "denominator": den, "log_scale": ls,
                    "channel_previous": z(), "lif1_membrane": z(), "lif2_membrane": z()})
    return out


def _embed(sd: dict, cfg: StepConfig, ids: Tensor) -> Tensor:
    e = sd["embedding.weight"][ids]
    if not cfg.spike_embedding:
        return e
    return (cfg.surrogate_slope * e >= 0).to(e.dtype)


def model_forward_step(sd: dict, cfg: StepConfig, ids: Tensor,
                       state: list[dict]) -> tuple[Tensor, list[dict]]:
    """``language.py:1434-1453``: logits [B, V] and the new state (copied)."""
    state = [dict(s) for s in state]
    x = _embed(sd, cfg, ids)
    for layer in range(cfg.n_layer):
        x = block_step(sd, cfg, layer, x, state[layer])
    return _linear(sd, "head", _ln(sd, "ln_out", x)), state


def model_sequence_logits(sd: dict, cfg: StepConfig, ids: Tensor) -> Tensor:
    """``language.py:1455-1467`` forward (eval) on [B, T] ids -> [B, T, V]."""
    x = _embed(sd, cfg, ids)

    def lif(t: Tensor) -> Tensor:
        if not cfg.spiking:
            return t
        return L.lif_loop(t, tau=cfg.lif_tau, threshold=cfg.lif_threshold, reset=cfg.lif_reset,
                          slope=cfg.surrogate_slope)

    for layer in range(cfg.n_layer):
        p = f"blocks.{layer}"
        if layer == 0:
            x = _ln(sd, f"{p}.ln0", x)
        h = _ln(sd, f"{p}.ln1", x)
        k_in, v_in, r_in = (TM.mix_with_previous(h, sd[f"{p}.att.time_mix_{n}"])
                            for n in ("k", "v", "r"))
        wkv = W.wkv_loop(_linear(sd, f"{p}.att.key", k_in), _linear(sd, f"{p}.att.value", v_in),
                         sd[f"{p}.att.time_decay"], sd[f"{p}.att.time_first"])
        att = _linear(sd, f"{p}.att.output",
                      torch.sigmoid(_linear(sd, f"{p}.att.receptance", r_in)) * wkv)
        x = x + lif(att)
        h = _ln(sd, f"{p}.ln2", x)
        k_in = TM.mix_with_previous(h, sd[f"{p}.ffn.time_mix_k"])
        r_in = TM.mix_with_previous(h, sd[f"{p}.ffn.time_mix_r"])
        key = torch.relu(_linear(sd, f"{p}.ffn.key", k_in)).square()
        ffn = torch.sigmoid(_linear(sd, f"{p}.ffn.receptance", r_in)) * _linear(
            sd, f"{p}.ffn.value", key)
        x = x + lif(ffn)
    return _linear(sd, "head", _ln(sd, "ln_out", x))
