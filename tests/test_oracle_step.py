"""Pins the CPU oracle of the recurrent step (oracle/step.py).

The reference's own check (tests/test_language.py:437-459): a model stepped
token by token from the initial state gives the sequence forward's logits at
every position, with the LIF threshold at 0 so that both LIFs spike.  The
sequence forward uses the independently pinned WKV loop and LIF loop.
"""

from __future__ import annotations

import pytest
import torch

from oracle import step as S
from spikegpt_myelin_amd.model import SpikeGPTConfig, SpikeLanguageModel


def _model_sd(seed: int, *, vocab=11, layers=2, embd=16, threshold=0.0, spiking=True,
              spike_embedding=True, scale=30.0):
    torch.manual_seed(seed)
    cfg = SpikeGPTConfig(vocab_size=vocab, context_length=8, n_layer=layers, n_embd=embd,
                         dropout=0.0, lif_threshold=threshold, spiking=spiking,
                         spike_embedding=spike_embedding)
    model = SpikeLanguageModel(cfg)
    sd = {k: v.detach().clone() for k, v in model.state_dict().items()}
    for k in sd:
        # Larger projections than the init so that spikes and resets happen.
        if k.endswith(("key.weight", "value.weight", "receptance.weight", "output.weight")):
            sd[k] *= scale
    return cfg, sd


@pytest.mark.parametrize("spiking,spike_embedding", [(True, True), (False, True), (True, False)])
def test_step_matches_sequence_forward(spiking, spike_embedding):
    cfg, sd = _model_sd(0, spiking=spiking, spike_embedding=spike_embedding)
    sc = S.StepConfig.of(cfg)
    ids = torch.randint(0, cfg.vocab_size, (3, 8), generator=torch.Generator().manual_seed(1))
    full = S.model_sequence_logits(sd, sc, ids)
    state = S.initial_state(sc, ids.shape[0])
    steps = []
    for t in range(ids.shape[1]):
        logits, state = S.model_forward_step(sd, sc, ids[:, t], state)
        steps.append(logits)
    torch.testing.assert_close(torch.stack(steps, 1), full, atol=1e-5, rtol=1e-5)
    if spiking:
        assert any(bool((s["lif1_membrane"] != 0).any()) for s in state)


def test_lif_step_spikes_and_resets():
    cfg = S.StepConfig(n_layer=1, n_embd=2, lif_tau=2.0, lif_threshold=1.0, lif_reset=0.25)
    m = torch.zeros(1, 2)
    x = torch.tensor([[0.75, 2.0]])
    s, m = S.lif_step(x, m, cfg)
    assert s.tolist() == [[0.0, 1.0]] and m.tolist() == [[0.75, 0.25]]
    s, m = S.lif_step(x, m, cfg)  # 0.375 + 0.75 = 1.125 >= 1 -> spike, reset
    assert s.tolist() == [[1.0, 1.0]] and m.tolist() == [[0.25, 0.25]]


def test_oracle_step_catches_a_dropped_state_update():
    cfg, sd = _model_sd(2)
    sc = S.StepConfig.of(cfg)
    ids = torch.randint(0, cfg.vocab_size, (2, 6), generator=torch.Generator().manual_seed(3))
    full = S.model_sequence_logits(sd, sc, ids)
    state = S.initial_state(sc, 2)
    steps = []
    for t in range(6):
        logits, new = S.model_forward_step(sd, sc, ids[:, t], state)
        for s_new, s_old in zip(new, state):
            s_new["channel_previous"] = s_old["channel_previous"]  # planted mistake
        state = new
        steps.append(logits)
    assert not torch.allclose(torch.stack(steps, 1), full, atol=1e-4)
