"""The fused one-token block step (block_step_row / block_step_wkv through
spikegpt_myelin_amd.generation) against the CPU oracle of the reference's
eager step, against the model's own sequence forward (the reference's check,
tests/test_language.py:437-459), and the captured HIP graph against the
eager step on every replay."""

from __future__ import annotations

import pytest
import torch

from oracle import step as S
from spikegpt_myelin_amd import generation as G
from spikegpt_myelin_amd.model import SpikeGPTConfig, SpikeLanguageModel

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda", 0)


def _model(embd: int, *, layers=2, vocab=50, seed=0, scale=30.0, threshold=0.0, ctx=16,
           spiking=True):
    torch.manual_seed(seed)
    cfg = SpikeGPTConfig(vocab_size=vocab, context_length=ctx, n_layer=layers, n_embd=embd,
                         dropout=0.0, lif_threshold=threshold, spiking=spiking)
    model = SpikeLanguageModel(cfg)
    with torch.no_grad():
        for name, p in model.named_parameters():
            # Larger projections than the init so that both LIFs spike and reset.
            if name.endswith(("key.weight", "value.weight", "receptance.weight",
                              "output.weight")):
                p.mul_(scale)
    return model.to(DEV).eval()


def _cpu_sd(model):
    return {k: v.detach().float().cpu() for k, v in model.state_dict().items()}


def _oracle_state_slots(state):
    return [torch.stack([s[n] for n in G.SLOTS]) for s in state]


@pytest.mark.parametrize("embd,spiking", [(96, True), (768, True), (96, False)])
def test_forward_step_matches_oracle(embd, spiking):
    model = _model(embd, spiking=spiking)
    sd, sc = _cpu_sd(model), S.StepConfig.of(model.config)
    B, T = 4, 6
    ids = torch.randint(0, model.config.vocab_size, (B, T),
                        generator=torch.Generator().manual_seed(1))
    state = model.initial_state(batch_size=B)
    ostate = S.initial_state(sc, B)
    print(f"forward_step vs oracle: C={embd} B={B} T={T}", flush=True)
    for t in range(T):
        logits, state = model.forward_step(ids[:, t].to(DEV), state)
        ologits, ostate = S.model_forward_step(sd, sc, ids[:, t], ostate)
        torch.testing.assert_close(logits.cpu(), ologits, atol=2e-4, rtol=1e-4)
    got = state.packed.cpu()
    for layer, want in enumerate(_oracle_state_slots(ostate)):
        # The state accumulates fp32 projections (K up to 4C) summed in another
        # order than the CPU's; the membranes reach a few units.
        torch.testing.assert_close(got[layer], want, atol=1e-3, rtol=1e-3)
    assert bool((got[:, G.SLOTS.index("lif1_membrane")] != 0).any()) == spiking


def test_step_matches_hip_sequence_forward():
    model = _model(128, layers=3)
    B, T = 3, 12
    ids = torch.randint(0, model.config.vocab_size, (B, T), device=DEV,
                        generator=torch.Generator(device=DEV).manual_seed(2))
    with torch.no_grad():
        full = model(ids)
    state = model.initial_state(batch_size=B)
    steps = []
    for t in range(T):
        logits, state = model.forward_step(ids[:, t], state)
        steps.append(logits)
    torch.testing.assert_close(torch.stack(steps, 1), full, atol=5e-4, rtol=1e-4)


def test_forward_step_leaves_input_state_and_accepts_unpacked_state():
    model = _model(96)
    ids = torch.tensor([3, 7], device=DEV)
    s0 = model.initial_state(batch_size=2)
    l1, s1 = model.forward_step(ids, s0)
    before = s1.packed.clone()
    # A hand-built state (separate tensors, no packed buffer) gives the same step.
    loose = G.SpikeLanguageModelState(blocks=tuple(
        G.SpikeGPTBlockState(
            time_mix=G.SpikeTimeMixState(*(t.clone() for t in (
                b.time_mix.previous, b.time_mix.numerator, b.time_mix.denominator,
                b.time_mix.log_scale))),
            ffn_pre=None,
            channel_mix=G.SpikeChannelMixState(b.channel_mix.previous.clone()),
            lif1=G.SpikingSequenceLIFState(b.lif1.membrane.clone()),
            lif2=G.SpikingSequenceLIFState(b.lif2.membrane.clone()))
        for b in s1.blocks))
    l2a, s2a = model.forward_step(ids, s1)
    l2b, s2b = model.forward_step(ids, loose)
    assert torch.equal(s1.packed, before)
    torch.testing.assert_close(l2b, l2a, atol=1e-6, rtol=1e-6)
    torch.testing.assert_close(s2b.packed, s2a.packed, atol=1e-6, rtol=1e-6)
    with pytest.raises(IndexError):
        model.forward_step(torch.tensor([0, 50], device=DEV), s1)


@pytest.mark.parametrize("layer", [0, 1])
def test_block_step_matches_oracle(layer):
    model = _model(96)
    sd, sc = _cpu_sd(model), S.StepConfig.of(model.config)
    block = model.blocks[layer]
    B = 5
    x = torch.randn(B, 96, generator=torch.Generator().manual_seed(4))
    st = block.initial_state(batch_size=B)
    ost = S.initial_state(sc, 1)[0]
    for t in range(3):
        xt = x * (t + 1)
        y, st = block.step(xt.to(DEV), st)
        oy = S.block_step(sd, sc, layer, xt, ost)
        torch.testing.assert_close(y.cpu(), oy, atol=2e-4, rtol=1e-4)
    torch.testing.assert_close(st.lif2.membrane.cpu(), ost["lif2_membrane"], atol=2e-4, rtol=1e-4)


def test_step_graph_replays_match_eager():
    model = _model(256, layers=2)
    B = 8
    g = G.StepGraph(model, B)
    state = model.initial_state(batch_size=B)
    gen = torch.Generator(device=DEV).manual_seed(5)
    for t in range(6):
        ids = torch.randint(0, model.config.vocab_size, (B,), device=DEV, generator=gen)
        glog = g.step(ids).clone()
        # Eager work and a synchronisation between replays.
        elog, state = model.forward_step(ids, state)
        torch.cuda.synchronize()
        torch.testing.assert_close(glog, elog, atol=1e-5, rtol=1e-5)
    torch.testing.assert_close(g.state().packed, state.packed, atol=1e-5, rtol=1e-5)
    g.reset()
    ids = torch.arange(B, device=DEV) % model.config.vocab_size
    l0, _ = model.forward_step(ids, model.initial_state(batch_size=B))
    torch.testing.assert_close(g.step(ids), l0, atol=1e-5, rtol=1e-5)


def test_generate_cached_graph_eager_and_uncached_agree():
    model = _model(64, layers=2, ctx=12, vocab=20)
    ids = torch.randint(0, 20, (2, 4), device=DEV, generator=torch.Generator(device=DEV).manual_seed(6))
    a = model.generate(ids, max_new_tokens=6, sampling="greedy")
    b = model.generate(ids, max_new_tokens=6, sampling="greedy", use_graph=False)
    c = model.generate(ids, max_new_tokens=6, sampling="greedy", use_cache=False)
    assert a.shape == (2, 10) and torch.equal(a[:, :4], ids)
    assert torch.equal(a, b) and torch.equal(a, c)
    streamed = torch.cat(list(model.generate_stream(ids, max_new_tokens=6, sampling="greedy")), 1)
    assert torch.equal(streamed, a[:, 4:])


def test_checkpoint_round_trip_runs_the_same_model(tmp_path):
    from spikegpt_myelin_amd import checkpoint as K

    model = _model(64, layers=2, ctx=12, vocab=20)
    vocab = K.CharacterVocabulary(tokens=tuple(chr(97 + i) for i in range(20)))
    path = tmp_path / "m.pt"
    K.save_spike_language_checkpoint(path, model, vocab, metadata={"note": "gpu"})
    ck = K.load_spike_language_checkpoint(path, map_location="cpu")
    loaded = ck.model.to(DEV).eval()
    ids = vocab.encode("abcdefgh").view(2, 4).to(DEV)
    with torch.no_grad():
        torch.testing.assert_close(loaded(ids), model(ids), atol=0, rtol=0)
    assert torch.equal(loaded.generate(ids, max_new_tokens=4, sampling="greedy"),
                       model.generate(ids, max_new_tokens=4, sampling="greedy"))
