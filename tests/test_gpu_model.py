"""End-model parity: the SpikeGPT model on the HIP WKV, LIF and token-shift
kernels against the same model (identical weights and batch) with all three
replaced by the CPU oracle's formulations.

Bars: loss within 0.2 % relative (the end-model bar), under bf16 autocast
and in fp32, where the loss is not chaotic (the measured noise floor is given
at the 41M-depth test); in the firing regime of the 41M depth, each layer's
halves teacher-forced against the oracle (bars at TEACHER_FORCED_TOL);
parameter gradients in fp32 with cosine similarity > 0.999 (the spike
threshold makes gradients discontinuous, so an elementwise bound would test
rounding luck, not the kernels).
"""

from __future__ import annotations

import copy

import pytest
import torch

from oracle import lif as L
from oracle import timemix as TM
from oracle import wkv4 as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _model(n_layer=2, n_embd=128, vocab=256, ctx=64, seed=0):
    from spikegpt_myelin_amd.model import SpikeGPTConfig, SpikeLanguageModel

    torch.manual_seed(seed)
    cfg = SpikeGPTConfig(vocab_size=vocab, context_length=ctx, n_layer=n_layer, n_embd=n_embd,
                         dropout=0.0)
    return SpikeLanguageModel(cfg)


def _batch(b, t, vocab=256, seed=1):
    g = torch.Generator().manual_seed(seed)
    ids = torch.randint(0, vocab, (b, t + 1), generator=g)
    return ids[:, :-1].contiguous(), ids[:, 1:].contiguous()


def _oracle_wkv(key, value, time_decay, time_first):
    # The oracle runs on the CPU; autograd carries gradients across the copies.
    y = O.wkv_forward_op(key.cpu(), value.cpu(), time_decay.cpu(), time_first.cpu())
    return y.to(key.device)


def _oracle_lif(x, *, tau, threshold, reset, surrogate_slope):
    return L.lif_loop(x.cpu(), tau, threshold, reset, surrogate_slope).to(x.device)


def _oracle_mix(x, mixes):
    od = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else None
    with torch.autocast("cuda", enabled=False):
        outs = TM.shift_mix(x.float().cpu(), mixes.float().cpu(), od)
    return [o.to(x.device) for o in outs]


def _oracle_ln(x, norm):
    # torch's layer norm in fp32, as autocast runs it
    return torch.nn.functional.layer_norm(x.float(), norm.normalized_shape, norm.weight,
                                          norm.bias, norm.eps)


def _patch_oracle(mp, wkv=_oracle_wkv):
    """Route the model's WKV, LIF, token-shift mix, fused layer norm + mix and
    gates through the oracle's formulations (``wkv``: the WKV to use)."""
    import spikegpt_myelin_amd.model as M

    mp.setattr(M, "weighted_key_value_gated",
               lambda k, v, td, tf, r: torch.sigmoid(r) * wkv(k, v, td, tf))
    mp.setattr(M, "lif_sequence", _oracle_lif)
    mp.setattr(M, "lif_residual", lambda residual, x, **kw: residual + _oracle_lif(x, **kw))
    mp.setattr(M, "token_shift_mix", _oracle_mix)
    mp.setattr(M, "layer_norm_shift_mix", lambda x, norm, mix: _oracle_mix(_oracle_ln(x, norm), mix))
    mp.setattr(M, "layer_norm_shift_mix_fork",
               lambda x, norm, mix: [*_oracle_mix(_oracle_ln(x, norm), mix), x])
    mp.setattr(M, "relu_square", lambda x: torch.relu(x).square())
    mp.setattr(M, "sigmoid_gate", lambda r, x: torch.sigmoid(r) * x)


def _loss(model, ids, tgt, autocast, oracle, monkeypatch):
    with monkeypatch.context() as mp:
        if oracle:
            _patch_oracle(mp)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            loss, _ = model(ids, tgt)
    return loss


@pytest.mark.parametrize("autocast", [True, False])
def test_loss_matches_oracle_recurrences(autocast, monkeypatch):
    model = _model().to(DEV)
    # Perturb the small random init so that spikes actually fire.
    with torch.no_grad():
        for p in model.parameters():
            if p.ndim == 2:
                p.mul_(8.0)
    ids, tgt = (x.to(DEV) for x in _batch(4, 64))
    with torch.no_grad():
        hip = _loss(model, ids, tgt, autocast, False, monkeypatch)
        ref = _loss(model, ids, tgt, autocast, True, monkeypatch)
    rel = abs(float(hip) - float(ref)) / abs(float(ref))
    assert rel < 2e-3, f"loss {float(hip):.6f} vs oracle {float(ref):.6f} (rel {rel:.2e})"


@pytest.mark.parametrize("autocast,scale", [(True, 1.0), (False, 1.0), (True, 4.0), (False, 4.0)])
def test_loss_matches_oracle_recurrences_at_41m_depth(autocast, scale, monkeypatch):
    # The 41M configuration itself: 12 layers, 512 channels, byte vocabulary,
    # random init (scale 1), and with the projection weights scaled by 4 so
    # that the time mixes' outputs approach the LIF threshold; B=2, T=512
    # keeps the CPU oracle's twelve layers of loops within seconds.  Larger
    # scales put the 12-layer spiking model in a regime where the loss is not
    # a parity measure: at scale 8, the oracle model with its layer norm
    # summed in fp64 instead of fp32 (no kernel involved) moves its own loss
    # by 2-3e-3 under bf16 autocast, and a 2^-14 relative nudge of the WKV
    # output moves it by up to 5e-3 in fp32 (spikes near the threshold flip
    # and the flips compound over the layers); at scale 4 both stay below
    # 2.5e-4.  The firing regime is compared layer by layer, teacher-forced,
    # in test_layers_match_oracle_teacher_forced_at_41m_depth.
    model = _model(n_layer=12, n_embd=512, vocab=256, ctx=1024, seed=3).to(DEV)
    if scale != 1.0:
        with torch.no_grad():
            for p in model.parameters():
                if p.ndim == 2:
                    p.mul_(scale)
    ids, tgt = (x.to(DEV) for x in _batch(2, 512, seed=11))
    print(f"41M depth: autocast={autocast} scale={scale}", flush=True)
    with torch.no_grad():
        hip = _loss(model, ids, tgt, autocast, False, monkeypatch)
        ref = _loss(model, ids, tgt, autocast, True, monkeypatch)
    rel = abs(float(hip) - float(ref)) / abs(float(ref))
    print(f"41M depth loss {float(hip):.6f} vs oracle {float(ref):.6f} (rel {rel:.2e})")
    assert rel < 2e-3, f"loss {float(hip):.6f} vs oracle {float(ref):.6f} (rel {rel:.2e})"


def _time_mix_half(block, x):
    """The block's first half on ``x`` (model.py SpikeGPTBlock.forward): the
    time mix's output before its LIF, and the residual with the spikes added.
    Every op is looked up on the model module, so patches apply."""
    import spikegpt_myelin_amd.model as M

    residual = block.ln0(x) if block.ln0 is not None else x
    *mixed, residual = M.layer_norm_shift_mix_fork(residual, block.ln1, block.att.mixes())
    pre = block.att.project(*mixed)
    return pre, M._add_lif(residual, block.lif1, pre)


def _channel_mix_half(block, x):
    import spikegpt_myelin_amd.model as M

    *mixed, residual = M.layer_norm_shift_mix_fork(x, block.ln2, block.ffn.mixes())
    pre = block.ffn.project(*mixed)
    return pre, M._add_lif(residual, block.lif2, pre)


def _wkv_dropped_bonus(key, value, time_decay, time_first):
    # planted mistake: the current token's bonus e^(u + k) taken as e^k
    return _oracle_wkv(key, value, time_decay, torch.zeros_like(time_first))


def _wkv_decay_twice(key, value, time_decay, time_first):
    # planted mistake: the decay applied twice per step (w -> 2 w)
    return _oracle_wkv(key, value, time_decay + 0.6931471805599453, time_first)


def _teacher_forced(model, ids, autocast, wkv=_oracle_wkv):
    """Per layer: the oracle model's block input, then both halves on the HIP
    path and on the oracle path from the same oracle inputs.  Returns a list
    of (hip_att, ora_att, hip_att_out, ora_att_out, hip_ffn, ora_ffn,
    hip_out, ora_out) per layer."""
    out = []
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        x = model.embed_tokens(ids)
        for block in model.blocks:
            h_att, h_mid = _time_mix_half(block, x)
            with pytest.MonkeyPatch.context() as mp:
                _patch_oracle(mp, wkv)
                o_att, o_mid = _time_mix_half(block, x)
                o_ffn, o_out = _channel_mix_half(block, o_mid)
            h_ffn, h_out = _channel_mix_half(block, o_mid)
            out.append((h_att, o_att, h_mid, o_mid, h_ffn, o_ffn, h_out, o_out))
            x = o_out
    return out


def _normwise(got, ref):
    got, ref = got.double(), ref.double()
    return float((got - ref).norm() / ref.norm()) if float(ref.norm()) > 0 else float(got.norm())


# Bars of the teacher-forced comparison.  bf16 autocast: each half's output
# before its LIF within 2e-3 normwise and 2e-2 * max|ref| elementwise (measured
# on MI355X at most 4.8e-4 and 5.4e-3 over the twelve layers), at most 1e-3 of
# the spikes flipped (measured 3.8e-5: membranes within a bf16 rounding of the
# threshold).  fp32: 1e-5 normwise and elementwise relative to max|ref|
# (measured 1.1e-6 and 1.4e-6), at most 1e-4 of the spikes flipped (measured
# one in 524,288).  Planted mistakes in the oracle's WKV give 0.24-0.96
# normwise in every layer, so the time-mix bar is met by a margin of more than
# 100 against either.
TEACHER_FORCED_TOL = {True: (2e-3, 2e-2, 1e-3), False: (1e-5, 1e-5, 1e-4)}


@pytest.mark.parametrize("autocast", [True, False])
def test_layers_match_oracle_teacher_forced_at_41m_depth(autocast):
    # The firing regime of the 41M configuration (projection weights scaled
    # by 8: 17-22 % of the time mixes' and 37-39 % of the channel mixes'
    # outputs cross the LIF threshold), compared layer by layer with the
    # oracle model's own block input fed to both paths: each half's
    # continuous output before its LIF (the time mix carries the WKV
    # recurrence) and the spikes each LIF adds.  Teacher forcing keeps a
    # spike flipped in one layer from changing the next layer's input, which
    # is what makes the loss of this configuration chaotic (see the 41M-depth
    # loss test).
    norm_tol, max_tol, flip_tol = TEACHER_FORCED_TOL[autocast]
    model = _model(n_layer=12, n_embd=512, vocab=256, ctx=1024, seed=3).to(DEV)
    with torch.no_grad():
        for p in model.parameters():
            if p.ndim == 2:
                p.mul_(8.0)
    ids, _ = (x.to(DEV) for x in _batch(2, 512, seed=11))
    print(f"teacher-forced 41M depth autocast={autocast}", flush=True)
    layers = _teacher_forced(model, ids, autocast)
    for i, (h_att, o_att, h_mid, o_mid, h_ffn, o_ffn, h_out, o_out) in enumerate(layers):
        for half, got, ref, h_spk, o_spk in (("time mix", h_att, o_att, h_mid, o_mid),
                                             ("channel mix", h_ffn, o_ffn, h_out, o_out)):
            err = _normwise(got, ref)
            ref64 = ref.double()
            mx = float((got.double() - ref64).abs().max() / ref64.abs().max())
            flips = float(((h_spk - o_spk).abs() > 0.5).double().mean())
            fired = float((ref.float() >= 1.0).double().mean())
            print(f"layer {i:2d} {half}: normwise {err:.2e}, max {mx:.2e}, flips {flips:.2e}, "
                  f"over threshold {fired:.3f}")
            assert fired > 0.05, f"layer {i} {half}: the LIF hardly fires ({fired:.3f})"
            assert err < norm_tol, f"layer {i} {half}: normwise {err:.2e}"
            assert mx < max_tol, f"layer {i} {half}: max error / max|ref| {mx:.2e}"
            assert flips < flip_tol, f"layer {i} {half}: {flips:.2e} of the spikes flipped"
    # Power: the same comparison against an oracle with a planted mistake.
    for name, wkv in (("dropped bonus", _wkv_dropped_bonus), ("decay twice", _wkv_decay_twice)):
        bad = _teacher_forced(model, ids, autocast, wkv)
        errs = [_normwise(h[0], m[1]) for h, m in zip(layers, bad)]
        print(f"oracle with {name}: time mix normwise per layer " +
              " ".join(f"{e:.1e}" for e in errs))
        assert min(errs) > 50 * TEACHER_FORCED_TOL[True][0], f"{name}: {min(errs):.2e}"


def test_loss_matches_oracle_recurrences_at_216m_shape(monkeypatch):
    # The 216M-class architecture (language.py:297-298: 18 layers x 768,
    # GPT-2 BPE vocabulary 50277), random init, bf16 autocast; B=1, T=256.
    # At 768 channels the block takes the two-kernel layer norm + token shift
    # path (the fused kernel holds at most 512 channels per row).
    model = _model(n_layer=18, n_embd=768, vocab=50277, ctx=1024, seed=4).to(DEV)
    ids, tgt = (x.to(DEV) for x in _batch(1, 256, vocab=50277, seed=12))
    with torch.no_grad():
        hip = _loss(model, ids, tgt, True, False, monkeypatch)
        ref = _loss(model, ids, tgt, True, True, monkeypatch)
    rel = abs(float(hip) - float(ref)) / abs(float(ref))
    print(f"216M shape loss {float(hip):.6f} vs oracle {float(ref):.6f} (rel {rel:.2e})")
    assert rel < 2e-3, f"loss {float(hip):.6f} vs oracle {float(ref):.6f} (rel {rel:.2e})"


def test_gradient_checkpointing_gives_the_same_loss_and_gradients():
    # language.py:1396-1404: with checkpointing on, each block is recomputed
    # in the backward; the kernels are deterministic, so every value matches.
    model = _model(n_layer=3, n_embd=128).to(DEV)
    twin = copy.deepcopy(model)
    twin.set_gradient_checkpointing(True)
    ids, tgt = (x.to(DEV) for x in _batch(4, 64, seed=13))
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss_a, _ = model(ids, tgt)
        loss_b, _ = twin(ids, tgt)
    loss_a.backward()
    loss_b.backward()
    assert torch.equal(loss_a, loss_b)
    for (name, p), q in zip(model.named_parameters(), twin.parameters()):
        assert torch.equal(p.grad, q.grad), name


def test_gradients_match_oracle_recurrences(monkeypatch):
    model = _model(n_layer=2, n_embd=64).to(DEV)
    with torch.no_grad():
        for p in model.parameters():
            if p.ndim == 2:
                p.mul_(8.0)
    twin = copy.deepcopy(model)
    ids, tgt = (x.to(DEV) for x in _batch(2, 48, seed=5))
    _loss(model, ids, tgt, False, False, monkeypatch).backward()
    _loss(twin, ids, tgt, False, True, monkeypatch).backward()
    for (name, p), q in zip(model.named_parameters(), twin.parameters()):
        a, b = p.grad.double().flatten(), q.grad.double().flatten()
        if float(b.norm()) == 0.0:
            assert float(a.norm()) == 0.0, name
            continue
        cos = float(a @ b / (a.norm() * b.norm()))
        assert cos > 0.999, f"{name}: cosine {cos:.6f}"


def test_training_steps_reduce_the_loss():
    model = _model(n_layer=2, n_embd=128).to(DEV)
    opt = torch.optim.AdamW(model.parameters(), lr=3e-3, fused=True)
    ids, tgt = (x.to(DEV) for x in _batch(8, 64, seed=9))
    losses = []
    for _ in range(30):
        opt.zero_grad(set_to_none=True)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss, _ = model(ids, tgt)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(model.parameters(), 1.0)
        opt.step()
        losses.append(float(loss))
    assert all(torch.isfinite(torch.tensor(losses)))
    assert losses[-1] < losses[0] - 0.5, losses


@pytest.mark.parametrize("autocast", [True, False])
def test_split_k_linear_matches_linear(autocast):
    from spikegpt_myelin_amd.model import SplitKLinear

    torch.manual_seed(3)
    ref = torch.nn.Linear(512, 384, bias=False).to(DEV)
    lin = SplitKLinear(512, 384, bias=False).to(DEV)
    lin.load_state_dict(ref.state_dict())
    x = torch.randn(4, 8192, 512, device=DEV)  # 32768 rows: 16 slices of 2048
    gy = torch.randn(4, 8192, 384, device=DEV)
    outs = []
    for m in (ref, lin):
        xi = x.clone().requires_grad_(True)
        with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
            y = m(xi)
        y.backward(gy.to(y.dtype))
        outs.append((y.detach().float(), xi.grad.float(), m.weight.grad.float()))
    (y0, gx0, gw0), (y1, gx1, gw1) = outs
    # Forward and input gradient run the same GEMMs; the weight gradient sums
    # 16 fp32 slices instead of one fp32 accumulation.
    tol = dict(rtol=2e-2, atol=2e-2) if autocast else dict(rtol=1e-4, atol=1e-4)
    assert torch.allclose(y1, y0, **tol)
    assert torch.allclose(gx1, gx0, **tol)
    rel = float((gw1 - gw0).norm() / gw0.norm())
    assert rel < (1e-2 if autocast else 1e-5), rel


def test_reduce_overhead_compiled_model_matches_eager():
    # The reference's trainer compiles the whole model with
    # torch.compile(model, mode="reduce-overhead", fullgraph=True)
    # (examples/example_utils.py:166-169): one graph, inductor, and the
    # forward and backward each captured in a HIP graph and replayed.  A new
    # batch every step (so a replay that reused stale inputs would show); the
    # compiled model's loss and gradients against the eager model's.
    # Inductor generates its own kernels for the torch ops between the HIP
    # ops (embedding, layer norms, head, cross entropy), so the bar is the
    # end-model one: loss within 2e-3, gradient cosine > 0.999.
    from hip_graphs import recorded_hip_graphs, reset
    from torch._dynamo.utils import counters

    reset()
    counters.clear()
    model = _model(n_layer=2, n_embd=128).to(DEV)
    with torch.no_grad():
        for p in model.parameters():
            if p.ndim == 2:
                p.mul_(8.0)
    twin = copy.deepcopy(model)
    compiled = torch.compile(twin, mode="reduce-overhead", fullgraph=True)
    for step in range(5):
        print(f"reduce-overhead model step {step}", flush=True)
        ids, tgt = (x.to(DEV) for x in _batch(4, 64, seed=30 + step))
        losses = []
        for m, params in ((model, model), (compiled, twin)):
            params.zero_grad(set_to_none=True)
            with torch.autocast("cuda", dtype=torch.bfloat16):
                loss, _ = m(ids, tgt)
            loss.backward()
            losses.append(float(loss.detach()))
        torch.cuda.synchronize()
        rel = abs(losses[1] - losses[0]) / abs(losses[0])
        print(f"step {step}: eager {losses[0]:.6f} compiled {losses[1]:.6f} (rel {rel:.2e})")
        assert rel < 2e-3, f"step {step}: loss rel {rel:.2e}"
        for (name, p), q in zip(model.named_parameters(), twin.parameters()):
            a, b = p.grad.double().flatten(), q.grad.double().flatten()
            if float(a.norm()) == 0.0:
                assert float(b.norm()) == 0.0, name
                continue
            cos = float(a @ b / (a.norm() * b.norm()))
            assert cos > 0.999, f"step {step} {name}: cosine {cos:.6f}"
    assert counters["inductor"]["cudagraph_skips"] == 0, dict(counters["inductor"])
    assert recorded_hip_graphs() >= 2  # the forward and the backward graph
    torch._dynamo.reset()
