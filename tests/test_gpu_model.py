"""End-model parity: the SpikeGPT model on the HIP WKV, LIF and token-shift
kernels against the same model (identical weights and batch) with all three
replaced by the CPU oracle's formulations.

Bars: loss within 0.2 % relative (the end-model bar), under bf16 autocast
and in fp32; parameter gradients in fp32 with cosine similarity > 0.999 (the
spike threshold makes gradients discontinuous, so an elementwise bound would
test rounding luck, not the kernels).
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


def _loss(model, ids, tgt, autocast, oracle, monkeypatch):
    import spikegpt_myelin_amd.model as M

    with monkeypatch.context() as mp:
        if oracle:
            mp.setattr(M, "weighted_key_value_gated",
                       lambda k, v, td, tf, r: torch.sigmoid(r) * _oracle_wkv(k, v, td, tf))
            mp.setattr(M, "lif_sequence", _oracle_lif)
            mp.setattr(M, "lif_residual", lambda residual, x, **kw: residual + _oracle_lif(x, **kw))
            mp.setattr(M, "token_shift_mix", _oracle_mix)
            # The block's fused layer norm + mix becomes torch's layer norm
            # (fp32, as autocast runs it) and the oracle's mix.
            mp.setattr(M, "layer_norm_shift_mix", lambda x, norm, mix: _oracle_mix(
                torch.nn.functional.layer_norm(x.float(), norm.normalized_shape, norm.weight,
                                               norm.bias, norm.eps), mix))
            mp.setattr(M, "layer_norm_shift_mix_fork", lambda x, norm, mix: [*_oracle_mix(
                torch.nn.functional.layer_norm(x.float(), norm.normalized_shape, norm.weight,
                                               norm.bias, norm.eps), mix), x])
            mp.setattr(M, "relu_square", lambda x: torch.relu(x).square())
            mp.setattr(M, "sigmoid_gate", lambda r, x: torch.sigmoid(r) * x)
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


@pytest.mark.parametrize("autocast,scale", [(True, 1.0), (False, 1.0), (True, 4.0), (True, 8.0),
                                            (False, 8.0)])
def test_loss_matches_oracle_recurrences_at_41m_depth(autocast, scale, monkeypatch):
    # The 41M configuration itself: 12 layers, 512 channels, byte vocabulary,
    # random init (scale 1), and with the projection weights scaled up so
    # that the LIFs fire and the recurrences shape the output (scales 4, 8);
    # B=2, T=512 keeps the CPU oracle's twelve layers of loops within seconds.
    import spikegpt_myelin_amd.model as M

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
        with monkeypatch.context() as mp:
            # Power of the check: the same model with the time mix's
            # recurrence output zeroed.
            mp.setattr(M, "weighted_key_value_gated", lambda k, v, td, tf, r: torch.zeros_like(k))
            with torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
                no_wkv, _ = model(ids, tgt)
    rel = abs(float(hip) - float(ref)) / abs(float(ref))
    moved = abs(float(no_wkv) - float(ref)) / abs(float(ref))
    print(f"41M depth loss {float(hip):.6f} vs oracle {float(ref):.6f} (rel {rel:.2e}); "
          f"without the recurrence {float(no_wkv):.6f} (rel {moved:.2e})")
    assert rel < 2e-3, f"loss {float(hip):.6f} vs oracle {float(ref):.6f} (rel {rel:.2e})"
    if scale >= 8.0:
        # here the recurrence moves the loss by far more than the bar
        assert moved > 10 * 2e-3, f"the recurrence hardly moves the loss ({moved:.2e})"


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
