"""Host-side logic of the one-token step: the per-model workspace cache and the
shape checks made before any raw pointer reaches a kernel (no GPU needed)."""

from __future__ import annotations

import gc

import pytest
import torch

from spikegpt_myelin_amd import generation as G
from spikegpt_myelin_amd.model import SpikeGPTConfig, SpikeLanguageModel

CPU = torch.device("cpu")


def _model(n_embd, vocab=50, layers=2):
    return SpikeLanguageModel(SpikeGPTConfig(vocab_size=vocab, context_length=8, n_layer=layers,
                                             n_embd=n_embd))


def test_workspace_follows_the_model_not_its_id():
    # A freed model's id is usually reused by the next object; a cache keyed
    # on id() would hand the wider model's buffers to a narrower model.
    m1 = _model(64)
    ws1 = G.workspace_for(m1, 3, CPU)
    assert ws1.dims == (3, 64, m1.blocks[0].ffn.key.out_features, 50)
    assert G.workspace_for(m1, 3, CPU) is ws1
    del m1
    gc.collect()
    m2 = _model(32, vocab=20)
    ws2 = G.workspace_for(m2, 3, CPU)
    assert ws2.dims == (3, 32, m2.blocks[0].ffn.key.out_features, 20)
    assert ws2.residual.shape == (3, 32) and ws2.logits.shape == (3, 20)
    # a new batch size gets new buffers
    assert G.workspace_for(m2, 5, CPU).dims[0] == 5


def test_workspace_cache_does_not_keep_models_alive():
    m = _model(16)
    G.workspace_for(m, 2, CPU)
    n = len(G._WS_CACHE)
    del m
    gc.collect()
    assert len(G._WS_CACHE) == n - 1


def test_mismatched_workspace_or_state_is_rejected_before_launch():
    m = _model(32)
    other = _model(64)
    ws_wrong = G.workspace_for(other, 2, CPU)
    src = torch.zeros(2, len(G.SLOTS), 2, 32)
    with pytest.raises(ValueError, match="workspace"):
        G._check_workspace(m, ws_wrong, 2, src, src)
    ws = G.StepWorkspace(*G._model_dims(m, 2), CPU)
    G._check_workspace(m, ws, 2, src, src)
    with pytest.raises(ValueError, match="state src"):
        G._check_workspace(m, ws, 2, torch.zeros(2, len(G.SLOTS), 2, 16), src)


def test_row_arguments_are_shape_checked():
    residual = torch.zeros(2, 32)
    with pytest.raises(ValueError, match="out\\[0\\]"):
        G._row(G.PRE_NONE, residual=residual, stream=0, outs=(torch.zeros(2, 16),))
    ln = torch.nn.LayerNorm(16)
    with pytest.raises(ValueError, match="ln.weight"):
        G._row(G.PRE_NONE, residual=residual, stream=0, ln=ln)
    with pytest.raises(ValueError, match="prev_in"):
        G._row(G.PRE_NONE, residual=residual, stream=0, prev_in=torch.zeros(3, 32))


def test_gradient_checkpointing_flag():
    # language.py:1376, 1396-1404: the config flag sets the model's attribute,
    # set_gradient_checkpointing toggles it.
    m = SpikeLanguageModel(SpikeGPTConfig(vocab_size=10, context_length=4, n_layer=1, n_embd=8,
                                          gradient_checkpointing=True))
    assert m.gradient_checkpointing is True
    m.set_gradient_checkpointing(False)
    assert m.gradient_checkpointing is False
    m.set_gradient_checkpointing()
    assert m.gradient_checkpointing is True


def test_tensors_off_the_gpu_are_rejected_before_launch():
    # The step kernels take raw addresses: a host tensor (or one on another
    # device than the model) must raise ValueError, never reach a kernel.
    cuda0 = torch.device("cuda", 0)
    with pytest.raises(ValueError, match="expected a tensor on cuda:0"):
        G._need(torch.zeros(2, 3), (2, 3), "state src", device=cuda0)
    residual = torch.zeros(2, 32)
    with pytest.raises(ValueError, match="HIP GPU"):
        G._row(G.PRE_NONE, residual=residual, stream=0, outs=(torch.zeros(2, 32),))
    with pytest.raises(ValueError, match="prev_in: expected a tensor on"):
        G._row(G.PRE_NONE, residual=residual, stream=0,
               prev_in=torch.zeros(2, 32, device="meta"))
    m = _model(32)
    ws = G.StepWorkspace(*G._model_dims(m, 2), CPU)
    src = torch.zeros(2, len(G.SLOTS), 2, 32)
    with pytest.raises(ValueError, match="state dst: expected a tensor on cpu"):
        G._check_workspace(m, ws, 2, src, src.to("meta"))
    ids = torch.zeros(2, dtype=torch.int64)
    with pytest.raises(ValueError, match="HIP GPU"):
        G.model_step(m, ids, src, src, ws)
    with pytest.raises(ValueError, match="HIP GPU"):
        G.block_step(m.blocks[0], torch.zeros(2, 32), src[0], src[0],
                     G.StepWorkspace(*G._model_dims(m, 2), CPU))
