"""Recurrent one-token steps and generation on the gfx950 block-step kernels.

The reference generates with ``SpikeLanguageModel.forward_step``
(``src/spikegpt/language.py:1434-1453``), which runs every block's
``SpikeGPTBlock.step`` (``:1301-1335``) in eager PyTorch: ~60 element-wise
launches per layer around seven projections.  Here a layer is four HIP
launches (``block_step_row`` x2, ``block_step_wkv``, ``relu_square_forward``)
plus the projections (hipBLASLt GEMMs into preallocated buffers), and
:class:`StepGraph` captures a whole model step into one HIP graph so that a
generated token costs one graph launch.

State.  The recurrent state of all layers lives in ONE fp32 tensor
``[n_layer, 7, B, C]``; slot order is :data:`SLOTS`.  The reference's state
dataclasses (``language.py:182-230``) are provided with the same names and
fields, as views into that tensor, so code that inspects a state keeps
working; a state assembled from separate tensors is packed on entry.

Arithmetic is fp32 throughout (the reference's step runs in the parameters'
dtype, fp32 for a trained model), so a step matches the sequence forward of
the same model to fp32 rounding.  Dropout is not applied: a step runs with
eval semantics, as ``generate`` (``:1486-1487``) does; steps are inference
only (no autograd through the state).
"""

from __future__ import annotations

import ctypes
import weakref
from dataclasses import dataclass, field
from typing import TYPE_CHECKING, Iterator

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib

if TYPE_CHECKING:  # pragma: no cover
    from .model import SpikeGPTBlock, SpikeLanguageModel

# Per-layer state slots of the packed tensor.
SLOTS = ("time_previous", "numerator", "denominator", "log_scale", "channel_previous",
         "lif1_membrane", "lif2_membrane")
_TPREV, _NUM, _DEN, _LS, _CPREV, _LIF1, _LIF2 = range(7)

PRE_EMBED, PRE_LIF, PRE_GATE_LIF, PRE_NONE = 0, 1, 2, 3

_LOG_SCALE_INIT = torch.finfo(torch.float32).min  # language.py:969-974


# ----------------------------------------------------------- state types ----
@dataclass(frozen=True)
class SpikeTimeMixState:
    """``language.py:182-189``."""

    previous: Tensor
    numerator: Tensor
    denominator: Tensor
    log_scale: Tensor


@dataclass(frozen=True)
class SpikeChannelMixState:
    """``language.py:201-205``."""

    previous: Tensor


@dataclass(frozen=True)
class SpikingSequenceLIFState:
    """``language.py:208-212``."""

    membrane: Tensor


@dataclass(frozen=True)
class SpikeGPTBlockState:
    """``language.py:215-223`` (``ffn_pre`` is always None: the
    ``rwkv-ffn-pre`` variant is not served)."""

    time_mix: SpikeTimeMixState | None
    ffn_pre: SpikeChannelMixState | None
    channel_mix: SpikeChannelMixState
    lif1: SpikingSequenceLIFState
    lif2: SpikingSequenceLIFState


@dataclass(frozen=True)
class SpikeLanguageModelState:
    """``language.py:226-230``; ``packed`` is the ``[n_layer, 7, B, C]`` fp32
    tensor the block views point into (None for a hand-built state)."""

    blocks: tuple[SpikeGPTBlockState, ...]
    packed: Tensor | None = field(default=None, repr=False, compare=False)


def _block_views(layer: Tensor) -> SpikeGPTBlockState:
    return SpikeGPTBlockState(
        time_mix=SpikeTimeMixState(previous=layer[_TPREV], numerator=layer[_NUM],
                                   denominator=layer[_DEN], log_scale=layer[_LS]),
        ffn_pre=None,
        channel_mix=SpikeChannelMixState(previous=layer[_CPREV]),
        lif1=SpikingSequenceLIFState(membrane=layer[_LIF1]),
        lif2=SpikingSequenceLIFState(membrane=layer[_LIF2]),
    )


def state_from_packed(packed: Tensor) -> SpikeLanguageModelState:
    """State whose block tensors are views of ``packed`` ``[L, 7, B, C]``."""
    return SpikeLanguageModelState(blocks=tuple(_block_views(packed[i])
                                                for i in range(packed.shape[0])),
                                   packed=packed)


def initial_packed(n_layer: int, batch_size: int, channels: int,
                   device: torch.device) -> Tensor:
    """Zero state with the WKV log-scale at ``finfo(float32).min``."""
    packed = torch.zeros(n_layer, len(SLOTS), batch_size, channels, device=device,
                         dtype=torch.float32)
    packed[:, _LS].fill_(_LOG_SCALE_INIT)
    return packed


def _block_tensors(bs: SpikeGPTBlockState) -> list[Tensor]:
    if bs.time_mix is None or not isinstance(bs.time_mix, SpikeTimeMixState):
        raise NotImplementedError("the block step serves the RWKV time mix only")
    tm = bs.time_mix
    return [tm.previous, tm.numerator, tm.denominator, tm.log_scale, bs.channel_mix.previous,
            bs.lif1.membrane, bs.lif2.membrane]


def pack_state(state: SpikeLanguageModelState) -> Tensor:
    """The ``[L, 7, B, C]`` fp32 tensor behind ``state`` (packed on demand)."""
    p = state.packed
    if p is not None and p.dtype == torch.float32 and p.is_contiguous():
        ok = all(t.data_ptr() == p[i, j].data_ptr() and t.shape == p[i, j].shape
                 for i, bs in enumerate(state.blocks) for j, t in enumerate(_block_tensors(bs)))
        if ok and len(state.blocks) == p.shape[0]:
            return p
    return torch.stack([torch.stack([t.float() for t in _block_tensors(bs)])
                        for bs in state.blocks]).contiguous()


# ---------------------------------------------------------- launch glue ----
def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _need(t: Tensor | None, shape: tuple, name: str, dtype: torch.dtype = torch.float32,
          device: torch.device | None = None) -> None:
    """Raise unless ``t`` (if given) is a contiguous ``dtype`` tensor of ``shape``
    on ``device`` (when given).  The kernels receive raw addresses, so a host
    tensor must be refused here rather than handed to the GPU."""
    if t is None:
        return
    if tuple(t.shape) != tuple(shape) or t.dtype != dtype or not t.is_contiguous():
        raise ValueError(f"{name}: expected a contiguous {dtype} tensor of shape "
                         f"{tuple(shape)}; got {t.dtype} {tuple(t.shape)}")
    if device is not None and t.device != device:
        raise ValueError(f"{name}: expected a tensor on {device}; got one on {t.device}")


def _gpu_device(t: Tensor, name: str) -> torch.device:
    """The HIP device of ``t``; a host (or meta) tensor raises ValueError."""
    if t.device.type != "cuda":
        raise ValueError(f"{name}: the step kernels run on a HIP GPU; got a tensor on {t.device}")
    return t.device


def _row(pre: int, *, residual: Tensor, stream: int, ln: torch.nn.LayerNorm | None = None,
         mix: tuple[Tensor, ...] = (), prev_in: Tensor | None = None,
         prev_out: Tensor | None = None, outs: tuple[Tensor, ...] = (), ids: Tensor | None = None,
         embedding: Tensor | None = None, embedding_slope: float = 1.0,
         embedding_spike: bool = True, ln0: torch.nn.LayerNorm | None = None,
         add: Tensor | None = None, gate: Tensor | None = None, mem_in: Tensor | None = None,
         mem_out: Tensor | None = None, lif=None) -> None:
    a = _lib.StepRowArgs()
    B, C = residual.shape
    dev = residual.device
    # Every tensor is handed to the kernel as a raw pointer: check that each
    # one has the [B, C] row shape (or [C] / [vocab, C]) the kernel indexes,
    # on the residual's device, and (below) that this device is a GPU.
    for name, t in (("prev_in", prev_in), ("prev_out", prev_out), ("add", add), ("gate", gate),
                    ("mem_in", mem_in), ("mem_out", mem_out)):
        _need(t, (B, C), name, device=dev)
    for j, o in enumerate(outs):
        _need(o, (B, C), f"out[{j}]", device=dev)
    for mod, name in ((ln, "ln"), (ln0, "ln0")):
        if mod is not None:
            _need(mod.weight, (C,), f"{name}.weight", device=dev)
            _need(mod.bias, (C,), f"{name}.bias", device=dev)
    for j, m in enumerate(mix):
        if m.numel() != C or m.dtype != torch.float32:
            raise ValueError(f"mixing vector {j} has {m.numel()} elements; the row has {C}")
        if m.device != dev:
            raise ValueError(f"mixing vector {j}: expected a tensor on {dev}; got one on {m.device}")
    if ids is not None:
        _need(ids, (B,), "ids", torch.int64, device=dev)
        if embedding is None or embedding.ndim != 2 or embedding.shape[1] != C:
            raise ValueError(f"embedding must be [vocab, {C}]")
        _need(embedding, tuple(embedding.shape), "embedding", device=dev)
    _gpu_device(residual, "residual")
    a.batch, a.channels = B, C
    a.residual = residual.data_ptr()
    if ids is not None:
        a.ids = ids.data_ptr()
        a.embedding = embedding.data_ptr()
        a.vocab = embedding.shape[0]
        a.embedding_slope = embedding_slope
        a.embedding_spike = int(embedding_spike)
    if ln0 is not None:
        a.ln0_weight, a.ln0_bias = ln0.weight.data_ptr(), ln0.bias.data_ptr()
    if add is not None:
        a.add = add.data_ptr()
        a.gate = _ptr(gate)
        a.membrane_in, a.membrane_out = mem_in.data_ptr(), mem_out.data_ptr()
        if lif is None:
            a.spiking = 0
        else:
            a.spiking = 1
            a.lif_decay, a.lif_threshold = lif.decay, lif.threshold
            a.lif_reset, a.lif_slope = lif.reset, lif.surrogate_slope
    if ln is not None:
        a.ln_weight, a.ln_bias = ln.weight.data_ptr(), ln.bias.data_ptr()
        a.ln_eps = ln.eps
    elif ln0 is not None:
        a.ln_eps = ln0.eps
    else:
        a.ln_eps = 1e-5
    if mix:
        for j, m in enumerate(mix):
            a.mix[j] = m.data_ptr()
        a.n_mix = len(mix)
        a.previous_in, a.previous_out = prev_in.data_ptr(), prev_out.data_ptr()
    for j, o in enumerate(outs):
        a.out[j] = o.data_ptr()
    lib = _lib.load()
    _lib.check(_lib.timed("block_step_row", residual.device,
                          lambda: lib.block_step_row(pre, ctypes.byref(a), stream)),
               "block_step_row")


class StepWorkspace:
    """Activation buffers of one step for batch ``B`` (reused every step)."""

    def __init__(self, B: int, C: int, hidden: int, vocab: int, device: torch.device) -> None:
        self.dims = (B, C, hidden, vocab)
        f = dict(device=device, dtype=torch.float32)
        self.residual = torch.empty(B, C, **f)
        self.mixed = torch.empty(3, B, C, **f)    # k, v, r inputs (channel mix: k, r)
        self.proj = torch.empty(3, B, C, **f)     # k, v, r projections
        self.gated = torch.empty(B, C, **f)
        self.att = torch.empty(B, C, **f)
        self.ffn_key = torch.empty(B, hidden, **f)
        self.ffn_act = torch.empty(B, hidden, **f)  # relu(key)^2
        self.ffn_value = torch.empty(B, C, **f)
        self.ffn_gate = torch.empty(B, C, **f)
        self.normed = torch.empty(B, C, **f)
        self.logits = torch.empty(B, vocab, **f)


def _lif_module(mod):
    from .model import SpikingSequenceLIF

    return mod if isinstance(mod, SpikingSequenceLIF) else None


def _mm(x: Tensor, linear: torch.nn.Linear, out: Tensor) -> Tensor:
    return torch.mm(x, linear.weight.t(), out=out)


def _time_mix_half(block: "SpikeGPTBlock", src: Tensor, dst: Tensor, ws: StepWorkspace,
                   stream: int) -> None:
    """Projections, WKV + gate and output projection of one block; the row
    kernel that produced ws.mixed[0..2] already ran."""
    att = block.att
    _mm(ws.mixed[0], att.key, ws.proj[0])
    _mm(ws.mixed[1], att.value, ws.proj[1])
    _mm(ws.mixed[2], att.receptance, ws.proj[2])
    B, C = ws.residual.shape
    lib = _lib.load()
    rc = _lib.timed("block_step_wkv", src.device, lambda: lib.block_step_wkv(
        ws.proj[0].data_ptr(), ws.proj[1].data_ptr(), ws.proj[2].data_ptr(),
        att.time_decay.data_ptr(), att.time_first.data_ptr(),
        src[_NUM].data_ptr(), src[_DEN].data_ptr(), src[_LS].data_ptr(),
        dst[_NUM].data_ptr(), dst[_DEN].data_ptr(), dst[_LS].data_ptr(),
        ws.gated.data_ptr(), B, C, stream))
    _lib.check(rc, "block_step_wkv")
    _mm(ws.gated, att.output, ws.att)


def _channel_mix_half(block: "SpikeGPTBlock", src: Tensor, dst: Tensor, ws: StepWorkspace,
                      stream: int) -> None:
    """First LIF + LN2 + token shift, then the channel-mix projections up to
    (not including) the gate, which the next row kernel applies."""
    ffn = block.ffn
    _row(PRE_LIF, residual=ws.residual, stream=stream, ln=block.ln2, mix=_mixes(ffn),
         prev_in=src[_CPREV], prev_out=dst[_CPREV], outs=(ws.mixed[0], ws.mixed[1]),
         add=ws.att, mem_in=src[_LIF1], mem_out=dst[_LIF1], lif=_lif_module(block.lif1))
    _mm(ws.mixed[0], ffn.key, ws.ffn_key)
    lib = _lib.load()
    n = ws.ffn_key.numel()
    rc = _lib.timed("relu_square", src.device, lambda: lib.relu_square_forward(
        ws.ffn_key.data_ptr(), ws.ffn_act.data_ptr(), n, _lib.DTYPE_F32, stream))
    _lib.check(rc, "relu_square_forward")
    _mm(ws.ffn_act, ffn.value, ws.ffn_value)
    _mm(ws.mixed[1], ffn.receptance, ws.ffn_gate)


def _mixes(mod) -> tuple[Tensor, ...]:
    """Mixing vectors ([1, 1, C] fp32 parameters) of a time mix (k, v, r) or a
    channel mix (k, r), passed to the kernel by address."""
    names = ("time_mix_k", "time_mix_v", "time_mix_r") if hasattr(mod, "time_mix_v") else (
        "time_mix_k", "time_mix_r")
    out = tuple(getattr(mod, n) for n in names)
    for m in out:
        if not m.is_contiguous():
            raise ValueError("mixing vectors must be contiguous")
    return out


def _check_model(model: "SpikeLanguageModel") -> None:
    for p in model.parameters():
        if p.dtype != torch.float32 or not p.is_cuda:
            raise NotImplementedError(
                "the block-step kernels run fp32 models on the GPU; got a parameter of "
                f"dtype {p.dtype} on {p.device}")
    if model.config.n_embd % 4 != 0 or model.config.n_embd > 4096:
        raise NotImplementedError("the block-step kernels take n_embd % 4 == 0, <= 4096")


@torch.no_grad()
def model_step(model: "SpikeLanguageModel", ids: Tensor, src: Tensor, dst: Tensor,
               ws: StepWorkspace) -> Tensor:
    """Advance every layer by one token: reads state ``src``, writes ``dst``
    (may be the same tensor), returns ``ws.logits`` [B, vocab]."""
    cfg = model.config
    _check_workspace(model, ws, ids.shape[0], src, dst)
    dev = _gpu_device(model.embedding.weight, "model parameters")
    _need(ids, (ids.shape[0],), "ids", torch.int64, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    blocks = list(model.blocks)
    L = len(blocks)
    first = blocks[0]
    _row(PRE_EMBED, residual=ws.residual, stream=stream, ids=ids,
         embedding=model.embedding.weight, embedding_slope=cfg.surrogate_slope,
         embedding_spike=cfg.spike_embedding, ln0=first.ln0, ln=first.ln1,
         mix=_mixes(first.att), prev_in=src[0, _TPREV], prev_out=dst[0, _TPREV],
         outs=(ws.mixed[0], ws.mixed[1], ws.mixed[2]))
    for i, block in enumerate(blocks):
        if i > 0:
            prev = blocks[i - 1]
            _row(PRE_GATE_LIF, residual=ws.residual, stream=stream, ln=block.ln1,
                 mix=_mixes(block.att), prev_in=src[i, _TPREV], prev_out=dst[i, _TPREV],
                 outs=(ws.mixed[0], ws.mixed[1], ws.mixed[2]), add=ws.ffn_value,
                 gate=ws.ffn_gate, mem_in=src[i - 1, _LIF2], mem_out=dst[i - 1, _LIF2],
                 lif=_lif_module(prev.lif2))
        _time_mix_half(block, src[i], dst[i], ws, stream)
        _channel_mix_half(block, src[i], dst[i], ws, stream)
    _row(PRE_GATE_LIF, residual=ws.residual, stream=stream, ln=model.ln_out,
         outs=(ws.normed,), add=ws.ffn_value, gate=ws.ffn_gate, mem_in=src[L - 1, _LIF2],
         mem_out=dst[L - 1, _LIF2], lif=_lif_module(blocks[-1].lif2))
    return _mm(ws.normed, model.head, ws.logits)


@torch.no_grad()
def block_step(block: "SpikeGPTBlock", inputs: Tensor, src: Tensor, dst: Tensor,
               ws: StepWorkspace) -> Tensor:
    """One block's step on its input ``inputs`` [B, C]; state slot rows
    ``src``/``dst`` [7, B, C]; returns the new residual (``ws.residual``)."""
    B, C = inputs.shape
    if ws.dims[:3] != (B, C, block.ffn.key.out_features):
        raise ValueError(f"step workspace sized for (B, C, hidden) = {ws.dims[:3]}; the block "
                         f"and batch need {(B, C, block.ffn.key.out_features)}")
    dev = _gpu_device(block.att.time_decay, "block parameters")
    _need(inputs, (B, C), "inputs", device=dev)
    _need(src, (len(SLOTS), B, C), "state src", device=dev)
    _need(dst, (len(SLOTS), B, C), "state dst", device=dev)
    _need(ws.residual, (B, C), "workspace", device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws.residual.copy_(inputs)
    _row(PRE_NONE, residual=ws.residual, stream=stream, ln0=block.ln0, ln=block.ln1,
         mix=_mixes(block.att), prev_in=src[_TPREV], prev_out=dst[_TPREV],
         outs=(ws.mixed[0], ws.mixed[1], ws.mixed[2]))
    _time_mix_half(block, src, dst, ws, stream)
    _channel_mix_half(block, src, dst, ws, stream)
    _row(PRE_GATE_LIF, residual=ws.residual, stream=stream, add=ws.ffn_value, gate=ws.ffn_gate,
         mem_in=src[_LIF2], mem_out=dst[_LIF2], lif=_lif_module(block.lif2))
    return ws.residual


def _model_dims(model: "SpikeLanguageModel", batch: int) -> tuple[int, int, int, int]:
    cfg = model.config
    return (batch, cfg.n_embd, model.blocks[0].ffn.key.out_features, cfg.vocab_size)


def _check_workspace(model: "SpikeLanguageModel", ws: StepWorkspace, batch: int,
                     src: Tensor, dst: Tensor) -> None:
    """The workspace and the state buffers must have the model's sizes: the
    kernels index them by the model's B and C."""
    dims = _model_dims(model, batch)
    if ws.dims != dims:
        raise ValueError(f"step workspace sized for (B, C, hidden, vocab) = {ws.dims}; "
                         f"the model and batch need {dims}")
    want = (model.config.n_layer, len(SLOTS), batch, model.config.n_embd)
    dev = model.embedding.weight.device
    for name, t in (("src", src), ("dst", dst)):
        _need(t, want, f"state {name}", device=dev)
    _need(ws.residual, (batch, model.config.n_embd), "step workspace", device=dev)


# Step workspaces per live model (weak keys: a workspace never outlives its
# model, and a new model never finds an old model's buffers).
_WS_CACHE: "weakref.WeakKeyDictionary" = weakref.WeakKeyDictionary()


def workspace_for(model: "SpikeLanguageModel", batch: int, device: torch.device) -> StepWorkspace:
    dims = _model_dims(model, batch)
    key = (dims, torch.device(device))
    per_model = _WS_CACHE.get(model)
    ws = None if per_model is None else per_model.get(key)
    if ws is None:
        ws = StepWorkspace(*dims, device)
        _WS_CACHE[model] = {key: ws}  # one workspace per model (the last batch size)
    return ws


# ------------------------------------------------------- public helpers ----
def initial_state(model: "SpikeLanguageModel", *, batch_size: int,
                  device: torch.device | None = None,
                  dtype: torch.dtype | None = None) -> SpikeLanguageModelState:
    """``SpikeLanguageModel.initial_state`` (``language.py:1410-1432``); the
    state is fp32 whatever ``dtype`` says (the kernels keep fp32 state)."""
    dev = model.embedding.weight.device if device is None else torch.device(device)
    return state_from_packed(initial_packed(model.config.n_layer, batch_size,
                                            model.config.n_embd, dev))


def forward_step(model: "SpikeLanguageModel", input_ids: Tensor,
                 state: SpikeLanguageModelState) -> tuple[Tensor, SpikeLanguageModelState]:
    """``SpikeLanguageModel.forward_step`` (``language.py:1434-1453``):
    logits [B, vocab] and a new state (the input state is left unchanged)."""
    if input_ids.ndim != 1:
        raise ValueError(f"input_ids must have shape [B]; got {input_ids.shape}")
    _check_model(model)
    if not input_ids.is_cuda:
        raise RuntimeError("forward_step runs on the GPU; input_ids is on the CPU")
    if bool(((input_ids < 0) | (input_ids >= model.config.vocab_size)).any()):
        raise IndexError("input_ids out of range of the vocabulary")
    ids = input_ids.to(torch.int64).contiguous()
    src = pack_state(state)
    B = ids.shape[0]
    if src.shape != (model.config.n_layer, len(SLOTS), B, model.config.n_embd):
        raise ValueError(f"state of shape {tuple(src.shape)} does not fit batch {B}")
    dst = torch.empty_like(src)
    ws = workspace_for(model, B, ids.device)
    logits = model_step(model, ids, src, dst, ws).clone()
    return logits, state_from_packed(dst)


class StepGraph:
    """A whole-model step for a fixed batch, captured in one HIP graph.

    ``step(ids)`` copies ``ids`` into the graph's input, replays it and returns
    the logits tensor (overwritten by the next step).  The state lives in the
    graph's own buffer and is updated in place; ``state()`` returns a copy
    in the reference's dataclass form and ``reset(state)`` loads one.
    """

    def __init__(self, model: "SpikeLanguageModel", batch_size: int,
                 state: SpikeLanguageModelState | None = None) -> None:
        _check_model(model)
        self.model = model
        dev = model.embedding.weight.device
        cfg = model.config
        self.ids = torch.zeros(batch_size, dtype=torch.int64, device=dev)
        self.packed = initial_packed(cfg.n_layer, batch_size, cfg.n_embd, dev)
        self.ws = StepWorkspace(batch_size, cfg.n_embd, model.blocks[0].ffn.key.out_features,
                                cfg.vocab_size, dev)
        # Warm up (library handles, GEMM workspaces) outside the capture, on a
        # side stream as graph capture requires, then capture.
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side), torch.no_grad():
            for _ in range(2):
                model_step(model, self.ids, self.packed, self.packed, self.ws)
        torch.cuda.current_stream(dev).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph), torch.no_grad():
            self.logits = model_step(model, self.ids, self.packed, self.packed, self.ws)
        self.reset(state)

    def reset(self, state: SpikeLanguageModelState | None = None) -> None:
        cfg = self.model.config
        if state is None:
            self.packed.copy_(initial_packed(cfg.n_layer, self.ids.shape[0], cfg.n_embd,
                                             self.packed.device))
        else:
            self.packed.copy_(pack_state(state))

    def step(self, input_ids: Tensor) -> Tensor:
        self.ids.copy_(input_ids.reshape(-1), non_blocking=True)
        self.graph.replay()
        return self.logits

    def state(self) -> SpikeLanguageModelState:
        return state_from_packed(self.packed.clone())


def sample_next_token(logits: Tensor, *, temperature: float, top_k: int | None,
                      sampling: str) -> Tensor:
    """``_sample_next_token`` (``language.py:356-376``): temperature, top-k
    filter, then greedy argmax or a multinomial draw; [B, 1] int64."""
    next_logits = logits / temperature
    if top_k is not None:
        k = min(top_k, next_logits.shape[-1])
        kth = torch.topk(next_logits, k, dim=-1).values[:, -1:]
        next_logits = next_logits.masked_fill(next_logits < kth, float("-inf"))
    if sampling == "greedy":
        return next_logits.argmax(dim=-1, keepdim=True)
    return torch.multinomial(F.softmax(next_logits, dim=-1), num_samples=1)


def _check_generate_args(input_ids: Tensor, max_new_tokens: int, temperature: float,
                         top_k: int | None, sampling: str) -> None:
    # language.py:1474-1485
    if max_new_tokens < 0:
        raise ValueError("max_new_tokens must be non-negative")
    if temperature <= 0.0:
        raise ValueError("temperature must be positive")
    if top_k is not None and top_k <= 0:
        raise ValueError("top_k must be positive when provided")
    if sampling not in ("multinomial", "greedy"):
        raise ValueError("sampling must be 'multinomial' or 'greedy'")
    if input_ids.ndim != 2:
        raise ValueError(f"input_ids must have shape [B, T]; got {input_ids.shape}")
    if input_ids.shape[1] == 0:
        raise ValueError("input_ids must contain at least one context token")


def generate_tokens(model: "SpikeLanguageModel", input_ids: Tensor, *, max_new_tokens: int,
                    temperature: float, top_k: int | None, sampling: str,
                    use_graph: bool) -> Iterator[Tensor]:
    """Yields the ``max_new_tokens`` sampled tokens ([B, 1] each) after
    consuming the context through the recurrent state."""
    _check_generate_args(input_ids, max_new_tokens, temperature, top_k, sampling)
    B, T = input_ids.shape
    if bool(((input_ids < 0) | (input_ids >= model.config.vocab_size)).any()):
        raise IndexError("input_ids out of range of the vocabulary")
    if use_graph:
        g = StepGraph(model, B)
        step = g.step
    else:
        state = initial_state(model, batch_size=B)

        def step(ids: Tensor) -> Tensor:
            nonlocal state
            out, state = forward_step(model, ids, state)
            return out
    logits = None
    for t in range(T):
        logits = step(input_ids[:, t])
    for _ in range(max_new_tokens):
        nxt = sample_next_token(logits, temperature=temperature, top_k=top_k, sampling=sampling)
        yield nxt
        logits = step(nxt[:, 0])
