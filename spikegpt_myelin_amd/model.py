"""SpikeGPT language model around the HIP WKV and LIF kernels.

Host-side mirror of the reference model (``src/spikegpt/language.py``) for the
training and evaluation path: same class names, constructor arguments,
parameter names and initialisation, so that a state dict moves between the
two.  Every sequential recurrence runs in the gfx950 kernels -- the WKV time
mix through ``myelin::wkv_forward{,_bf16io}`` (``SpikeTimeMix.forward``,
``language.py:1015-1036``) and the spiking activations through
``myelin::lif_sequence_forward`` (``SpikingSequenceLIF.forward``,
``language.py:848-918``), and the token-shift mixes that feed the
projections through one fused ``myelin::layer_norm_shift_mix`` pass per
block half (the half's layer norm and its token-shift mixes,
``language.py:344-353, 1341-1356``), and the squared ReLU and receptance gates
through ``myelin::relu_square`` / ``myelin::sigmoid_gate``; linear layers
(with split-K weight gradients), the first block's ``ln0``, ``ln_out`` and
the loss are PyTorch-ROCm (hipBLASLt GEMMs).

Supported configuration: ``model_type="rwkv"``, ``attention="rwkv"``,
``spike_input=False`` (the reference defaults, ``language.py:234-256``).
Other variants raise ``NotImplementedError``.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
import torch.utils.checkpoint
from torch import Tensor, nn

from . import generation
from .gates import relu_square, sigmoid_gate
from .generation import (SpikeChannelMixState, SpikeGPTBlockState, SpikeLanguageModelState,
                         SpikeTimeMixState, SpikingSequenceLIFState, StepWorkspace, block_step,
                         initial_packed, pack_state, state_from_packed)
from .lif import atan_surrogate, lif_residual, lif_sequence, serves_surrogate
from .splitk import split_k_sum
from .timemix import layer_norm_shift_mix, layer_norm_shift_mix_fork, token_shift_mix
from .language import weighted_key_value
from .wkv import GATED_TIME_MIX, weighted_key_value_gated


@dataclass
class SpikeGPTConfig:
    """``SpikeGPTConfig`` of ``language.py:234-281`` (same fields and defaults)."""

    vocab_size: int
    context_length: int
    n_layer: int = 4
    n_embd: int = 128
    dropout: float = 0.03
    model_type: str = "rwkv"
    attention: str = "rwkv"
    n_head: int = 8
    rope_base: float = 10000.0
    lif_tau: float = 2.0
    lif_threshold: float = 1.0
    lif_reset: float = 0.0
    surrogate_slope: float = 2.0
    spike_embedding: bool = True
    spiking: bool = True
    spike_input: bool = False
    gradient_checkpointing: bool = False

    def validate(self) -> None:
        if self.vocab_size <= 0:
            raise ValueError("vocab_size must be positive")
        if self.context_length <= 0:
            raise ValueError("context_length must be positive")
        if self.n_layer <= 0:
            raise ValueError("n_layer must be positive")
        if self.n_embd <= 0:
            raise ValueError("n_embd must be positive")
        if self.dropout < 0.0 or self.dropout >= 1.0:
            raise ValueError("dropout must be in [0, 1)")
        if self.lif_tau <= 0.0:
            raise ValueError("lif_tau must be positive")
        if self.model_type != "rwkv" or self.attention != "rwkv" or self.spike_input:
            raise NotImplementedError(
                "this build serves model_type='rwkv', attention='rwkv', spike_input=False"
            )


class _HeavisideAtan(torch.autograd.Function):
    """Hard spike with the arctan surrogate gradient (the embedding spike of
    ``language.py:1386-1394``): forward ``[x >= 0]``, backward
    ``0.5 / (1 + (pi/2 x)^2)``."""

    @staticmethod
    def forward(ctx, x: Tensor) -> Tensor:  # noqa: D102
        ctx.save_for_backward(x)
        return (x >= 0).to(x.dtype)

    @staticmethod
    def backward(ctx, grad: Tensor) -> Tensor:  # noqa: D102
        (x,) = ctx.saved_tensors
        q = (torch.pi / 2) * x.float()
        return (grad.float() * (0.5 / (1.0 + q * q))).to(grad.dtype)


class _SplitKLinearFn(torch.autograd.Function):
    """``x @ weight.T`` whose weight gradient sums S independent GEMMs over
    slices of the B*T rows (fp32 outputs, then the fixed-order fp32 sum of
    :func:`split_k_sum`).  With
    B*T = 65536 rows and a 512x512 weight, the one-GEMM weight gradient has
    only a few dozen output tiles for 256 CUs; S slices give S times as many.
    Forward and input gradient are the ordinary GEMMs; the computation dtype
    is the active CUDA autocast dtype, as ``nn.Linear`` under autocast."""

    @staticmethod
    def forward(ctx, x: Tensor, weight: Tensor, splits: int) -> Tensor:  # noqa: D102
        dt = torch.get_autocast_dtype("cuda") if torch.is_autocast_enabled("cuda") else x.dtype
        with torch.autocast("cuda", enabled=False):
            xc, wc = x.to(dt), weight.to(dt)
            y = torch.matmul(xc, wc.t())
        ctx.save_for_backward(xc, wc)
        ctx.splits = splits
        ctx.weight_dtype = weight.dtype
        return y

    @staticmethod
    def backward(ctx, grad: Tensor):  # noqa: D102
        xc, wc = ctx.saved_tensors
        grad = grad.to(wc.dtype)
        with torch.autocast("cuda", enabled=False):
            gx = torch.matmul(grad, wc)
            rows = grad.numel() // grad.shape[-1]
            s = ctx.splits
            g3 = grad.reshape(s, rows // s, grad.shape[-1])
            x3 = xc.reshape(s, rows // s, xc.shape[-1])
            # [S, out, in] = g3^T @ x3: the transposed view is the left
            # operand; the right one is contiguous.
            parts = torch.bmm(g3.transpose(1, 2), x3, out_dtype=torch.float32)
        return gx, split_k_sum(parts).to(ctx.weight_dtype), None


class SplitKLinear(nn.Linear):
    """``nn.Linear`` (same parameters and state-dict names) with the split-K
    weight gradient of :class:`_SplitKLinearFn` when the input has enough
    rows; falls back to ``nn.Linear`` otherwise (and on non-CUDA tensors)."""

    min_rows_per_split = 2048
    splits = 16

    def forward(self, x: Tensor) -> Tensor:
        rows = x.numel() // x.shape[-1]
        if (self.bias is not None or not x.is_cuda or not torch.is_grad_enabled()
                or rows % self.splits != 0 or rows // self.splits < self.min_rows_per_split):
            return super().forward(x)
        return _SplitKLinearFn.apply(x, self.weight, self.splits)


class SpikingSequenceLIF(nn.Module):
    """``language.py:766-918``: LIF over ``[B, T, C]`` in one HIP kernel.

    The constructor takes the reference's arguments (``:769-781``).  What the
    kernels compute is the reference's fused path for the arctan surrogate
    with a Heaviside forward; ``fused`` and ``recompute`` are accepted and
    change nothing in the values: the reference's per-step loop (``fused=False``)
    performs the same float32 operations in the same order as the kernels,
    and the kernels always recompute inside 32-step blocks from membrane
    records (the reference's ``recompute`` trades memory the same way).  A
    surrogate other than the arctan one, or ``hard_forward=False`` (a smooth
    forward ``spike = surrogate(c)``), raises ``NotImplementedError`` here,
    so such a module never reaches the kernels."""

    def __init__(self, *, tau: float = 2.0, threshold: float = 1.0, reset: float = 0.0,
                 surrogate=atan_surrogate, surrogate_slope: float = 2.0,
                 hard_forward: bool = True, fused: bool = True, recompute: bool = False) -> None:
        super().__init__()
        if tau <= 0.0:
            raise ValueError("tau must be positive")
        if not serves_surrogate(surrogate, hard_forward):
            what = ("hard_forward=False (smooth forward spikes)" if not hard_forward
                    else f"surrogate {getattr(surrogate, '__name__', surrogate)!r}")
            raise NotImplementedError(
                f"SpikingSequenceLIF: the HIP LIF kernels serve the arctan surrogate with "
                f"hard_forward=True; {what} is not served")
        self.tau = tau
        self.threshold = threshold
        self.reset = reset
        self.surrogate = surrogate
        self.surrogate_slope = surrogate_slope
        self.hard_forward = hard_forward
        self.fused = fused
        self.recompute = recompute

    @property
    def decay(self) -> float:
        return 1.0 - (1.0 / self.tau)

    def forward(self, inputs: Tensor) -> Tensor:
        if inputs.ndim != 3:
            raise ValueError(f"inputs must have shape [B, T, C]; got {inputs.shape}")
        return lif_sequence(inputs, tau=self.tau, threshold=self.threshold, reset=self.reset,
                            surrogate_slope=self.surrogate_slope)


def _add_lif(residual: Tensor, lif: nn.Module, x: Tensor) -> Tensor:
    """``residual + lif(x)``; a spiking LIF writes its spikes straight into the
    fp32 residual (``myelin::lif_residual_forward``)."""
    if isinstance(lif, SpikingSequenceLIF):
        return lif_residual(residual, x, tau=lif.tau, threshold=lif.threshold, reset=lif.reset,
                            surrogate_slope=lif.surrogate_slope)
    return residual + lif(x)


class SpikeTimeMix(nn.Module):
    """``language.py:921-1036``: token-shift mixes, k/v/r projections, WKV,
    ``sigmoid(r) * wkv`` and the output projection."""

    def __init__(self, n_embd: int, n_layer: int, layer_id: int) -> None:
        super().__init__()
        if n_embd <= 0:
            raise ValueError("n_embd must be positive")
        attn = n_embd
        ratio_0_to_1 = layer_id / max(1, n_layer - 1)
        ratio_1_to_almost0 = 1.0 - (layer_id / n_layer)
        position = torch.arange(n_embd, dtype=torch.float32) / n_embd
        # Initialisation of language.py:938-950.
        decay_speed = -5.0 + 8.0 * torch.pow(
            torch.arange(attn, dtype=torch.float32) / max(1, attn - 1), 0.7 + 1.3 * ratio_0_to_1
        )
        zigzag = torch.tensor([(i + 1) % 3 - 1 for i in range(attn)], dtype=torch.float32)
        self.time_decay = nn.Parameter(decay_speed)
        self.time_first = nn.Parameter(torch.ones(attn) * -1.2039728 + zigzag * 0.5)
        self.time_mix_k = nn.Parameter(torch.pow(position, ratio_1_to_almost0).view(1, 1, -1))
        self.time_mix_v = nn.Parameter(
            (torch.pow(position, ratio_1_to_almost0) + 0.3 * ratio_0_to_1).view(1, 1, -1)
        )
        self.time_mix_r = nn.Parameter(torch.pow(position, 0.5 * ratio_1_to_almost0).view(1, 1, -1))
        self.key = SplitKLinear(n_embd, attn, bias=False)
        self.value = SplitKLinear(n_embd, attn, bias=False)
        self.receptance = SplitKLinear(n_embd, attn, bias=False)
        self.output = SplitKLinear(attn, n_embd, bias=False)

    def mixes(self) -> Tensor:
        """The k, v, r mixing vectors stacked ``[3, C]``."""
        return torch.stack([self.time_mix_k.view(-1), self.time_mix_v.view(-1),
                            self.time_mix_r.view(-1)])

    def forward(self, inputs: Tensor) -> Tensor:
        return self.project(*token_shift_mix(inputs, self.mixes()))

    def project(self, k_in: Tensor, v_in: Tensor, r_in: Tensor) -> Tensor:
        """Everything after the token-shift mixes (``language.py:1019-1036``)."""
        key = self.key(k_in)
        value = self.value(v_in)
        receptance = self.receptance(r_in)
        if GATED_TIME_MIX:
            # sigmoid(r) * wkv with the gate folded into the WKV kernels.
            gated = weighted_key_value_gated(key, value, self.time_decay, self.time_first,
                                             receptance)
        else:
            gated = sigmoid_gate(receptance, weighted_key_value(key, value, self.time_decay,
                                                                self.time_first))
        return self.output(gated)


class SpikeChannelMix(nn.Module):
    """``language.py:1145-1196``: squared-ReLU feed-forward with a receptance gate."""

    def __init__(self, n_embd: int, n_layer: int, layer_id: int) -> None:
        super().__init__()
        ratio_1_to_almost0 = 1.0 - (layer_id / n_layer)
        position = torch.arange(n_embd, dtype=torch.float32) / n_embd
        self.time_mix_k = nn.Parameter(torch.pow(position, ratio_1_to_almost0).view(1, 1, -1))
        self.time_mix_r = nn.Parameter(torch.pow(position, ratio_1_to_almost0).view(1, 1, -1))
        self.key = SplitKLinear(n_embd, 4 * n_embd, bias=False)
        self.receptance = SplitKLinear(n_embd, n_embd, bias=False)
        self.value = SplitKLinear(4 * n_embd, n_embd, bias=False)

    def mixes(self) -> Tensor:
        """The k, r mixing vectors stacked ``[2, C]``."""
        return torch.stack([self.time_mix_k.view(-1), self.time_mix_r.view(-1)])

    def forward(self, inputs: Tensor) -> Tensor:
        return self.project(*token_shift_mix(inputs, self.mixes()))

    def project(self, k_in: Tensor, r_in: Tensor) -> Tensor:
        """Everything after the token-shift mixes (``language.py:1192-1196``)."""
        key = relu_square(self.key(k_in))
        return sigmoid_gate(self.receptance(r_in), self.value(key))


class SpikeGPTBlock(nn.Module):
    """``language.py:1223-1360``: ``x + LIF(att(ln1 x))``, then ``+ LIF(ffn(ln2 x))``."""

    def __init__(self, config: SpikeGPTConfig, layer_id: int) -> None:
        super().__init__()
        self.config = config
        self.layer_id = layer_id
        self.ln0 = nn.LayerNorm(config.n_embd) if layer_id == 0 else None
        self.ln1 = nn.LayerNorm(config.n_embd)
        self.ln2 = nn.LayerNorm(config.n_embd)
        self.att = SpikeTimeMix(config.n_embd, config.n_layer, layer_id)
        self.ffn = SpikeChannelMix(config.n_embd, config.n_layer, layer_id)

        def make_lif() -> nn.Module:
            if not config.spiking:
                return nn.Identity()
            return SpikingSequenceLIF(tau=config.lif_tau, threshold=config.lif_threshold,
                                      reset=config.lif_reset,
                                      surrogate_slope=config.surrogate_slope)

        self.lif1 = make_lif()
        self.lif2 = make_lif()
        self.dropout = nn.Dropout(config.dropout)

    def initial_state(self, *, batch_size: int, device: torch.device | None = None,
                      dtype: torch.dtype | None = None) -> SpikeGPTBlockState:
        """``language.py:1270-1299``: zero state, log-scale at finfo(fp32).min
        (fp32 whatever ``dtype`` says)."""
        dev = self.ln1.weight.device if device is None else torch.device(device)
        return state_from_packed(initial_packed(1, batch_size, self.config.n_embd, dev)).blocks[0]

    def step(self, inputs: Tensor, state: SpikeGPTBlockState) -> tuple[Tensor, SpikeGPTBlockState]:
        """``language.py:1301-1335``: one token through the block (the fused
        block-step kernels, fp32, eval semantics)."""
        if inputs.ndim != 2:
            raise ValueError(f"inputs must have shape [B, C]; got {inputs.shape}")
        src = pack_state(SpikeLanguageModelState(blocks=(state,)))[0]
        dst = torch.empty_like(src)
        ws = StepWorkspace(inputs.shape[0], self.config.n_embd, self.ffn.key.out_features, 1,
                           inputs.device)
        out = block_step(self, inputs.float().contiguous(), src, dst, ws)
        return out.clone(), state_from_packed(dst.unsqueeze(0)).blocks[0]

    def forward(self, inputs: Tensor) -> Tensor:
        # att(ln1(x)) and ffn(ln2(x)) with each layer norm folded into the
        # half's token-shift kernel; the residual stream is taken back from
        # that op (layer_norm_shift_mix_fork), so its two gradients are summed
        # inside the fused backward kernel.
        residual = self.ln0(inputs) if self.ln0 is not None else inputs
        *mixed, residual = layer_norm_shift_mix_fork(residual, self.ln1, self.att.mixes())
        residual = _add_lif(residual, self.lif1, self.att.project(*mixed))
        *mixed, residual = layer_norm_shift_mix_fork(residual, self.ln2, self.ffn.mixes())
        residual = _add_lif(residual, self.lif2, self.ffn.project(*mixed))
        return self.dropout(residual)


class SpikeLanguageModel(nn.Module):
    """``language.py:1363-1480``: spiking embedding, blocks, ``ln_out``, head."""

    def __init__(self, config: SpikeGPTConfig) -> None:
        super().__init__()
        config.validate()
        self.config = config
        self.embedding = nn.Embedding(config.vocab_size, config.n_embd)
        self.blocks = nn.ModuleList(SpikeGPTBlock(config, i) for i in range(config.n_layer))
        self.ln_out = nn.LayerNorm(config.n_embd)
        self.head = SplitKLinear(config.n_embd, config.vocab_size, bias=False)
        self.gradient_checkpointing = config.gradient_checkpointing
        self.apply(self._init_weights)

    @staticmethod
    def _init_weights(module: nn.Module) -> None:
        # language.py:1378-1384
        if isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=1.0e-3)
        elif isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=0.01)
            if module.bias is not None:
                nn.init.zeros_(module.bias)

    def embed_tokens(self, input_ids: Tensor) -> Tensor:
        embeddings = self.embedding(input_ids)
        if not self.config.spike_embedding:
            return embeddings
        return _HeavisideAtan.apply(self.config.surrogate_slope * embeddings)

    def forward(self, input_ids: Tensor, targets: Tensor | None = None):
        if input_ids.ndim != 2:
            raise ValueError(f"input_ids must have shape [B, T]; got {input_ids.shape}")
        if input_ids.shape[1] > self.config.context_length:
            raise ValueError(
                "input sequence length exceeds context_length; "
                f"got {input_ids.shape[1]} and {self.config.context_length}"
            )
        hidden = self.embed_tokens(input_ids)
        for block in self.blocks:
            hidden = self._run_block(block, hidden)
        if targets is None:
            return self.head(self.ln_out(hidden))
        return self.loss_tail(hidden, targets)

    def set_gradient_checkpointing(self, enabled: bool = True) -> None:
        """``language.py:1396-1399``: block-level activation checkpointing."""
        self.gradient_checkpointing = enabled

    def _run_block(self, block: nn.Module, hidden: Tensor) -> Tensor:
        """``language.py:1401-1404``: with checkpointing on (training, grad
        enabled), a block keeps only its input and is recomputed in the
        backward; the HIP ops' autograd Functions recompute like any other."""
        if self.gradient_checkpointing and self.training and torch.is_grad_enabled():
            return torch.utils.checkpoint.checkpoint(block, hidden, use_reentrant=False)
        return block(hidden)

    def loss_tail(self, hidden: Tensor, targets: Tensor) -> tuple[Tensor, Tensor]:
        """``language.py:1469-1480``: ``ln_out -> head -> cross_entropy``."""
        logits = self.head(self.ln_out(hidden))
        loss = F.cross_entropy(logits.reshape(-1, logits.shape[-1]), targets.reshape(-1))
        return loss, logits

    # ------------------------------------------------ recurrent generation --
    def initial_state(self, *, batch_size: int, device: torch.device | None = None,
                      dtype: torch.dtype | None = None) -> SpikeLanguageModelState:
        """``language.py:1410-1432`` (fp32 state whatever ``dtype`` says)."""
        return generation.initial_state(self, batch_size=batch_size, device=device, dtype=dtype)

    def forward_step(self, input_ids: Tensor,
                     state: SpikeLanguageModelState) -> tuple[Tensor, SpikeLanguageModelState]:
        """``language.py:1434-1453``: one token for every batch row through
        the fused block-step kernels; returns logits [B, vocab] and the new
        state (the given state is not modified)."""
        return generation.forward_step(self, input_ids, state)

    @torch.no_grad()
    def generate(self, input_ids: Tensor, *, max_new_tokens: int, temperature: float = 1.0,
                 top_k: int | None = None, sampling: str = "multinomial",
                 use_cache: bool = True, use_graph: bool = True) -> Tensor:
        """``language.py:1455-1524``.  ``use_cache`` runs the recurrent state
        (``use_graph``: one captured HIP graph per token); otherwise the
        context window is recomputed with the sequence forward each token."""
        was_training = self.training
        self.eval()
        try:
            if use_cache:
                new = list(generation.generate_tokens(
                    self, input_ids, max_new_tokens=max_new_tokens, temperature=temperature,
                    top_k=top_k, sampling=sampling, use_graph=use_graph))
                return torch.cat([input_ids, *new], dim=1)
            generation._check_generate_args(input_ids, max_new_tokens, temperature, top_k,
                                            sampling)
            output = input_ids
            for _ in range(max_new_tokens):
                logits = self(output[:, -self.config.context_length:])
                nxt = generation.sample_next_token(logits[:, -1], temperature=temperature,
                                                   top_k=top_k, sampling=sampling)
                output = torch.cat((output, nxt), dim=1)
            return output
        finally:
            if was_training:
                self.train()

    def generate_stream(self, input_ids: Tensor, *, max_new_tokens: int,
                        temperature: float = 1.0, top_k: int | None = None,
                        sampling: str = "multinomial", use_graph: bool = True):
        """``language.py:1526-1573``: yields one [B, 1] token per step, sampled
        as :meth:`generate` with ``use_cache=True``."""
        was_training = self.training
        self.eval()
        try:
            with torch.no_grad():
                yield from generation.generate_tokens(
                    self, input_ids, max_new_tokens=max_new_tokens, temperature=temperature,
                    top_k=top_k, sampling=sampling, use_graph=use_graph)
        finally:
            if was_training:
                self.train()
