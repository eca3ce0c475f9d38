"""Checkpoint format ``"myelin.spike_language_checkpoint.v1"`` and vocabularies.

Reads and writes the reference's SpikeGPT checkpoints
(``src/spikegpt/language.py:1741-1801``): one ``torch.save`` payload, a dict
with

* ``"format"``: ``"myelin.spike_language_checkpoint.v1"``;
* ``"config"``: the ``SpikeGPTConfig`` fields as a plain dict (``:1664-1703``);
* ``"vocabulary"``: ``{"type": "byte"}``, ``{"type": "character", "tokens":
  [...]}`` or ``{"type": "bpe", "tokenizer_json": ..., "vocab_size": n}``
  (``:1706-1738``);
* ``"state_dict"``: the model's parameters under the reference's names (this
  package's model uses the same names);
* ``"metadata"``: a dict; optional ``"optimizer_state_dict"``.

Loading uses ``torch.load(..., weights_only=True)``, which rebuilds tensors
and plain containers only and executes nothing from the file.  Keys saved
from a ``torch.compile``d model carry ``._orig_mod.`` segments; they are
stripped, as the reference's loader does (``:1783-1788``).
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field
from os import PathLike
from typing import Any, Mapping, Union

import torch
from torch import Tensor

from .model import SpikeGPTConfig, SpikeLanguageModel

FORMAT = "myelin.spike_language_checkpoint.v1"

__all__ = [
    "FORMAT", "CharacterVocabulary", "ByteVocabulary", "BPEVocabulary", "LanguageVocabulary",
    "SpikeLanguageCheckpoint", "spikegpt_config_to_dict", "spikegpt_config_from_dict",
    "language_vocabulary_to_dict", "language_vocabulary_from_dict",
    "save_spike_language_checkpoint", "load_spike_language_checkpoint",
]


# ------------------------------------------------------------ vocabularies --
@dataclass(frozen=True)
class CharacterVocabulary:
    """Sorted set of characters (``language.py:54-82``)."""

    tokens: tuple[str, ...]

    @classmethod
    def from_text(cls, text: str) -> "CharacterVocabulary":
        if not text:
            raise ValueError("text must not be empty")
        return cls(tuple(sorted(set(text))))

    @property
    def size(self) -> int:
        return len(self.tokens)

    @property
    def token_to_id(self) -> dict[str, int]:
        return {t: i for i, t in enumerate(self.tokens)}

    def encode(self, text: str) -> Tensor:
        index = self.token_to_id
        missing = sorted(set(text) - set(index))
        if missing:
            raise ValueError(f"text contains out-of-vocabulary characters: {missing}")
        return torch.tensor([index[ch] for ch in text], dtype=torch.long)

    def decode(self, token_ids: Tensor) -> str:
        return "".join(self.tokens[i] for i in token_ids.tolist())


@dataclass(frozen=True)
class ByteVocabulary:
    """UTF-8 bytes, 256 ids (``language.py:85-106``)."""

    @classmethod
    def from_text(cls, text: str) -> "ByteVocabulary":
        if not text:
            raise ValueError("text must not be empty")
        return cls()

    @property
    def size(self) -> int:
        return 256

    def encode(self, text: str) -> Tensor:
        if not text:
            raise ValueError("text must not be empty")
        return torch.tensor(list(text.encode("utf-8")), dtype=torch.long)

    def decode(self, token_ids: Tensor) -> str:
        return bytes(token_ids.detach().cpu().tolist()).decode("utf-8", errors="replace")


@dataclass(frozen=True)
class BPEVocabulary:
    """A ``tokenizers`` BPE tokenizer stored inline as its JSON
    (``language.py:109-158``); needs the ``tokenizers`` package, imported on
    first use."""

    tokenizer_json: str
    vocab_size: int
    _tokenizer: Any = field(init=False, repr=False, compare=False, default=None)

    def __post_init__(self) -> None:
        from tokenizers import Tokenizer

        object.__setattr__(self, "_tokenizer", Tokenizer.from_str(self.tokenizer_json))

    @classmethod
    def from_tokenizer_file(cls, path: Union[str, PathLike]) -> "BPEVocabulary":
        from tokenizers import Tokenizer

        tok = Tokenizer.from_file(str(path))
        return cls(tokenizer_json=tok.to_str(), vocab_size=tok.get_vocab_size())

    @property
    def size(self) -> int:
        return self.vocab_size

    def encode(self, text: str) -> Tensor:
        if not text:
            raise ValueError("text must not be empty")
        return torch.tensor(self._tokenizer.encode(text).ids, dtype=torch.long)

    def encode_batch(self, texts: list[str]) -> list[list[int]]:
        return [e.ids for e in self._tokenizer.encode_batch(texts)]

    def decode(self, token_ids: Tensor) -> str:
        return self._tokenizer.decode(token_ids.detach().cpu().tolist())


LanguageVocabulary = Union[CharacterVocabulary, ByteVocabulary, BPEVocabulary]


@dataclass(frozen=True)
class SpikeLanguageCheckpoint:
    """A loaded checkpoint (``language.py:172-179``)."""

    model: SpikeLanguageModel
    vocabulary: LanguageVocabulary
    metadata: dict[str, object]
    optimizer_state_dict: dict[str, Any] | None = None


# ------------------------------------------------------------- validation --
def _mapping(value: object, name: str) -> Mapping[str, object]:
    if not isinstance(value, Mapping):
        raise ValueError(f"{name} must be a mapping")
    return value


def _typed(value: object, name: str, kind) -> Any:
    # The reference's checks (language.py:1640-1661): isinstance against bool,
    # int, int | float or str; numeric values come back as float.
    ok = isinstance(value, (int, float)) if kind is float else isinstance(value, kind)
    if not ok:
        what = {bool: "a bool", int: "an int", float: "numeric", str: "a string"}[kind]
        raise ValueError(f"{name} must be {what}")
    return float(value) if kind is float else value


# (field, type, default): defaults keep older checkpoints loadable (:1670-1703).
_CONFIG_FIELDS = (
    ("vocab_size", int, None), ("context_length", int, None), ("n_layer", int, 4),
    ("n_embd", int, 128), ("dropout", float, 0.03), ("model_type", str, "rwkv"),
    ("attention", str, "rwkv"), ("n_head", int, 8), ("rope_base", float, 10000.0),
    ("lif_tau", float, 2.0), ("lif_threshold", float, 1.0), ("lif_reset", float, 0.0),
    ("surrogate_slope", float, 2.0), ("spike_embedding", bool, True), ("spiking", bool, True),
    ("spike_input", bool, False), ("gradient_checkpointing", bool, False),
)


def spikegpt_config_to_dict(config: SpikeGPTConfig) -> dict[str, object]:
    """``language.py:1664-1667``."""
    return dict(asdict(config))


def spikegpt_config_from_dict(data: Mapping[str, object]) -> SpikeGPTConfig:
    """``language.py:1670-1703``; raises ``ValueError`` on a malformed field and
    ``NotImplementedError`` for a variant this package does not run."""
    values = {}
    for name, kind, default in _CONFIG_FIELDS:
        raw = data.get(name, default) if default is not None else data.get(name)
        values[name] = _typed(raw, f"config.{name}", kind)
    config = SpikeGPTConfig(**values)
    config.validate()
    return config


def language_vocabulary_to_dict(vocabulary: LanguageVocabulary) -> dict[str, object]:
    """``language.py:1706-1717``."""
    if isinstance(vocabulary, ByteVocabulary):
        return {"type": "byte"}
    if isinstance(vocabulary, BPEVocabulary):
        return {"type": "bpe", "tokenizer_json": vocabulary.tokenizer_json,
                "vocab_size": vocabulary.vocab_size}
    return {"type": "character", "tokens": list(vocabulary.tokens)}


def language_vocabulary_from_dict(data: Mapping[str, object]) -> LanguageVocabulary:
    """``language.py:1720-1738``."""
    kind = _typed(data.get("type"), "vocabulary.type", str)
    if kind == "byte":
        return ByteVocabulary()
    if kind == "bpe":
        return BPEVocabulary(
            tokenizer_json=_typed(data.get("tokenizer_json"), "vocabulary.tokenizer_json", str),
            vocab_size=_typed(data.get("vocab_size"), "vocabulary.vocab_size", int))
    if kind != "character":
        raise ValueError(f"unsupported vocabulary type: {kind}")
    tokens = data.get("tokens")
    if not isinstance(tokens, list) or not all(isinstance(t, str) for t in tokens):
        raise ValueError("character vocabulary tokens must be a list of strings")
    if not tokens:
        raise ValueError("character vocabulary tokens must not be empty")
    return CharacterVocabulary(tokens=tuple(tokens))


# ------------------------------------------------------------------ files --
def save_spike_language_checkpoint(path: Union[str, PathLike], model: SpikeLanguageModel,
                                   vocabulary: LanguageVocabulary, *,
                                   metadata: Mapping[str, object] | None = None,
                                   optimizer: torch.optim.Optimizer | None = None) -> None:
    """``language.py:1741-1760``: one ``torch.save`` payload."""
    payload: dict[str, object] = {
        "format": FORMAT,
        "config": spikegpt_config_to_dict(model.config),
        "vocabulary": language_vocabulary_to_dict(vocabulary),
        "state_dict": model.state_dict(),
        "metadata": dict(metadata or {}),
    }
    if optimizer is not None:
        payload["optimizer_state_dict"] = optimizer.state_dict()
    torch.save(payload, path)


def load_spike_language_checkpoint(
        path: Union[str, PathLike], *,
        map_location: str | torch.device | None = None) -> SpikeLanguageCheckpoint:
    """``language.py:1763-1801``, with the restricted (``weights_only``) loader."""
    payload = torch.load(path, map_location=map_location, weights_only=True)
    if not isinstance(payload, Mapping):
        raise ValueError("checkpoint payload must be a mapping")
    if payload.get("format") != FORMAT:
        raise ValueError("unsupported SpikeLanguageModel checkpoint format")
    config = spikegpt_config_from_dict(_mapping(payload.get("config"), "config"))
    vocabulary = language_vocabulary_from_dict(_mapping(payload.get("vocabulary"), "vocabulary"))
    raw = payload.get("state_dict")
    if not isinstance(raw, Mapping):
        raise ValueError("checkpoint state_dict must be a mapping")
    state_dict = {k.replace("._orig_mod.", "."): v for k, v in raw.items()}
    model = SpikeLanguageModel(config)
    model.load_state_dict(state_dict)
    metadata = dict(_mapping(payload.get("metadata", {}), "metadata"))
    opt = payload.get("optimizer_state_dict")
    opt = None if opt is None else dict(_mapping(opt, "optimizer_state_dict"))
    return SpikeLanguageCheckpoint(model=model, vocabulary=vocabulary, metadata=metadata,
                                   optimizer_state_dict=opt)
