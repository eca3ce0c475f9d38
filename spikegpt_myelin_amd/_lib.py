"""ctypes binding of libwkv_hip.so (the C ABI declared in include/wkv_hip.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime
torch already loaded (both carry the soname ``libamdhip64.so.7``); the stream
handles torch hands out are then valid in the library.  There is no fallback:
if the shared library is missing the first call raises ``RuntimeError`` naming
the build command.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  -- must load torch's HIP runtime first

LIB_PATH = Path(__file__).resolve().parent / "libwkv_hip.so"

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2

_TORCH_TO_CODE = {
    torch.float32: DTYPE_F32,
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
}

_P = ctypes.c_void_p


class StepRowArgs(ctypes.Structure):
    """``wkv_step_row_args`` of ``include/wkv_hip.h`` (argument block of
    ``block_step_row``); pointer fields hold device addresses as ints."""

    _fields_ = [
        ("ids", _P), ("embedding", _P), ("vocab", ctypes.c_int64),
        ("embedding_slope", ctypes.c_float), ("embedding_spike", ctypes.c_int),
        ("ln0_weight", _P), ("ln0_bias", _P),
        ("add", _P), ("gate", _P), ("membrane_in", _P), ("membrane_out", _P),
        ("lif_decay", ctypes.c_float), ("lif_threshold", ctypes.c_float),
        ("lif_reset", ctypes.c_float), ("lif_slope", ctypes.c_float),
        ("spiking", ctypes.c_int),
        ("residual", _P), ("ln_weight", _P), ("ln_bias", _P), ("ln_eps", ctypes.c_float),
        ("mix", _P * 3), ("n_mix", ctypes.c_int), ("previous_in", _P), ("previous_out", _P),
        ("out", _P * 3), ("batch", ctypes.c_int64), ("channels", ctypes.c_int64),
    ]


# Every exported entry point: name -> (restype, argtypes).
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_SZ = ctypes.c_size_t
_F = ctypes.c_float
SIGNATURES = {
    "wkv4_forward_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "wkv4_forward": (_INT, [_P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _INT, _P]),
    "wkv4_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64, _INT]),
    "wkv4_backward": (
        _INT,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _INT, _P],
    ),
    "wkv4_backward_noalloc": (
        _INT,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _INT, _P],
    ),
    "wkv4_checkpoint_bytes": (_SZ, [_I64, _I64, _I64]),
    "wkv4_forward_checkpointed": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _INT, _P]),
    "wkv4_backward_checkpointed_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "wkv4_forward_gated_checkpointed": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _INT, _P]),
    "wkv4_backward_gated_checkpointed": (
        _INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _INT, _P]),
    "wkv4_backward_checkpointed": (
        _INT,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _INT, _P],
    ),
    "wkv4_decode_step": (_INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _INT, _P]),
    "wkv7_forward": (_INT, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P]),
    "wkv7_checkpoint_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "wkv7_forward_checkpointed": (
        _INT,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _INT, _P],
    ),
    "wkv7_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "wkv7_backward": (
        _INT,
        [_P] * 16 + [_P, _SZ, _I64, _I64, _I64, _I64, _INT, _P],
    ),
    "wkv7_backward_checkpointed": (
        _INT,
        [_P] * 16 + [_I64, _I64, _I64, _I64, _INT, _P],
    ),
    "lif_checkpoint_bytes": (_SZ, [_I64, _I64, _I64]),
    "lif_forward_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "lif_forward": (
        _INT,
        [_P, _P, _P, _P, _SZ, _I64, _I64, _I64, _F, _F, _F, _F, _INT, _P],
    ),
    "lif_backward_workspace_bytes": (_SZ, [_I64, _I64, _I64]),
    "lif_backward": (
        _INT,
        [_P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _F, _F, _F, _F, _INT, _P],
    ),
    "lif_residual_forward": (
        _INT, [_P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _F, _F, _F, _F, _INT, _P]),
    "lif_residual_backward": (
        _INT, [_P, _P, _P, _P, _P, _SZ, _I64, _I64, _I64, _F, _F, _F, _F, _INT, _P]),
    "token_shift_mix_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "token_shift_mix_forward": (
        _INT,
        [_P, _INT, _P, _I64, _P, _P, _P, _INT, _I64, _I64, _I64, _P],
    ),
    "token_shift_mix_backward": (
        _INT,
        [_P, _INT, _P, _I64, _P, _P, _P, _INT, _P, _P, _P, _SZ, _I64, _I64, _I64, _P],
    ),
    "split_k_sum": (_INT, [_P, _P, _I64, _I64, _P]),
    "relu_square_forward": (_INT, [_P, _P, _I64, _INT, _P]),
    "relu_square_backward": (_INT, [_P, _P, _P, _I64, _INT, _P]),
    "sigmoid_gate_forward": (_INT, [_P, _P, _P, _I64, _INT, _P]),
    "sigmoid_gate_backward": (_INT, [_P, _P, _P, _P, _P, _I64, _INT, _P]),
    "layer_norm_shift_mix_forward": (
        _INT, [_P, _P, _P, _F, _P, _I64, _P, _P, _P, _INT, _P, _P, _I64, _I64, _I64, _P]),
    "layer_norm_shift_mix_workspace_bytes": (_SZ, [_I64, _I64, _I64, _I64]),
    "layer_norm_shift_mix_backward": (
        _INT, [_P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _INT, _P, _P, _P, _P, _SZ, _I64, _I64,
               _I64, _P]),
    "block_step_row": (_INT, [_INT, ctypes.POINTER(StepRowArgs), _P]),
    "block_step_wkv": (_INT, [_P] * 12 + [_I64, _I64, _P]),
    "wkv_time_next_call": (_INT, [_P, _P]),
    "wkv_time_next_kernel": (_INT, [_P, _P, _INT]),
    "wkv_last_error_string": (ctypes.c_char_p, []),
    "wkv_version": (ctypes.c_char_p, []),
}

# Optional timing hook: when set to a list, every C ABI launch made through
# ``timed`` appends (name, start_event, end_event), the events carried by the
# launch's first and last kernel dispatch (``wkv_time_next_call``).  None (the
# default) costs nothing.
EVENT_LOG: list | None = None

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library with typed entry points."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m spikegpt_myelin_amd.build` "
                "(the WKV ops have no non-HIP implementation)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_TO_CODE[dtype]
    except KeyError:
        raise TypeError(f"WKV kernels take float32, bfloat16 or float16 tensors; got {dtype}") from None


def check(rc: int, what: str) -> None:
    """Map a nonzero C ABI status to ``RuntimeError`` with the library's message."""
    if rc != 0:
        msg = load().wkv_last_error_string().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def aligned(t: torch.Tensor) -> torch.Tensor:
    """``t`` contiguous with a 16-byte-aligned base address (copied if not)."""
    t = t.contiguous()
    if t.data_ptr() % 16:
        t = t.clone()
    return t


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def timed(name: str, device: torch.device, call):
    """Run ``call()`` (one C ABI entry point); when ``EVENT_LOG`` is a list,
    time its kernels with events bound to their dispatches."""
    if EVENT_LOG is None:
        return call()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    arm_events(start, end)
    rc = call()
    EVENT_LOG.append((name, start, end))
    return rc


def arm_events(start: torch.cuda.Event, end: torch.cuda.Event, kernel: int | None = None) -> None:
    """Bind ``start``/``end`` to the first/last kernel dispatch of the next C ABI
    call on this thread (kernel start and end timestamps, no marker packets),
    or, with ``kernel``, both to that call's ``kernel``-th dispatch alone."""
    for ev in (start, end):
        if ev.cuda_event == 0:
            # torch creates the HIP event lazily at its first record.
            ev.record(torch.cuda.current_stream())
    if kernel is None:
        load().wkv_time_next_call(start.cuda_event, end.cuda_event)
    else:
        check(load().wkv_time_next_kernel(start.cuda_event, end.cuda_event, kernel),
              "wkv_time_next_kernel")


def stream_of(t: torch.Tensor) -> int:
    """The calling thread's current HIP stream on ``t``'s device (the raw
    handle, without building a ``torch.cuda.Stream`` object per call)."""
    return torch._C._cuda_getCurrentRawStream(t.get_device())


def require_gpu(*tensors: torch.Tensor) -> None:
    """The ops run only on a HIP device; there is no CPU implementation."""
    for t in tensors:
        if t.device.type != "cuda":
            raise RuntimeError(
                "myelin WKV ops run on the GPU (HIP) only; got a tensor on "
                f"{t.device}. Move inputs to the GPU."
            )
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"all tensors must be on one device; got {dev} and {t.device}")
