"""ctypes binding of libmi_attn.so, the gfx950 C-ABI library.

The library is loaded lazily on first use and there is no fallback: if it is
missing or a call fails, a RuntimeError says why. Pointers are passed as
integers (``tensor.data_ptr()``), the HIP stream as the raw handle of torch's
current stream on the tensor's device, read at call time so calls from any
thread (AsyncEngine's worker) launch on that thread's current stream.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libmi_attn.so"

MI_OK = 0
DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F32 = ctypes.c_float

# (restype, argtypes) of every entry point declared in include/mi_attn.h and
# include/mi_model.h.
SIGNATURES = {
    "mi_last_error": (ctypes.c_char_p, []),
    "mi_abi_version": (_I32, []),
    "mi_kv_append": (
        _I32,
        [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _P, _I32, _I32,
         _I32, _I32, _I32, _I32, _I32, _P],
    ),
    "mi_paged_decode_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32]),
    "mi_paged_decode": (
        _I32,
        [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _I32, _P, _P, _I64, _I64,
         _P, _I64, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P],
    ),
    "mi_paged_decode_append": (
        _I32,
        [_P, _I64, _I64, _P, _I64, _I64,
         _P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _I32, _P, _P, _I64, _I64,
         _P, _I64, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P],
    ),
    "mi_paged_decode_noalloc_max_bytes": (_I64, []),
    "mi_paged_decode_append_noalloc": (
        _I32,
        [_P, _I64, _I64, _P, _I64, _I64,
         _P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _I64, _I32, _P, _P, _I64, _I64,
         _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P],
    ),
    "mi_qk_norm_rope_append": (
        _I32,
        [_P, _I64, _P, _P, _F32, _P, _P, _I32, _P, _I32, _P, _P, _I64, _I64, _P, _I64, _I64,
         _P, _P, _I64, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P],
    ),
    "mi_decode_plan_bytes": (_I64, [_I32, _I32, _I32]),
    "mi_decode_plan": (_I32, [_P, _I32, _I32, _I32, _I32, _I32, _P, _I64, _P]),
    "mi_paged_prefill": (
        _I32,
        [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I32, _P, _I64,
         _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P],
    ),
    "mi_paged_prefill_workspace_bytes": (_I64, [_I32, _I32, _I32, _I32, _I32, _I32]),
    "mi_paged_prefill_planned": (
        _I32,
        [_P, _I64, _I64, _P, _P, _I64, _I64, _I64, _P, _P, _P, _I64, _I32, _P, _I64,
         _I64, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _F32, _I32, _P, _I64, _I32,
         _P],
    ),
    "mi_paged_prefill_plan": (
        _I32,
        [_P, _P, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _P, _I64, _P],
    ),
    "mi_gather_kv": (
        _I32,
        [_P, _P, _I64, _I64, _I64, _P, _I64, _I32, _P, _I32, _I32, _P, _P, _I32, _I32,
         _I32, _I32, _I32, _P],
    ),
    "mi_greedy_argmax_state_bytes": (_I64, [_I32]),
    "mi_greedy_argmax": (_I32, [_P, _I64, _I32, _I32, _I32, _P, _P, _I64, _P]),
    "mi_step_metadata": (
        _I32,
        [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _P, _I64, _I32, _P, _P, _P, _P,
         _P],
    ),
    "mi_linear": (_I32, [_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _I32, _P]),
    "mi_linear_swiglu": (_I32, [_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _I32, _I32, _P]),
    "mi_rms_norm_residual": (
        _I32, [_P, _I64, _P, _I64, _P, _F32, _P, _I64, _P, _I64, _I32, _I32, _I32, _P]),
    "mi_silu_mul": (_I32, [_P, _I64, _P, _I64, _I32, _I32, _I32, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Load (once) and return the library; RuntimeError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIBRARY_PATH.exists():
                raise RuntimeError(
                    f"{LIBRARY_PATH.name} is not built; run "
                    "`python -m microinfer_amd.csrc.build` (hipcc, gfx950)"
                )
            lib = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def last_error() -> str:
    return load().mi_last_error().decode(errors="replace")


def check(status: int, what: str) -> None:
    if status != MI_OK:
        raise RuntimeError(f"{what} failed (status {status}): {last_error()}")


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def stream_handle(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def require_device(*tensors: torch.Tensor, what: str) -> None:
    """The product path runs only on the GPU: no CPU fallback exists."""
    for tensor in tensors:
        if tensor is not None and not tensor.is_cuda:
            raise RuntimeError(
                f"{what} runs on the HIP device only; got a {tensor.device} tensor"
            )
