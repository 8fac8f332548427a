"""Dense decoder-layer ops through the HIP library: projections at decode
batch sizes, RMSNorm with the residual sum, and the SwiGLU gate.

The reference runs these as torch in Python: ``FuseLayerNorm``
(microinfer/layer/norm.py:20-35; ``_compiled_add_rms_norm`` :13-16 when its
ops are compiled), the FFN's SwiGLU (``_compiled_swiglu``,
microinfer/layer/transformer.py:12-15, ``FFN.forward`` :82-88) and every
projection as ``F.linear``. Each function here is one HIP launch with the
same result up to float32 summation order; ``supported_*`` tell the caller
when a request is outside what the kernels take (32-bit tensors, more than
64 rows for a projection, unaligned rows) and ``prefer_hip_linear`` when the
HIP projection is measured faster than torch's, so the caller keeps torch for
the rest.
"""

from __future__ import annotations

import torch

from microinfer_amd import _lib

_HALF = (torch.bfloat16, torch.float16)
LINEAR_MAX_ROWS = 64


def _rows_aligned(t: torch.Tensor) -> bool:
    es = t.element_size()
    return (t.dim() == 2 and t.stride(1) == 1 and t.data_ptr() % 16 == 0
            and (t.stride(0) * es) % 16 == 0)


def supported_linear(x: torch.Tensor, weight: torch.Tensor) -> bool:
    return (x.is_cuda and x.dtype in _HALF and weight.dtype == x.dtype and x.dim() == 2
            and weight.dim() == 2 and 0 < x.shape[0] <= LINEAR_MAX_ROWS
            and x.shape[1] == weight.shape[1] and weight.shape[0] % 16 == 0
            and x.shape[1] % 32 == 0 and _rows_aligned(x) and _rows_aligned(weight))


def prefer_hip_linear(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether ``hip_linear`` beats torch's product for this request.

    Measured on MI355X (hipGraph-replayed, the Qwen3-0.6B projections, us per
    launch, HIP against hipBLASLt): at 64 rows QKV 8.1 / 8.5, output 6.1 /
    8.0, gate/up 10.4 / 11.9, down 8.1 / 9.7; at 8 rows 4.1 / 5.9, 5.3 /
    8.1, 6.2 / 8.0, 7.0 / 9.1. The vocabulary projection (151936 columns)
    stays on hipBLASLt past 16 rows (64 rows: 138 against 85)."""
    if not supported_linear(x, weight):
        return False
    return x.shape[0] <= 16 or weight.shape[0] <= 32768


def hip_linear(x: torch.Tensor, weight: torch.Tensor, *,
               out: torch.Tensor | None = None) -> torch.Tensor:
    """``F.linear(x, weight)`` for ``x [m <= 64, k]``, ``weight [n, k]``."""
    _lib.require_device(x, weight, out, what="dense projection")
    if not supported_linear(x, weight):
        raise ValueError("hip_linear: x [m <= 64, k] and weight [n % 16 == 0, k % 32 == 0] "
                         "of one 16-bit dtype with 16-byte aligned rows are required")
    m, k = x.shape
    n = weight.shape[0]
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=x.device)
    elif out.shape != (m, n) or out.dtype != x.dtype or not _rows_aligned(out):
        raise ValueError("hip_linear: out must be [m, n] of x's dtype with aligned rows")
    _lib.check(_lib.load().mi_linear(
        x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), out.data_ptr(),
        out.stride(0), m, n, k, _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)),
        "mi_linear")
    return out


def hip_linear_swiglu(x: torch.Tensor, gate_up: torch.Tensor, *,
                      out: torch.Tensor | None = None) -> torch.Tensor:
    """``F.silu(gate) * up`` of ``gate, up = F.linear(x, gate_up).chunk(2, -1)``
    (``FFN.forward``, transformer.py:82-88) in one launch: ``gate_up [2 I, k]``
    holds the gate's rows then the up projection's; the result ``[m, I]`` is
    ``hip_silu_mul(hip_linear(x, gate_up))`` bit for bit."""
    _lib.require_device(x, gate_up, out, what="gate/up projection")
    if not supported_linear(x, gate_up) or gate_up.shape[0] % 32:
        raise ValueError("hip_linear_swiglu: x [m <= 64, k] and gate_up [2 I, k] (I % 16 == 0, "
                         "k % 32 == 0) of one 16-bit dtype with 16-byte aligned rows are "
                         "required")
    m, k = x.shape
    inter = gate_up.shape[0] // 2
    if out is None:
        out = torch.empty((m, inter), dtype=x.dtype, device=x.device)
    elif out.shape != (m, inter) or out.dtype != x.dtype or not _rows_aligned(out):
        raise ValueError("hip_linear_swiglu: out must be [m, I] of x's dtype with aligned rows")
    _lib.check(_lib.load().mi_linear_swiglu(
        x.data_ptr(), x.stride(0), gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(),
        out.stride(0), m, inter, k, _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)),
        "mi_linear_swiglu")
    return out


def supported_rows(*tensors: torch.Tensor) -> bool:
    """Whether the norm / SwiGLU kernels take these ``[rows, dim]`` tensors."""
    first = tensors[0]
    return all(t is None or (t.is_cuda and t.dtype == first.dtype and t.dtype in _HALF
                             and _rows_aligned(t)) for t in tensors)


def hip_rms_norm_residual(x: torch.Tensor, residual: torch.Tensor | None, weight: torch.Tensor,
                          eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """``FuseLayerNorm.forward`` (norm.py:26-35): returns
    ``(rms_norm(x + residual) * weight, x + residual)``; with no residual the
    sum is ``x`` itself (returned, not copied)."""
    _lib.require_device(x, residual, weight, what="RMSNorm")
    rows, dim = x.shape
    if not supported_rows(x, residual) or weight.dtype != x.dtype or weight.shape != (dim,) \
            or dim % 8 or dim > 8192 or weight.data_ptr() % 16:
        raise ValueError("hip_rms_norm_residual: 16-bit [rows, dim % 8 == 0] tensors with "
                         "aligned rows and a matching [dim] weight are required")
    out = torch.empty_like(x)
    combined = x if residual is None else torch.empty_like(x)
    _lib.check(_lib.load().mi_rms_norm_residual(
        x.data_ptr(), x.stride(0), 0 if residual is None else residual.data_ptr(),
        0 if residual is None else residual.stride(0), weight.data_ptr(), float(eps),
        out.data_ptr(), out.stride(0), 0 if residual is None else combined.data_ptr(),
        combined.stride(0), rows, dim, _lib.dtype_code(x.dtype),
        _lib.stream_handle(x.device)), "mi_rms_norm_residual")
    return out, combined


def hip_silu_mul(gate_up: torch.Tensor) -> torch.Tensor:
    """``F.silu(gate) * up`` with ``gate, up = gate_up.chunk(2, dim=-1)``
    (transformer.py:12-15)."""
    _lib.require_device(gate_up, what="SwiGLU")
    rows, width = gate_up.shape
    if not supported_rows(gate_up) or width % 16:
        raise ValueError("hip_silu_mul: a 16-bit [rows, 2 * inter] tensor with inter % 8 == 0 "
                         "and aligned rows is required")
    inter = width // 2
    out = torch.empty((rows, inter), dtype=gate_up.dtype, device=gate_up.device)
    _lib.check(_lib.load().mi_silu_mul(
        gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), out.stride(0), rows, inter,
        _lib.dtype_code(gate_up.dtype), _lib.stream_handle(gate_up.device)), "mi_silu_mul")
    return out
