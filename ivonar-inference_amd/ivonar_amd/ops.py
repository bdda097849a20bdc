"""Tensor-level calls into the ternary HIP library (the secondary boundary, quantization.py:177-178).

Every function takes and returns torch tensors on a ROCm device, launches on
the current stream and never synchronises.  The shapes follow the reference:

* ``quantize_rows(x [M, K])`` -> (q8 int8 [M, C*64], xsum int32 [M, C],
  scale fp32 [M]) with C = ceil(K/64), the activation scratch the GEMV and
  GEMM entry points read (q8 layout private to the library);
* ``gemv(matrix, x [K])`` -> y [N]: the decode GEMV (M = 1);
* ``gemm(matrix, q8, xsum, scale)`` -> y [M, N]: int8 MFMA over M tokens;
* ``ternary_linear(x [..., K], matrix)`` -> [..., N]: GEMV for one token,
  quantize + MFMA GEMM otherwise;
* ``group_partials(matrix, q8, xsum)`` -> int32 [N, G]: the GEMV's exact
  per-128-group partial sums (test export).
"""

from __future__ import annotations

import torch
from torch import Tensor

from .matrix import Matrix
from .runtime import KernelError, check, current_stream, float32, initialise, int32, library, pointer

MODE_PLAIN, MODE_NORM, MODE_ATTN = 0, 1, 2
CHUNK = 64

_GEMV_NAMES = {
    ("plain", "store"): "gemv_plain_store",
    ("plain", "residual"): "gemv_plain_residual",
    ("norm", "store"): "gemv_norm_store",
    ("norm", "silu_pair"): "gemv_norm_silu_pair",
    ("attn", "residual"): "gemv_attn_residual",
}
_GEMM_NAMES = {"store": "gemm_tile_store", "residual": "gemm_tile_residual", "silu_pair": "gemm_tile_silu_pair"}


def _require_device(*tensors: Tensor | None) -> torch.device:
    device = None
    for tensor in tensors:
        if tensor is None:
            continue
        if tensor.device.type != "cuda":
            raise KernelError("ternary kernels need tensors on a ROCm device")
        if device is None:
            device = tensor.device
    if device is None:
        raise KernelError("no device tensor given")
    initialise(device.index if device.index is not None else torch.cuda.current_device())
    return device


def activation_buffers(m: int, n: int, device: torch.device) -> tuple[Tensor, Tensor, Tensor]:
    chunks = (n + CHUNK - 1) // CHUNK
    return (
        torch.empty((m, chunks * CHUNK), dtype=torch.int8, device=device),
        torch.empty((m, chunks), dtype=torch.int32, device=device),
        torch.empty((m,), dtype=torch.float32, device=device),
    )


def quantize_rows(
    x: Tensor, mode: int = MODE_PLAIN, aux: Tensor | None = None, eps: float = 1e-6, splits: int = 1,
    n: int | None = None, out: tuple[Tensor, Tensor, Tensor] | None = None,
) -> tuple[Tensor, Tensor, Tensor]:
    """Per-token int8 quantization of the rows of x (fp32 [M, in_stride]); n inputs per row."""
    device = _require_device(x, aux)
    if x.dtype != torch.float32 or x.stride(-1) != 1:
        raise KernelError("quantize_rows needs fp32 rows with unit stride")
    rows = x.reshape(-1, x.shape[-1]) if x.ndim != 2 else x
    m = rows.shape[0]
    width = int(n if n is not None else rows.shape[1])
    q8, xsum, scale = out if out is not None else activation_buffers(m, width, device)
    check(
        library().ivonar_quantize_rows(
            current_stream(device), mode, pointer(rows), int32(rows.stride(0)), pointer(aux), int32(width),
            float32(eps), int32(splits), int32(m), pointer(q8), pointer(xsum), pointer(scale),
        ),
        "ivonar_quantize_rows",
    )
    return q8, xsum, scale


def gemv(
    matrix: Matrix, x: Tensor, out: Tensor | None = None, mode: str = "plain", epilogue: str = "store",
    aux: Tensor | None = None, eps: float = 1e-6, splits: int = 1,
) -> Tensor:
    """Decode GEMV of one token through the reference-named entry point for (mode, epilogue)."""
    device = _require_device(x, matrix.packed)
    name = _GEMV_NAMES.get((mode, epilogue))
    if name is None:
        raise KernelError(f"no GEMV entry point for mode={mode!r} epilogue={epilogue!r}")
    for tensor in (x, aux):
        if tensor is not None and (tensor.dtype != torch.float32 or tensor.stride(-1) != 1):
            raise KernelError(f"{name} needs fp32 activations with unit stride")
    rows_out = matrix.rows // 2 if epilogue == "silu_pair" else matrix.rows
    if out is None:
        if epilogue == "residual":
            raise KernelError("a residual GEMV needs the output tensor it adds into")
        out = torch.empty(rows_out, dtype=torch.float32, device=device)
    function = getattr(library(), name)
    check(
        function(
            current_stream(device), pointer(x), pointer(aux), pointer(None), pointer(None), pointer(None),
            pointer(matrix.packed), pointer(matrix.scales), pointer(matrix.bias), pointer(out),
            int32(matrix.rows), int32(matrix.in_features), int32(matrix.row_bytes), int32(matrix.groups),
            int32(matrix.lanes), int32(splits), float32(eps), pointer(None), int32(0),
        ),
        name,
    )
    return out


def gemv_prequant(matrix: Matrix, q8: Tensor, xsum: Tensor, scale: Tensor, out: Tensor | None = None) -> Tensor:
    """gemv_prequant_store: one token from pre-quantized activations."""
    device = _require_device(q8, matrix.packed)
    if out is None:
        out = torch.empty(matrix.rows, dtype=torch.float32, device=device)
    check(
        library().gemv_prequant_store(
            current_stream(device), pointer(None), pointer(None), pointer(q8), pointer(xsum), pointer(scale),
            pointer(matrix.packed), pointer(matrix.scales), pointer(matrix.bias), pointer(out),
            int32(matrix.rows), int32(matrix.in_features), int32(matrix.row_bytes), int32(matrix.groups),
            int32(matrix.lanes), int32(1), float32(1e-6), pointer(None), int32(0),
        ),
        "gemv_prequant_store",
    )
    return out


def gemm(
    matrix: Matrix, q8: Tensor, xsum: Tensor, scale: Tensor, out: Tensor | None = None, epilogue: str = "store",
    m: int | None = None, out_stride: int | None = None,
) -> Tensor:
    """int8 MFMA GEMM over m pre-quantized token rows (gemm_tile_* entry points)."""
    device = _require_device(q8, matrix.packed)
    rows = int(q8.shape[0]) if m is None else int(m)
    width = matrix.rows // 2 if epilogue == "silu_pair" else matrix.rows
    if out is None:
        if epilogue == "residual":
            raise KernelError("a residual GEMM needs the output tensor it adds into")
        out = torch.empty((rows, width), dtype=torch.float32, device=device)
    stride = int(out_stride if out_stride is not None else (out.stride(0) if out.ndim == 2 else width))
    name = _GEMM_NAMES[epilogue]
    check(
        getattr(library(), name)(
            current_stream(device), pointer(q8), pointer(xsum), pointer(scale), pointer(matrix.packed),
            pointer(matrix.scales), pointer(matrix.bias), pointer(out), int32(matrix.rows),
            int32(matrix.in_features), int32(matrix.row_bytes), int32(matrix.groups), int32(matrix.lanes),
            int32(stride), int32(rows),
        ),
        name,
    )
    return out


def group_partials(matrix: Matrix, q8: Tensor, xsum: Tensor) -> Tensor:
    device = _require_device(q8, matrix.packed)
    groups = (matrix.in_features + 127) // 128
    out = torch.empty((matrix.rows, groups), dtype=torch.int32, device=device)
    check(
        library().gemv_group_partials(
            current_stream(device), pointer(q8), pointer(xsum), pointer(matrix.packed), int32(matrix.rows),
            int32(matrix.in_features), int32(matrix.row_bytes), int32(groups), pointer(out),
        ),
        "gemv_group_partials",
    )
    return out


def embed(matrix: Matrix, tokens: Tensor, out: Tensor | None = None) -> Tensor:
    """Rows tokens[t] of the packed matrix decoded to fp32 [m, in_features] (embed_tile)."""
    device = _require_device(tokens, matrix.packed)
    if tokens.dtype != torch.int64:
        raise KernelError("token ids must be int64")
    m = int(tokens.numel())
    if out is None:
        out = torch.empty((m, matrix.in_features), dtype=torch.float32, device=device)
    check(
        library().embed_tile(
            current_stream(device), pointer(tokens), pointer(matrix.packed), pointer(matrix.scales), pointer(out),
            int32(matrix.in_features), int32(matrix.row_bytes), int32(matrix.groups), int32(m),
        ),
        "embed_tile",
    )
    return out


def argmax(values: Tensor, out: Tensor | None = None) -> Tensor:
    device = _require_device(values)
    if out is None:
        out = torch.empty(1, dtype=torch.int64, device=device)
    check(library().ivonar_argmax(current_stream(device), pointer(values), int32(values.numel()), pointer(out)),
          "ivonar_argmax")
    return out


def ternary_linear(x: Tensor, matrix: Matrix) -> Tensor:
    """y = ternary linear layer of x [..., K] (GEMV for one token, MFMA GEMM otherwise)."""
    device = _require_device(x, matrix.packed)
    if x.shape[-1] != matrix.in_features:
        raise KernelError(f"input width {x.shape[-1]} does not match the layer's {matrix.in_features}")
    lead = x.shape[:-1]
    rows = x.reshape(-1, matrix.in_features).float().contiguous()
    m = rows.shape[0]
    if m == 1:
        return gemv(matrix, rows[0]).reshape(*lead, matrix.rows)
    q8, xsum, scale = quantize_rows(rows)
    out = torch.empty((m, matrix.rows), dtype=torch.float32, device=device)
    gemm(matrix, q8, xsum, scale, out=out)
    return out.reshape(*lead, matrix.rows)
