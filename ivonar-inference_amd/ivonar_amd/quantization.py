"""Ternary weight semantics and the TernaryLinear module (mirrors the reference's quantization.py).

Packed format (``quantization.py:10-32``): ``packed_weight`` is uint8
``[out_features, ceil(in_features / 4)]``; byte b of a row holds inputs
4b..4b+3, input 4b+k in bits 2k..2k+1 as code = w + 1 with w in {-1, 0, +1}
(code 3 is reserved); ``weight_scales`` is fp16 ``[out_features,
ceil(in_features / 128)]``; ``bias`` is fp32 ``[out_features]`` or None.

``TernaryLinear.forward`` (``quantization.py:177-178``) runs on the MI355X
kernels: activations are quantized per token to int8 by absmax, dot products
are exact integers per 128-input group, and fp32 scales are applied after.
It has no CPU path; calling it on a non-ROCm tensor raises ``KernelError``.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F
from torch import Tensor, nn

TERNARY_GROUP_SIZE = 128


def unpack_ternary_codes(packed: Tensor, in_features: int) -> Tensor:
    """uint8 packed rows -> int8 ternary values in {-1, 0, +1} (quantization.py:13-18)."""
    fields = [(packed >> shift) & 0x03 for shift in (0, 2, 4, 6)]
    values = torch.stack(fields, dim=-1).reshape(*packed.shape[:-1], -1)
    return values[..., :in_features].to(torch.int8) - 1


def pack_ternary_codes(values: Tensor) -> Tensor:
    """int ternary values [..., K] in {-1, 0, +1} -> packed uint8 [..., ceil(K/4)]."""
    codes = (values.to(torch.int16) + 1).to(torch.uint8)
    k = codes.shape[-1]
    pad = (-k) % 4
    if pad:
        codes = F.pad(codes, (0, pad), value=1)
    quads = codes.reshape(*codes.shape[:-1], -1, 4)
    return quads[..., 0] | (quads[..., 1] << 2) | (quads[..., 2] << 4) | (quads[..., 3] << 6)


def dequantize_ternary_codes(codes: Tensor, scales: Tensor, group_size: int, dtype: torch.dtype) -> Tensor:
    """values * per-group scale, as ``dtype`` (semantics of quantization.py:21-32).

    Each input's scale is its group's, repeated ``group_size`` times along the
    row and cut to the row's width; the product is formed in fp32."""
    width = int(codes.shape[-1])
    per_input = scales.float().repeat_interleave(int(group_size), dim=-1)[..., :width]
    return (codes.float() * per_input).to(dtype)


def _require_shape(what: str, tensor: Tensor, expected: tuple[int, ...]) -> None:
    if tuple(tensor.shape) != expected:
        raise ValueError(f"invalid {what} shape: expected {expected}, got {tuple(tensor.shape)}")


class TernaryLinear(nn.Module):
    """Packed ternary linear layer with the reference's constructor contract (quantization.py:119-147).

    ``packed_weight`` uint8 [out_features, ceil(in_features/4)], ``weight_scales``
    [out_features, ceil(in_features/group_size)], ``bias`` [out_features] or
    None; the shapes are checked with the reference's messages and the
    tensors kept as buffers (bias in fp32)."""

    def __init__(
        self,
        packed_weight: Tensor,
        weight_scales: Tensor,
        in_features: int,
        bias: Tensor | None = None,
        eps: float = 1e-5,
        group_size: int = TERNARY_GROUP_SIZE,
    ) -> None:
        super().__init__()
        if packed_weight.dtype != torch.uint8 or packed_weight.dim() != 2:
            raise ValueError("packed_weight must be a two-dimensional uint8 tensor")
        rows = int(packed_weight.shape[0])
        width, groups = int(in_features), -(-int(in_features) // int(group_size))
        _require_shape("packed", packed_weight, (rows, -(-width // 4)))
        _require_shape("scale", weight_scales, (rows, groups))
        if bias is not None:
            _require_shape("bias", bias, (rows,))
        self.in_features, self.out_features = width, rows
        self.group_size, self.eps = int(group_size), float(eps)
        buffers = {
            "packed_weight": packed_weight.contiguous(),
            "weight_scales": weight_scales.contiguous(),
            "bias": None if bias is None else bias.detach().float().clone(),
        }
        for name, tensor in buffers.items():
            self.register_buffer(name, tensor)
        self._matrix = None

    def unpacked_weight(self, dtype: torch.dtype = torch.float32) -> Tensor:
        codes = unpack_ternary_codes(self.packed_weight, self.in_features)
        return dequantize_ternary_codes(codes, self.weight_scales, self.group_size, dtype)

    def matrix(self):
        """The device-resident, row-padded kernel operand of this layer (built once)."""
        from .matrix import Matrix

        device = self.packed_weight.device
        if self._matrix is None or self._matrix.packed.device != device:
            self._matrix = Matrix([self], device)
        return self._matrix

    def _apply(self, fn, recurse: bool = True):
        module = super()._apply(fn, recurse)
        self._matrix = None
        return module

    def forward(self, x: Tensor) -> Tensor:
        from .ops import ternary_linear

        if self.group_size != TERNARY_GROUP_SIZE:
            raise ValueError(f"ternary kernels need group size {TERNARY_GROUP_SIZE}")
        return ternary_linear(x, self.matrix())
