"""Kernel operands: fused, row-padded ternary matrices (mirrors the reference's kernel_decoder.py:46-142).

``Matrix`` stacks or interleaves projections that share an input (QKV
fusion; gate/up interleave with row 2j = gate j, row 2j+1 = up j), pads each
packed row with zero bytes to a multiple of 16 (zero codes meet zero-padded
activations, so the padding adds nothing), and places packed weights, fp16
scales and the fp32 bias on the device in the layout the kernels read in
place.  ``lanes`` keeps the reference's launch hint (``_lanes_for``) for
callers that pass it on; the kernels choose their own lane split.
"""

from __future__ import annotations

from collections.abc import Sequence

import torch
import torch.nn.functional as F
from torch import Tensor

from .quantization import TERNARY_GROUP_SIZE
from .runtime import KernelError

CHUNK = 64
THREADS = 256
NARROW_WIDTH = 4 * THREADS
ROW_ALIGNMENT = 16
TARGET_THREADS = 5120
WIDE_CHUNKS = NARROW_WIDTH // CHUNK


def _lanes_for(chunks: int, rows: int, max_lanes: int) -> int:
    """The reference's launch hint (kernel_decoder.py:46-50)."""
    lanes = 2
    while lanes < max_lanes and (rows * lanes < TARGET_THREADS or (chunks > WIDE_CHUNKS and chunks > 2 * lanes)):
        lanes *= 2
    return lanes


def _stack(tensors: Sequence[Tensor], interleave: bool) -> Tensor:
    if len(tensors) == 1:
        return tensors[0]
    if interleave:
        return torch.stack(tensors, dim=1).reshape(-1, *tensors[0].shape[1:])
    return torch.cat(tensors, dim=0)


class Matrix:
    __slots__ = ("packed", "scales", "bias", "rows", "in_features", "row_bytes", "groups", "chunks", "lanes")

    def __init__(
        self,
        projections: Sequence,
        device: torch.device,
        interleave: bool = False,
        max_lanes: int = 32,
        lanes: int = 0,
    ) -> None:
        first = projections[0]
        in_features = int(first.in_features)
        rows = int(first.out_features)
        for projection in projections:
            if int(projection.in_features) != in_features:
                raise KernelError("fused projections must share their input width")
            if interleave and int(projection.out_features) != rows:
                raise KernelError("interleaved projections must share their output width")
            if int(projection.group_size) != TERNARY_GROUP_SIZE:
                raise KernelError(f"ternary kernels need group size {TERNARY_GROUP_SIZE}")
        packed = _stack([projection.packed_weight for projection in projections], interleave)
        row_bytes = int(packed.shape[1])
        padded = (row_bytes + ROW_ALIGNMENT - 1) // ROW_ALIGNMENT * ROW_ALIGNMENT
        if padded != row_bytes:
            packed = F.pad(packed, (0, padded - row_bytes))
        self.packed = packed.contiguous().to(device)
        scales = _stack([projection.weight_scales for projection in projections], interleave)
        if scales.dtype != torch.float16:
            raise KernelError("ternary kernels need float16 group scales")
        self.scales = scales.contiguous().to(device)
        biases = [projection.bias for projection in projections]
        if all(bias is None for bias in biases):
            self.bias: Tensor | None = None
        elif any(bias is None for bias in biases):
            raise KernelError("fused projections must all carry a bias or none")
        else:
            self.bias = _stack([bias.float() for bias in biases], interleave).contiguous().to(device)
        self.rows = int(self.packed.shape[0])
        self.in_features = in_features
        self.row_bytes = padded
        self.groups = int(self.scales.shape[1])
        self.chunks = (in_features + CHUNK - 1) // CHUNK
        self.lanes = lanes if lanes else _lanes_for(self.chunks, self.rows, max_lanes)

    @classmethod
    def from_tensors(
        cls, packed: Tensor, scales: Tensor, in_features: int, bias: Tensor | None = None, device=None
    ) -> "Matrix":
        """A matrix from raw packed uint8 [N, ceil(K/4)] (or already padded) and fp16 scales [N, G]."""

        class _Projection:
            pass

        projection = _Projection()
        projection.packed_weight = packed
        projection.weight_scales = scales
        projection.bias = bias
        projection.in_features = int(in_features)
        projection.out_features = int(packed.shape[0])
        projection.group_size = TERNARY_GROUP_SIZE
        return cls([projection], torch.device(device) if device is not None else packed.device)

    @property
    def grid(self) -> int:
        rows_per_block = THREADS // self.lanes
        return (self.rows + rows_per_block - 1) // rows_per_block

    @property
    def wide(self) -> bool:
        return self.in_features > NARROW_WIDTH

    @property
    def scale_bits(self) -> Tensor:
        return self.scales.view(torch.int16)
