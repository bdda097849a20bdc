"""Kernel operands: ternary projections fused into one device matrix.

A decoder launches one kernel for several projections that read the same
input (QKV, gate/up).  ``Matrix`` places them in one device operand in the
layout the kernels read in place (reference ``kernel_decoder.py:84-142``):

* stacked: the projections' rows one after the other;
* interleaved (gate/up): row ``count*j + i`` is row j of projection i, so a
  silu-pair epilogue finds gate j and up j in rows 2j and 2j+1;
* every packed row padded with zero bytes to a multiple of 16 (zero bytes
  are code 0 against zero-padded activations, so the padding adds nothing);
* fp16 group scales and an fp32 bias (all projections carry one or none).

The destination tensors are allocated once on the device at their final
size and each projection is copied into its rows (a strided row slice when
interleaved), so no fused copy is ever built on the host.  ``lanes`` is the
reference's launch hint (``kernel_decoder.py:46-50``), which callers pass on
unchanged; this library's kernels choose their own lane split.
"""

from __future__ import annotations

from collections.abc import Sequence
from dataclasses import dataclass

import torch
from torch import Tensor

from .quantization import TERNARY_GROUP_SIZE
from .runtime import KernelError

CHUNK = 64
THREADS = 256
NARROW_WIDTH = 4 * THREADS  # inputs above which the reference launches its *_wide kernels
ROW_ALIGNMENT = 16
TARGET_THREADS = 5120
WIDE_CHUNKS = NARROW_WIDTH // CHUNK


def _lanes_for(chunks: int, rows: int, max_lanes: int) -> int:
    """The reference's threads-per-row hint (kernel_decoder.py:46-50).

    The smallest power of two from 2 up at which the launch has at least
    TARGET_THREADS threads and, for rows wider than WIDE_CHUNKS chunks, each
    lane takes at most two chunks; ``max_lanes`` caps it."""
    for lanes in (2, 4, 8, 16, 32, 64, 128):
        enough_threads = rows * lanes >= TARGET_THREADS
        short_enough = chunks <= WIDE_CHUNKS or chunks <= 2 * lanes
        if lanes >= max_lanes or (enough_threads and short_enough):
            return lanes
    return 128


@dataclass(frozen=True)
class _Part:
    """One projection's host (or device) tensors as the fusion reads them."""

    packed: Tensor
    scales: Tensor
    bias: Tensor | None
    in_features: int
    rows: int
    group_size: int


def _part(projection) -> _Part:
    return _Part(projection.packed_weight, projection.weight_scales, projection.bias, int(projection.in_features),
                 int(projection.out_features), int(getattr(projection, "group_size", TERNARY_GROUP_SIZE)))


def _check_parts(parts: Sequence[_Part], interleave: bool) -> None:
    if not parts:
        raise KernelError("a matrix needs at least one projection")
    width, rows = parts[0].in_features, parts[0].rows
    if any(part.in_features != width for part in parts):
        raise KernelError("fused projections must share their input width")
    if interleave and any(part.rows != rows for part in parts):
        raise KernelError("interleaved projections must share their output width")
    if any(part.group_size != TERNARY_GROUP_SIZE for part in parts):
        raise KernelError(f"ternary kernels need group size {TERNARY_GROUP_SIZE}")
    if any(part.scales.dtype != torch.float16 for part in parts):
        raise KernelError("ternary kernels need float16 group scales")
    with_bias = [part.bias is not None for part in parts]
    if any(with_bias) and not all(with_bias):
        raise KernelError("fused projections must all carry a bias or none")


def _row_slices(parts: Sequence[_Part], interleave: bool):
    """Destination rows of each projection: a strided slice when interleaved, a range when stacked."""
    if interleave:
        count = len(parts)
        return [slice(index, None, count) for index in range(count)]
    slices, start = [], 0
    for part in parts:
        slices.append(slice(start, start + part.rows))
        start += part.rows
    return slices


class Matrix:
    """A fused, row-padded ternary operand on one device (see the module docstring)."""

    __slots__ = ("packed", "scales", "bias", "rows", "in_features", "row_bytes", "groups", "chunks", "lanes")

    def __init__(
        self,
        projections: Sequence,
        device: torch.device,
        interleave: bool = False,
        max_lanes: int = 32,
        lanes: int = 0,
    ) -> None:
        self._fill([_part(projection) for projection in projections], torch.device(device), interleave)
        self.lanes = lanes if lanes else _lanes_for(self.chunks, self.rows, max_lanes)

    def _fill(self, parts: list[_Part], device: torch.device, interleave: bool) -> None:
        _check_parts(parts, interleave)
        total = sum(part.rows for part in parts)
        packed_width = max(int(part.packed.shape[1]) for part in parts)
        groups = int(parts[0].scales.shape[1])
        if any(int(part.scales.shape[1]) != groups for part in parts):
            raise KernelError("fused projections must share their scale group count")
        row_bytes = -(-packed_width // ROW_ALIGNMENT) * ROW_ALIGNMENT
        packed = torch.zeros((total, row_bytes), dtype=torch.uint8, device=device)
        scales = torch.empty((total, groups), dtype=torch.float16, device=device)
        bias = torch.empty(total, dtype=torch.float32, device=device) if parts[0].bias is not None else None
        for part, rows in zip(parts, _row_slices(parts, interleave)):
            packed[rows, : part.packed.shape[1]] = part.packed
            scales[rows] = part.scales
            if bias is not None:
                bias[rows] = part.bias.float()
        self.packed = packed
        self.scales = scales
        self.bias = bias
        self.rows = total
        self.in_features = parts[0].in_features
        self.row_bytes = row_bytes
        self.groups = groups
        self.chunks = -(-self.in_features // CHUNK)

    @classmethod
    def from_tensors(
        cls, packed: Tensor, scales: Tensor, in_features: int, bias: Tensor | None = None, device=None,
        lanes: int = 0, max_lanes: int = 32,
    ) -> "Matrix":
        """A matrix from raw packed uint8 [N, >= ceil(K/4)] (padded or not) and fp16 scales [N, G]."""
        matrix = cls.__new__(cls)
        part = _Part(packed, scales, bias, int(in_features), int(packed.shape[0]), TERNARY_GROUP_SIZE)
        matrix._fill([part], torch.device(device) if device is not None else packed.device, False)
        matrix.lanes = lanes if lanes else _lanes_for(matrix.chunks, matrix.rows, max_lanes)
        return matrix

    @property
    def grid(self) -> int:
        """Blocks of the reference's launch for this operand (its 256-thread blocks of 256/lanes rows)."""
        return -(-self.rows // (THREADS // self.lanes))

    @property
    def wide(self) -> bool:
        """Whether the reference launches the *_wide variant (more than 1024 inputs)."""
        return self.in_features > NARROW_WIDTH

    @property
    def scale_bits(self) -> Tensor:
        return self.scales.view(torch.int16)
