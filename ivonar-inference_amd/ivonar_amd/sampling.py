"""Device sampling state and launches (reference: decoder.py:324-371 sampling rule and
configure_sampling; kernel_decoder.py:213-224 and :619-681 the logit_bounds / sample_token launches).

``DeviceSampler`` owns the buffers the two kernels read and write (temperature, penalty,
inverse_penalty, top_k, seen, bounds, uniform, token), validates the rule on the host as the
reference's ``configure_sampling`` does, and launches both kernels on the current stream.  Nothing
here synchronises except ``sample()``, which returns the token as a Python int.
"""

from __future__ import annotations

from typing import Iterable

import torch
from torch import Tensor

from .runtime import KernelError, check, current_stream, int32, library, pointer

SAMPLE_THREADS = 1024  # largest top-k one sampling block handles (kernel_decoder.py:25)
BOUND_GROUP = 64       # logits per bound (kernel_decoder.py:26)
MAX_VOCAB = 1 << 18


class DeviceSampler:
    """Temperature / repetition-penalty / top-k sampling of one sequence on the device."""

    def __init__(self, vocab: int, device: torch.device | str, max_top_k: int = 256) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise KernelError("the device sampler needs a ROCm device")
        if not 0 < vocab <= MAX_VOCAB:
            raise KernelError(f"vocab {vocab} outside 1..{MAX_VOCAB}")
        if not 0 < max_top_k <= SAMPLE_THREADS:
            raise KernelError(f"max_top_k {max_top_k} outside 1..{SAMPLE_THREADS}")
        lib = library()
        check(lib.ivonar_define(b"MAX_TOPK", int(max_top_k)), "define MAX_TOPK")
        self.vocab = int(vocab)
        self.max_top_k = int(max_top_k)
        self.device = device
        self.temperature = torch.ones(1, dtype=torch.float32, device=device)
        self.penalty = torch.ones(1, dtype=torch.float32, device=device)
        self.inverse_penalty = torch.ones(1, dtype=torch.float32, device=device)
        self.top_k = torch.ones(1, dtype=torch.int64, device=device)
        self.seen = torch.zeros((1, vocab), dtype=torch.bool, device=device)
        self.bounds = torch.zeros((vocab + BOUND_GROUP - 1) // BOUND_GROUP, dtype=torch.float32, device=device)
        self.uniform = torch.zeros(1, dtype=torch.float32, device=device)
        self.token = torch.zeros(1, dtype=torch.int64, device=device)

    def configure_sampling(self, temperature: float, top_k: int, repetition_penalty: float = 1.0,
                           penalized_ids: Iterable[int] = ()) -> None:
        """The rule of decoder.py:340-361: a non-positive temperature or penalty is a ValueError, a top_k
        outside 1..max_top_k selects max_top_k, and the in-vocabulary ids of `penalized_ids` are marked
        as already generated (the rest are ignored)."""
        if any(value <= 0 for value in (temperature, repetition_penalty)):
            raise ValueError("temperature and repetition_penalty must be positive")
        k = int(top_k)
        if not 1 <= k <= self.max_top_k:
            k = self.max_top_k
        penalty = float(repetition_penalty)
        for buffer, value in ((self.temperature, float(temperature)), (self.penalty, penalty),
                              (self.inverse_penalty, 1.0 / penalty), (self.top_k, k)):
            buffer.fill_(value)
        ids = torch.as_tensor([int(i) for i in penalized_ids], dtype=torch.int64)
        marked = torch.zeros((1, self.vocab), dtype=torch.bool)
        marked[0, ids[(ids >= 0) & (ids < self.vocab)]] = True
        self.seen.copy_(marked)

    def launch(self, logits: Tensor, uniform: Tensor | None = None, token: Tensor | None = None,
               history: Tensor | None = None) -> None:
        """logit_bounds then sample_token on the current stream; draws with `uniform` (default: this
        sampler's buffer), writes `token` (default: this sampler's) and `history` if given."""
        if logits.device != self.device or logits.dtype != torch.float32 or logits.numel() < self.vocab:
            raise KernelError("logits must be float32 on the sampler's device with at least vocab entries")
        if not logits.is_contiguous():
            raise KernelError("logits must be contiguous")
        lib = library()
        stream = current_stream(self.device)
        check(lib.logit_bounds(stream, pointer(logits), pointer(self.temperature), pointer(self.penalty),
                               pointer(self.inverse_penalty), pointer(self.seen), pointer(self.bounds),
                               int32(self.vocab)), "logit_bounds")
        check(lib.sample_token(stream, pointer(logits), pointer(self.bounds), pointer(self.temperature),
                               pointer(self.penalty), pointer(self.inverse_penalty), pointer(self.seen),
                               pointer(self.top_k), pointer(self.uniform if uniform is None else uniform),
                               pointer(self.token if token is None else token), pointer(history),
                               int32(self.vocab)), "sample_token")

    def sample(self, logits: Tensor) -> int:
        """kernel_decoder.py:669-681: a fresh uniform, both launches, the token read back."""
        self.uniform.uniform_()
        self.launch(logits)
        return int(self.token[0])
