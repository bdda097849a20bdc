"""Decode and prefill driver for a stack of ternary linear layers (mirrors the reference's kernel_decoder.py).

The reference's ``KernelDecoder`` (``kernel_decoder.py:179-283``, ``:303-368``)
builds one ``Launch`` per op and replays the list per token (decode) and per
32-token tile (prefill).  ``StackDecoder`` builds the same launch pattern for
the ternary linear path, with the same entry points and argument lists, through
this package's ``runtime`` (the C ABI of the MI355X library):

decode step (``kernel_decoder.py:233-269``)::

    embed_token                                   token -> residual
    per layer:
      gemv_norm_store       entry (fused QKV)     residual -> mixer_in   (RMSNorm prologue)
      gemv_plain_residual   out                   V third of mixer_in -> residual +=
      gemv_norm_silu_pair   gate/up (interleaved) residual -> ffn_mid    (RMSNorm prologue)
      gemv_plain_residual   down                  ffn_mid -> residual +=
    gemv_norm_store                               residual -> logits (tied token matrix, RMSNorm fused)
    ivonar_argmax                                 logits -> next token (greedy)
      or, with sampling: uniform_(), logit_bounds, sample_token (kernel_decoder.py:619-681)

prefill tile (``kernel_decoder.py:303-368``): ``embed_tile``, per layer
``quantize_tile_norm`` + ``gemm_tile_store``, ``quantize_tile_plain`` +
``gemm_tile_residual``, ``quantize_tile_norm`` + ``gemm_tile_silu_pair``,
``quantize_tile_plain`` + ``gemm_tile_residual``, then ``gather_token``; the
head and the first token's selection run once, after the last tile (the
reference runs its head in every tile and samples after the prompt).

The mixers (recurrent scan, latent attention) are not part of this path: the
output projection reads the V third of the entry projection's output instead
of a mixer's output.  Greedy tokens are written on the device into a ring of
``burst`` slots, so a burst of decode steps runs as one HIP graph replay with
a single read-back, as the reference's burst graphs do (``kernel_decoder.py:694-735``).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np
import torch

from . import runtime
from .matrix import Matrix, _lanes_for
from .quantization import TernaryLinear
from .runtime import KernelError, Launch, float32, int32, pointer
from .sampling import DeviceSampler
from .synthetic import LinearStackWeights

TILE = 32
SELF_CHECK_TOLERANCE = 0.25  # kernel_decoder.py:38
THREADS = 256
HEAD_LANES = 4
CHUNK = 64
BURST = 16


def _linear(layer) -> TernaryLinear:
    return TernaryLinear(torch.from_numpy(np.ascontiguousarray(layer.packed)),
                         torch.from_numpy(np.ascontiguousarray(layer.scales)), layer.in_features,
                         None if layer.bias is None else torch.from_numpy(layer.bias))


@dataclass
class _LayerOps:
    entry: Matrix
    out: Matrix
    gate_up: Matrix
    down: Matrix
    mixer_norm: torch.Tensor
    ffn_norm: torch.Tensor


class _TorchOp:
    """A torch call in a launch list (runs on torch's current stream, which is the launch stream)."""

    __slots__ = ("function",)

    def __init__(self, function) -> None:
        self.function = function

    def __call__(self, stream: int) -> None:
        del stream
        self.function()


class StackDecoder:
    def __init__(self, weights: LinearStackWeights, device: str | torch.device = "cuda", burst: int = BURST,
                 sampling: bool = False, max_top_k: int = 256) -> None:
        device = torch.device(device)
        if device.type != "cuda":
            raise KernelError("the ternary decoder needs a ROCm device")
        config = weights.config
        self.config = config
        self.device = device
        self.burst = int(burst)
        hidden, dense, vocab = config.hidden, config.dense, config.vocab
        max_chunks = (max(hidden, dense) + CHUNK - 1) // CHUNK
        self.module = runtime.compile_module(None, {"HEAD_DIM": 64, "MAX_CHUNKS": max_chunks, "TILE": TILE}, device)
        self.token_matrix = Matrix([_linear(weights.token)], device, lanes=HEAD_LANES)
        self.layers: list[_LayerOps] = []
        for layer in weights.layers:
            self.layers.append(_LayerOps(
                entry=Matrix([_linear(layer.qkv)], device),
                out=Matrix([_linear(layer.out)], device),
                gate_up=Matrix([_linear(layer.gate), _linear(layer.up)], device, interleave=True, max_lanes=16),
                down=Matrix([_linear(layer.down)], device),
                mixer_norm=torch.from_numpy(layer.mixer_norm).to(device),
                ffn_norm=torch.from_numpy(layer.ffn_norm).to(device),
            ))
        self.final_norm = torch.from_numpy(weights.final_norm).to(device)
        f32 = dict(dtype=torch.float32, device=device)
        self.residual = torch.zeros(hidden, **f32)
        self.mixer_in = torch.zeros(config.qkv, **f32)
        self.ffn_mid = torch.zeros(dense, **f32)
        self.logits = torch.zeros(vocab, **f32)
        self.q8 = torch.zeros(max_chunks * CHUNK, dtype=torch.int8, device=device)
        self.q8sum = torch.zeros(max_chunks, dtype=torch.int32, device=device)
        self.q8scale = torch.zeros(1, **f32)
        self.history = torch.zeros(self.burst, dtype=torch.int64, device=device)
        # sampling state (kernel_decoder.py:213-224): one uniform per ring slot, drawn inside the step
        self.sampler = DeviceSampler(vocab, device, max_top_k) if sampling else None
        self.uniforms = torch.zeros(self.burst, **f32)
        self.drawn_uniforms: list[float] = []  # with sampling: the uniform of every token advance_many returned
        # prefill tile buffers (kernel_decoder.py:308-319)
        self.tile_tokens = torch.zeros(TILE, dtype=torch.int64, device=device)
        self.tile_valid = torch.zeros(1, dtype=torch.int64, device=device)
        self.residual_tile = torch.zeros(TILE, hidden, **f32)
        self.mixer_in_tile = torch.zeros(TILE, config.qkv, **f32)
        self.ffn_tile = torch.zeros(TILE, dense, **f32)
        self.q8_tile = torch.zeros(TILE, max_chunks * CHUNK, dtype=torch.int8, device=device)
        self.xsum_tile = torch.zeros(TILE, max_chunks, dtype=torch.int32, device=device)
        self.scale_tile = torch.zeros(TILE, **f32)
        # The head is one GEMV with the RMSNorm prologue fused (the reference runs quantize_norm and
        # gemv_prequant_store, kernel_decoder.py:265-267; the logits are the same bits either way).
        self._head = [self._gemv("gemv_norm_store", self.token_matrix, self.residual, self.final_norm, self.logits,
                                 eps=config.eps)]
        self._steps = [self._build_step(slot) for slot in range(self.burst)]
        self._tile = self._build_tile()
        self._first = self._head + self._select(self.burst - 1)  # after the last tile
        self._graph: torch.cuda.CUDAGraph | None = None
        self._tile_graph: torch.cuda.CUDAGraph | None = None
        self.position = 0

    # ------------------------------------------------------------------ launch builders

    def _gemv(self, name: str, matrix: Matrix, source, aux, output, eps: float = 1e-6, splits: int = 1,
              prequant: bool = False) -> Launch:
        """kernel_decoder.py:562-584 (the prefetch slots are passed empty)."""
        args = [
            pointer(source), pointer(aux),
            pointer(self.q8 if prequant else None), pointer(self.q8sum if prequant else None),
            pointer(self.q8scale if prequant else None),
            pointer(matrix.packed), pointer(matrix.scales), pointer(matrix.bias), pointer(output),
            int32(matrix.rows), int32(matrix.in_features), int32(matrix.row_bytes), int32(matrix.groups),
            int32(matrix.lanes), int32(splits), float32(eps), pointer(None), int32(0),
        ]
        if matrix.wide and not prequant:
            name += "_wide"
        return Launch(self.module.kernel(name), (matrix.grid, 1, 1), (THREADS, 1, 1), args)

    def _quantize(self, name: str, source, aux, width: int, eps: float = 1e-6) -> Launch:
        """kernel_decoder.py:611-618."""
        args = [pointer(source), pointer(aux), int32(width), float32(eps), int32(1),
                pointer(self.q8), pointer(self.q8sum), pointer(self.q8scale)]
        if width > 4 * THREADS:
            name += "_wide"
        return Launch(self.module.kernel(name), (1, 1, 1), (THREADS, 1, 1), args)

    def _quantize_tile(self, name: str, source, width: int, in_stride: int, aux=None, eps: float = 1e-6) -> Launch:
        """kernel_decoder.py:370-386."""
        args = [pointer(source), int32(in_stride), pointer(aux), int32(width), float32(eps), int32(1),
                pointer(self.q8_tile), pointer(self.xsum_tile), pointer(self.scale_tile)]
        if width > 4 * THREADS:
            name += "_wide"
        return Launch(self.module.kernel(name), (TILE, 1, 1), (THREADS, 1, 1), args)

    def _gemm_tile(self, name: str, matrix: Matrix, output, out_stride: int) -> Launch:
        """kernel_decoder.py:388-397."""
        args = [pointer(self.q8_tile), pointer(self.xsum_tile), pointer(self.scale_tile),
                pointer(matrix.packed), pointer(matrix.scales), pointer(matrix.bias), pointer(output),
                int32(matrix.rows), int32(matrix.in_features), int32(matrix.row_bytes), int32(matrix.groups),
                int32(matrix.lanes), int32(out_stride), int32(TILE)]
        if matrix.wide:
            name += "_wide"
        return Launch(self.module.kernel(name), (matrix.grid, 1, 1), (THREADS, 1, 1), args)

    def _select(self, slot: int) -> list:
        """The next token into ring slot `slot`: greedy argmax, or a draw of the device sampler with a
        fresh uniform (kernel_decoder.py:669-681)."""
        history = self.history[slot:slot + 1]
        vocab = self.config.vocab
        sampler = self.sampler
        if sampler is None:
            args = [pointer(self.logits), int32(vocab), pointer(history)]
            return [Launch(self.module.kernel("ivonar_argmax"), (1, 1, 1), (1024, 1, 1), args)]
        uniform = self.uniforms[slot:slot + 1]
        groups = (vocab + 63) // 64
        bounds_args = [pointer(self.logits), pointer(sampler.temperature), pointer(sampler.penalty),
                       pointer(sampler.inverse_penalty), pointer(sampler.seen), pointer(sampler.bounds), int32(vocab)]
        sample_args = [pointer(self.logits), pointer(sampler.bounds), pointer(sampler.temperature),
                       pointer(sampler.penalty), pointer(sampler.inverse_penalty), pointer(sampler.seen),
                       pointer(sampler.top_k), pointer(uniform), pointer(sampler.token), pointer(history), int32(vocab)]
        return [_TorchOp(uniform.uniform_),
                Launch(self.module.kernel("logit_bounds"), (groups, 1, 1), (64, 1, 1), bounds_args),
                Launch(self.module.kernel("sample_token"), (1, 1, 1), (1024, 1, 1), sample_args)]

    def configure_sampling(self, temperature: float, top_k: int, repetition_penalty: float = 1.0,
                           penalized_ids=()) -> None:
        """decoder.py:334-361 (the decoder must have been created with sampling=True)."""
        if self.sampler is None:
            raise RuntimeError("this decoder was created without sampling")
        self.sampler.configure_sampling(temperature, top_k, repetition_penalty, penalized_ids)

    def _build_step(self, slot: int) -> list[Launch]:
        """One greedy decode step reading the token in slot-1 of the ring and writing slot."""
        config = self.config
        hidden = config.hidden
        previous = self.history[(slot - 1) % self.burst:(slot - 1) % self.burst + 1]
        token = self.token_matrix
        launches = [Launch(self.module.kernel("embed_token"), ((hidden + THREADS - 1) // THREADS, 1, 1), (THREADS, 1, 1),
                           [pointer(previous), pointer(token.packed), pointer(token.scales), pointer(self.residual),
                            int32(hidden), int32(token.row_bytes), int32(token.groups)])]
        values = self.mixer_in.narrow(0, 2 * hidden, hidden)
        for ops in self.layers:
            launches.append(self._gemv("gemv_norm_store", ops.entry, self.residual, ops.mixer_norm, self.mixer_in,
                                       eps=config.eps))
            launches.append(self._gemv("gemv_plain_residual", ops.out, values, None, self.residual))
            launches.append(self._gemv("gemv_norm_silu_pair", ops.gate_up, self.residual, ops.ffn_norm,
                                       self.ffn_mid, eps=config.eps))
            launches.append(self._gemv("gemv_plain_residual", ops.down, self.ffn_mid, None, self.residual))
        launches.extend(self._head)
        launches.extend(self._select(slot))
        return launches

    def _build_tile(self) -> list[Launch]:
        """One 32-token prefill tile, ending with its last valid token's residual in ``self.residual``."""
        config = self.config
        hidden, dense, qkv = config.hidden, config.dense, config.qkv
        token = self.token_matrix
        launches = [Launch(self.module.kernel("embed_tile"), ((hidden + THREADS - 1) // THREADS, TILE, 1),
                           (THREADS, 1, 1),
                           [pointer(self.tile_tokens), pointer(token.packed), pointer(token.scales),
                            pointer(self.residual_tile), int32(hidden), int32(token.row_bytes), int32(token.groups),
                            int32(TILE)])]
        values = self.mixer_in_tile.narrow(1, 2 * hidden, hidden)
        for ops in self.layers:
            launches.append(self._quantize_tile("quantize_tile_norm", self.residual_tile, hidden, hidden,
                                                ops.mixer_norm, eps=config.eps))
            launches.append(self._gemm_tile("gemm_tile_store", ops.entry, self.mixer_in_tile, qkv))
            launches.append(self._quantize_tile("quantize_tile_plain", values, hidden, qkv))
            launches.append(self._gemm_tile("gemm_tile_residual", ops.out, self.residual_tile, hidden))
            launches.append(self._quantize_tile("quantize_tile_norm", self.residual_tile, hidden, hidden,
                                                ops.ffn_norm, eps=config.eps))
            launches.append(self._gemm_tile("gemm_tile_silu_pair", ops.gate_up, self.ffn_tile, dense))
            launches.append(self._quantize_tile("quantize_tile_plain", self.ffn_tile, dense, dense))
            launches.append(self._gemm_tile("gemm_tile_residual", ops.down, self.residual_tile, hidden))
        launches.append(Launch(self.module.kernel("gather_token"), ((hidden + THREADS - 1) // THREADS, 1, 1),
                               (THREADS, 1, 1),
                               [pointer(self.residual_tile), pointer(self.residual), int32(hidden),
                                pointer(self.tile_valid)]))
        return launches

    # ------------------------------------------------------------------ running

    def _run(self, launches: list[Launch]) -> None:
        stream = runtime.current_stream(self.device)
        for launch in launches:
            launch(stream)

    @torch.no_grad()
    def prefill(self, input_ids) -> torch.Tensor:
        """Runs the prompt in 32-token tiles (kernel_decoder.py:456-479), then the head on its last token:
        the logits are left in ``self.logits`` and the first token (greedy, or drawn by the sampler) in
        the ring's last slot."""
        ids = torch.as_tensor(input_ids, dtype=torch.int64).reshape(-1)
        length = int(ids.numel())
        if length == 0:
            raise ValueError("the prompt must not be empty")
        if int(ids.min()) < 0 or int(ids.max()) >= self.config.vocab:
            raise IndexError(f"token id is out of range for vocab_size={self.config.vocab}")
        ids = ids.to(self.device)
        for start in range(0, length, TILE):
            chunk = ids[start:start + TILE]
            count = int(chunk.numel())
            self.tile_tokens.zero_()
            self.tile_tokens[:count].copy_(chunk)
            self.tile_valid.fill_(count)
            if self._tile_graph is not None:
                self._tile_graph.replay()  # one replay per tile (kernel_decoder.py:444-447)
            else:
                self._run(self._tile)
        self._run(self._first)
        self.position = 0
        return self.logits

    @torch.no_grad()
    def step(self) -> None:
        """One eager greedy step: consumes the last token, appends the next one to the ring."""
        self._run(self._steps[self.position % self.burst])
        self.position += 1

    @torch.no_grad()
    def capture(self) -> bool:
        """Records one burst of decode steps into a HIP graph (kernel_decoder.py:694-719).  With sampling,
        the uniforms are drawn inside the graph, fresh on every replay; the sampler's `seen` is restored
        after the warm-up and the capture, as the ring is.  Then records the prefill tile program as a
        second graph (kernel_decoder.py:482-509), which prefill() replays once per 32-token tile after
        filling the device buffers tile_tokens and tile_valid; the residual the last prefill left is
        restored after its warm-up and capture."""
        if self.position % self.burst != 0:
            raise KernelError("capture at a burst boundary")
        saved = self.history.clone()
        seen = None if self.sampler is None else self.sampler.seen.clone()
        stream = torch.cuda.Stream(device=self.device)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            for slot in range(self.burst):
                self._run(self._steps[slot])
        torch.cuda.current_stream(self.device).wait_stream(stream)
        torch.cuda.synchronize(self.device)
        self.history.copy_(saved)
        if seen is not None:
            self.sampler.seen.copy_(seen)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for slot in range(self.burst):
                self._run(self._steps[slot])
        torch.cuda.synchronize(self.device)
        self.history.copy_(saved)
        if seen is not None:
            self.sampler.seen.copy_(seen)
        self._graph = graph
        self._tile_graph = self._capture_tile(stream)
        return True

    def _capture_tile(self, stream: torch.cuda.Stream) -> torch.cuda.CUDAGraph:
        residual, valid = self.residual.clone(), self.tile_valid.clone()
        self.tile_valid.fill_(TILE)
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            self._run(self._tile)
        torch.cuda.current_stream(self.device).wait_stream(stream)
        torch.cuda.synchronize(self.device)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            self._run(self._tile)
        torch.cuda.synchronize(self.device)
        self.residual.copy_(residual)
        self.tile_valid.copy_(valid)
        return graph

    @torch.no_grad()
    def advance_many(self, count: int) -> list[int]:
        """``count`` greedy tokens after the last one produced: whole bursts replay the graph with one
        read-back each (kernel_decoder.py:722-735); the rest run eagerly."""
        tokens: list[int] = []
        sampling = self.sampler is not None
        while count - len(tokens) >= self.burst and self._graph is not None and self.position % self.burst == 0:
            self._graph.replay()
            self.position += self.burst
            tokens.extend(self.history.tolist())
            if sampling:
                self.drawn_uniforms.extend(self.uniforms.tolist())
        while len(tokens) < count:
            slot = self.position % self.burst
            self.step()
            tokens.append(int(self.history[slot]))
            if sampling:
                self.drawn_uniforms.append(float(self.uniforms[slot]))
        return tokens

    def reset(self) -> None:
        """Back to an empty sequence (decoder.py:463-466): position 0, an empty token ring, no token seen."""
        self.position = 0
        self.history.zero_()
        if self.sampler is not None:
            self.sampler.seen.zero_()

    @torch.no_grad()
    def self_check(self) -> None:
        """Runs one prompt through the prefill tiles and through single decode steps and requires both to
        agree (kernel_decoder.py:524-549), so a GPU the kernels do not run correctly on fails while loading.

        The prompt has TILE + TILE // 2 + 1 random ids in [2, vocab): prefill() takes it whole (the tile
        GEMMs), then the first id alone, after which every further id is written into the ring slot the
        next step reads and one step consumes it (the GEMVs).  Both end with the logits of the prompt's last
        id; they must be finite, not all zero, and within a relative norm of SELF_CHECK_TOLERANCE, and the
        token the last step selected must lie in the vocabulary.  The decoder is reset afterwards.  Raises
        KernelError."""
        vocab = int(self.config.vocab)
        length = TILE + TILE // 2 + 1
        ids = torch.randint(2, max(vocab, 3), (length,), generator=torch.Generator().manual_seed(0)) % vocab
        whole = self.prefill(ids).clone()
        self.prefill(ids[:1])
        for index in range(1, length):
            self.history[(self.position - 1) % self.burst].fill_(int(ids[index]))
            self.step()
        stepped = self.logits.clone()
        selected = int(self.history[(self.position - 1) % self.burst])
        self.reset()
        scale = float(whole.norm())
        if not (bool(torch.isfinite(whole).all()) and bool(torch.isfinite(stepped).all())) or scale == 0.0:
            raise KernelError("the ternary kernels produced invalid numbers on this GPU")
        difference = float((whole - stepped).norm()) / scale
        if difference > SELF_CHECK_TOLERANCE:
            raise KernelError(f"the ternary kernels disagree with themselves on this GPU ({difference:.1e})")
        if not 0 <= selected < vocab:
            raise KernelError("the ternary sampler returned an invalid token on this GPU")

    @torch.no_grad()
    def generate(self, prompt_ids, count: int) -> list[int]:
        """The first token from the prompt's last position, then count-1 steps (greedy, or drawn by the
        device sampler as configured)."""
        self.prefill(prompt_ids)
        first = int(self.history[self.burst - 1])
        return [first] + self.advance_many(count - 1)
