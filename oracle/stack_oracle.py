"""Greedy decoding of a ternary linear stack on the CPU.  TEST INFRASTRUCTURE ONLY.

Only the tests and ``bench.py``'s token check use this module, and only as the
checker of the decoder's tokens and logits.

It restates the decode step and the 32-token prefill tile of the decoder
(the reference's ``kernel_decoder.py:233-269`` and ``:303-368``, without the
mixers: the output projection reads the V third of the fused entry
projection) from the oracle's primitives:

* quantizers: ``orc_quantize_rows`` (PLAIN; NORM = RMSNorm with clip +-8
  first, reference ``ternary.cu:395-409``);
* integer core: ``orc_partials_i8``, exact per-128-group int32 dot products
  of the ternary values with the int8 activations;
* fp32 finish: ``orc_finish`` in the decode GEMV's order (lane pairs, the
  lane count from the GEMV plan) or the token GEMM's order (K-splits from the
  GEMM plan), both pinned against ``orc_gemv_pairs`` / ``orc_gemm_split``.

The plans are passed in as callables, ``gemv_lanes(rows, k)`` and
``gemm_splits(m, rows, k)``; they are parameters of the kernels' summation
order, not computations of the checker.
"""

from __future__ import annotations

from collections.abc import Callable

import numpy as np

import ternary_oracle as T

TILE = 32


class _Projection:
    """int8 ternary values [rows, K] and fp16 scale bits [rows, G] of one fused operand."""

    def __init__(self, values: np.ndarray, scale_bits: np.ndarray, k: int) -> None:
        self.values = np.ascontiguousarray(values, dtype=np.int8)
        self.scale_bits = np.ascontiguousarray(scale_bits, dtype=np.uint16)
        self.k = int(k)
        self.rows = int(values.shape[0])


def _values(layer, codes) -> np.ndarray:
    if codes is None:
        codes = T.unpack_codes(layer.packed, layer.in_features)
    return codes.astype(np.int8) - np.int8(1)


class StackOracle:
    def __init__(self, weights, gemv_lanes: Callable[[int, int], int], gemm_splits: Callable[[int, int, int], int],
                 oracle: T.Oracle | None = None) -> None:
        self.oracle = oracle or T.oracle()
        self.config = weights.config
        codes = weights.codes or {}
        self._gemv_lanes = gemv_lanes
        self._gemm_splits = gemm_splits

        def single(name: str, layer) -> _Projection:
            return _Projection(_values(layer, codes.get(name)), layer.scales.view(np.uint16), layer.in_features)

        self.token = single("token", weights.token)
        self.token_packed = np.ascontiguousarray(weights.token.packed)
        self.layers = []
        for index, layer in enumerate(weights.layers):
            gate = _values(layer.gate, codes.get(f"{index}.gate"))
            up = _values(layer.up, codes.get(f"{index}.up"))
            # interleaved rows: 2j = gate j, 2j+1 = up j (the decoder's gate/up operand)
            gate_up = np.stack([gate, up], axis=1).reshape(-1, gate.shape[1])
            gate_up_scales = np.stack([layer.gate.scales.view(np.uint16), layer.up.scales.view(np.uint16)],
                                      axis=1).reshape(-1, layer.gate.scales.shape[1])
            self.layers.append(dict(
                qkv=single(f"{index}.qkv", layer.qkv),
                out=single(f"{index}.out", layer.out),
                gate_up=_Projection(gate_up, gate_up_scales, layer.gate.in_features),
                down=single(f"{index}.down", layer.down),
                mixer_norm=np.ascontiguousarray(layer.mixer_norm, dtype=np.float32),
                ffn_norm=np.ascontiguousarray(layer.ffn_norm, dtype=np.float32),
            ))
        self.final_norm = np.ascontiguousarray(weights.final_norm, dtype=np.float32)

    # ----------------------------------------------------------------- one linear

    def _linear(self, projection: _Projection, x: np.ndarray, mode: int, aux, epi: int, out: np.ndarray,
                tile: bool) -> np.ndarray:
        """One projection for one token row: quantize, exact partials, fp32 finish in the kernel's order."""
        k = projection.k
        q8, _, scale = self.oracle.quantize_rows(mode, x, k, aux=aux, eps=self.config.eps)
        partials = self.oracle.partials_i8(projection.values, T.q8_linear(q8[0], k))
        if tile:
            splits = self._gemm_splits(TILE, projection.rows, k)  # 0: one token, run as the decode GEMV
            order, param = (1, splits) if splits else (0, self._gemv_lanes(projection.rows, k))
        else:
            order, param = 0, self._gemv_lanes(projection.rows, k)
        return self.oracle.finish(order, param, epi, partials, projection.scale_bits, scale, None, out, k,
                                  out.shape[-1])

    def _layer(self, ops: dict, residual: np.ndarray, tile: bool) -> None:
        hidden, dense = self.config.hidden, self.config.dense
        mixer_in = np.zeros(3 * hidden, dtype=np.float32)
        self._linear(ops["qkv"], residual, T.MODE_NORM, ops["mixer_norm"], T.EPI_STORE, mixer_in, tile)
        self._linear(ops["out"], mixer_in[2 * hidden:], T.MODE_PLAIN, None, T.EPI_RESIDUAL, residual, tile)
        ffn = np.zeros(dense, dtype=np.float32)
        self._linear(ops["gate_up"], residual, T.MODE_NORM, ops["ffn_norm"], T.EPI_SILU_PAIR, ffn, tile)
        self._linear(ops["down"], ffn, T.MODE_PLAIN, None, T.EPI_RESIDUAL, residual, tile)

    def _head(self, residual: np.ndarray) -> np.ndarray:
        logits = np.zeros(self.config.vocab, dtype=np.float32)
        return self._linear(self.token, residual, T.MODE_NORM, self.final_norm, T.EPI_STORE, logits, False)

    def _embed(self, token: int) -> np.ndarray:
        return self.oracle.embed(np.array([token], dtype=np.int64), self.token_packed, self.token.scale_bits,
                                 self.config.hidden)[0].copy()

    # ----------------------------------------------------------------- decoding

    def prefill_logits(self, prompt) -> np.ndarray:
        """Logits of the prompt's last token through the tile path (rows of a tile are independent)."""
        residual = self._embed(int(prompt[-1]))
        for ops in self.layers:
            self._layer(ops, residual, tile=True)
        return self._head(residual)

    def step_logits(self, token: int) -> np.ndarray:
        residual = self._embed(int(token))
        for ops in self.layers:
            self._layer(ops, residual, tile=False)
        return self._head(residual)

    def generate(self, prompt, count: int, keep_logits: bool = False):
        logits = self.prefill_logits(prompt)
        tokens = [self.oracle.argmax(logits)]
        history = [logits] if keep_logits else None
        while len(tokens) < count:
            logits = self.step_logits(tokens[-1])
            tokens.append(self.oracle.argmax(logits))
            if history is not None:
                history.append(logits)
        return (tokens, history) if keep_logits else tokens

    def generate_sampled(self, prompt, uniforms, temperature: float, top_k: int, repetition_penalty: float = 1.0,
                         penalized_ids=(), max_top_k: int = 256):
        """Tokens drawn by the sampling rule (decoder.py:324-361): token j uses uniforms[j]; the seen set
        starts from penalized_ids and gains every drawn token."""
        vocab = self.config.vocab
        seen = np.zeros(vocab, dtype=np.uint8)
        for token in penalized_ids:
            if 0 <= int(token) < vocab:
                seen[int(token)] = 1
        effective = int(top_k) if 0 < int(top_k) <= max_top_k else max_top_k
        penalty = np.float32(repetition_penalty)
        inverse = np.float32(1.0 / float(repetition_penalty))
        tokens = []
        logits = self.prefill_logits(prompt)
        for j, u in enumerate(uniforms):
            if j:
                logits = self.step_logits(tokens[-1])
            token, _, _ = self.oracle.sample_token(logits, seen, np.float32(temperature), penalty, inverse,
                                                   effective, max_top_k, np.float32(u))
            tokens.append(token)
        return tokens
