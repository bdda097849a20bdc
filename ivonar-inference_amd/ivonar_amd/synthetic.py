"""Seeded synthetic ternary layers and activations for the benchmark workloads.

There are no checkpoints here, so every workload uses random-init packed
weights with the stated statistics.  Codes are drawn categorically over
{0, 1, 2} (code = w + 1) and packed four per byte in the reference layout;
fp16 group scales that would round to zero are raised to the smallest
positive fp16 value, since packed checkpoints require positive scales
(reference loader.py:106-112).  Generators are numpy PCG64 streams seeded by
the workload number.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

GROUP = 128
SMALLEST_HALF = np.float16(np.finfo(np.float16).smallest_subnormal)


@dataclass
class Layer:
    """One packed ternary matrix on the host: packed uint8 [N, ceil(K/4)], fp16 scales [N, G]."""

    packed: np.ndarray
    scales: np.ndarray
    in_features: int
    bias: np.ndarray | None = None

    @property
    def rows(self) -> int:
        return int(self.packed.shape[0])

    @property
    def scale_bits(self) -> np.ndarray:
        return self.scales.view(np.uint16)


def sample_codes(rng: np.random.Generator, rows: int, k: int, p=(0.3, 0.4, 0.3)) -> np.ndarray:
    """uint8 codes [rows, k] with P(code 0, 1, 2) = p (w = code - 1)."""
    u = rng.random((rows, k), dtype=np.float32)
    return ((u >= np.float32(p[0])).astype(np.uint8) + (u >= np.float32(p[0] + p[1])).astype(np.uint8))


def pack_codes(codes: np.ndarray) -> np.ndarray:
    rows, k = codes.shape
    width = math.ceil(k / 4)
    if k % 4:
        codes = np.concatenate([codes, np.ones((rows, width * 4 - k), dtype=np.uint8)], axis=1)
    q = codes.reshape(rows, width, 4)
    return (q[..., 0] | (q[..., 1] << 2) | (q[..., 2] << 4) | (q[..., 3] << 6)).astype(np.uint8)


def to_half_scales(values: np.ndarray) -> np.ndarray:
    half = values.astype(np.float16)
    return np.where(half > 0, half, SMALLEST_HALF).astype(np.float16)


def abs_normal_scales(rng: np.random.Generator, rows: int, groups: int, sigma: float, offset: float = 0.0):
    return to_half_scales(np.abs(rng.normal(0.0, sigma, size=(rows, groups))) + offset)


def lognormal_scales(rng: np.random.Generator, rows: int, groups: int, mu: float, sigma: float):
    return to_half_scales(np.exp(rng.normal(mu, sigma, size=(rows, groups))))


def ternary_layer(
    rng: np.random.Generator, rows: int, k: int, p=(0.3, 0.4, 0.3), scale: str = "abs_normal", sigma: float = 0.02,
    offset: float = 1e-4, mu: float = -4.0, with_codes: bool = False,
):
    """A packed layer; with_codes also returns the uint8 codes [rows, k]."""
    codes = sample_codes(rng, rows, k, p)
    groups = math.ceil(k / GROUP)
    if scale == "lognormal":
        scales = lognormal_scales(rng, rows, groups, mu, sigma)
    else:
        scales = abs_normal_scales(rng, rows, groups, sigma, offset)
    layer = Layer(pack_codes(codes), scales, k)
    return (layer, codes) if with_codes else layer


# Workloads -----------------------------------------------------------------

GEMV_SHAPE = (1024, 4096)  # single ternary linear at M=1: K -> N
STRESS_SHAPES = ((8192, 28672), (28672, 8192))  # large-shape HBM stress at M=1
PREFILL_SHAPES = ((1024, 4096), (4096, 1024))  # prefill tile GEMM shapes
SWEEP_SHAPE = (4096, 14336)
SWEEP_M = (1, 2, 4, 8, 16, 32, 64, 128, 512, 2048)


def single_linear(seed: int = 0):
    """K=1024 -> N=4096, p=(0.3,0.4,0.3), scale |N(0,0.02)|+1e-4, x ~ N(0,1) [1, 1024]."""
    rng = np.random.default_rng(seed)
    k, n = GEMV_SHAPE
    layer = ternary_layer(rng, n, k, sigma=0.02, offset=1e-4)
    x = rng.standard_normal((1, k)).astype(np.float32)
    return layer, x


def stress_layers(seed: int = 3):
    """8192->28672 and 28672->8192, scale |N(0,0.01)|, x ~ N(0,1)."""
    rng = np.random.default_rng(seed)
    out = []
    for k, n in STRESS_SHAPES:
        layer = ternary_layer(rng, n, k, sigma=0.01, offset=0.0)
        out.append((layer, rng.standard_normal((1, k)).astype(np.float32)))
    return out


def prefill_activations(rng: np.random.Generator, length: int, k: int, outlier_fraction: float = 0.01):
    """N(0,1) [length, k] with a fixed 1% of channels scaled by 20."""
    x = rng.standard_normal((length, k)).astype(np.float32)
    channels = np.sort(np.random.default_rng(1000 + k).choice(k, max(1, int(k * outlier_fraction)), replace=False))
    x[:, channels] *= np.float32(20.0)
    return x


def prefill_layers(seed: int = 2):
    rng = np.random.default_rng(seed)
    return [(ternary_layer(rng, n, k, sigma=0.02, offset=1e-4), k) for k, n in PREFILL_SHAPES]


def sweep_layer(seed: int = 4):
    """4096->14336 with p(0)=0.6, p(+-1)=0.2, lognormal(-4, 0.5) scales."""
    rng = np.random.default_rng(seed)
    k, n = SWEEP_SHAPE
    return ternary_layer(rng, n, k, p=(0.2, 0.6, 0.2), scale="lognormal", mu=-4.0, sigma=0.5), rng


def student_t(rng: np.random.Generator, shape, dof: float = 3.0) -> np.ndarray:
    return rng.standard_t(dof, size=shape).astype(np.float32)


# Decoder-shaped stack -------------------------------------------------------


@dataclass
class StackConfig:
    """A decoder's ternary linear path: per layer a fused QKV entry (norm prologue), an output
    projection fed by the V third of the entry's output (the mixer is not part of this path), a
    gated MLP (gate and up interleaved, silu pair) and a down projection; a tied ternary
    embedding / LM head over the vocabulary."""

    vocab: int = 32000
    hidden: int = 1024
    layers: int = 24
    dense: int = 4096
    eps: float = 1e-6

    @property
    def qkv(self) -> int:
        return 3 * self.hidden


@dataclass
class StackLayer:
    qkv: Layer
    out: Layer
    gate: Layer
    up: Layer
    down: Layer
    mixer_norm: np.ndarray
    ffn_norm: np.ndarray


@dataclass
class LinearStackWeights:
    config: StackConfig
    token: Layer
    layers: list
    final_norm: np.ndarray
    codes: dict | None = None  # name -> uint8 codes [rows, K] when kept

    def named_layers(self):
        yield "token", self.token
        for index, layer in enumerate(self.layers):
            for name in ("qkv", "out", "gate", "up", "down"):
                yield f"{index}.{name}", getattr(layer, name)


def decoder_stack(config: StackConfig | None = None, seed: int = 1, keep_codes: bool = False) -> LinearStackWeights:
    """Random-init weights: codes p=(0.3,0.4,0.3), scales |N(0,0.02)|+1e-4, norm weights 1+0.1*N(0,1)."""
    config = config or StackConfig()
    rng = np.random.default_rng(seed)
    codes: dict | None = {} if keep_codes else None

    def make(name: str, rows: int, k: int) -> Layer:
        layer, c = ternary_layer(rng, rows, k, sigma=0.02, offset=1e-4, with_codes=True)
        if codes is not None:
            codes[name] = c
        return layer

    def norm() -> np.ndarray:
        return (1.0 + 0.1 * rng.standard_normal(config.hidden)).astype(np.float32)

    token = make("token", config.vocab, config.hidden)
    layers = []
    for index in range(config.layers):
        layers.append(StackLayer(
            qkv=make(f"{index}.qkv", config.qkv, config.hidden),
            out=make(f"{index}.out", config.hidden, config.hidden),
            gate=make(f"{index}.gate", config.dense, config.hidden),
            up=make(f"{index}.up", config.dense, config.hidden),
            down=make(f"{index}.down", config.hidden, config.dense),
            mixer_norm=norm(),
            ffn_norm=norm(),
        ))
    return LinearStackWeights(config, token, layers, norm(), codes)


def prompt_ids(vocab: int, length: int = 36, seed: int = 1) -> list[int]:
    """Random prompt ids in [2, vocab)."""
    return [int(v) for v in np.random.default_rng(10_000 + seed).integers(2, vocab, size=length)]


# Packed checkpoints ----------------------------------------------------------


def checkpoint_config(vocab: int = 300, hidden: int = 256, layer_types=("mamba", "mla"), dense: int = 512,
                      latent: int = 128, heads: int = 4, state_dim: int = 16) -> dict:
    """A configuration dictionary that satisfies the packed-checkpoint contract (reference config.py:6-74)."""
    return {
        "architecture": "ivonar_native_ternary", "architecture_version": 1, "ternary_group_size": 128,
        "ternary_storage": "q2_g128", "activation_quantization": "int8_per_token",
        "output_head_type": "tied_ternary_embedding_head", "mla_rope_layout": "decoupled_direct_rope",
        "mamba_implementation": "ivonar_mamba3_conv_et_mimo", "mamba_variant": "MIMO", "tie_embeddings": True,
        "name": "synthetic", "vocab_size": vocab, "seq_len": 512, "hidden_dim": hidden,
        "num_layers": len(layer_types), "num_heads": heads, "state_dim": state_dim,
        "layer_types": list(layer_types), "dense_intermediate_dim": dense, "mla_latent_dim": latent,
    }


def checkpoint_state(config: dict, seed: int = 0) -> dict:
    """A model_state with the reference's key names and shapes for `config` (random ternary codes,
    positive fp16 scales, norms near 1; the mixers' own tensors are small random arrays).  Output
    widths of the mixer projections are this generator's choice: the checkpoint format fixes only
    their input widths."""
    import torch

    rng = np.random.default_rng(seed)
    hidden, dense, latent = config["hidden_dim"], config["dense_intermediate_dim"], config["mla_latent_dim"]
    heads, state_dim = config["num_heads"], config["state_dim"]
    state: dict = {}

    def linear(prefix: str, rows: int, k: int) -> None:
        state[f"{prefix}.packed_weight"] = torch.from_numpy(pack_codes(sample_codes(rng, rows, k)))
        state[f"{prefix}.weight_scales"] = torch.from_numpy(
            to_half_scales(np.abs(rng.normal(0.0, 0.02, size=(rows, math.ceil(k / GROUP)))) + 1e-4))

    def vector(key: str, n: int, base: float = 1.0, spread: float = 0.1) -> None:
        state[key] = torch.from_numpy((base + spread * rng.standard_normal(n)).astype(np.float32))

    linear("token_io.projection", config["vocab_size"], hidden)
    for index, kind in enumerate(config["layer_types"]):
        prefix = f"blocks.{index}"
        if kind == "mamba":
            linear(f"{prefix}.mixer.in_proj", 2 * hidden + 2 * heads * state_dim, hidden)
            linear(f"{prefix}.mixer.bc_dt_proj", 2 * heads * state_dim + heads, hidden)
            linear(f"{prefix}.mixer.out_proj", hidden, hidden)
            vector(f"{prefix}.mixer.log_decay", heads, 0.0, 1.0)
            vector(f"{prefix}.mixer.theta", heads, 0.0, 1.0)
            vector(f"{prefix}.mixer.skip", hidden, 0.0, 1.0)
            vector(f"{prefix}.mixer.conv_weight", hidden * 4, 0.0, 0.1)
            vector(f"{prefix}.mixer.conv_bias", hidden, 0.0, 0.1)
        else:
            linear(f"{prefix}.mixer.q_proj", hidden, hidden)
            linear(f"{prefix}.mixer.kv_down_proj", latent, hidden)
            linear(f"{prefix}.mixer.k_nope_up_proj", hidden, latent)
            linear(f"{prefix}.mixer.k_rope_proj", 64, hidden)
            linear(f"{prefix}.mixer.v_up_proj", hidden, latent)
            linear(f"{prefix}.mixer.out_proj", hidden, hidden)
        linear(f"{prefix}.ffn.gate_proj", dense, hidden)
        linear(f"{prefix}.ffn.up_proj", dense, hidden)
        linear(f"{prefix}.ffn.down_proj", hidden, dense)
        vector(f"{prefix}.mixer_norm.weight", hidden)
        vector(f"{prefix}.ffn_norm.weight", hidden)
    vector("final_norm.weight", hidden)
    return state


def write_checkpoint(path, config: dict | None = None, state: dict | None = None, seed: int = 0,
                     tokenizer_sha256: str | None = "0" * 64, **extra) -> dict:
    """Writes a packed checkpoint in the reference's payload layout (loader.py:222-258) with torch.save;
    returns the payload."""
    import torch

    config = config or checkpoint_config()
    payload = {"format": "ivonar_packed_ternary_inference", "schema_version": 1, "config": config,
               "model_state": state if state is not None else checkpoint_state(config, seed),
               "tokenizer_sha256": tokenizer_sha256, "lineup": "synthetic", "stage": "test", "phase": "packed",
               "step": 7}
    payload.update(extra)
    torch.save(payload, path)
    return payload
