"""Packed checkpoints for the ternary linear path (reference: loader.py:94-258 loading and validation,
config.py:6-74 the configuration contract, kernel_decoder.py:53-142 and :230-262 the Matrix groups).

``load_checkpoint(path)`` reads an Ivonar packed checkpoint with ``torch.load(weights_only=True)``
(nothing in the file is executed), checks its format, schema, tokenizer hash and configuration contract,
that every state entry is a tensor of the right dtype and that the key set is exactly the model's, and
returns the ternary linear path on the host.  ``LinearPath.matrices(device)`` uploads it as device
``Matrix`` groups fused the way the reference decoder launches them, and validates every operand on the
device (``ivonar_validate_ternary``: reserved code 3, non-finite or non-positive scales):

* token matrix: ``token_io.projection`` (4 lanes, the LM head and the embedding);
* per ``mamba`` block: ``entry`` = [in_proj, bc_dt_proj], ``out`` = [out_proj];
* per ``mla`` block: ``entry`` = [q_proj, kv_down_proj, k_rope_proj], ``up`` = [k_nope_up_proj, v_up_proj],
  ``out`` = [out_proj];
* per block: ``gate_up`` = [gate_proj, up_proj] interleaved (16 lanes at most), ``down`` = [down_proj].

The mixers' own tensors (decay, theta, skip, convolution) are required and counted as used, as the
reference's model builder does, and are handed back untouched in ``mixer_tensors``: the mixers are not
part of this path.  Errors are the reference's ``RuntimeError`` / ``ValueError`` messages.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import torch
from torch import Tensor

from .matrix import Matrix
from .quantization import TernaryLinear
from .runtime import KernelError, check, current_stream, library, pointer

PACKED_FORMAT = "ivonar_packed_ternary_inference"
PACKED_SCHEMA_VERSION = 1
HEAD_LANES = 4

# config.py:6-17: what a checkpoint must declare to run on the ternary kernels.
REQUIRED_CONTRACT = {
    "architecture": "ivonar_native_ternary",
    "architecture_version": 1,
    "ternary_group_size": 128,
    "ternary_storage": "q2_g128",
    "activation_quantization": "int8_per_token",
    "output_head_type": "tied_ternary_embedding_head",
    "mla_rope_layout": "decoupled_direct_rope",
    "mamba_implementation": "ivonar_mamba3_conv_et_mimo",
    "mamba_variant": "MIMO",
    "tie_embeddings": True,
}

FLAG_RESERVED_CODE, FLAG_NONFINITE_SCALE, FLAG_NONPOSITIVE_SCALE = 1, 2, 4


@dataclass(frozen=True)
class CheckpointConfig:
    """config.py:20-74: the configuration fields running the model needs."""

    name: str
    vocab_size: int
    seq_len: int
    hidden_dim: int
    num_layers: int
    num_heads: int
    state_dim: int
    layer_types: tuple[str, ...]
    dense_dim: int
    latent_dim: int
    base_context: int
    final_context: int
    rope_base: float
    longrope_scaling: str

    @classmethod
    def from_payload(cls, config: Any) -> "CheckpointConfig":
        if not isinstance(config, dict):
            raise ValueError("checkpoint config is invalid")
        mismatches = [f"{key}={config.get(key)!r}" for key, expected in REQUIRED_CONTRACT.items()
                      if config.get(key) != expected]
        if mismatches:
            raise ValueError("incompatible Ivonar checkpoint: " + ", ".join(mismatches))
        if int(config.get("num_experts", 0)) > 0:
            raise ValueError("mixture-of-experts checkpoints are not supported")
        hidden = int(config["hidden_dim"])
        layers = int(config["num_layers"])
        kinds = tuple(str(kind) for kind in config.get("layer_types") or ())
        if not kinds:
            kinds = tuple("mamba" for _ in range(layers))
        if len(kinds) != layers or any(kind not in {"mamba", "mla"} for kind in kinds):
            raise ValueError("layer_types must name mamba or mla for every layer")
        return cls(
            name=str(config.get("name", "")),
            vocab_size=int(config["vocab_size"]),
            seq_len=int(config["seq_len"]),
            hidden_dim=hidden,
            num_layers=layers,
            num_heads=int(config["num_heads"]),
            state_dim=int(config["state_dim"]),
            layer_types=kinds,
            dense_dim=int(config.get("dense_intermediate_dim", 0)
                          or max(int(config.get("intermediate_dim", 0)), 4 * hidden)),
            latent_dim=int(config.get("mla_latent_dim", 0) or max(128, hidden // 4)),
            base_context=int(config.get("base_context", 8192)),
            final_context=int(config.get("final_context", 8192)),
            rope_base=float(config.get("rope_base", 10000.0)),
            longrope_scaling=str(config.get("longrope_scaling", "linear")),
        )


def _check_entries(state: dict[str, Any]) -> None:
    """loader.py:94-112, the host part: every entry a tensor, packed buffers uint8, scales float16."""
    for key, value in state.items():
        if not isinstance(value, Tensor):
            raise RuntimeError(f"model_state entry is not a tensor: {key}")
        if key.endswith(".packed_weight") and value.dtype != torch.uint8:
            raise RuntimeError(f"packed ternary buffer must be uint8: {key}")
        if key.endswith(".weight_scales") and value.dtype != torch.float16:
            raise RuntimeError(f"g128 scale buffer must be float16: {key}")


class _StateReader:
    """Hands out state tensors by key and reports what was never asked for (loader.py:115-145)."""

    def __init__(self, state: dict[str, Tensor]) -> None:
        self.state = state
        self.used: set[str] = set()

    def take(self, key: str) -> Tensor:
        if key not in self.state:
            raise RuntimeError(f"model_state is missing {key}")
        self.used.add(key)
        return self.state[key]

    def take_optional(self, key: str) -> Tensor | None:
        if key not in self.state:
            return None
        self.used.add(key)
        return self.state[key]

    def linear(self, prefix: str, in_features: int) -> TernaryLinear:
        return TernaryLinear(self.take(f"{prefix}.packed_weight"), self.take(f"{prefix}.weight_scales"), in_features,
                             bias=self.take_optional(f"{prefix}.bias"))

    def unused(self) -> list[str]:
        return sorted(set(self.state) - self.used)


_MAMBA_TENSORS = ("log_decay", "theta", "skip", "conv_weight", "conv_bias")

# The fused operand groups of a block and their projections, in launch order (kernel_decoder.py:236-262).
_FFN = (("gate_up", ("gate_proj", "up_proj")), ("down", ("down_proj",)))
GROUPS = {
    "mamba": (("entry", ("in_proj", "bc_dt_proj")), ("out", ("out_proj",))) + _FFN,
    "mla": (("entry", ("q_proj", "kv_down_proj", "k_rope_proj")), ("up", ("k_nope_up_proj", "v_up_proj")),
            ("out", ("out_proj",))) + _FFN,
}


@dataclass
class BlockLinears:
    """One block's ternary projections, by the names of the reference's modules."""

    kind: str
    projections: dict[str, TernaryLinear]
    mixer_norm: Tensor
    ffn_norm: Tensor
    mixer_tensors: dict[str, Tensor] = field(default_factory=dict)


@dataclass
class LinearPath:
    """The ternary linear path of a checkpoint (host tensors) and its metadata."""

    config: CheckpointConfig
    token: TernaryLinear
    blocks: list[BlockLinears]
    final_norm: Tensor
    path: Path | None = None
    lineup: str | None = None
    stage: str | None = None
    phase: str | None = None
    step: int = 0
    tokenizer_sha256: str | None = None

    def matrices(self, device: torch.device | str, validate: bool = True):
        """(token matrix, per-block dict of Matrix) on `device`, fused as the reference decoder's
        launches are (kernel_decoder.py:230-262); with `validate`, every uploaded operand is checked
        on the device first."""
        device = torch.device(device)
        token = Matrix([self.token], device, lanes=HEAD_LANES)
        named = [("token_io.projection", token)]
        groups = []
        for index, block in enumerate(self.blocks):
            p = block.projections
            layer = {}
            for group, members in GROUPS[block.kind]:
                interleave = group == "gate_up"
                layer[group] = Matrix([p[name] for name in members], device, interleave=interleave,
                                      max_lanes=16 if interleave else 32)
                named.append((f"blocks.{index} {group} ({', '.join(members)})", layer[group]))
            groups.append(layer)
        if validate:
            validate_matrices(named)
        return token, groups


def build_linear_path(config: CheckpointConfig, state: dict[str, Any]) -> LinearPath:
    """loader.py:148-219 for the ternary linear path: the same keys, shapes and unused-entry check."""
    _check_entries(state)
    reader = _StateReader(state)
    hidden = config.hidden_dim
    token = reader.linear("token_io.projection", hidden)
    if token.out_features != config.vocab_size:
        raise RuntimeError(f"token weight has {token.out_features} rows, config says {config.vocab_size}")
    blocks = []
    for index, kind in enumerate(config.layer_types):
        prefix = f"blocks.{index}"
        projections: dict[str, TernaryLinear] = {}
        mixer_tensors: dict[str, Tensor] = {}
        if kind == "mamba":
            projections["in_proj"] = reader.linear(f"{prefix}.mixer.in_proj", hidden)
            projections["bc_dt_proj"] = reader.linear(f"{prefix}.mixer.bc_dt_proj", hidden)
            projections["out_proj"] = reader.linear(f"{prefix}.mixer.out_proj", hidden)
            for name in _MAMBA_TENSORS:
                mixer_tensors[name] = reader.take(f"{prefix}.mixer.{name}")
        else:
            projections["q_proj"] = reader.linear(f"{prefix}.mixer.q_proj", hidden)
            projections["kv_down_proj"] = reader.linear(f"{prefix}.mixer.kv_down_proj", hidden)
            projections["k_nope_up_proj"] = reader.linear(f"{prefix}.mixer.k_nope_up_proj", config.latent_dim)
            projections["k_rope_proj"] = reader.linear(f"{prefix}.mixer.k_rope_proj", hidden)
            projections["v_up_proj"] = reader.linear(f"{prefix}.mixer.v_up_proj", config.latent_dim)
            projections["out_proj"] = reader.linear(f"{prefix}.mixer.out_proj", hidden)
        projections["gate_proj"] = reader.linear(f"{prefix}.ffn.gate_proj", hidden)
        projections["up_proj"] = reader.linear(f"{prefix}.ffn.up_proj", hidden)
        projections["down_proj"] = reader.linear(f"{prefix}.ffn.down_proj", config.dense_dim)
        blocks.append(BlockLinears(kind, projections, reader.take(f"{prefix}.mixer_norm.weight"),
                                   reader.take(f"{prefix}.ffn_norm.weight"), mixer_tensors))
    final_norm = reader.take("final_norm.weight")
    unused = reader.unused()
    if unused:
        raise RuntimeError(f"model_state has entries the model does not use: {', '.join(unused[:5])}")
    return LinearPath(config, token, blocks, final_norm)


def load_checkpoint(path: str | Path, expected_tokenizer_sha256: str | None = None) -> LinearPath:
    """loader.py:222-258 up to the model build: the payload checks, then ``build_linear_path``."""
    model_file = Path(path)
    payload = torch.load(model_file, map_location="cpu", weights_only=True)
    if not isinstance(payload, dict):
        raise RuntimeError(f"invalid Ivonar checkpoint: {model_file}")
    if payload.get("format") != PACKED_FORMAT or payload.get("schema_version") != PACKED_SCHEMA_VERSION:
        raise RuntimeError(f"unsupported checkpoint format; expected {PACKED_FORMAT} schema {PACKED_SCHEMA_VERSION}")
    config = CheckpointConfig.from_payload(payload.get("config"))
    tokenizer_sha256 = str(payload["tokenizer_sha256"]) if payload.get("tokenizer_sha256") else None
    if expected_tokenizer_sha256 is not None:
        if tokenizer_sha256 is None:
            raise RuntimeError("checkpoint is missing tokenizer_sha256")
        if tokenizer_sha256 != str(expected_tokenizer_sha256):
            raise RuntimeError(
                f"tokenizer SHA-256 mismatch: expected {expected_tokenizer_sha256}, found {tokenizer_sha256}")
    state = payload.get("model_state")
    if not isinstance(state, dict):
        raise RuntimeError("checkpoint model_state is invalid")
    linear_path = build_linear_path(config, state)
    linear_path.path = model_file
    linear_path.lineup = str(payload["lineup"]) if payload.get("lineup") is not None else None
    linear_path.stage = str(payload["stage"]) if payload.get("stage") is not None else None
    linear_path.phase = str(payload["phase"]) if payload.get("phase") is not None else None
    linear_path.step = int(payload.get("step", 0) or 0)
    linear_path.tokenizer_sha256 = tokenizer_sha256
    return linear_path


def validation_flags(packed: Tensor, scales: Tensor) -> Tensor:
    """Launches ``ivonar_validate_ternary`` over one device operand on the current stream; returns the
    int32 flags tensor (not yet synchronised)."""
    if packed.device.type != "cuda" or scales.device.type != "cuda":
        raise KernelError("the checkpoint checks run on a ROCm device")
    if packed.dtype != torch.uint8 or scales.dtype != torch.float16:
        raise KernelError("packed must be uint8 and scales float16")
    packed = packed.contiguous()
    scales = scales.contiguous()
    flags = torch.zeros(1, dtype=torch.int32, device=packed.device)
    check(library().ivonar_validate_ternary(current_stream(packed.device), pointer(packed), packed.numel(),
                                            pointer(scales), scales.numel(), pointer(flags)),
          "ivonar_validate_ternary")
    return flags


def validate_matrices(named: list[tuple[str, Matrix]]) -> None:
    """The reference's packed-buffer checks (loader.py:98-112) on device operands, one read-back for all."""
    if not named:
        return
    flags = torch.cat([validation_flags(matrix.packed, matrix.scales) for _, matrix in named]).cpu().tolist()
    for (name, _), value in zip(named, flags):
        if value & FLAG_RESERVED_CODE:
            raise RuntimeError(f"packed ternary buffer contains the reserved code 3: {name}")
        if value & FLAG_NONFINITE_SCALE:
            raise RuntimeError(f"g128 scale buffer must contain only finite values: {name}")
        if value & FLAG_NONPOSITIVE_SCALE:
            raise RuntimeError(f"g128 scale buffer must contain only positive values: {name}")
