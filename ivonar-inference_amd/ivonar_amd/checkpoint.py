"""Packed checkpoints for the ternary linear path (reference: loader.py:94-258 loading and validation,
config.py:6-74 the configuration contract, kernel_decoder.py:53-142 and :230-262 the Matrix groups).

``load_checkpoint(path)`` reads an Ivonar packed checkpoint with ``torch.load(weights_only=True)``
(nothing in the file is executed), checks its format, schema, tokenizer hash and configuration contract,
every state entry (a tensor of the right dtype; packed buffers free of the reserved code 3, scales finite
and positive) and that the key set is exactly the model's, and returns the ternary linear path on the
host.  ``LinearPath.matrices(device)`` uploads it as device
``Matrix`` groups fused the way the reference decoder launches them, and checks every uploaded operand
again on the device (``ivonar_validate_ternary``), so operands built from host tensors that never went
through the loader are covered too:

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


def _dense_width(config: dict[str, Any], hidden: int) -> int:
    return int(config.get("dense_intermediate_dim", 0) or max(int(config.get("intermediate_dim", 0)), 4 * hidden))


def _latent_width(config: dict[str, Any], hidden: int) -> int:
    return int(config.get("mla_latent_dim", 0) or max(128, hidden // 4))


# The configuration fields (config.py:20-74): field name, payload key, type, and the default when the key
# is optional (None: required).  Widths that depend on others are filled in afterwards.
_CONFIG_FIELDS = (
    ("name", "name", str, ""),
    ("vocab_size", "vocab_size", int, None),
    ("seq_len", "seq_len", int, None),
    ("hidden_dim", "hidden_dim", int, None),
    ("num_layers", "num_layers", int, None),
    ("num_heads", "num_heads", int, None),
    ("state_dim", "state_dim", int, None),
    ("base_context", "base_context", int, 8192),
    ("final_context", "final_context", int, 8192),
    ("rope_base", "rope_base", float, 10000.0),
    ("longrope_scaling", "longrope_scaling", str, "linear"),
)
_LAYER_KINDS = ("mamba", "mla")


@dataclass(frozen=True)
class CheckpointConfig:
    """The configuration fields running the model needs (semantics of config.py:20-74)."""

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
        """Parse and check a payload's ``config`` dict: the contract, no experts, one known kind per layer."""
        if not isinstance(config, dict):
            raise ValueError("checkpoint config is invalid")
        wrong = [f"{key}={config.get(key)!r}" for key in REQUIRED_CONTRACT if config.get(key) != REQUIRED_CONTRACT[key]]
        if wrong:
            raise ValueError("incompatible Ivonar checkpoint: " + ", ".join(wrong))
        if int(config.get("num_experts", 0)) > 0:
            raise ValueError("mixture-of-experts checkpoints are not supported")
        values = {name: kind(config[key] if default is None else config.get(key, default))
                  for name, key, kind, default in _CONFIG_FIELDS}
        kinds = tuple(map(str, config.get("layer_types") or ())) or ("mamba",) * values["num_layers"]
        if len(kinds) != values["num_layers"] or not set(kinds) <= set(_LAYER_KINDS):
            raise ValueError("layer_types must name mamba or mla for every layer")
        hidden = values["hidden_dim"]
        return cls(layer_types=kinds, dense_dim=_dense_width(config, hidden), latent_dim=_latent_width(config, hidden),
                   **values)

    def width(self, source: str) -> int:
        """Input width of a projection by the name of its source: hidden, latent or dense."""
        return {"hidden": self.hidden_dim, "latent": self.latent_dim, "dense": self.dense_dim}[source]


# Reserved-code test per byte value: a byte holds code 3 when both bits of one of its four fields are set.
_RESERVED_BYTES = torch.tensor([any((value >> shift) & 3 == 3 for shift in (0, 2, 4, 6)) for value in range(256)])


def _holds_reserved_code(packed: Tensor) -> bool:
    """Whether any byte of a packed buffer carries code 3 (one histogram of the byte values)."""
    if packed.numel() == 0:
        return False
    counts = torch.bincount(packed.reshape(-1).to(torch.int64) if packed.device.type != "cpu"
                            else packed.reshape(-1), minlength=256)
    return bool(counts.cpu()[_RESERVED_BYTES].any())


def _check_entries(state: dict[str, Any]) -> None:
    """The reference's per-entry checks (loader.py:94-112), in the state's order: every entry a tensor; packed
    buffers uint8 with no reserved code; g128 scales float16, finite and positive."""
    for key, value in state.items():
        if not isinstance(value, Tensor):
            raise RuntimeError(f"model_state entry is not a tensor: {key}")
        if key.endswith(".packed_weight"):
            if value.dtype != torch.uint8:
                raise RuntimeError(f"packed ternary buffer must be uint8: {key}")
            if _holds_reserved_code(value):
                raise RuntimeError(f"packed ternary buffer contains the reserved code 3: {key}")
        elif key.endswith(".weight_scales"):
            if value.dtype != torch.float16:
                raise RuntimeError(f"g128 scale buffer must be float16: {key}")
            if value.numel() and not bool(torch.isfinite(value).all()):
                raise RuntimeError(f"g128 scale buffer must contain only finite values: {key}")
            if value.numel() and not bool((value > 0).all()):
                raise RuntimeError(f"g128 scale buffer must contain only positive values: {key}")


# The ternary projections of a block, by module name and the width of their input, in the order the
# reference builds its modules (loader.py:156-190); then the mixer's own tensors and the norms.
_MIXER_PROJECTIONS = {
    "mamba": (("in_proj", "hidden"), ("bc_dt_proj", "hidden"), ("out_proj", "hidden")),
    "mla": (("q_proj", "hidden"), ("kv_down_proj", "hidden"), ("k_nope_up_proj", "latent"),
            ("k_rope_proj", "hidden"), ("v_up_proj", "latent"), ("out_proj", "hidden")),
}
_FFN_PROJECTIONS = (("gate_proj", "hidden"), ("up_proj", "hidden"), ("down_proj", "dense"))
_MIXER_TENSORS = {"mamba": ("log_decay", "theta", "skip", "conv_weight", "conv_bias"), "mla": ()}

# The fused operand groups of a block and their projections, in launch order (kernel_decoder.py:236-262).
_FFN_GROUPS = (("gate_up", ("gate_proj", "up_proj")), ("down", ("down_proj",)))
GROUPS = {
    "mamba": (("entry", ("in_proj", "bc_dt_proj")), ("out", ("out_proj",))) + _FFN_GROUPS,
    "mla": (("entry", ("q_proj", "kv_down_proj", "k_rope_proj")), ("up", ("k_nope_up_proj", "v_up_proj")),
            ("out", ("out_proj",))) + _FFN_GROUPS,
}


@dataclass(frozen=True)
class _Entry:
    """One state key the model reads: a projection's part, a mixer tensor or a norm."""

    key: str
    required: bool = True


def _projection_entries(prefix: str) -> list[_Entry]:
    return [_Entry(f"{prefix}.packed_weight"), _Entry(f"{prefix}.weight_scales"), _Entry(f"{prefix}.bias", False)]


def _block_layout(kind: str, index: int) -> list[tuple[str, str, str]]:
    """(state prefix, projection name, input source) of every projection of block `index`."""
    prefix = f"blocks.{index}"
    return ([(f"{prefix}.mixer.{name}", name, source) for name, source in _MIXER_PROJECTIONS[kind]]
            + [(f"{prefix}.ffn.{name}", name, source) for name, source in _FFN_PROJECTIONS])


def _expected_entries(config: CheckpointConfig) -> list[_Entry]:
    """Every key the model reads, in the order the reference's builder takes them: the token matrix; per
    block the mixer's projections and tensors, the feed-forward projections and the two norms; the final
    norm."""
    entries = _projection_entries("token_io.projection")
    for index, kind in enumerate(config.layer_types):
        prefix = f"blocks.{index}"
        for name, _ in _MIXER_PROJECTIONS[kind]:
            entries += _projection_entries(f"{prefix}.mixer.{name}")
        entries += [_Entry(f"{prefix}.mixer.{name}") for name in _MIXER_TENSORS[kind]]
        for name, _ in _FFN_PROJECTIONS:
            entries += _projection_entries(f"{prefix}.ffn.{name}")
        entries += [_Entry(f"{prefix}.mixer_norm.weight"), _Entry(f"{prefix}.ffn_norm.weight")]
    entries.append(_Entry("final_norm.weight"))
    return entries


def _check_keys(config: CheckpointConfig, state: dict[str, Tensor]) -> None:
    """The key set must be exactly the model's: nothing required missing, nothing left over."""
    expected = _expected_entries(config)
    for entry in expected:
        if entry.required and entry.key not in state:
            raise RuntimeError(f"model_state is missing {entry.key}")
    known = {entry.key for entry in expected}
    unused = sorted(key for key in state if key not in known)
    if unused:
        raise RuntimeError(f"model_state has entries the model does not use: {', '.join(unused[:5])}")


def _linear(state: dict[str, Tensor], prefix: str, in_features: int) -> TernaryLinear:
    return TernaryLinear(state[f"{prefix}.packed_weight"], state[f"{prefix}.weight_scales"], in_features,
                         bias=state.get(f"{prefix}.bias"))


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
        on the device as well."""
        device = torch.device(device)
        token = Matrix([self.token], device, lanes=HEAD_LANES)
        named = [("token_io.projection", token)]
        groups = []
        for index, block in enumerate(self.blocks):
            layer = {}
            for group, members in GROUPS[block.kind]:
                interleave = group == "gate_up"
                layer[group] = Matrix([block.projections[name] for name in members], device, interleave=interleave,
                                      max_lanes=16 if interleave else 32)
                named.append((f"blocks.{index} {group} ({', '.join(members)})", layer[group]))
            groups.append(layer)
        if validate:
            validate_matrices(named)
        return token, groups


def build_linear_path(config: CheckpointConfig, state: dict[str, Any]) -> LinearPath:
    """The ternary linear path of a packed state dict (loader.py:146-203 for these modules): the
    entry checks, the exact key set, then every projection with its shape checks."""
    _check_entries(state)
    _check_keys(config, state)
    token = _linear(state, "token_io.projection", config.hidden_dim)
    if token.out_features != config.vocab_size:
        raise RuntimeError(f"token weight has {token.out_features} rows, config says {config.vocab_size}")
    blocks = []
    for index, kind in enumerate(config.layer_types):
        projections = {name: _linear(state, prefix, config.width(source))
                       for prefix, name, source in _block_layout(kind, index)}
        mixer = {name: state[f"blocks.{index}.mixer.{name}"] for name in _MIXER_TENSORS[kind]}
        blocks.append(BlockLinears(kind, projections, state[f"blocks.{index}.mixer_norm.weight"],
                                   state[f"blocks.{index}.ffn_norm.weight"], mixer))
    return LinearPath(config, token, blocks, state["final_norm.weight"])


def _read_payload(model_file: Path) -> dict[str, Any]:
    """The checkpoint dict, loaded without executing anything from the file, with its format checked."""
    payload = torch.load(model_file, map_location="cpu", weights_only=True)
    if not isinstance(payload, dict):
        raise RuntimeError(f"invalid Ivonar checkpoint: {model_file}")
    if (payload.get("format"), payload.get("schema_version")) != (PACKED_FORMAT, PACKED_SCHEMA_VERSION):
        raise RuntimeError(f"unsupported checkpoint format; expected {PACKED_FORMAT} schema {PACKED_SCHEMA_VERSION}")
    return payload


def _check_tokenizer(found: str | None, expected: str | None) -> None:
    if expected is None:
        return
    if found is None:
        raise RuntimeError("checkpoint is missing tokenizer_sha256")
    if found != str(expected):
        raise RuntimeError(f"tokenizer SHA-256 mismatch: expected {expected}, found {found}")


def _optional_text(payload: dict[str, Any], key: str) -> str | None:
    value = payload.get(key)
    return None if value is None else str(value)


def load_checkpoint(path: str | Path, expected_tokenizer_sha256: str | None = None) -> LinearPath:
    """Read a packed checkpoint (the checks of loader.py:222-242 with the reference's messages) and
    return its ternary linear path with the payload's metadata."""
    model_file = Path(path)
    payload = _read_payload(model_file)
    config = CheckpointConfig.from_payload(payload.get("config"))
    tokenizer = str(payload["tokenizer_sha256"]) if payload.get("tokenizer_sha256") else None
    _check_tokenizer(tokenizer, expected_tokenizer_sha256)
    state = payload.get("model_state")
    if not isinstance(state, dict):
        raise RuntimeError("checkpoint model_state is invalid")
    linear_path = build_linear_path(config, state)
    linear_path.path = model_file
    linear_path.lineup, linear_path.stage, linear_path.phase = (
        _optional_text(payload, key) for key in ("lineup", "stage", "phase"))
    linear_path.step = int(payload.get("step", 0) or 0)
    linear_path.tokenizer_sha256 = tokenizer
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
