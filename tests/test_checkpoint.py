"""Packed-checkpoint loading for the ternary linear path on the host (reference loader.py:94-258,
config.py:6-74): the payload, contract and key checks with the reference's messages."""

from __future__ import annotations

import pytest
import torch

from ivonar_amd import checkpoint as C
from ivonar_amd import synthetic


def _write(tmp_path, **kwargs):
    path = tmp_path / "model.pt"
    payload = synthetic.write_checkpoint(path, **kwargs)
    return path, payload


def test_loads_mixed_blocks_and_metadata(tmp_path):
    path, payload = _write(tmp_path)
    linear = C.load_checkpoint(path, expected_tokenizer_sha256="0" * 64)
    config = payload["config"]
    assert linear.config.layer_types == ("mamba", "mla")
    assert linear.config.dense_dim == config["dense_intermediate_dim"]
    assert (linear.lineup, linear.stage, linear.phase, linear.step) == ("synthetic", "test", "packed", 7)
    assert linear.token.out_features == config["vocab_size"] and linear.token.in_features == config["hidden_dim"]
    mamba, mla = linear.blocks
    assert set(mamba.projections) == {"in_proj", "bc_dt_proj", "out_proj", "gate_proj", "up_proj", "down_proj"}
    assert set(mamba.mixer_tensors) == {"log_decay", "theta", "skip", "conv_weight", "conv_bias"}
    assert mla.projections["k_nope_up_proj"].in_features == config["mla_latent_dim"]
    assert mla.projections["down_proj"].in_features == config["dense_intermediate_dim"]
    state = payload["model_state"]
    assert torch.equal(mla.projections["q_proj"].packed_weight, state["blocks.1.mixer.q_proj.packed_weight"])
    assert torch.equal(linear.final_norm, state["final_norm.weight"])


def test_config_defaults_follow_the_reference():
    config = synthetic.checkpoint_config(hidden=256)
    del config["dense_intermediate_dim"], config["mla_latent_dim"], config["layer_types"]
    parsed = C.CheckpointConfig.from_payload(config)
    assert parsed.dense_dim == 4 * 256 and parsed.latent_dim == 128
    assert parsed.layer_types == ("mamba", "mamba")
    assert (parsed.base_context, parsed.final_context, parsed.rope_base, parsed.longrope_scaling) == \
        (8192, 8192, 10000.0, "linear")


@pytest.mark.parametrize("change,message", [
    ({"tie_embeddings": False}, "incompatible Ivonar checkpoint: tie_embeddings=False"),
    ({"ternary_group_size": 64}, "incompatible Ivonar checkpoint: ternary_group_size=64"),
    ({"num_experts": 2}, "mixture-of-experts checkpoints are not supported"),
    ({"layer_types": ["mamba", "attention"]}, "layer_types must name mamba or mla for every layer"),
    ({"layer_types": ["mamba"]}, "layer_types must name mamba or mla for every layer"),
])
def test_contract_violations_are_refused(change, message):
    config = synthetic.checkpoint_config()
    config.update(change)
    with pytest.raises(ValueError, match=message):
        C.CheckpointConfig.from_payload(config)
    with pytest.raises(ValueError, match="checkpoint config is invalid"):
        C.CheckpointConfig.from_payload(["not", "a", "dict"])


def test_payload_checks(tmp_path):
    path, _ = _write(tmp_path, format="other")
    with pytest.raises(RuntimeError, match="unsupported checkpoint format"):
        C.load_checkpoint(path)
    path, _ = _write(tmp_path, schema_version=2)
    with pytest.raises(RuntimeError, match="unsupported checkpoint format"):
        C.load_checkpoint(path)
    path, _ = _write(tmp_path, tokenizer_sha256="ab" * 32)
    with pytest.raises(RuntimeError, match="tokenizer SHA-256 mismatch"):
        C.load_checkpoint(path, expected_tokenizer_sha256="cd" * 32)
    assert C.load_checkpoint(path).tokenizer_sha256 == "ab" * 32
    path, _ = _write(tmp_path, tokenizer_sha256=None)
    with pytest.raises(RuntimeError, match="checkpoint is missing tokenizer_sha256"):
        C.load_checkpoint(path, expected_tokenizer_sha256="cd" * 32)
    path, _ = _write(tmp_path, model_state=[1, 2])
    with pytest.raises(RuntimeError, match="checkpoint model_state is invalid"):
        C.load_checkpoint(path)
    torch.save([1, 2, 3], tmp_path / "list.pt")
    with pytest.raises(RuntimeError, match="invalid Ivonar checkpoint"):
        C.load_checkpoint(tmp_path / "list.pt")


def _state():
    return synthetic.checkpoint_state(synthetic.checkpoint_config(), seed=3)


def _build(state):
    return C.build_linear_path(C.CheckpointConfig.from_payload(synthetic.checkpoint_config()), state)


def test_state_checks():
    state = _state()
    state["blocks.0.mixer.theta"] = 3.0
    with pytest.raises(RuntimeError, match="model_state entry is not a tensor: blocks.0.mixer.theta"):
        _build(state)
    state = _state()
    state["blocks.1.ffn.up_proj.packed_weight"] = state["blocks.1.ffn.up_proj.packed_weight"].to(torch.int16)
    with pytest.raises(RuntimeError, match="packed ternary buffer must be uint8"):
        _build(state)
    state = _state()
    state["token_io.projection.weight_scales"] = state["token_io.projection.weight_scales"].float()
    with pytest.raises(RuntimeError, match="g128 scale buffer must be float16"):
        _build(state)
    state = _state()
    del state["blocks.1.mixer.v_up_proj.weight_scales"]
    with pytest.raises(RuntimeError, match="model_state is missing blocks.1.mixer.v_up_proj.weight_scales"):
        _build(state)
    state = _state()
    state["blocks.0.extra"] = torch.zeros(1)
    with pytest.raises(RuntimeError, match="model_state has entries the model does not use: blocks.0.extra"):
        _build(state)
    state = _state()
    state["token_io.projection.packed_weight"] = state["token_io.projection.packed_weight"][:-1]
    state["token_io.projection.weight_scales"] = state["token_io.projection.weight_scales"][:-1]
    with pytest.raises(RuntimeError, match="token weight has 299 rows, config says 300"):
        _build(state)
    state = _state()
    state["blocks.0.ffn.down_proj.packed_weight"] = state["blocks.0.ffn.down_proj.packed_weight"][:, :-1]
    with pytest.raises(ValueError):
        _build(state)


def test_optional_bias_is_taken():
    state = _state()
    state["blocks.0.mixer.out_proj.bias"] = torch.zeros(256)
    linear = _build(state)
    assert linear.blocks[0].projections["out_proj"].bias is not None


def test_device_groups_need_a_rocm_device():
    from ivonar_amd.runtime import KernelError

    linear = _build(_state())
    with pytest.raises(KernelError):
        linear.matrices("cpu")


@pytest.mark.parametrize("where", [0, "middle", -1])
def test_reserved_code_and_bad_scales_are_refused_at_load(where):
    """loader.py:94-112 runs at load time: a byte carrying code 3 anywhere, an infinite, NaN, zero or
    negative scale is refused with the reference's message."""
    key = "blocks.1.ffn.down_proj"
    for field, value, message in [
        ("packed_weight", 0b11_01_01_01, "contains the reserved code 3"),
        ("packed_weight", 0b01_11_01_01, "contains the reserved code 3"),
        ("packed_weight", 0b11_10_10_10, "contains the reserved code 3"),
        ("weight_scales", float("inf"), "must contain only finite values"),
        ("weight_scales", float("nan"), "must contain only finite values"),
        ("weight_scales", 0.0, "must contain only positive values"),
        ("weight_scales", -0.01, "must contain only positive values"),
    ]:
        state = _state()
        tensor = state[f"{key}.{field}"].clone()
        flat = tensor.view(-1)
        index = flat.numel() // 2 if where == "middle" else where
        flat[index] = value
        state[f"{key}.{field}"] = tensor
        with pytest.raises(RuntimeError, match=f"{message}: {key}.{field}"):
            _build(state)


def test_reserved_byte_table_matches_the_field_decoding():
    from ivonar_amd.quantization import unpack_ternary_codes

    every_byte = torch.arange(256, dtype=torch.uint8).reshape(256, 1)
    fields = unpack_ternary_codes(every_byte, 4) + 1  # codes 0..3 of each byte's four inputs
    assert torch.equal(C._RESERVED_BYTES, (fields == 3).any(dim=1))
    assert int(C._RESERVED_BYTES.sum()) == 256 - 81  # 3**4 bytes use codes 0..2 only
