"""Device side of checkpoint loading: ivonar_validate_ternary against host brute force, and the fused
Matrix groups of a loaded checkpoint against the oracle's GEMV over the same rows."""

from __future__ import annotations

import numpy as np
import pytest

import ternary_oracle as T

pytestmark = pytest.mark.gpu


def _flags(cuda, packed: np.ndarray, scales: np.ndarray) -> int:
    import torch

    from ivonar_amd import checkpoint as C

    p = torch.from_numpy(np.ascontiguousarray(packed)).to(cuda)
    s = torch.from_numpy(np.ascontiguousarray(scales)).to(cuda)
    flags = C.validation_flags(p, s)
    torch.cuda.synchronize()
    return int(flags[0])


def _brute(packed: np.ndarray, scales: np.ndarray) -> int:
    flags = 0
    if ((packed & (packed >> 1) & 0x55) != 0).any():
        flags |= 1
    bits = scales.view(np.uint16).astype(np.uint32)
    if ((bits & 0x7C00) == 0x7C00).any():
        flags |= 2
    if (((bits & 0x8000) != 0) | (bits == 0)).any():
        flags |= 4
    return flags


@pytest.mark.parametrize("nbytes,nscales", [(1, 1), (15, 7), (16, 8), (4099, 1031), (1 << 20, 1 << 17),
                                             ((64 << 20) + 5, (1 << 22) + 3)])
def test_validation_flags_match_brute_force(cuda, nbytes, nscales):
    rng = np.random.default_rng(nbytes % 1000)
    codes = rng.integers(0, 3, size=nbytes * 4, dtype=np.uint8).reshape(-1, 4)
    packed = (codes[:, 0] | (codes[:, 1] << 2) | (codes[:, 2] << 4) | (codes[:, 3] << 6)).astype(np.uint8)
    scales = (np.abs(rng.standard_normal(nscales)) * 0.02 + 1e-3).astype(np.float16)
    print(f"validate bytes={nbytes} scales={nscales}", flush=True)
    assert _flags(cuda, packed, scales) == 0 == _brute(packed, scales)
    for where in (0, nbytes // 2, nbytes - 1):
        for field in (0, 3):
            bad = packed.copy()
            bad[where] |= np.uint8(3 << (2 * field))
            assert _flags(cuda, bad, scales) == 1 == _brute(bad, scales)
    for where in (0, nscales - 1):
        for value, flag in ((np.inf, 2), (-np.inf, 6), (np.nan, 2), (0.0, 4), (-0.0, 4), (-1e-3, 4)):
            bad = scales.copy()
            bad[where] = np.float16(value)
            assert _flags(cuda, packed, bad) == flag == _brute(packed, bad), (where, value)


def test_loaded_groups_match_the_oracle(cuda, oracle, tmp_path):
    """Every fused group of a mamba and an mla block: the GEMV over the device Matrix equals the oracle's
    GEMV over the host projections stacked (or, for gate/up, interleaved) the reference's way."""
    import torch

    from ivonar_amd import checkpoint as C
    from ivonar_amd import ops, runtime, synthetic

    path = tmp_path / "model.pt"
    synthetic.write_checkpoint(path, seed=11)
    linear = C.load_checkpoint(path)
    token, groups = linear.matrices(cuda)
    rng = np.random.default_rng(5)
    cases = [("token", [linear.token], token, False)]
    for block, layer in zip(linear.blocks, groups):
        for name, members in C.GROUPS[block.kind]:
            cases.append((name, [block.projections[m] for m in members], layer[name], name == "gate_up"))
    for name, projections, matrix, interleave in cases:
        k = projections[0].in_features
        packs = [p.packed_weight.numpy() for p in projections]
        scales = [p.weight_scales.numpy().view(np.uint16) for p in projections]
        if interleave:
            packed = np.stack(packs, axis=1).reshape(-1, packs[0].shape[1])
            scale_bits = np.stack(scales, axis=1).reshape(-1, scales[0].shape[1])
        else:
            packed, scale_bits = np.concatenate(packs), np.concatenate(scales)
        assert matrix.rows == packed.shape[0]
        x = rng.standard_normal(k).astype(np.float32)
        y = ops.gemv(matrix, torch.from_numpy(x).to(cuda)).cpu().numpy()
        q8, xsum, sx = oracle.quantize_rows(T.MODE_PLAIN, x, k)
        lanes, _ = runtime.gemv_plan(matrix.rows, k)
        expected = oracle.gemv_pairs(T.EPI_STORE, q8[0], xsum[0], sx[0], T.pad_rows16(packed), scale_bits, None,
                                     np.zeros(matrix.rows, np.float32), k, lanes)
        np.testing.assert_array_equal(y, expected, err_msg=name)


def test_reserved_code_in_a_checkpoint_is_refused(cuda, tmp_path):
    """The loader refuses a corrupt checkpoint on the host (loader.py:94-112); operands corrupted after
    loading are refused by the device check when they are uploaded."""
    import torch

    from ivonar_amd import checkpoint as C
    from ivonar_amd import synthetic

    config = synthetic.checkpoint_config()
    state = synthetic.checkpoint_state(config, seed=2)
    key = "blocks.1.mixer.kv_down_proj.packed_weight"
    state[key] = state[key].clone()
    state[key][3, 5] |= 0xC0
    synthetic.write_checkpoint(tmp_path / "bad.pt", config=config, state=state)
    with pytest.raises(RuntimeError, match=f"reserved code 3: {key}"):
        C.load_checkpoint(tmp_path / "bad.pt")
    synthetic.write_checkpoint(tmp_path / "good.pt", config=config, state=synthetic.checkpoint_state(config, seed=2))
    linear = C.load_checkpoint(tmp_path / "good.pt")
    linear.blocks[1].projections["kv_down_proj"].packed_weight[3, 5] |= 0xC0
    with pytest.raises(RuntimeError, match=r"reserved code 3: blocks.1 entry \(q_proj, kv_down_proj, k_rope_proj\)"):
        linear.matrices(cuda)
    linear = C.load_checkpoint(tmp_path / "good.pt")
    linear.blocks[0].projections["down_proj"].weight_scales[0, 0] = float("inf")
    with pytest.raises(RuntimeError, match="only finite values: blocks.0 down"):
        linear.matrices(cuda)
    assert torch.cuda.is_available()
