"""Host-side checks that need no GPU: the C ABI library loads and exports every declared symbol,
the Python mirror of the reference FFI is consistent with it, and host logic behaves."""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest
import torch

HEADER = Path(__file__).resolve().parent.parent / "include" / "ivonar_ternary.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:hipError_t|const char\*|int|void)\s+(\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_library_exports_every_declared_entry_point():
    from ivonar_amd import runtime

    lib = runtime.library()
    declared = _declared_functions()
    assert len(declared) >= 40
    missing = [name for name in declared if not hasattr(lib, name)]
    assert not missing, missing


def test_python_signatures_cover_the_launchable_entry_points():
    from ivonar_amd import runtime

    declared = set(_declared_functions())
    assert set(runtime.SIGNATURES) <= declared
    for name in declared:
        if name.startswith(("gemv_", "gemm_tile_", "quantize_", "embed_", "gather_", "logit_", "sample_")):
            assert name in runtime.SIGNATURES, name


def test_reference_kernel_names_are_all_present():
    """Every ternary-linear kernel the reference decoder launches (ternary.cu) has an entry point."""
    from ivonar_amd import runtime

    reference = [f"gemv_{k}{w}" for k in ("plain_store", "plain_residual", "norm_store", "norm_silu_pair",
                                          "attn_residual") for w in ("", "_wide")]
    reference += ["gemv_prequant_store", "quantize_norm", "quantize_norm_wide", "embed_token", "embed_tile",
                  "gather_token"]
    reference += [f"quantize_tile_{k}{w}" for k in ("plain", "norm", "attn") for w in ("", "_wide")]
    reference += [f"gemm_tile_{k}{w}" for k in ("store", "residual", "silu_pair") for w in ("", "_wide")]
    reference += ["logit_bounds", "sample_token"]
    lib = runtime.library()
    assert all(hasattr(lib, name) for name in reference)
    assert all(name in runtime.SIGNATURES for name in reference)


def test_token_finish_limit_range():
    """The in-launch finish limit of the K-sliced token GEMV: 0..992, returning the previous value."""
    from ivonar_amd import runtime

    lib = runtime.library()
    assert lib.ivonar_token_finish_limit(992) == 992
    assert lib.ivonar_token_finish_limit(993) == -1
    assert lib.ivonar_token_finish_limit(-1) == -1
    assert lib.ivonar_token_finish_limit(0) == 992
    assert lib.ivonar_token_finish_limit(992) == 0


def test_host_only_calls():
    from ivonar_amd import runtime

    lib = runtime.library()
    assert lib.ivonar_abi_version() == runtime.ABI_VERSION
    assert lib.ivonar_define(b"NOT_A_DEFINE", 3) != 0
    assert lib.ivonar_define(b"TILE", 0) != 0
    assert lib.ivonar_define(b"TILE", 32) == 0
    assert lib.ivonar_define(b"MAX_TOPK", 1025) != 0
    assert lib.ivonar_define(b"MAX_TOPK", 256) == 0
    assert lib.ivonar_define(b"GEMV_WAIT_SPINS", 1) != 0  # no in-launch wait to bound any more
    assert lib.ivonar_error_string(1)
    assert runtime.gemm_plan(2048, 4096, 1024) == 1
    assert runtime.gemm_plan(1, 4096, 1024) == 0  # one token: the decode GEMV
    assert runtime.gemm_plan(2, 4096, 1024) >= 1
    for n, expected in [(8, 2), (64, 2), (100, 2), (1024, 16), (4096, 64), (8192, 64), (28672, 64)]:
        lanes, per_lane = runtime.gemv_plan(100, n)
        assert lanes == expected and per_lane == 2


def test_sampler_refuses_the_cpu():
    from ivonar_amd import runtime
    from ivonar_amd.sampling import DeviceSampler

    with pytest.raises(runtime.KernelError):
        DeviceSampler(32000, "cpu")


def test_launch_checks_argument_count():
    from ivonar_amd import runtime

    kernel = runtime.Kernel(None, "gemv_plain_store")
    with pytest.raises(runtime.KernelError):
        runtime.Launch(kernel, (1, 1, 1), (256, 1, 1), [runtime.int32(1)])


def test_compile_module_refuses_a_cpu_device():
    from ivonar_amd import runtime

    with pytest.raises(runtime.KernelError):
        runtime.compile_module(None, {"TILE": 32}, torch.device("cpu"))


def test_reference_lane_hints():
    """_lanes_for gives the reference's launch hints at the benchmark shapes (kernel_decoder.py:46-50)."""
    from ivonar_amd.matrix import _lanes_for

    assert _lanes_for(16, 4096, 32) == 2        # K=1024 -> N=4096
    assert _lanes_for(16, 1024, 32) == 8        # out projection
    assert _lanes_for(16, 8192, 16) == 2        # gate/up, max 16 lanes
    assert _lanes_for(64, 1024, 32) == 32       # down projection K=4096
    assert _lanes_for(128, 28672, 32) == 32     # K=8192 -> N=28672
    assert _lanes_for(448, 8192, 32) == 32      # K=28672 -> N=8192


def test_matrix_pads_stacks_and_interleaves_on_the_host():
    from ivonar_amd.matrix import Matrix
    from ivonar_amd.quantization import TernaryLinear

    g = torch.Generator().manual_seed(0)

    def layer(rows, k, bias=True):
        packed = torch.randint(0, 256, (rows, (k + 3) // 4), generator=g, dtype=torch.uint8)
        scales = (torch.rand(rows, (k + 127) // 128, generator=g) * 0.05 + 0.01).half()
        return TernaryLinear(packed, scales, k, torch.randn(rows, generator=g) if bias else None)

    gate, up = layer(6, 24), layer(6, 24)
    fused = Matrix([gate, up], torch.device("cpu"), interleave=True)
    assert fused.row_bytes == 16 and fused.rows == 12 and fused.groups == 1
    assert torch.equal(fused.packed[0::2, :6], gate.packed_weight)
    assert torch.equal(fused.packed[1::2, :6], up.packed_weight)
    assert not fused.packed[:, 6:].any()
    assert torch.equal(fused.bias[1::2], up.bias)
    stacked = Matrix([gate, up], torch.device("cpu"))
    assert torch.equal(stacked.packed[6:, :6], up.packed_weight)
    with pytest.raises(Exception):
        Matrix([gate, layer(6, 24, bias=False)], torch.device("cpu"))


def test_ternary_linear_checks_shapes_and_refuses_cpu_tensors():
    from ivonar_amd.quantization import TernaryLinear, pack_ternary_codes, unpack_ternary_codes
    from ivonar_amd.runtime import KernelError

    values = torch.randint(-1, 2, (5, 10), dtype=torch.int8)
    packed = pack_ternary_codes(values)
    assert torch.equal(unpack_ternary_codes(packed, 10), values)
    scales = torch.full((5, 1), 0.02, dtype=torch.float16)
    with pytest.raises(ValueError):
        TernaryLinear(packed[:, :2], scales, 10)
    with pytest.raises(ValueError):
        TernaryLinear(packed, scales.repeat(1, 2), 10)
    layer = TernaryLinear(packed, scales, 10)
    dense = layer.unpacked_weight()
    assert torch.allclose(dense, values.float() * 0.02, atol=1e-4)
    with pytest.raises(KernelError):
        layer(torch.randn(2, 10))


def test_synthetic_layers_follow_the_stated_statistics():
    from ivonar_amd import synthetic

    rng = np.random.default_rng(0)
    layer, codes = synthetic.ternary_layer(rng, 512, 1024, with_codes=True)
    freq = np.bincount(codes.ravel(), minlength=3) / codes.size
    assert np.allclose(freq, (0.3, 0.4, 0.3), atol=0.01)
    assert (layer.scales > 0).all() and not (codes == 3).any()
    assert layer.packed.shape == (512, 256) and layer.scales.shape == (512, 8)


def test_decoder_refuses_a_cpu_device():
    from ivonar_amd.decoder import StackDecoder
    from ivonar_amd.runtime import KernelError
    from ivonar_amd.synthetic import StackConfig, decoder_stack

    weights = decoder_stack(StackConfig(vocab=64, hidden=128, layers=1, dense=256), seed=0)
    with pytest.raises(KernelError):
        StackDecoder(weights, "cpu")


def test_sampling_rule_on_host_buffers():
    """configure_sampling's rule (decoder.py:340-361) on host-resident buffers: the top-k clamp, the
    penalized ids marked as seen (out-of-vocabulary ids ignored), and the error on a non-positive value."""
    from ivonar_amd.sampling import DeviceSampler

    sampler = object.__new__(DeviceSampler)
    sampler.vocab, sampler.max_top_k, sampler.device = 10, 4, torch.device("cpu")
    sampler.temperature, sampler.penalty, sampler.inverse_penalty = torch.ones(1), torch.ones(1), torch.ones(1)
    sampler.top_k = torch.ones(1, dtype=torch.int64)
    sampler.seen = torch.ones((1, 10), dtype=torch.bool)
    sampler.configure_sampling(0.5, 0, 2.0, penalized_ids=[3, 3, -1, 10, 9])
    assert sampler.top_k.item() == 4 and sampler.temperature.item() == 0.5
    assert sampler.penalty.item() == 2.0 and sampler.inverse_penalty.item() == 0.5
    assert sampler.seen[0].nonzero().flatten().tolist() == [3, 9]
    sampler.configure_sampling(1.0, 3)
    assert sampler.top_k.item() == 3 and not sampler.seen.any()
    sampler.configure_sampling(1.0, 5)
    assert sampler.top_k.item() == 4
    for temperature, penalty in ((0.0, 1.0), (1.0, -2.0)):
        with pytest.raises(ValueError):
            sampler.configure_sampling(temperature, 3, penalty)
