"""The Python FFI mirror exposes everything the reference decoder takes from its kernel runtime.

The reference's ``kernel_decoder.py`` binds its kernels through ``kernels/runtime.py``: it imports
``KernelError, Launch, float32, int32, pointer`` (``kernel_decoder.py:13-14``), calls
``runtime.compile_module(source, defines, device)`` (``:216``) and four methods of
``runtime.driver()``: ``persisting_capacity(device)`` (``:226``), ``reserve_persisting(device, nbytes)``
(``:274``), ``bind(device)`` (``:448,552,677,684``) and ``persist_on_stream(stream, base, nbytes)``
(``:518``).  Swapping the module for ``ivonar_amd.runtime`` must leave every one of those calls
resolvable with the same arguments.
"""

from __future__ import annotations

import inspect

import pytest
import torch

from ivonar_amd import runtime

# (attribute of the runtime module, positional parameters the reference's call passes)
MODULE_CALLS = [
    ("compile_module", ["source", "defines", "device"]),
    ("pointer", ["tensor"]),
    ("int32", ["value"]),
    ("float32", ["value"]),
]
DRIVER_CALLS = [
    ("persisting_capacity", 1),   # kernel_decoder.py:226
    ("reserve_persisting", 2),    # :274
    ("bind", 1),                  # :448, :552, :677, :684
    ("persist_on_stream", 3),     # :518
]


def _accepts(function, count: int) -> bool:
    signature = inspect.signature(function)
    try:
        signature.bind(*range(count))
    except TypeError:
        return False
    return True


def test_module_level_names():
    assert issubclass(runtime.KernelError, RuntimeError)
    for name, params in MODULE_CALLS:
        function = getattr(runtime, name)
        assert _accepts(function, len(params)), name
    assert _accepts(runtime.Launch, 4) and _accepts(runtime.Launch, 5)  # kernel, grid, block, args[, shared]
    assert callable(runtime.driver)


def test_driver_methods_and_one_driver_per_process():
    first = runtime.driver()
    assert first is runtime.driver()
    for name, count in DRIVER_CALLS:
        method = getattr(first, name)
        assert _accepts(method, count), name


def test_ctypes_arguments_are_read_at_call_time():
    value = runtime.int32(3)
    value.value = 7
    assert value.value == 7
    assert runtime.pointer(None).value in (None, 0)
    assert runtime.float32(0.5).value == 0.5


@pytest.mark.skipif(torch.cuda.is_available(), reason="checks the refusal without a ROCm device")
def test_driver_refuses_without_a_device():
    with pytest.raises(runtime.KernelError):
        runtime.driver().persisting_capacity(0)
    with pytest.raises(runtime.KernelError):
        runtime.driver().bind(0)


def test_persist_on_stream_refuses_a_window():
    driver = runtime.driver()
    driver.persist_on_stream(1, 4096, 0)  # an empty window is accepted
    with pytest.raises(runtime.KernelError):
        driver.persist_on_stream(1, 4096, 1 << 20)
    with pytest.raises(runtime.KernelError):
        driver.persist_on_stream(1, 4096, -1)


def test_modules_keep_their_own_defines():
    small = runtime.Module((0, (("HEAD_DIM", 16),)), {"HEAD_DIM": 16})
    default = runtime.Module((0, ()), {})
    assert dict(small.define_values)["HEAD_DIM"] == 16
    assert dict(default.define_values)["HEAD_DIM"] == 64
    assert dict(default.define_values)["TILE"] == 32


def test_launches_of_modules_with_different_defines_do_not_interleave(monkeypatch):
    """Two threads launch kernels of modules with different HEAD_DIM / TILE over and over; the
    library's process-wide define values must be the launching module's at every launch (the values
    are made current and the kernel launched under one lock).  A recording stand-in replaces the
    library, so no device is needed."""
    import threading
    import time

    current: dict[str, int] = {}
    seen: list[tuple[str, tuple]] = []

    class FakeLibrary:
        def ivonar_define(self, name: bytes, value: int) -> int:
            current[name.decode()] = int(value)
            time.sleep(1e-4)  # let the other thread run between defines
            return 0

    def fake_kernel(tag):
        def function(stream, *args):
            seen.append((tag, tuple(sorted(current.items()))))
            time.sleep(1e-4)
            return 0
        return function

    monkeypatch.setattr(runtime, "library", lambda: FakeLibrary())
    monkeypatch.setattr(runtime, "_applied_defines", None)
    modules = {
        "a": runtime.Module(("a",), {"HEAD_DIM": 64, "TILE": 32}),
        "b": runtime.Module(("b",), {"HEAD_DIM": 128, "TILE": 16}),
    }
    launches = {tag: runtime.Launch(runtime.Kernel(fake_kernel(tag), "gather_token", module), (1, 1, 1), (1, 1, 1),
                                    [None] * len(runtime.SIGNATURES["gather_token"]))
                for tag, module in modules.items()}

    def worker(tag):
        for _ in range(100):
            launches[tag](0)

    threads = [threading.Thread(target=worker, args=(tag,)) for tag in launches]
    for thread in threads:
        thread.start()
    for thread in threads:
        thread.join()
    assert len(seen) == 200
    for tag, values in seen:
        assert values == modules[tag].define_values, f"launch of module {tag} ran with {values}"
