"""Kernel FFI of the MI355X ternary library (mirrors the reference's kernels/runtime.py).

The reference compiles ``ternary.cu`` with NVRTC and launches kernels through
the CUDA driver with ctypes (``kernels/runtime.py:225-324``).  Here the
kernels are prebuilt HIP code for gfx950 in ``_lib/libivonar_ternary.so``,
whose C-ABI entry points carry the reference kernels' names and argument
orders with the stream first (``include/ivonar_ternary.h``).  The Python
surface keeps the reference's shape so callers need no change:

* ``compile_module(source, defines, device)`` -> ``Module`` (source is not
  compiled; the defines HEAD_DIM / TILE / MAX_CHUNKS are applied);
* ``Module.kernel(name)`` -> ``Kernel``;
* ``Launch(kernel, grid, block, args, shared=0)(stream)``: grid, block and
  shared memory are the caller's hints and the library computes its own;
* ``pointer`` / ``int32`` / ``float32`` build the ctypes arguments; they are
  read at call time, so in-place updates (the reference's prefetch slots,
  ``kernel_decoder.py:589-603``) are seen;
* every failure raises ``KernelError`` (``runtime.py:26-27``).

There is no CPU or second-backend fallback: without the built library or a
ROCm device, ``compile_module`` raises.
"""

from __future__ import annotations

import ctypes
import threading
from collections.abc import Iterable, Mapping
from ctypes import c_float, c_int, c_void_p
from pathlib import Path

import torch

LIBRARY = Path(__file__).resolve().parent / "_lib" / "libivonar_ternary.so"
ABI_VERSION = 1


class KernelError(RuntimeError):
    pass


_P, _I, _F = c_void_p, c_int, c_float
_GEMV = [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _F, _P, _I]
_QUANT = [_P, _P, _I, _F, _I, _P, _P, _P]
_QUANT_TILE = [_P, _I, _P, _I, _F, _I, _P, _P, _P]
_GEMM = [_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I]

#: Argument types (after the stream) of every launchable entry point.
SIGNATURES: dict[str, list] = {
    **{name: _GEMV for name in (
        "gemv_plain_store", "gemv_plain_residual", "gemv_norm_store", "gemv_norm_silu_pair", "gemv_attn_residual",
        "gemv_prequant_store", "gemv_plain_store_wide", "gemv_plain_residual_wide", "gemv_norm_store_wide",
        "gemv_norm_silu_pair_wide", "gemv_attn_residual_wide", "ivonar_gemv_plain_store_noalloc",
    )},
    "quantize_norm": _QUANT,
    "quantize_norm_wide": _QUANT,
    **{name: _QUANT_TILE for name in (
        "quantize_tile_plain", "quantize_tile_plain_wide", "quantize_tile_norm", "quantize_tile_norm_wide",
        "quantize_tile_attn", "quantize_tile_attn_wide",
    )},
    **{name: _GEMM for name in (
        "gemm_tile_store", "gemm_tile_residual", "gemm_tile_silu_pair", "gemm_tile_store_wide",
        "gemm_tile_residual_wide", "gemm_tile_silu_pair_wide",
    )},
    "embed_token": [_P, _P, _P, _P, _I, _I, _I],
    "embed_tile": [_P, _P, _P, _P, _I, _I, _I, _I],
    "gather_token": [_P, _P, _I, _P],
    "gemv_group_partials": [_P, _P, _P, _I, _I, _I, _I, _P],
    "ivonar_quantize_rows": [_I, _P, _I, _P, _I, _F, _I, _I, _P, _P, _P],
    "ivonar_argmax": [_P, _I, _P],
    "logit_bounds": [_P, _P, _P, _P, _P, _P, _I],
    "sample_token": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I],
    "ivonar_stream_read": [_P, ctypes.c_longlong, _P],
    "ivonar_validate_ternary": [_P, ctypes.c_longlong, _P, ctypes.c_longlong, _P],
}

_lock = threading.Lock()
_library: ctypes.CDLL | None = None
_initialised: set[int] = set()
_modules: dict[tuple, "Module"] = {}


def library() -> ctypes.CDLL:
    """Load the HIP library once (after torch, so it binds torch's HIP runtime)."""
    global _library
    with _lock:
        if _library is None:
            if not LIBRARY.is_file():
                raise KernelError(f"the ternary HIP library is not built ({LIBRARY}); run the package build first")
            try:
                lib = ctypes.CDLL(str(LIBRARY))
            except OSError as exc:
                raise KernelError(f"the ternary HIP library could not be loaded: {exc}") from exc
            lib.ivonar_abi_version.restype = c_int
            if lib.ivonar_abi_version() != ABI_VERSION:
                raise KernelError("the ternary HIP library has an unexpected ABI version")
            lib.ivonar_error_string.argtypes = [c_int]
            lib.ivonar_error_string.restype = ctypes.c_char_p
            lib.ivonar_init.argtypes = [c_int]
            lib.ivonar_init.restype = c_int
            lib.ivonar_define.argtypes = [ctypes.c_char_p, c_int]
            lib.ivonar_define.restype = c_int
            lib.ivonar_gemv_plan.argtypes = [c_int, c_int, ctypes.POINTER(c_int), ctypes.POINTER(c_int)]
            lib.ivonar_gemv_plan.restype = None
            lib.ivonar_gemm_plan.argtypes = [c_int, c_int, c_int]
            lib.ivonar_gemm_plan.restype = c_int
            lib.ivonar_stream_read_sink_words.argtypes = []
            lib.ivonar_stream_read_sink_words.restype = c_int
            lib.ivonar_token_finish_limit.argtypes = [c_int]
            lib.ivonar_token_finish_limit.restype = c_int
            for name, argtypes in SIGNATURES.items():
                function = getattr(lib, name)
                function.argtypes = [c_void_p, *argtypes]
                function.restype = c_int
            _library = lib
        return _library


def check(status: int, what: str = "HIP call") -> None:
    if status != 0:
        message = library().ivonar_error_string(int(status))
        raise KernelError(f"{what} failed with HIP error {status}: {message.decode() if message else 'unknown'}")


def gemv_plan(rows: int, n: int) -> tuple[int, int]:
    """(lanes per row, rows per lane) of the decode GEMV for a K = n row."""
    lanes, per_lane = c_int(), c_int()
    library().ivonar_gemv_plan(int(rows), int(n), ctypes.byref(lanes), ctypes.byref(per_lane))
    return int(lanes.value), int(per_lane.value)


def gemm_plan(m: int, rows: int, n: int) -> int:
    """K-splits of the token GEMM for m tokens (fixes its fp32 summation order)."""
    return int(library().ivonar_gemm_plan(int(m), int(rows), int(n)))


def initialise(device_index: int) -> None:
    """Allocate the library's per-device scratch (outside any graph capture)."""
    with _lock:
        if device_index in _initialised:
            return
    current = torch.cuda.current_device()
    if current != device_index:
        torch.cuda.set_device(device_index)
    try:
        check(library().ivonar_init(int(device_index)), "ivonar_init")
    finally:
        if current != device_index:
            torch.cuda.set_device(current)
    with _lock:
        _initialised.add(device_index)


class Kernel:
    __slots__ = ("function", "name", "module")

    def __init__(self, function, name: str, module: "Module | None" = None) -> None:
        self.function = function
        self.name = name
        self.module = module


class Launch:
    """One recorded call of an entry point; ``launch(stream)`` runs it on a HIP stream handle."""

    __slots__ = ("kernel", "grid", "block", "shared", "_args")

    def __init__(
        self,
        kernel: Kernel,
        grid: tuple[int, int, int],
        block: tuple[int, int, int],
        args: Iterable[object],
        shared: int = 0,
    ) -> None:
        self.kernel = kernel
        self.grid = tuple(int(value) for value in grid)
        self.block = tuple(int(value) for value in block)
        self.shared = int(shared)
        self._args = tuple(args)
        expected = len(SIGNATURES[kernel.name])
        if len(self._args) != expected:
            raise KernelError(f"{kernel.name} takes {expected} arguments, got {len(self._args)}")

    def __call__(self, stream: int) -> None:
        module = self.kernel.module
        # The define values live once per process in the library: making a
        # module's values current and launching its kernel happen under one
        # lock, so a launch of another module cannot switch them in between.
        with _launch_lock:
            if module is not None and _applied_defines is not module.define_values:
                module.apply_defines()
            status = self.kernel.function(c_void_p(stream), *self._args)
        if status != 0:
            check(status, self.kernel.name)


_DEFINES = ("HEAD_DIM", "TILE", "MAX_CHUNKS", "MAX_TOPK")
_LIBRARY_DEFAULTS = {"HEAD_DIM": 64, "TILE": 32, "MAX_CHUNKS": 70, "MAX_TOPK": 256}
# The define values the library currently holds (the tuple of the module that set them last).
_applied_defines: tuple | None = None
_launch_lock = threading.Lock()


class Module:
    """One configuration of the library: the reference's -D defines of ``compile_module``.

    The library keeps one set of define values per process; every launch of a
    module's kernel first makes that module's values current (a few host
    calls, only when another module's launch ran in between), so modules with
    different HEAD_DIM or TILE can be used side by side as in the reference,
    where each define set is its own compiled module (``runtime.py:301-324``).
    """

    def __init__(self, key: tuple, defines: Mapping[str, object]) -> None:
        self.key = key
        self.defines = dict(defines)
        values = dict(_LIBRARY_DEFAULTS)
        values.update({name: int(defines[name]) for name in _DEFINES if name in defines})
        self.define_values = tuple(sorted(values.items()))
        self._kernels: dict[str, Kernel] = {}

    def apply_defines(self) -> None:
        global _applied_defines
        lib = library()
        for name, value in self.define_values:
            check(lib.ivonar_define(name.encode(), int(value)), f"define {name}")
        _applied_defines = self.define_values

    def kernel(self, name: str) -> Kernel:
        kernel = self._kernels.get(name)
        if kernel is None:
            if name not in SIGNATURES:
                raise KernelError(f"the ternary library has no entry point {name!r}")
            kernel = Kernel(getattr(library(), name), name, self)
            self._kernels[name] = kernel
        return kernel


def compile_module(
    source: str | None, defines: Mapping[str, object], device: torch.device, name: str = "ivonar"
) -> Module:
    """Bind the prebuilt library for ``device`` and apply the reference's -D defines.

    ``source`` is accepted for signature compatibility and ignored.  The
    module's HEAD_DIM, TILE, MAX_CHUNKS and MAX_TOPK are made current before
    each of its launches.
    """
    del source, name
    device = torch.device(device)
    if device.type != "cuda":
        raise KernelError("ternary kernels need a ROCm device")
    if not torch.cuda.is_available():
        raise KernelError("no ROCm device is available for the ternary kernels")
    index = device.index if device.index is not None else torch.cuda.current_device()
    library()
    initialise(index)
    key = (index, tuple(sorted((k, int(v)) for k, v in defines.items() if k in _DEFINES)))
    with _lock:
        module = _modules.get(key)
        if module is None:
            module = Module(key, defines)
            _modules[key] = module
    with _launch_lock:
        module.apply_defines()  # rejects out-of-range values here, as NVRTC would at compile time
    return module


def pointer(tensor: torch.Tensor | None) -> c_void_p:
    return c_void_p(0 if tensor is None else tensor.data_ptr())


def int32(value: int) -> c_int:
    return c_int(int(value))


def float32(value: float) -> c_float:
    return c_float(float(value))


def current_stream(device: torch.device | None = None) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


class Driver:
    """The device-context half of the reference's driver object (``kernels/runtime.py:140-191``).

    The reference decoder calls four of its methods around its launches
    (``kernel_decoder.py:226,274,448,518,552,677,684``):

    * ``bind(device_index)`` makes the device current for the calling thread
      before a launch sequence (the reference retains the CUDA primary
      context and sets it current); here the HIP runtime's per-thread current
      device is set, once per thread and device;
    * ``persisting_capacity(device_index)`` is the persisting-L2 budget.  It
      is 0 here: MI355X has no access-policy window, and its 256 MB Infinity
      Cache keeps recently read weights without a hint, so the reference
      decoder builds no arena and never calls the next two;
    * ``reserve_persisting(device_index, nbytes)`` and
      ``persist_on_stream(stream, base, nbytes)`` check their arguments and
      set nothing.  A request above the capacity raises ``KernelError``, the
      error the reference's caller already handles by switching persistence
      off (``kernel_decoder.py:273-277``, ``:517-521``).
    """

    def __init__(self) -> None:
        self._bound: dict[int, int] = {}
        self._reserved: dict[int, int] = {}
        self._lock = threading.Lock()

    def check(self, status: int) -> None:
        check(status, "HIP call")

    def _device(self, device_index: int) -> int:
        index = int(device_index)
        if not torch.cuda.is_available():
            raise KernelError("no ROCm device is available for the ternary kernels")
        if index < 0 or index >= torch.cuda.device_count():
            raise KernelError(f"HIP device {index} does not exist")
        return index

    def bind(self, device_index: int) -> None:
        thread = threading.get_ident()
        index = int(device_index)
        if self._bound.get(thread) == index:
            return
        torch.cuda.set_device(self._device(index))
        with self._lock:
            self._bound[thread] = index

    def persisting_capacity(self, device_index: int) -> int:
        self._device(device_index)
        return 0

    def reserve_persisting(self, device_index: int, nbytes: int) -> None:
        index = self._device(device_index)
        if int(nbytes) < 0:
            raise KernelError("a persisting-L2 reservation cannot be negative")
        if int(nbytes) > self.persisting_capacity(index):
            raise KernelError(f"device {index} has no persisting-L2 window for {int(nbytes)} bytes")
        with self._lock:
            self._reserved[index] = max(self._reserved.get(index, 0), int(nbytes))

    def persist_on_stream(self, stream: int, base: int, nbytes: int) -> None:
        if int(nbytes) < 0 or int(base) < 0 or int(stream) < 0:
            raise KernelError("an access window needs a stream, a base address and a non-negative size")
        if int(nbytes) > 0:
            raise KernelError("this device has no access-policy window to persist weights in")


_driver: Driver | None = None


def driver() -> Driver:
    """The process's ``Driver`` (one per process, as the reference's ``runtime.driver()``)."""
    global _driver
    with _lock:
        if _driver is None:
            _driver = Driver()
        return _driver
