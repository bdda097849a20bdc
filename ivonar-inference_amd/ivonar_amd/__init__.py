"""MI355X-native ternary linear layer (drop-in for Ivonar's ternary kernel path).

Hand-written HIP kernels for gfx950 behind a C ABI (``include/ivonar_ternary.h``)
with the reference kernels' entry-point names; this package is the Python
host side that mirrors the reference's kernel FFI (``runtime``), its packed
format and ``TernaryLinear`` (``quantization``), its fused kernel operands
(``matrix``) and a decode/prefill driver for stacks of ternary linear layers
(``decoder``).
"""

from .runtime import KernelError, Launch, Module, compile_module, float32, int32, pointer

__all__ = ["KernelError", "Launch", "Module", "compile_module", "float32", "int32", "pointer"]
