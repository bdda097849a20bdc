"""Build the HIP library (libivonar_ternary.so) for gfx950, in the source tree.

The HIP sources under ``csrc/`` are compiled to position-independent objects
with hipcc for gfx950 and linked with the system C++ linker against the HIP
runtime that PyTorch-ROCm ships (``torch/lib/libamdhip64.so``), so the
library and torch share one runtime: torch's streams and device pointers are
valid inside it and its launches can be recorded into torch's HIP graphs.

Flags: ``-ffp-contract=off`` (every fused multiply-add in the kernels is an
explicit ``fmaf``, which keeps the fp32 order reproducible on the CPU) and
``-Xclang -target-feature -Xclang -packed-fp32-ops`` (no packed fp32 VALU
instructions) and ``-mllvm -amdgpu-mfma-vgpr-form`` (MFMA results in ordinary
VGPRs: the kernels convert every int32 MFMA tile with VALU instructions, which
would otherwise first copy it out of the accumulation registers, and the
smaller register footprint keeps two waves per SIMD).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE.parent / "csrc"
INCLUDE = PACKAGE.parent.parent / "include"
LIBRARY = PACKAGE / "_lib" / "libivonar_ternary.so"
ARCH = "gfx950"
SOURCES = ("quantize.hip", "gemv.hip", "gemv_tokens.hip", "gemm.hip", "gemm_wide.hip", "gemm_skinny.hip", "embed.hip", "sample.hip", "stream_read.hip",
           "validate.hip", "capi.hip")
HIP_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fno-gpu-rdc",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
    "-Wall",
    "-Wno-unused-result",
)


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.is_file():
        return str(candidate)
    found = shutil.which("hipcc")
    if found is None:
        raise RuntimeError("hipcc was not found; the ternary library needs ROCm's hipcc to build")
    return found


def torch_hip_runtime() -> Path:
    """Directory and file of the HIP runtime that torch loads."""
    import torch

    lib = Path(torch.__file__).resolve().parent / "lib" / "libamdhip64.so"
    if not lib.is_file():
        raise RuntimeError(f"torch does not ship a HIP runtime at {lib}; a ROCm build of torch is required")
    return lib


def _compile(source: Path, output: Path, hipcc: str) -> None:
    command = [hipcc, *HIP_FLAGS, f"-I{INCLUDE}", "-c", str(source), "-o", str(output)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stdout}\n{result.stderr}")
    noise = [line for line in result.stderr.splitlines() if "packed-fp32-ops" not in line and line.strip()]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def check_waits(objects) -> None:
    """Refuse code whose hand-placed vmcnt waits leave a VGPR access ahead of its load (asmcheck), and
    kernels that spill registers to scratch."""
    from .asmcheck import check_object, kernels_with_scratch

    hazards = [hazard for obj in objects for hazard in check_object(Path(obj))]
    if hazards:
        listing = "\n".join(str(hazard) for hazard in hazards[:20])
        raise RuntimeError(f"{len(hazards)} VGPR accesses precede the wait for their load:\n{listing}")
    spills = [entry for obj in objects for entry in kernels_with_scratch(Path(obj))]
    if spills:
        listing = "\n".join(f"{name}: {size} bytes" for name, size in spills[:20])
        raise RuntimeError(f"{len(spills)} kernels spill registers to scratch:\n{listing}")


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    hipcc = _hipcc()
    runtime = torch_hip_runtime()
    out_dir = LIBRARY.parent
    obj_dir = PACKAGE.parent / "_build"
    out_dir.mkdir(parents=True, exist_ok=True)
    obj_dir.mkdir(parents=True, exist_ok=True)
    objects = [obj_dir / (Path(name).stem + ".o") for name in SOURCES]
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as pool:
        list(pool.map(lambda pair: _compile(CSRC / pair[0], pair[1], hipcc), zip(SOURCES, objects)))
    check_waits(objects)
    temporary = LIBRARY.with_suffix(f".so.tmp{os.getpid()}")
    link = [
        os.environ.get("CXX", "g++"),
        "-shared",
        "-o",
        str(temporary),
        *map(str, objects),
        str(runtime),
        f"-Wl,-rpath,{runtime.parent}",
        "-Wl,--no-undefined",
    ]
    result = subprocess.run(link, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking {LIBRARY.name} failed:\n{result.stdout}\n{result.stderr}")
    temporary.replace(LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
