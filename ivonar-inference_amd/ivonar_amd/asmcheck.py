"""Post-build check of hand-placed memory waits in this library's own gfx950 code objects.

Several kernels issue their global loads as inline assembly and place the
``s_waitcnt vmcnt(N)`` that covers each load by hand, so the compiler does not
know which registers are still being filled.  It may therefore copy, read or
reuse such a register before the wait: the read sees the register's old
contents and the result is wrong only when the load is slow.  This module
finds such accesses in the compiled code.

Model (the gfx9 vector-memory counter): every vector memory instruction
(load, store, atomic; global, buffer, flat, scratch) increments ``vmcnt``;
loads return their data in issue order; ``s_waitcnt vmcnt(N)`` stalls until
at most N of them are outstanding, so every load with N or more younger
vector memory instructions behind it has landed.  For each load that writes
VGPRs the analysis keeps its position counted from the youngest (0 = just
issued).  A wait ``vmcnt(N)`` retires the loads at positions >= N.  Any other
instruction that names a VGPR of a pending load (as a source or a
destination) is reported.  Branches are followed as a control-flow graph and
the states of merging paths are joined by keeping, per register, its
youngest possible position, so a register counts as pending if it is pending
on any path (a loop is iterated to a fixed point).

The code object is taken from the build's object files
(``.hip_fatbin`` section, gfx950 entry) and disassembled with ROCm's LLVM
tools; only code compiled from this repository is read.  The same code
objects' metadata also names any kernel that asks for private (scratch)
memory, i.e. spills registers (``kernels_with_scratch``).
"""

from __future__ import annotations

import os
import re
import subprocess
import tempfile
from dataclasses import dataclass, field
from pathlib import Path

TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
_POSITION_CAP = 64  # vmcnt holds at most 63: a load this old is retired by any wait

_VMEM_PREFIXES = ("global_", "buffer_", "flat_", "scratch_")
_LINE = re.compile(r"^\s+([a-z_0-9]+)(?:\s+(.*?))?\s*//\s*([0-9A-Fa-f]+):(.*)$")
_LABEL = re.compile(r"^([0-9a-f]+) <(.+)>:$")
_VREG = re.compile(r"(?<![a-z_0-9])v(?:\[(\d+):(\d+)\]|(\d+)(?![0-9]))")
_TARGET_ADDR = re.compile(r"<(.+)\+0x([0-9a-f]+)>")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")


@dataclass
class Instruction:
    address: int
    mnemonic: str
    operands: str
    comment: str = ""

    def vgprs(self) -> list[int]:
        regs: list[int] = []
        for low, high, single in _VREG.findall(self.operands):
            if single:
                regs.append(int(single))
            else:
                regs.extend(range(int(low), int(high) + 1))
        return regs


@dataclass
class Hazard:
    function: str
    address: int
    text: str
    registers: list[int]

    def __str__(self) -> str:
        return f"{self.function} +0x{self.address:x}: {self.text} touches v{self.registers} before its load landed"


@dataclass
class Function:
    name: str
    start: int
    body: list[Instruction] = field(default_factory=list)


def _is_vmem(mnemonic: str) -> bool:
    return mnemonic.startswith(_VMEM_PREFIXES)


def _load_destination(ins: Instruction) -> list[int]:
    """VGPRs a vector memory instruction writes when its data returns (empty for stores and LDS DMA)."""
    m = ins.mnemonic
    if "_lds" in m or re.search(r"\blds\b", ins.operands):
        return []
    returns = "_load" in m or ("_atomic" in m and re.search(r"\b(glc|sc0)\b", ins.operands) is not None)
    if not returns:
        return []
    first = ins.operands.split(",")[0].strip()
    match = _VREG.fullmatch(first)
    if match is None:
        return []
    low, high, single = match.groups()
    return [int(single)] if single else list(range(int(low), int(high) + 1))


def parse_disassembly(text: str) -> list[Function]:
    functions: list[Function] = []
    current: Function | None = None
    for line in text.splitlines():
        label = _LABEL.match(line)
        if label:
            current = Function(label.group(2), int(label.group(1), 16))
            functions.append(current)
            continue
        if current is None:
            continue
        ins = _LINE.match(line)
        if ins:
            current.body.append(Instruction(int(ins.group(3), 16), ins.group(1), ins.group(2) or "", ins.group(4)))
    return functions


def _successors(fn: Function, index: int, by_address: dict[int, int]) -> list[int]:
    ins = fn.body[index]
    m = ins.mnemonic
    following = [index + 1] if index + 1 < len(fn.body) else []
    if m in ("s_endpgm", "s_setpc_b64"):
        return []
    if m.startswith("s_cbranch") or m == "s_branch":
        target = _TARGET_ADDR.search(ins.comment)
        jump: list[int] = []
        if target is not None:
            address = fn.start + int(target.group(2), 16)
            if address in by_address:
                jump = [by_address[address]]
        return jump if m == "s_branch" else jump + following
    return following


def _join(a: dict[int, int], b: dict[int, int]) -> dict[int, int]:
    out = dict(a)
    for reg, pos in b.items():
        out[reg] = min(out.get(reg, pos), pos)
    return out


def check_function(fn: Function) -> list[Hazard]:
    """Every access to a VGPR whose vector memory load may not have landed."""
    if not fn.body:
        return []
    by_address = {ins.address: i for i, ins in enumerate(fn.body)}
    # Join points: the entry, every branch target and every instruction after a branch.
    leaders = {0}
    for i in range(len(fn.body)):
        succ = _successors(fn, i, by_address)
        if succ != [i + 1]:
            leaders.update(succ)
    state_in: dict[int, dict[int, int]] = {0: {}}
    work = [0]
    hazards: dict[int, Hazard] = {}
    while work:
        index = work.pop()
        pending = dict(state_in[index])
        # Run the straight-line stretch from `index` to the next branch or join point.
        while True:
            ins = fn.body[index]
            m = ins.mnemonic
            if m == "s_waitcnt":
                count = _VMCNT.search(ins.operands)
                if count is not None:
                    limit = int(count.group(1))
                    pending = {r: p for r, p in pending.items() if p < limit}
            elif _is_vmem(m):
                dest = _load_destination(ins)
                dest_set = set(dest)
                touched = [r for r in ins.vgprs() if r in pending and r not in dest_set]
                # An address or data register still being filled by an older load.
                if touched:
                    hazards.setdefault(ins.address, Hazard(fn.name, ins.address - fn.start,
                                                           f"{m} {ins.operands}", sorted(set(touched))))
                # A load over a pending load's registers is safe: loads land in issue order.
                pending = {r: min(p + 1, _POSITION_CAP) for r, p in pending.items()}
                for r in dest:
                    pending[r] = 0
            else:
                touched = [r for r in ins.vgprs() if r in pending]
                if touched:
                    hazards.setdefault(ins.address, Hazard(fn.name, ins.address - fn.start,
                                                           f"{m} {ins.operands}", sorted(set(touched))))
            successors = _successors(fn, index, by_address)
            if successors == [index + 1] and index + 1 not in leaders:
                index += 1
                continue
            for nxt in successors:
                merged = _join(state_in[nxt], pending) if nxt in state_in else pending
                if nxt not in state_in or merged != state_in[nxt]:
                    state_in[nxt] = merged
                    work.append(nxt)
            break
    return sorted(hazards.values(), key=lambda h: h.address)


def _llvm_tool(name: str) -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "llvm" / "bin" / name
    if not path.is_file():
        raise RuntimeError(f"{path} not found; the wait check needs ROCm's LLVM tools")
    return str(path)


def _device_code(obj: Path, tmp: str) -> Path | None:
    """The gfx950 code object embedded in one of this build's object files (None: host-only object)."""
    fatbin = Path(tmp) / "fatbin"
    code = Path(tmp) / "code.o"
    dumped = subprocess.run([_llvm_tool("llvm-objcopy"), f"--dump-section=.hip_fatbin={fatbin}", str(obj)],
                            capture_output=True, text=True)
    if dumped.returncode != 0:
        if "not found" in dumped.stderr:
            return None
        raise RuntimeError(f"llvm-objcopy failed on {obj}: {dumped.stderr}")
    subprocess.run([_llvm_tool("clang-offload-bundler"), "--unbundle", "--type=o", f"--input={fatbin}",
                    f"--targets={TARGET}", f"--output={code}"], check=True, capture_output=True)
    return code


def disassemble_object(obj: Path) -> str:
    """gfx950 disassembly of the device code embedded in one of this build's object files."""
    with tempfile.TemporaryDirectory() as tmp:
        code = _device_code(obj, tmp)
        if code is None:
            return ""
        result = subprocess.run([_llvm_tool("llvm-objdump"), "-d", "--mcpu=gfx950", str(code)], check=True,
                                capture_output=True, text=True)
        return result.stdout


def kernels_with_scratch(obj: Path) -> list[tuple[str, int]]:
    """Kernels of the object whose code object metadata asks for private (scratch) memory per lane:
    register spills, which also make every dispatch set up scratch.  (name, bytes) pairs."""
    with tempfile.TemporaryDirectory() as tmp:
        code = _device_code(obj, tmp)
        if code is None:
            return []
        notes = subprocess.run([_llvm_tool("llvm-readelf"), "--notes", str(code)], check=True,
                               capture_output=True, text=True).stdout
    found = []
    for entry in notes.split(".name:")[1:]:
        size = re.search(r"\.private_segment_fixed_size:\s+(\d+)", entry)
        if size is not None and int(size.group(1)) > 0:
            found.append((entry.split("\n", 1)[0].strip(), int(size.group(1))))
    return found


def check_object(obj: Path, name_filter: str | None = None) -> list[Hazard]:
    hazards: list[Hazard] = []
    for fn in parse_disassembly(disassemble_object(obj)):
        if name_filter is not None and name_filter not in fn.name:
            continue
        hazards.extend(check_function(fn))
    return hazards
