"""Compile the gfx950 HIP library ``libfastmm_amd.so`` in-tree.

``python -m rdna3_fastmm._build`` (or ``__graft_entry__.build()``) regenerates
nothing: the per-scheme programs in ``csrc/generated`` are checked in and a
test keeps them equal to the generator's output. Every source is compiled
with ``-ffp-contract=off`` (the transforms must round exactly like the fp32
straight-line programs) and without packed-fp32 instructions.

The 16x16x32 leaf-GEMM kernels issue their MFMAs as inline asm, whose result
latency the compiler cannot see. The build therefore also emits the device
assembly of ``leaf_gemm.hip`` and refuses to produce the library if any
compiler-generated instruction touches an accumulator register written by an
asm MFMA before a fence (three ``s_nop 7``) has covered its latency. The
thin-row kernel issues its global loads as inline asm with hand-written
``s_waitcnt vmcnt`` waits; the same check refuses a build in which any
instruction reads or writes a load's destination registers while that load
can still be in flight.
"""

from __future__ import annotations

from concurrent.futures import ThreadPoolExecutor
import os
from pathlib import Path
import re
import shutil
import subprocess
import sys

PACKAGE_DIR = Path(__file__).resolve().parent
SOURCE_DIR = PACKAGE_DIR.parent / "csrc"
INCLUDE_DIR = PACKAGE_DIR.parent.parent / "include"
BUILD_DIR = PACKAGE_DIR.parent / "_build"
LIBRARY_NAME = "libfastmm_amd.so"
LIBRARY_PATH = PACKAGE_DIR / LIBRARY_NAME
TORCH_OPS_SOURCE = "torch_ops.cpp"
TORCH_OPS_PATH = PACKAGE_DIR / "libfastmm_torch.so"
ARCH = "gfx950"

SOURCES = ("abi_common.cpp", "transforms.hip", "leaf_gemm.hip")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{SOURCE_DIR}",
    f"-I{INCLUDE_DIR}",
]


def _hipcc() -> str:
    candidate = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(candidate).exists():
        raise RuntimeError("hipcc not found; the fastmm library needs ROCm to build")
    return candidate


def _compile(source: str) -> Path:
    target = BUILD_DIR / (Path(source).stem + ".o")
    language = ["-x", "hip"] if source.endswith(".cpp") else []
    command = [_hipcc(), *COMMON_FLAGS, *language, "-c", str(SOURCE_DIR / source), "-o", str(target)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"compiling {source} failed:\n{result.stderr}")
    return target


ASM_CHECKED_SOURCE = "leaf_gemm.hip"
ASM_CHECKED_KERNELS = re.compile(r"^(_ZN6fastmm6mfma16\S*):", re.MULTILINE)
_AGPR = re.compile(r"\ba(?:\[(\d+):(\d+)\]|(\d+)\b)")


def _agprs(operands: str) -> set[int]:
    registers: set[int] = set()
    for low, high, single in _AGPR.findall(operands):
        if single:
            registers.add(int(single))
        else:
            registers.update(range(int(low), int(high) + 1))
    return registers


WRITE_TO_MFMA_WAIT_STATES = 4


def fence_violations(assembly: str) -> list[str]:
    """Compiler instructions that race an asm MFMA over an accumulator register.

    Scans each ``fastmm::mfma16`` kernel in program order, in both directions:

    * an MFMA marks its destination AGPRs pending; three consecutive
      ``s_nop 7`` (the fence's 24 wait states) clear them; any other
      instruction naming a pending AGPR is a violation (it would read or
      overwrite a result still in flight);
    * a non-MFMA write of an AGPR (``v_accvgpr_write/mov``, or a load into
      one before its ``s_waitcnt``) must be at least
      ``WRITE_TO_MFMA_WAIT_STATES`` wait states old when an MFMA reads that
      register as its accumulator input.

    Branches are followed in layout order, which covers loop bodies, their
    exits and the straight-line tails the compiler emits.
    """
    violations: list[str] = []
    for match in ASM_CHECKED_KERNELS.finditer(assembly):
        name = match.group(1)
        body = assembly[match.end():]
        body = body[: body.find("s_endpgm")]
        pending: set[int] = set()
        written_at: dict[int, int] = {}  # AGPR -> wait-state clock of a VALU write
        loaded: set[int] = set()  # AGPRs with a load in flight
        clock = 0
        nops = 0
        for line in body.splitlines():
            text = line.split(";", 1)[0].strip()
            if not text or text.endswith(":") or text.startswith("."):
                continue
            opcode, _, operands = text.partition(" ")
            fields = [field.strip() for field in operands.split(",")]
            if opcode.startswith("v_mfma"):
                accumulator_in = _agprs(fields[3]) if len(fields) > 3 else set()
                recent = {r for r in accumulator_in if clock - written_at.get(r, -10**9) < WRITE_TO_MFMA_WAIT_STATES}
                if recent or accumulator_in & loaded:
                    violations.append(f"{name}: {text} (accumulator input written just before)")
                pending |= _agprs(fields[0])
                nops = 0
                clock += 1
                continue
            if opcode == "s_nop":
                count = int(operands.strip() or 0)
                clock += count + 1
                nops = nops + 1 if count == 7 else 0
                if nops >= 3:
                    pending.clear()
                continue
            nops = 0
            clock += 1
            if opcode == "s_waitcnt":
                loaded.clear()
                continue
            if pending & _agprs(operands):
                violations.append(f"{name}: {text}")
            destination = _agprs(fields[0]) if fields else set()
            if opcode.startswith("v_accvgpr_write") or opcode.startswith("v_accvgpr_mov"):
                for register in destination:
                    written_at[register] = clock
            elif "load" in opcode:
                loaded |= destination
    return violations


ASM_LOAD_CHECKED_KERNELS = re.compile(r"^(_ZN6fastmm4thin\S*):", re.MULTILINE)
_VGPR = re.compile(r"(?<![a-z_])v(?:\[(\d+):(\d+)\]|(\d+)\b)")
_VMCNT = re.compile(r"vmcnt\((\d+)\)")
_VMEM_PREFIXES = ("global_", "buffer_", "flat_", "scratch_")


def _vgprs(operands: str) -> set[int]:
    registers: set[int] = set()
    for low, high, single in _VGPR.findall(operands):
        if single:
            registers.add(int(single))
        else:
            registers.update(range(int(low), int(high) + 1))
    return registers


def in_flight_load_violations(assembly: str, kernels: re.Pattern = ASM_LOAD_CHECKED_KERNELS) -> list[str]:
    """Instructions that touch a vector load's destination while the load may be in flight.

    Vector memory operations complete in issue order as far as ``vmcnt`` is
    concerned, so each kernel is scanned in layout order with a queue of the
    VMEM operations issued so far (stores hold a place in it without
    registers); ``s_waitcnt vmcnt(n)`` retires all but the newest ``n``. Any
    other instruction naming a VGPR of a queued load is a violation: it would
    read the register before the data arrives or overwrite it before the load
    lands. A load whose destination or address overlaps a queued load's
    destination is one too.
    """
    violations: list[str] = []
    for match in kernels.finditer(assembly):
        name = match.group(1)
        body = assembly[match.end():]
        body = body[: body.find("s_endpgm")]
        queue: list[set[int]] = []
        for line in body.splitlines():
            text = line.split(";", 1)[0].strip()
            if not text or text.endswith(":") or text.startswith("."):
                continue
            opcode, _, operands = text.partition(" ")
            if opcode == "s_waitcnt":
                counted = _VMCNT.search(operands)
                if counted:
                    del queue[: max(0, len(queue) - int(counted.group(1)))]
                continue
            in_flight = set().union(*queue) if queue else set()
            if opcode.startswith(_VMEM_PREFIXES):
                fields = [field.strip() for field in operands.split(",")]
                is_load = "_load" in opcode
                touched = _vgprs(operands)
                if touched & in_flight:
                    violations.append(f"{name}: {text}")
                queue.append(_vgprs(fields[0]) if is_load and fields else set())
                continue
            if _vgprs(operands) & in_flight:
                violations.append(f"{name}: {text}")
    return violations


def _check_device_assembly() -> None:
    target = BUILD_DIR / (Path(ASM_CHECKED_SOURCE).stem + ".s")
    command = [_hipcc(), *COMMON_FLAGS, "--cuda-device-only", "-S", str(SOURCE_DIR / ASM_CHECKED_SOURCE), "-o", str(target)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"assembling {ASM_CHECKED_SOURCE} failed:\n{result.stderr}")
    assembly = target.read_text()
    if not ASM_CHECKED_KERNELS.search(assembly):
        raise RuntimeError(f"{ASM_CHECKED_SOURCE}: no mfma16 kernels found to check")
    violations = fence_violations(assembly)
    if violations:
        listing = "\n".join(violations[:20])
        raise RuntimeError(f"{ASM_CHECKED_SOURCE}: accumulator accessed inside MFMA latency:\n{listing}")
    if not ASM_LOAD_CHECKED_KERNELS.search(assembly):
        raise RuntimeError(f"{ASM_CHECKED_SOURCE}: no thin-row kernels found to check")
    violations = in_flight_load_violations(assembly)
    if violations:
        listing = "\n".join(violations[:20])
        raise RuntimeError(f"{ASM_CHECKED_SOURCE}: load destination accessed while in flight:\n{listing}")


def build_torch_operators(verbose: bool = False) -> Path:
    """Compile the PyTorch-ROCm operator library over libfastmm_amd.so (host code only).

    A plain ``g++`` build against the installed torch headers and libraries
    (torch's include paths, its C++ ABI setting, c10/c10_hip/torch_hip), linked
    to ``libfastmm_amd.so`` next to it through ``$ORIGIN``. Loaded with
    ``torch.ops.load_library``.
    """
    import torch
    from torch.utils.cpp_extension import include_paths, library_paths

    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
    compiler = shutil.which("g++") or shutil.which("c++")
    if compiler is None:
        raise RuntimeError("no host C++ compiler found for the torch operator library")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    temporary = TORCH_OPS_PATH.with_suffix(".so.tmp")
    command = [
        compiler, "-O2", "-std=c++17", "-shared", "-fPIC", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{path}" for path in include_paths()], f"-I{rocm / 'include'}", f"-I{INCLUDE_DIR}",
        str(SOURCE_DIR / TORCH_OPS_SOURCE),
        *[f"-L{path}" for path in library_paths()], f"-L{rocm / 'lib'}", f"-L{PACKAGE_DIR}",
        "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_hip", "-ltorch", "-lamdhip64", "-lfastmm_amd",
        "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{path}" for path in library_paths()], "-o", str(temporary),
    ]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"building {TORCH_OPS_PATH.name} failed:\n{result.stderr}")
    os.replace(temporary, TORCH_OPS_PATH)
    if verbose:
        print(f"built {TORCH_OPS_PATH}")
    return TORCH_OPS_PATH


def build_library(verbose: bool = False) -> Path:
    """Compile every source, check the leaf-GEMM assembly, link, then build the torch
    operator library on top; returns the path of libfastmm_amd.so."""
    BUILD_DIR.mkdir(exist_ok=True)
    workers = min(len(SOURCES) + 1, max(1, (os.cpu_count() or 2) // 2))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        checked = pool.submit(_check_device_assembly)
        objects = list(pool.map(_compile, SOURCES))
        checked.result()
    temporary = LIBRARY_PATH.with_suffix(".so.tmp")
    command = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(temporary)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"linking {LIBRARY_NAME} failed:\n{result.stderr}")
    os.replace(temporary, LIBRARY_PATH)
    if verbose:
        print(f"built {LIBRARY_PATH}")
    build_torch_operators(verbose)
    return LIBRARY_PATH


if __name__ == "__main__":
    build_library(verbose=True)
    sys.exit(0)
