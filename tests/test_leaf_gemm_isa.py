"""Static checks of the 16x16x32 leaf-GEMM kernels' gfx950 assembly (CPU only).

The kernels issue their MFMAs as inline asm, so the compiler cannot see the
MFMA result latency; correctness then rests on no compiler-generated
instruction touching an accumulator inside that latency. These tests compile
``leaf_gemm.hip`` to device assembly with the library's own flags and check
that invariant (and that the checker catches a planted violation), plus the
shape of the main loop that the kernel's throughput depends on.
"""

from __future__ import annotations

import re
import subprocess

import pytest

from rdna3_fastmm import _build


@pytest.fixture(scope="module")
def assembly(tmp_path_factory) -> str:
    target = tmp_path_factory.mktemp("isa") / "leaf_gemm.s"
    command = [
        _build._hipcc(), *_build.COMMON_FLAGS, "--cuda-device-only", "-S",
        str(_build.SOURCE_DIR / "leaf_gemm.hip"), "-o", str(target),
    ]
    result = subprocess.run(command, capture_output=True, text=True)
    assert result.returncode == 0, result.stderr
    return target.read_text()


def _kernels(assembly: str) -> dict[str, str]:
    bodies = {}
    for match in _build.ASM_CHECKED_KERNELS.finditer(assembly):
        body = assembly[match.end():]
        bodies[match.group(1)] = body[: body.find("s_endpgm")]
    return bodies


def test_every_operand_and_product_variant_is_checked(assembly) -> None:
    # template arguments <operand, products>: (fp16, fp16), (fp16, fp32), (bf16, bf16), (bf16, fp32)
    names = set(_kernels(assembly))
    for variant in ("ILi1ELi1E", "ILi1ELi2E", "ILi0ELi0E", "ILi0ELi2E"):
        assert any(variant in n for n in names), (variant, names)
    # the persistent kernel's <stream products, strip> forms, for both 16-bit types
    for operand in ("ILi1ELi1E", "ILi0ELi0E"):
        for flags in ("Lb0ELb0E", "Lb1ELb0E", "Lb0ELb1E", "Lb1ELb1E"):
            assert any(f"persistent_kernel{operand}{flags}" in n for n in names), (operand, flags)


def test_no_accumulator_access_inside_mfma_latency(assembly) -> None:
    assert _build.fence_violations(assembly) == []


def test_checker_reports_a_missing_fence(assembly) -> None:
    # with the fences' nops shortened every epilogue read becomes a violation
    planted = assembly.replace("s_nop 7", "s_nop 6")
    assert len(_build.fence_violations(planted)) > 100


def test_checker_on_synthetic_listing() -> None:
    body = (
        "_ZN6fastmm6mfma16kE:\n"
        "\tv_mfma_f32_16x16x32_f16 a[0:3], v[0:3], v[4:7], a[0:3]\n"
        "\tv_accvgpr_read_b32 v9, a4\n"  # other register: fine
        "\tv_accvgpr_read_b32 v8, a2\n"  # inside the latency: violation
        "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n"
        "\tv_accvgpr_read_b32 v8, a2\n"  # after a fence: fine
        "\ts_endpgm\n"
    )
    assert _build.fence_violations(body) == ["_ZN6fastmm6mfma16kE: v_accvgpr_read_b32 v8, a2"]


def test_checker_on_accumulator_input_written_just_before() -> None:
    mfma = "\tv_mfma_f32_16x16x32_f16 a[4:7], v[0:3], v[4:7], a[0:3]\n"
    tail = "\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_endpgm\n"
    written = "_ZN6fastmm6mfma16kE:\n\tv_accvgpr_write_b32 a1, 0\n"
    assert len(_build.fence_violations(written + mfma + tail)) == 1
    # four wait states after the write: fine
    assert _build.fence_violations(written + "\ts_nop 3\n" + mfma + tail) == []
    # an AGPR load still in flight, then after its wait
    loaded = "_ZN6fastmm6mfma16kE:\n\tscratch_load_dwordx4 a[0:3], off, off\n"
    assert len(_build.fence_violations(loaded + "\ts_nop 7\n" + mfma + tail)) == 1
    assert _build.fence_violations(loaded + "\ts_waitcnt vmcnt(0)\n\ts_nop 3\n" + mfma + tail) == []


def _innermost_loops(body: str) -> list[list[str]]:
    """Opcodes of each innermost loop: a label and the last branch back to it,
    with no other such loop strictly inside."""
    lines = body.splitlines()
    labels = {}
    for i, line in enumerate(lines):
        if match := re.match(r"^(\.LBB\w+):", line):
            labels[match.group(1)] = i
    loops = {}
    for j, line in enumerate(lines):
        match = re.search(r"\bs_c?branch\w*\s+(\.LBB\w+)", line)
        if match and match.group(1) in labels and labels[match.group(1)] < j:
            loops[labels[match.group(1)]] = j  # the last branch back closes the loop
    spans = sorted(loops.items())
    inner = [(a, b) for a, b in spans if not any(a < a2 and b2 <= b for a2, b2 in spans if (a2, b2) != (a, b))]
    return [
        [line.split(";", 1)[0].split()[0] for line in lines[a + 1 : b + 1]
         if line.split(";", 1)[0].strip() and not line.strip().startswith(";") and not line.strip().endswith(":")]
        for a, b in inner
    ]


def test_main_loop_shape(assembly) -> None:
    for name, body in _kernels(assembly).items():
        # the K loop: four slices per iteration, each 64 MFMAs, 16 fragment reads
        # and 8 refills; the persistent kernel's strip form adds one MFMA, one
        # fragment read and one load per slice
        operand = re.search(r"kernelILi(\d)E", name).group(1)  # first template argument
        strip = re.search(r"persistent_kernelILi\dELi\dELb[01]ELb([01])E", name)
        extra = 4 if strip and strip.group(1) == "1" else 0
        mfma = "v_mfma_f32_16x16x32_bf16" if operand == "0" else "v_mfma_f32_16x16x32_f16"
        shapes = set()
        for opcodes in _innermost_loops(body):
            count = lambda prefix: sum(op.startswith(prefix) for op in opcodes)  # noqa: E731
            if count("v_mfma") == 0:
                continue
            shape = (count(mfma), count("ds_read_b128"), count("buffer_load_dwordx4"), count("s_barrier"))
            assert shape == (256 + extra, 64 + extra, 32 + extra, 4), (name, shape)
            for forbidden in ("v_accvgpr", "scratch_", "v_mov", "global_load", "flat_", "v_readlane", "v_writelane"):
                assert count(forbidden) == 0, (name, forbidden)
            shapes.add(shape[0] - extra)
        assert shapes == {256}, (name, shapes)


def _asm_vmcnt_waits(body: str) -> list[int]:
    """The vmcnt bounds of the kernel's own waits: those written as inline asm
    (between the ;;#ASMSTART / ;;#ASMEND markers), not the compiler's."""
    return [int(n) for block in re.findall(r";;#ASMSTART(.*?);;#ASMEND", body, re.S)
            for n in re.findall(r"s_waitcnt[^\n]*vmcnt\((\d+)\)", block)]


def _persistent_wait_violations(assembly: str) -> list[str]:
    """The persistent kernel's waits may leave only loads in flight: vmcnt also
    counts stores, and a store can complete before older loads, so a bound that
    allowed stores would not prove the awaited loads had landed. The kernel's own
    waits (the prologue's and every step's) are two steps of loads (16; 18 with
    the strip), the last one vmcnt(0), and no store precedes the first wait."""
    found = []
    for name, body in _kernels(assembly).items():
        flags = re.search(r"persistent_kernelILi\dELi\dELb[01]ELb([01])E", name)
        if not flags:
            continue
        loads = 18 if flags.group(1) == "1" else 16
        waits = _asm_vmcnt_waits(body)
        found += [f"{name}: vmcnt({n})" for n in waits[:-1] if n != loads]
        if waits[-1:] != [0]:
            found.append(f"{name}: the last wait is not vmcnt(0)")
        if "buffer_store" in body[: body.index("vmcnt(")]:
            found.append(f"{name}: a store before the first wait")
    return found


def test_persistent_waits_leave_only_loads_in_flight(assembly) -> None:
    assert _persistent_wait_violations(assembly) == []
    # a tile-start wait that lets the previous tile's stores stay in flight is caught
    at = assembly.index("s_waitcnt vmcnt(16)", re.search(r"_ZN6fastmm6mfma1617persistent_kernel\w*:", assembly).end())
    planted = assembly[:at] + "s_waitcnt vmcnt(48)" + assembly[at + len("s_waitcnt vmcnt(16)"):]
    assert len(_persistent_wait_violations(planted)) == 1


def test_thin_row_kernels_touch_no_load_in_flight(assembly) -> None:
    names = [m.group(1) for m in _build.ASM_LOAD_CHECKED_KERNELS.finditer(assembly)]
    for variant in ("ILi1ELi1E", "ILi1ELi2E", "ILi0ELi0E", "ILi0ELi2E"):
        assert any(variant in n for n in names), (variant, names)
    assert _build.in_flight_load_violations(assembly) == []


def test_load_checker_catches_a_planted_read(assembly) -> None:
    # copy a register of the first asm load's destination right after the load
    match = re.search(r"(\tglobal_load_dwordx4 v\[(\d+):\d+\], v\[\d+:\d+\], off\n)",
                      assembly[_build.ASM_LOAD_CHECKED_KERNELS.search(assembly).end():])
    assert match
    planted = assembly.replace(match.group(1), match.group(1) + f"\tv_mov_b32_e32 v250, v{match.group(2)}\n", 1)
    found = _build.in_flight_load_violations(planted)
    assert len(found) == 1 and f"v_mov_b32_e32 v250, v{match.group(2)}" in found[0]


def test_load_checker_on_synthetic_listing() -> None:
    head = "_ZN6fastmm4thinkE:\n"
    loads = "\tglobal_load_dwordx4 v[4:7], v[0:1], off\n\tglobal_load_dwordx4 v[8:11], v[2:3], off\n"
    use = "\tv_add_u32_e32 v20, v5, v9\n"
    end = "\ts_endpgm\n"
    assert len(_build.in_flight_load_violations(head + loads + use + end)) == 1
    # vmcnt(1) retires the older load only: v5 is ready, v9 is not
    assert len(_build.in_flight_load_violations(head + loads + "\ts_waitcnt vmcnt(1)\n" + use + end)) == 1
    assert _build.in_flight_load_violations(head + loads + "\ts_waitcnt vmcnt(1)\n\tv_mov_b32_e32 v20, v5\n" + end) == []
    assert _build.in_flight_load_violations(head + loads + "\ts_waitcnt vmcnt(0)\n" + use + end) == []
    # overwriting an address after issue is fine; overwriting a pending destination is not
    assert _build.in_flight_load_violations(head + loads + "\tv_mov_b32_e32 v0, 0\n" + end) == []
    assert len(_build.in_flight_load_violations(head + loads + "\tv_mov_b32_e32 v7, 0\n" + end)) == 1
    # a store holds a place in the count: after a load and a store, vmcnt(1) retires the load, vmcnt(2) does not
    store = "\tglobal_store_dwordx4 v[0:1], v[12:15], off\n"
    one = "\tglobal_load_dwordx4 v[4:7], v[0:1], off\n"
    assert _build.in_flight_load_violations(head + one + store + "\ts_waitcnt vmcnt(1)\n\tv_mov_b32_e32 v20, v5\n" + end) == []
    assert len(_build.in_flight_load_violations(head + one + store + "\ts_waitcnt vmcnt(2)\n\tv_mov_b32_e32 v20, v5\n" + end)) == 1
