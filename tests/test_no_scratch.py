"""No kernel of the built library uses scratch memory (CPU).

A kernel whose registers do not fit spills VGPRs to per-lane scratch memory
(the private segment): every spill is a store and a later load through the
vector memory path, and the hot kernels here are sized so that they need none
(register budgets from ``__launch_bounds__`` and ``amdgpu_waves_per_eu``,
loops that are not unrolled where the unrolled form spilled).  SGPR spills are
not counted: they go to lanes of a VGPR, not to memory.

This test reads the code-object metadata (``llvm-readelf --notes``, the ROCm
install's own) of every gfx950 bundle in libmhc_hip.so and checks, for every
kernel, a zero private segment, no VGPR spills and no dynamic stack.  The
parser is checked first on planted metadata.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "mhc-mlx_amd" / "mhc_mlx_amd" / "libmhc_hip.so"
OBJDUMP = Path("/opt/rocm/llvm/bin/llvm-objdump")
READELF = Path("/opt/rocm/llvm/bin/llvm-readelf")

_KEY = re.compile(r"^    \.(\w+):\s+(\S+)")


def kernels(notes: str) -> list[dict[str, str]]:
    """One dict of top-level keys per kernel entry of amdhsa.kernels (entries start with '  - .')."""
    out: list[dict[str, str]] = []
    for line in notes.splitlines():
        if line.startswith("  - ."):
            out.append({})
            line = "    " + line[4:]
        if out:
            m = _KEY.match(line)
            if m:
                out[-1][m.group(1)] = m.group(2)
    return [k for k in out if "symbol" in k]


def offenders(ks: list[dict[str, str]]) -> list[tuple[str, str, str, str]]:
    """(kernel, private segment bytes, VGPR spills, dynamic stack) for every kernel that uses scratch."""
    return [(k.get("name", "?"), k.get("private_segment_fixed_size", "?"), k.get("vgpr_spill_count", "?"),
             k.get("uses_dynamic_stack", "?"))
            for k in ks
            if k.get("private_segment_fixed_size") != "0" or k.get("vgpr_spill_count") != "0"
            or k.get("uses_dynamic_stack", "false") != "false"]


_PLANT = """\
amdhsa.kernels:
  - .agpr_count:     0
    .args:
      - .name:           x
        .offset:         0
    .name:           good
    .private_segment_fixed_size: 0
    .sgpr_spill_count: 12
    .symbol:         good.kd
    .uses_dynamic_stack: false
    .vgpr_spill_count: 0
  - .agpr_count:     0
    .name:           bad
    .private_segment_fixed_size: 156
    .symbol:         bad.kd
    .uses_dynamic_stack: false
    .vgpr_spill_count: 37
amdhsa.target:   amdgcn-amd-amdhsa--gfx950
"""


def test_parser_finds_planted_spills():
    ks = kernels(_PLANT)
    assert [k["name"] for k in ks] == ["good", "bad"]  # an argument's .name is not the kernel's
    assert offenders(ks) == [("bad", "156", "37", "false")]
    assert offenders(kernels(_PLANT.replace("156", "0").replace("37", "0"))) == []
    stack = _PLANT.replace("good.kd\n    .uses_dynamic_stack: false", "good.kd\n    .uses_dynamic_stack: true")
    assert [o[0] for o in offenders(kernels(stack))] == ["good", "bad"]


@pytest.mark.skipif(not LIB.exists() or not OBJDUMP.exists() or not READELF.exists(),
                    reason="libmhc_hip.so not built or the ROCm llvm tools absent")
def test_no_kernel_uses_scratch(tmp_path):
    lib = tmp_path / LIB.name
    shutil.copyfile(LIB, lib)
    # --offloading writes each bundle's code object next to its input
    subprocess.run([str(OBJDUMP), "--offloading", lib.name], cwd=tmp_path, check=True, capture_output=True)
    objs = sorted(tmp_path.glob("*gfx950"))
    assert objs, "no gfx950 code object in the library"
    ks: list[dict[str, str]] = []
    for o in objs:
        ks += kernels(subprocess.run([str(READELF), "--notes", str(o)], check=True, capture_output=True,
                                     text=True).stdout)
    assert len(ks) > 500  # the metadata was read
    assert any("mf64_bwd_kernel" in k["name"] for k in ks)
    bad = offenders(ks)
    assert bad == [], f"{len(bad)} of {len(ks)} kernels use scratch, first: {bad[:3]}"
