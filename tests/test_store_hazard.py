"""The built library's stores of more than 8 bytes against the store-data hazard (CPU).

A VMEM store of 12 or 16 bytes reads its data registers after it issues; an
instruction that writes one of those registers too soon changes what is
stored.  The compiler pads such a write after a FLAT store (one wait state) and
after a buffer store whose soffset is not an SGPR, but takes a buffer store
with an SGPR soffset as exempt.  On gfx950 it is not: the 32 < n <= 64 layer
backward, with a VALU write of a dx store's first data register in the next
instruction, stored that instruction's value in lanes 12..15 of 16-lane rows
when a second wave shared the SIMD (a run-to-run difference in dx).  Every
16-byte buffer store is now followed by an s_nop that reads its data
registers (``buf_store_b128``).

This test disassembles the gfx950 code objects of the built libmhc_hip.so
(llvm-objdump, the ROCm install's own) and checks every such store in every
kernel: no instruction writes a data register of a buffer store within two
wait states, or of a FLAT store within one.  The scanner is checked first on
planted sequences.
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

_STORE = re.compile(r"(buffer|global)_store_dwordx([34])\s+([^,\s]+),\s*([^,\s]+)")
_FUNC = re.compile(r"^[0-9a-f]+ <(\S+)>:")


def _regs(tok: str) -> set[int]:
    m = re.fullmatch(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.fullmatch(r"v(\d+)", tok)
    return {int(m.group(1))} if m else set()


def scan(text: str) -> list[tuple[str, str, str, int]]:
    """(kernel, store, writer, wait states between) for every store whose data registers an instruction
    writes too soon: within 2 wait states of a buffer store, within 1 of a FLAT store."""
    ins: list[tuple[str, str]] = []
    func = ""
    for raw in text.splitlines():
        m = _FUNC.match(raw)
        if m:
            func = m.group(1)
            continue
        t = raw.split("//")[0].strip()
        if t and not t.endswith(":"):
            ins.append((func, t))
    bad = []
    for i, (func, t) in enumerate(ins):
        m = _STORE.match(t)
        if not m:
            continue
        data = _regs(m.group(3) if m.group(1) == "buffer" else m.group(4))
        need = 2 if m.group(1) == "buffer" else 1
        ws = 0
        for f2, u in ins[i + 1:i + 8]:
            if f2 != func or ws >= need:
                break
            if u.startswith("s_nop"):
                ws += int(u.split()[1], 0) + 1 if len(u.split()) > 1 else 1
                continue
            if u.startswith("v_"):
                parts = u.split()
                if len(parts) > 1 and _regs(parts[1].rstrip(",")) & data:
                    bad.append((func, t, u, ws))
                    break
            ws += 1
    return bad


def test_scanner_finds_planted_writes():
    head = "0000000000001000 <k>:\n"
    hit = head + "\tbuffer_store_dwordx4 v[142:145], v146, s[8:11], s3 offen nt // 00\n\tv_add_u32_e32 v142, s62, v146 // 08\n"
    assert len(scan(hit)) == 1
    one = head + "\tbuffer_store_dwordx4 v[4:7], v1, s[8:11], s3 offen\n\tv_mov_b32_e32 v9, 0\n\tv_mul_f32_e32 v7, v2, v3\n"
    assert len(scan(one)) == 1  # one wait state is not enough after a buffer store
    mfma = head + "\tbuffer_store_dwordx4 v[56:59], v94, s[68:71], s2 offen nt\n\tv_mfma_f32_16x16x32_bf16 v[56:59], v[8:11], v[48:51], 0\n"
    assert len(scan(mfma)) == 1
    flat = head + "\tglobal_store_dwordx4 v[0:1], v[16:19], off nt\n\tv_cvt_f16_f32_e32 v16, v21\n"
    assert len(scan(flat)) == 1
    assert scan(flat.replace("\tv_cvt", "\ts_nop 0\n\tv_cvt")) == []  # the compiler's one wait state after FLAT
    assert scan(hit.replace("\tv_add", "\ts_nop 1\n\tv_add")) == []  # buf_store_b128's guard
    assert scan(head + "\tbuffer_store_dwordx4 v[4:7], v1, s[8:11], s3 offen\n\tv_add_u32_e32 v8, v1, v2\n") == []
    assert scan(head + "\tbuffer_store_dwordx2 v[4:5], v1, s[8:11], s3 offen\n\tv_mov_b32_e32 v4, 0\n") == []  # 8 bytes
    # the address of a FLAT store is its first operand, the data its second
    assert scan(head + "\tglobal_store_dwordx4 v[0:1], v[16:19], off\n\tv_lshl_add_u64 v[0:1], v[0:1], 0, s[2:3]\n") == []


@pytest.mark.skipif(not LIB.exists() or not OBJDUMP.exists(), reason="libmhc_hip.so not built or llvm-objdump absent")
def test_no_store_data_register_is_written_too_soon(tmp_path):
    lib = tmp_path / LIB.name
    shutil.copyfile(LIB, lib)
    # --offloading writes each bundle's code object next to its input
    subprocess.run([str(OBJDUMP), "--offloading", lib.name], cwd=tmp_path, check=True, capture_output=True)
    objs = sorted(tmp_path.glob("*gfx950"))
    assert objs, "no gfx950 code object in the library"
    bad, stores = [], 0
    for o in objs:
        text = subprocess.run([str(OBJDUMP), "-d", str(o)], check=True, capture_output=True, text=True).stdout
        stores += len(_STORE.findall(text))
        bad += scan(text)
    assert stores > 1000  # the disassembly was read
    assert bad == [], f"{len(bad)} stores, first: {bad[:3]}"
