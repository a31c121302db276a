"""Checks on the gfx950 machine code of the built library (CPU only).

The tile fetches issue global_load_lds_dwordx4 from inline asm that sets M0
itself (lrnnx_amd/csrc/tile_io.h).  That is only sound while the compiler
makes no other use of M0 in these kernels, so every M0 reference in the
disassembly must be one of the asm's own `s_mov_b32 m0, sN` writes directly
followed (after the s_nop) by the LDS DMA.  (The check that no kernel writes
through the scalar data cache lives in test_codeobj_smem.py.)
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "lrnnx_amd" / "liblrnnx_scan.so"
LLVM = Path("/opt/rocm/llvm/bin")
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tools():
    need = [LLVM / "llvm-objdump", LLVM / "clang-offload-bundler", LLVM / "llvm-objcopy"]
    return all(p.exists() for p in need)


_CACHE = {}


def disassemble(tmp):
    """Disassembly text of every gfx950 code object in the library (cached per process)."""
    if "text" in _CACHE:
        return _CACHE["text"]
    if not LIB.exists():
        pytest.skip("library not built")
    if not _tools():
        pytest.skip("ROCm llvm tools not found")
    fat = tmp / "fatbin"
    subprocess.run([str(LLVM / "llvm-objcopy"), "--dump-section", f".hip_fatbin={fat}", str(LIB), str(tmp / "x.so")],
                   check=True, capture_output=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundles in .hip_fatbin"
    texts = []
    for i, s in enumerate(starts):
        e = starts[i + 1] if i + 1 < len(starts) else len(data)
        bundle = tmp / f"b{i}.bin"
        bundle.write_bytes(data[s:e])
        obj = tmp / f"b{i}.co"
        r = subprocess.run([str(LLVM / "clang-offload-bundler"), "--type=o", "--unbundle",
                            "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={bundle}", f"--output={obj}"],
                           capture_output=True)
        if r.returncode != 0 or not obj.exists() or obj.stat().st_size == 0:
            continue
        d = subprocess.run([str(LLVM / "llvm-objdump"), "-d", "--mcpu=gfx950", str(obj)], capture_output=True,
                           text=True, check=True)
        texts.append(d.stdout)
    assert texts, "no gfx950 code objects found"
    _CACHE["text"] = "\n".join(texts)
    return _CACHE["text"]


@pytest.fixture(scope="module")
def disasm(tmp_path_factory):
    return disassemble(tmp_path_factory.mktemp("codeobj"))


def instructions(text):
    for line in text.splitlines():
        line = line.strip()
        if not line or line.endswith(">:") or line.startswith("Disassembly") or ":" in line.split(" ")[0]:
            continue
        yield line.split("//")[0].strip()


def test_m0_only_set_for_lds_dma(disasm):
    insts = [i for i in instructions(disasm) if i]
    n_dma = 0
    for k, ins in enumerate(insts):
        if not re.search(r"\bm0\b", ins):
            continue
        assert re.match(r"s_mov_b32 m0, s\d+$", ins), f"unexpected M0 use: {ins}"
        follow = [x for x in insts[k + 1:k + 3] if not x.startswith("s_nop")]
        assert follow and follow[0].startswith("global_load_lds_dwordx4"), f"M0 write not followed by LDS DMA: {ins}"
        n_dma += 1
    assert n_dma > 0
