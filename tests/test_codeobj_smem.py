"""No kernel of the library writes through the scalar data cache (CPU only;
disassembly of the built code objects, see test_codeobj.py)."""

import re

import pytest

from test_codeobj import disassemble, instructions


@pytest.fixture(scope="module")
def disasm(tmp_path_factory):
    return disassemble(tmp_path_factory.mktemp("codeobj_smem"))


def test_no_scalar_cache_writes(disasm):
    bad = re.compile(r"^(s_store_|s_buffer_store|s_atomic_|s_buffer_atomic|s_dcache_wb|s_dcache_discard|s_scratch_store)")
    hits = [i for i in instructions(disasm) if bad.match(i)]
    assert not hits, hits[:5]
