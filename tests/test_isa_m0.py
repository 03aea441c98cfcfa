"""The direct-to-LDS copy helpers (dma16 / dma16s / dma4 in
autoresearch_amd/csrc/ar_common.hpp) set m0 from inline asm and list it as
clobbered; clang ignores clobbers of reserved registers, so they are correct
only while no compiler-generated instruction in the same kernels uses m0.
This test compiles the two sources that use them to gfx950 assembly, with the
library's own flags, and checks that invariant: every m0 reference sits in
one of those asm blocks (s_mov_b32 m0 -> s_nop 0 -> global_load_lds_*), and
no instruction outside them reads or writes m0 explicitly or implicitly
(relative moves, messages, GWS / ordered / lane-id LDS forms, interpolation,
buffer-to-LDS loads, GPR index mode).  CPU only: hipcc cross-compiles."""
import concurrent.futures
import os
import re
import shutil
import subprocess
import tempfile

import pytest

from autoresearch_amd import build as B

SOURCES = ["ar_gemm.hip", "ar_flash.hip"]
# instructions that use m0 without naming it
IMPLICIT_M0 = re.compile(r"^(s_movrel|v_movrel|s_sendmsg|ds_gws|ds_ordered_count|ds_\w*_addtid|v_interp|"
                         r"buffer_load\w*\s.*\blds\b|s_set_gpr_idx)")

pytestmark = pytest.mark.skipif(not os.path.exists(B.HIPCC), reason="hipcc not available")


def _asm(src: str, out_dir: str) -> str:
    out = os.path.join(out_dir, os.path.basename(src) + ".s")
    cmd = [B.HIPCC, *B.CFLAGS, "--cuda-device-only", "-S", "-o", out, os.path.join(B.CSRC, src)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-4000:]
    with open(out) as f:
        return f.read()


def _check(text: str, name: str):
    in_asm = False
    block = []
    blocks = 0
    for raw in text.splitlines():
        line = raw.strip()
        if line == ";;#ASMSTART":
            in_asm, block = True, []
            continue
        if line == ";;#ASMEND":
            in_asm = False
            if any("m0" in x for x in block):
                # the only asm that touches m0: set it, one wait state, the copy
                assert len(block) == 3, (name, block)
                assert re.fullmatch(r"s_mov_b32 m0, s\d+", block[0]), (name, block)
                assert block[1] == "s_nop 0", (name, block)
                assert block[2].startswith("global_load_lds_dword"), (name, block)
                blocks += 1
            continue
        if not line or line.startswith(";") or line.startswith("."):
            continue
        if in_asm:
            block.append(line)
            continue
        if line.endswith(":"):
            continue
        assert not re.search(r"\bm0\b", line), f"{name}: compiler-generated m0 use: {line}"
        assert not IMPLICIT_M0.match(line), f"{name}: instruction with an implicit m0 operand: {line}"
    assert not in_asm, name
    return blocks


@pytest.fixture(scope="module")
def assembly():
    d = tempfile.mkdtemp(prefix="ar_isa_")
    try:
        with concurrent.futures.ThreadPoolExecutor(len(SOURCES)) as ex:
            texts = dict(zip(SOURCES, ex.map(lambda s: _asm(s, d), SOURCES)))
    finally:
        shutil.rmtree(d, ignore_errors=True)
    return texts


@pytest.mark.parametrize("src", SOURCES)
def test_m0_only_in_dma_helpers(assembly, src):
    n = _check(assembly[src], src)
    assert n > 0, f"{src}: no direct-to-LDS copies found (the check would be vacuous)"


def test_check_rejects_other_m0_uses():
    ok = "\t;;#ASMSTART\n\ts_mov_b32 m0, s4\n\ts_nop 0\n\tglobal_load_lds_dwordx4 v1, s[2:3]\n\t;;#ASMEND\n"
    assert _check(ok, "ok") == 1
    for bad in ["\ts_mov_b32 m0, -1\n",                    # a compiler-generated m0 write
                "\tv_movrels_b32_e32 v0, v1\n",            # implicit m0 (relative move)
                "\ts_sendmsg sendmsg(MSG_DEALLOC_VGPRS)\n",  # implicit m0 (message)
                ok.replace("s_nop 0", "s_nop 1\n\ts_mov_b32 s5, m0")]:  # a different asm block on m0
        with pytest.raises(AssertionError):
            _check(bad, "bad")
