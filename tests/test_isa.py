"""CPU: the built library's gfx950 code has no DPP read-after-write hazard.

gfx950 requires two wait states between a VALU instruction that writes a VGPR and a DPP instruction that reads it. The
compiler inserts them for the DPP it emits, but the IQ2_XXS block product issues v_dot4c_i32_i8 with a row_newbcast
DPP source from inline assembly (moe_device.h, dot4_bcast), which the compiler cannot see into. This test unbundles the
gfx950 code objects from libloki_moe.so, disassembles them with ROCm's llvm-objdump and checks every DPP instruction
against the instructions issued before it in straight-line code.
"""
import os
import re
import shutil
import struct
import subprocess
import tempfile

import pytest

import loki_amd

OBJDUMP = next((p for p in ("/opt/rocm/llvm/bin/llvm-objdump", shutil.which("llvm-objdump") or "") if p and os.path.exists(p)), None)
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def code_objects(path):
    """The gfx950 device images of every clang offload bundle in the shared library."""
    data = open(path, "rb").read()
    i = data.find(MAGIC)
    while i >= 0:
        n = struct.unpack_from("<Q", data, i + len(MAGIC))[0]
        p = i + len(MAGIC) + 8
        for _ in range(n):
            off, size, tl = struct.unpack_from("<QQQ", data, p)
            triple = data[p + 24:p + 24 + tl].decode()
            p += 24 + tl
            if "gfx950" in triple and size:
                yield data[i + off:i + off + size]
        i = data.find(MAGIC, i + 1)


def vregs(tok):
    m = re.match(r"v\[(\d+):(\d+)\]", tok)
    if m:
        return set(range(int(m.group(1)), int(m.group(2)) + 1))
    m = re.match(r"v(\d+)$", tok)
    return {int(m.group(1))} if m else set()


def dpp_hazards(lines):
    """(count of DPP instructions, list of hazards): a VALU write of a DPP instruction's source VGPR less than two
    wait states before it (s_nop N counts N + 1), scanning back through straight-line code only."""
    insts = []
    for l in lines:
        l = l.split("//")[0].strip()
        if not l or l.startswith(";"):
            continue
        insts.append(l)
    n, bad = 0, []
    for i, l in enumerate(insts):
        op = l.split()[0]
        if not op.endswith("_dpp") or l.endswith(":"):
            continue
        n += 1
        src = vregs(l.split(None, 1)[1].split(",")[1].strip().split()[0])
        ws, j = 0, i - 1
        while j >= 0 and ws < 2:
            p = insts[j]
            j -= 1
            if p.endswith(":") or p.startswith("s_branch") or p.startswith("s_cbranch") or p.startswith("s_setpc"):
                break
            t = p.split()
            if t[0] == "s_nop":
                ws += int(t[1], 0) + 1
                continue
            if t[0].startswith("v_") and len(t) > 1 and vregs(t[1].rstrip(",")) & src:
                bad.append("%s  ->  %s" % (p, l))
            ws += 1
    return n, bad


@pytest.mark.skipif(OBJDUMP is None, reason="llvm-objdump not found")
@pytest.mark.skipif(not os.path.exists(loki_amd.LIB_PATH), reason="libloki_moe.so not built")
def test_no_dpp_read_after_valu_write():
    total, bad, asm_dpp = 0, [], 0
    with tempfile.TemporaryDirectory() as d:
        for k, co in enumerate(code_objects(loki_amd.LIB_PATH)):
            f = os.path.join(d, "co%d.o" % k)
            open(f, "wb").write(co)
            out = subprocess.run([OBJDUMP, "-d", "--mcpu=gfx950", f], capture_output=True, text=True, check=True).stdout
            asm_dpp += out.count("v_dot4c_i32_i8_dpp")
            n, b = dpp_hazards(out.splitlines())
            total += n
            bad += b
    assert asm_dpp > 0, "the block product's v_dot4c_i32_i8_dpp not found in the library"
    assert total > asm_dpp
    assert not bad, "\n".join(bad[:20])


def test_checker_flags_a_planted_hazard():
    """The checker itself: a VALU write of the DPP source right before it is flagged; with s_nop 1 between, it is not."""
    planted = ["v_xad_u32 v18, v1, v2, v3", "v_dot4c_i32_i8_dpp v34, v18, v29 row_newbcast:0 row_mask:0xf bank_mask:0xf"]
    assert dpp_hazards(planted)[1]
    assert not dpp_hazards([planted[0], "s_nop 1", planted[1]])[1]
    assert not dpp_hazards(["v_xad_u32 v19, v1, v2, v3", planted[1]])[1]
    assert dpp_hazards(["v_mov_b32 v[18:19], 0", "s_nop 0", planted[1]])[1]
