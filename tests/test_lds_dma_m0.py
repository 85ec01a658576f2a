"""Build-time guard for the LDS-DMA inline assembly (CPU only).

thot_amd/csrc/lds_dma.hpp issues global_load_lds_dword[x4] from inline
assembly that sets M0 itself ("s_mov_b32 m0, sN" and the load in one
statement).  The compiler reserves M0 and does not track that write, so the
helpers are only safe while no code the compiler generates around them uses
M0.  This test compiles every source that includes the helpers to gfx950
device assembly with the library's own flags and checks that:
  * every write of M0 is one of ours (an s_mov_b32 m0 directly followed by a
    global_load_lds instruction), so the compiler never keeps a value of its
    own in M0 that an inline statement could overwrite;
  * no instruction that reads M0 implicitly (message, GWS, append/consume,
    relative moves, interpolation, addtid, trace data) appears at all.
"""
import os
import re
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(REPO, "thot_amd", "csrc")
HIPCC = "/opt/rocm/bin/hipcc"

IMPLICIT_M0 = re.compile(r"^\s*(s_sendmsg|s_ttracedata|ds_gws_|ds_append|ds_consume|v_movrel|s_movrel|v_interp|"
                         r"ds_read_addtid|ds_write_addtid|lds_param_load|lds_direct_load)")


def _users():
    out = []
    for f in sorted(os.listdir(CSRC)):
        if f.endswith(".hip"):
            text = open(os.path.join(CSRC, f)).read()
            if "lds_dma.hpp" in text or "gemm_dma.hpp" in text:
                out.append(f)
    return out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not available")
@pytest.mark.parametrize("src", _users())
def test_m0_is_only_set_for_lds_dma(src, tmp_path):
    from thot_amd.build import HIP_FLAGS
    flags = [f for f in HIP_FLAGS if f not in ("-fPIC",)]
    asm = tmp_path / (src + ".s")
    r = subprocess.run([HIPCC, *flags, "--cuda-device-only", "-S", os.path.join(CSRC, src), "-o", str(asm)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    lines = [l.split(";")[0].rstrip() for l in asm.read_text().splitlines()]
    insts = [l for l in lines if l.strip() and not l.lstrip().startswith((".", "//")) and not l.rstrip().endswith(":")]
    writes = 0
    for i, l in enumerate(insts):
        assert not IMPLICIT_M0.match(l), f"{src}: implicit M0 reader: {l.strip()}"
        if re.search(r"\bm0\b", l) is None:
            continue
        if l.lstrip().startswith("s_mov_b32 m0,"):
            writes += 1
            assert i + 1 < len(insts) and insts[i + 1].lstrip().startswith("global_load_lds"), \
                f"{src}: M0 write not followed by an LDS DMA: {l.strip()} / {insts[i + 1].strip()}"
        else:
            assert l.lstrip().startswith("global_load_lds"), f"{src}: other M0 use: {l.strip()}"
    assert writes > 0, f"{src}: expected the LDS-DMA helpers in the assembly"
