"""The direct-to-LDS copies own M0.

attention_flash.hip, attention_decode.hip and gdn_chunked.hip issue their global -> LDS copies
(buffer_load_dwordx4 ... lds) from inline asm that sets M0 itself, and the
flash kernel walks M0 from one copy to the next across the instructions in
between.  That is only sound while nothing else in those kernels reads or
writes M0, which the compiler does not know.  This test compiles both sources
to gfx950 assembly with the library's flags (a CPU-only cross-compile) and
requires every M0 reference to be one of the copies' own forms.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "kraken-infer_amd", "csrc")
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", f"-I{os.path.join(ROOT, 'include')}", f"-I{CSRC}",
         "--cuda-device-only", "-S"]
EXTRA = {"attention_flash.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"], "attention_decode.hip": [],
         "gdn_chunked.hip": [], "kquant.hip": []}
# Instructions that read M0 without naming it.
IMPLICIT = re.compile(r"^(s_movrel|v_movrel|ds_append|ds_consume|ds_gws|s_sendmsg|v_interp|"
                      r"ds_param|lds_direct|s_ttracedata)")
ALLOWED = [
    re.compile(r"^s_mov_b32 m0, s\d+$"),
    re.compile(r"^s_add_u32 m0, m0, 0x[0-9a-f]+$"),
    re.compile(r"^s_add_u32 m0, m0, \d+$"),
    re.compile(r"^buffer_load_dwordx4 v\d+, s\[\d+:\d+\], 0 offen (nt )?lds$"),
]


# SCC readers, and the scalar ALU instructions that write SCC (a conservative
# superset: every SOP1/SOP2/SOPC opcode family that sets it).
SCC_USE = re.compile(r"^(s_cbranch_scc[01]|s_cselect_b(32|64)|s_addc_u32|s_subb_u32|"
                     r"s_cmov_b(32|64)|s_cmovk_i32)\b")
SCC_DEF = re.compile(r"^s_(add|sub|addc|subb|min|max|and|or|xor|andn[12]|orn[12]|nand|nor|xnor|"
                     r"lshl|lshr|ashr|bfe|bfm|not|cmp|bitcmp|abs|absdiff|lshl\d_add|bcnt|ff[01]|"
                     r"flbit|quadmask|wqm|[a-z0-9]+_saveexec)[a-z0-9_]*\b")


def instructions(path):
    for line in path.read_text().splitlines():
        text = line.split(";")[0].strip()
        if text and not text.startswith(".") and not text.endswith(":"):
            yield text


def compile_isa(tmp_path, source):
    out = tmp_path / "k.s"
    subprocess.run([HIPCC, *FLAGS, *EXTRA[source], os.path.join(CSRC, source), "-o", str(out)],
                   check=True, capture_output=True)
    return out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
@pytest.mark.parametrize("source", sorted(EXTRA))
def test_m0_write_never_directly_precedes_an_lds_dma_load(tmp_path, source):
    """An M0 write needs one wait state before an LDS-DMA load reads it: the
    copies put an s_nop or other work in between, which the compiled code keeps."""
    prev = ""
    for text in instructions(compile_isa(tmp_path, source)):
        if " lds" in text and text.startswith(("buffer_", "global_")):
            assert not re.match(r"^s_(mov|add)_[bu]32 m0\b", prev), f"{source}: {prev} ; {text}"
        prev = text


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
@pytest.mark.parametrize("source", sorted(EXTRA))
def test_no_scc_value_lives_across_the_m0_add(tmp_path, source):
    """The copy asm's s_add_u32 on M0 writes SCC (declared clobbered): no SCC
    reader may take its value from that add, i.e. the last SCC writer before
    every reader is some other instruction."""
    last_def = ""
    for text in instructions(compile_isa(tmp_path, source)):
        if SCC_USE.match(text):
            assert not re.match(r"^s_add_u32 m0, m0\b", last_def), f"{source}: {last_def} ; {text}"
        if SCC_DEF.match(text):
            last_def = text


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
@pytest.mark.parametrize("source", sorted(EXTRA))
def test_m0_has_no_other_user(tmp_path, source):
    out = compile_isa(tmp_path, source)
    users = 0
    for text in instructions(out):
        assert not IMPLICIT.match(text), f"{source}: implicit M0 user: {text}"
        if " lds" in text and text.startswith(("buffer_", "global_")):
            assert any(p.match(text) for p in ALLOWED), f"{source}: other LDS-DMA load: {text}"
        if not re.search(r"\bm0\b", text):
            continue
        users += 1
        assert any(p.match(text) for p in ALLOWED), f"{source}: unexpected M0 use: {text}"
    assert users > 0, f"{source}: no M0 writes found (the copies moved?)"
