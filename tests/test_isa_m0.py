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
         "gdn_chunked.hip": []}
# Instructions that read M0 without naming it.
IMPLICIT = re.compile(r"^(s_movrel|v_movrel|ds_append|ds_consume|ds_gws|s_sendmsg|v_interp|"
                      r"ds_param|lds_direct|s_ttracedata)")
ALLOWED = [
    re.compile(r"^s_mov_b32 m0, s\d+$"),
    re.compile(r"^s_add_u32 m0, m0, 0x[0-9a-f]+$"),
    re.compile(r"^s_add_u32 m0, m0, \d+$"),
    re.compile(r"^buffer_load_dwordx4 v\d+, s\[\d+:\d+\], 0 offen (nt )?lds$"),
]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc is not installed")
@pytest.mark.parametrize("source", sorted(EXTRA))
def test_m0_has_no_other_user(tmp_path, source):
    out = tmp_path / "k.s"
    subprocess.run([HIPCC, *FLAGS, *EXTRA[source], os.path.join(CSRC, source), "-o", str(out)],
                   check=True, capture_output=True)
    users = 0
    for line in out.read_text().splitlines():
        text = line.split(";")[0].strip()
        if not text or text.startswith("."):
            continue
        assert not IMPLICIT.match(text), f"{source}: implicit M0 user: {text}"
        if " lds" in text and text.startswith(("buffer_", "global_")):
            assert any(p.match(text) for p in ALLOWED), f"{source}: other LDS-DMA load: {text}"
        if not re.search(r"\bm0\b", text):
            continue
        users += 1
        assert any(p.match(text) for p in ALLOWED), f"{source}: unexpected M0 use: {text}"
    assert users > 0, f"{source}: no M0 writes found (the copies moved?)"
