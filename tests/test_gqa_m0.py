"""Build check of the grouped-query K-logit kernel's inline DMA (CPU only).

k_logits_gqa.hip issues its global -> LDS DMA as inline assembly that sets
m0 (the LDS destination) itself: `s_mov_b32 m0, sN` then
`global_load_lds_dwordx4`.  The compiler treats m0 as reserved and does not
see the write, so the kernel is correct only while the compiled code keeps
nothing of its own in m0.  This test compiles the file to gfx950 assembly
with the library's flags and fails if any instruction other than those
pairs names m0, if any LDS DMA is not directly preceded by its own m0 write,
or if an instruction that reads m0 implicitly appears at all.
"""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "star-kv_amd", "csrc", "k_logits_gqa.hip")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# instructions that read m0 without naming it (LDS DMA, relative moves,
# interpolation, messages, GWS / append / ordered-count, add-tid LDS reads)
IMPLICIT_M0 = re.compile(r"^\s*(s_movrel|v_movrel|v_interp|s_sendmsg|ds_gws|ds_append|ds_consume|ds_ordered|"
                         r"ds_read_addtid|ds_write_addtid|buffer_load\S*.*\blds\b|global_load_lds|"
                         r"buffer_store_lds)")


def _asm(tmp_path):
    out = tmp_path / "k_logits_gqa.s"
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature",
                    "-Xclang", "-packed-fp32-ops", "--cuda-device-only", "-S", "-o", str(out), SRC],
                   check=True, capture_output=True)
    return out.read_text().splitlines()


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not installed")
def test_gqa_dma_is_the_only_m0_user(tmp_path):
    lines = [ln.split(";")[0].rstrip() for ln in _asm(tmp_path)]
    code = [ln for ln in lines if ln.strip() and not ln.strip().startswith(("#", ".", "//")) and
            not ln.strip().endswith(":")]
    pairs = 0
    for i, ln in enumerate(code):
        names_m0 = re.search(r"\bm0\b", ln) is not None
        if re.match(r"^\s*s_mov_b32\s+m0,\s+s\d+\s*$", ln):
            assert i + 1 < len(code) and re.match(r"^\s*global_load_lds_dwordx4\s", code[i + 1]), \
                f"m0 write not followed by the LDS DMA: {ln!r} / {code[i + 1] if i + 1 < len(code) else ''!r}"
            pairs += 1
            continue
        assert not names_m0, f"an instruction other than the DMA's own m0 write names m0: {ln!r}"
        if IMPLICIT_M0.match(ln):
            assert re.match(r"^\s*global_load_lds_dwordx4\s", ln) and i > 0 and \
                re.match(r"^\s*s_mov_b32\s+m0,", code[i - 1]), f"an m0 reader without its own m0 write: {ln!r}"
    assert pairs > 0, "no inline DMA found: the check no longer sees the kernel it guards"
