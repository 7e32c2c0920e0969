"""Build check: the decode hot path's kernels keep every value in registers (CPU only).

A VGPR spill inside a K-step or tile loop is a scratch round trip, and the
reload's memory wait also waits for the loop's own stores and loads: one
spilled 64-bit address in the int8 warp-specialised K-logit kernel cost 11 %
of its time at B16 S32768.  This test compiles the hot-path sources to
gfx950 assembly with the library's flags and fails if any of their kernels
that the decode path runs on aligned inputs reports a VGPR spill:
* every instantiation of the warp-specialised and grouped-query K-logit
  kernels, the raw-nibble P.V kernel and the split-S reduction / up-projection;
* the fused, aligned-row column-block P.V kernel for dense and group-64 V.
(The unaligned-row and per-token block-format P.V variants are not covered.)
"""
import concurrent.futures
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "star-kv_amd", "csrc")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "--cuda-device-only", "-S"]

# (source, mangled-name pattern every matching kernel of which must not spill)
CHECKS = [
    ("k_logits_ws.hip", r"k_logits_ws_kernel"),
    ("k_logits_gqa.hip", r"k_logits_gqa_kernel"),
    ("pv_latent.hip", r"pv_nib_kernel"),
    # pv_kernel<VT, NTW, FUSED = true, FAST = true, VQ = dense (0) or group-64 (2)>
    ("pv_latent.hip", r"pv_kernelI(DF16_|DF16b)Li\d+ELb1ELb1ELi[02]E"),
    ("up_proj.hip", r"up_proj_kernel|up_finish_kernel"),
]


def _spills(asm_text):
    """{kernel name: VGPR spill count} from the code object's metadata."""
    out, name = {}, None
    for ln in asm_text.splitlines():
        s = ln.strip()
        if s.startswith(".name:"):
            name = s.split()[1]
        elif s.startswith(".vgpr_spill_count:") and name is not None:
            out[name] = int(s.split()[1])
            name = None
    return out


def _compile(src, tmp_path):
    out = tmp_path / (src + ".s")
    subprocess.run([HIPCC, *FLAGS, "-o", str(out), os.path.join(CSRC, src)], check=True, capture_output=True)
    return src, out.read_text()


@pytest.mark.skipif(not shutil.which(HIPCC) and not os.path.exists(HIPCC), reason="hipcc not installed")
def test_hot_path_kernels_do_not_spill(tmp_path):
    srcs = sorted({s for s, _ in CHECKS})
    with concurrent.futures.ThreadPoolExecutor(len(srcs)) as ex:
        asm = dict(ex.map(lambda s: _compile(s, tmp_path), srcs))
    bad = []
    for src, pat in CHECKS:
        found = {k: v for k, v in _spills(asm[src]).items() if re.search(pat, k)}
        assert found, f"no kernel of {src} matches {pat}"
        bad += [(k, v) for k, v in found.items() if v]
    assert not bad, f"VGPR spills in hot-path kernels: {bad}"
