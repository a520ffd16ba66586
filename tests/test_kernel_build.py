"""Build-level checks of hand-written kernels whose correctness depends on the register allocation.

attn_bwd_dkdv_v4 keeps its dK/dV accumulators in AGPRs through inline-asm MFMAs whose latency the
compiler does not see: if the allocator ever moves those accumulators (v_accvgpr_read / write /
mov) or spills anything to scratch, a moved value can be read before its MFMA has written it, and
dV / dK come out wrong.  This compiles attention_bwd.hip for gfx950 exactly as the Makefile does
(device code only, to assembly; no GPU needed) and checks the kernel's allocation.
"""
import os
import re
import subprocess

import pytest

from conftest import PKG

HIPCC = "/opt/rocm/bin/hipcc"
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form=1"]


def _kernel_sections(asm):
    """{mangled kernel name: its assembly text up to and including the register summary}."""
    out = {}
    for m in re.finditer(r"^(_Z\w*attn_bwd_dkdv_v4\w*):", asm, flags=re.M):
        name = m.group(1)
        end = asm.find("; ScratchSize:", m.end())
        stop = asm.find("\n", end)
        out[name] = asm[m.start():stop]
    return out


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not installed")
def test_dkdv_accumulators_never_move(tmp_path):
    makefile = open(os.path.join(PKG, "Makefile")).read()
    # the per-file flag this check compiles with is still the Makefile's
    assert re.search(r"build/attention_bwd\.o:\s*FLAGS\s*\+=\s*-mllvm -amdgpu-mfma-vgpr-form=1", makefile)
    out = tmp_path / "attention_bwd.s"
    src = os.path.join(PKG, "csrc", "attention_bwd.hip")
    r = subprocess.run([HIPCC, *FLAGS, "--cuda-device-only", "-S", "-o", str(out), src],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-2000:]
    sections = _kernel_sections(out.read_text())
    assert len(sections) == 2, sorted(sections)  # bf16 and fp16 instantiations
    for name, text in sections.items():
        moves = re.findall(r"^\s*v_accvgpr_(?:read|write|mov)", text, flags=re.M)
        assert not moves, f"{name}: {len(moves)} accumulator moves"
        scratch = int(re.search(r"; ScratchSize: (\d+)", text).group(1))
        assert scratch == 0, f"{name}: {scratch} bytes of scratch"

