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



BUNDLER = "/opt/rocm/llvm/bin/clang-offload-bundler"
OBJCOPY = "/opt/rocm/llvm/bin/llvm-objcopy"
READELF = "/opt/rocm/llvm/bin/llvm-readelf"


def _kernel_metadata(obj, tmp_path):
    """[(kernel name, {field: int})] from the gfx950 code object embedded in one built object file."""
    stem = os.path.basename(obj)[:-2]
    fat, co = tmp_path / f"{stem}.fatbin", tmp_path / f"{stem}.co"
    sections = subprocess.run([READELF, "-S", obj], check=True, capture_output=True, text=True, timeout=120).stdout
    if ".hip_fatbin" not in sections:  # host-only object (the C ABI glue)
        return []
    subprocess.run([OBJCOPY, f"--dump-section=.hip_fatbin={fat}", obj, str(tmp_path / f"{stem}.copy.o")],
                   check=True, capture_output=True, timeout=120)
    subprocess.run([BUNDLER, "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={fat}",
                    f"--output={co}", "--unbundle"], check=True, capture_output=True, timeout=120)
    notes = subprocess.run([READELF, "--notes", str(co)], check=True, capture_output=True, text=True,
                           timeout=120).stdout
    out = []
    for block in re.split(r"\n\s+- \.", notes)[1:]:
        name = re.search(r"\.name:\s+(\S+)", "." + block)
        if not name:
            continue
        fields = {k: int(v) for k, v in re.findall(r"\.(private_segment_fixed_size|vgpr_spill_count|"
                                                    r"sgpr_spill_count):\s+(\d+)", "." + block)}
        out.append((name.group(1), fields))
    return out


@pytest.mark.skipif(not all(os.path.exists(t) for t in (BUNDLER, OBJCOPY, READELF)), reason="ROCm LLVM tools missing")
def test_no_kernel_spills_to_scratch(tmp_path):
    """No kernel of the built library spills registers or uses scratch memory: a spill in a hot loop or
    epilogue is a silent slowdown (the CE-statistics epilogue once spilled 55 VGPRs).  Reads the kernel
    descriptors of the objects the Makefile built (skipped when nothing is built)."""
    build = os.path.join(PKG, "build")
    objs = sorted(os.path.join(build, f) for f in os.listdir(build)) if os.path.isdir(build) else []
    objs = [o for o in objs if o.endswith(".o")]
    if not objs:
        pytest.skip("library not built")
    kernels = 0
    for obj in objs:
        for name, f in _kernel_metadata(obj, tmp_path):
            kernels += 1
            assert f.get("vgpr_spill_count", 0) == 0 and f.get("sgpr_spill_count", 0) == 0, (obj, name, f)
            assert f.get("private_segment_fixed_size", 0) == 0, (obj, name, f)
    assert kernels > 50, kernels
