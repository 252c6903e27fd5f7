"""Every HIP kernel of the library keeps its state in registers: no kernel
uses scratch (private) memory, which on these kernels would mean register
spills to memory inside streaming or MFMA loops.

The check reads the kernel metadata of the gfx950 code objects built in
gemma3.c_amd/_build (the objects libg3attn.so is linked from): the device
bundle of each object's .hip_fatbin section, then its AMDGPU metadata note
(.private_segment_fixed_size per kernel).  CPU only; skipped when the objects
or the ROCm LLVM tools are absent.
"""
import glob
import os
import re
import subprocess

import pytest

from helpers import REPO

BUILD = os.path.join(REPO, "gemma3.c_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
TOOLS = [os.path.join(LLVM, t) for t in ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf")]
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"

OBJS = sorted(p for p in glob.glob(os.path.join(BUILD, "*.o"))
              if os.path.basename(p)[:-2] in {os.path.basename(h)[:-4] for h in
                                              glob.glob(os.path.join(REPO, "gemma3.c_amd", "csrc", "*.hip"))})

pytestmark = pytest.mark.skipif(not OBJS or not all(os.path.exists(t) for t in TOOLS),
                                reason="built HIP objects or ROCm LLVM tools absent")


def kernel_metadata(obj, tmp_path):
    """[(kernel name, {field: int})] from the object's gfx950 code object."""
    fat = tmp_path / (os.path.basename(obj) + ".fatbin")
    co = tmp_path / (os.path.basename(obj) + ".co")
    subprocess.run([TOOLS[0], f"--dump-section=.hip_fatbin={fat}", obj], check=True, capture_output=True)
    subprocess.run([TOOLS[1], "--unbundle", "--type=o", f"--targets={TARGET}", f"--input={fat}",
                    f"--output={co}"], check=True, capture_output=True)
    notes = subprocess.run([TOOLS[2], "--notes", str(co)], check=True, capture_output=True, text=True).stdout
    # amdhsa.kernels is a list of maps, one per kernel: each starts at a
    # two-space "- " item; its keys sit at four spaces (the argument maps
    # nested in .args sit deeper)
    kernels, cur = [], None
    for line in notes.splitlines():
        m = re.match(r"(  - |    )\.([a-z_]+):\s+(\S+)$", line)
        if not m:
            continue
        lead, key, val = m.groups()
        if lead == "  - ":
            cur = {}
            kernels.append(cur)
        if cur is not None:
            cur[key] = val
    return [(k["name"], {f: int(v) for f, v in k.items()
                         if f in ("private_segment_fixed_size", "vgpr_count", "agpr_count", "group_segment_fixed_size")})
            for k in kernels if "name" in k]


@pytest.mark.parametrize("obj", OBJS, ids=[os.path.basename(o) for o in OBJS])
def test_no_kernel_uses_scratch(obj, tmp_path):
    kernels = kernel_metadata(obj, tmp_path)
    assert kernels, obj
    spilled = [(n, f["private_segment_fixed_size"]) for n, f in kernels if f.get("private_segment_fixed_size", 0)]
    assert not spilled, spilled


def test_prefill_kernels_fit_two_waves_per_simd(tmp_path):
    """The 16-queries-per-wave prefill kernels run two waves per SIMD: at most
    256 VGPRs and no AGPRs, and their LDS (the K / V rings, plus the key-scale
    ring of the fp8 cross policy) fits one workgroup per CU's 160 KiB."""
    obj = os.path.join(BUILD, "prefill.o")
    if obj not in OBJS:
        pytest.skip("prefill.o not built")
    found = 0
    for name, f in kernel_metadata(obj, tmp_path):
        if re.search(r"prefill_kernelILi\dELi1ELb", name):
            found += 1
            assert f["vgpr_count"] <= 256 and f.get("agpr_count", 0) == 0, (name, f)
            assert f["group_segment_fixed_size"] <= 160 * 1024, (name, f)
    assert found == 6, found
