"""The built library's gfx950 kernels use no scratch memory and spill no
vector registers.

A kernel that keeps values in scratch waits on every load with
`s_waitcnt vmcnt(0) lgkmcnt(0)`; hipcc produces one silently, for instance
when a select between two captured references of a lambda becomes a select
between two addresses in its closure (the staged prefill kernels once held
440 bytes of scratch that way and ran 2.6x slower).  This test reads the
code objects' metadata notes with ROCm's own tools (no GPU needed) and fails
on any kernel with a private segment or a VGPR spill."""
import os
import re
import subprocess

import pytest

import bmo_jetson_amd as bmo

LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tool(name):
    path = os.path.join(LLVM, name)
    if not os.path.exists(path):
        pytest.skip(f"{path} not present")
    return path


def _kernel_notes(tmp_path):
    """(name, private_segment_fixed_size, vgpr_spill_count, sgpr_spill_count)
    of every kernel in the library's gfx950 code objects."""
    objcopy, bundler, readelf = (_tool(n) for n in
                                 ("llvm-objcopy", "clang-offload-bundler", "llvm-readelf"))
    fat = tmp_path / "fat.bin"
    subprocess.run([objcopy, "-O", "binary", "--only-section=.hip_fatbin", bmo.LIB_PATH, str(fat)],
                   check=True)
    data = fat.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in .hip_fatbin"
    kernels = []
    for i, s in enumerate(starts):
        part = tmp_path / f"bundle{i}.bin"
        part.write_bytes(data[s:starts[i + 1] if i + 1 < len(starts) else len(data)])
        co = tmp_path / f"co{i}.o"
        listed = subprocess.run([bundler, "--type=o", f"--input={part}", "--list"],
                                capture_output=True, text=True, check=True).stdout.split()
        if TARGET not in listed:
            continue
        subprocess.run([bundler, "--type=o", f"--input={part}", f"--targets={TARGET}",
                        f"--output={co}", "--unbundle"], check=True)
        if co.stat().st_size == 0:
            continue
        notes = subprocess.run([readelf, "--notes", str(co)], capture_output=True, text=True,
                               check=True).stdout
        # metadata entries of one kernel sit between its "- .args:" list
        # item and the next; collect the keys of interest in order
        cur = {}
        for line in notes.splitlines():
            m = re.match(r"\s*-?\s*\.(name|private_segment_fixed_size|vgpr_spill_count|"
                         r"sgpr_spill_count):\s+(\S+)", line)
            if not m:
                continue
            key, val = m.group(1), m.group(2)
            if key == "name" and "name" in cur:
                kernels.append(cur)
                cur = {}
            cur[key] = val
        if "name" in cur:
            kernels.append(cur)
    return kernels


def test_no_kernel_uses_scratch_or_spills(tmp_path):
    kernels = _kernel_notes(tmp_path)
    names = [k["name"] for k in kernels]
    for family in ("append_kernel", "decode_kernel", "prefill_kernel", "gemv_kernel",
                   "stage_kernel", "commit_kernel"):
        assert any(family in n for n in names), f"{family} missing from the code objects"
    # (SGPR spills go to VGPR lanes, not memory, and are allowed)
    bad = [k for k in kernels
           if int(k.get("private_segment_fixed_size", "0")) != 0
           or int(k.get("vgpr_spill_count", "0")) != 0]
    assert not bad, f"kernels with scratch or VGPR spills: {bad}"
