"""Register budget of the shipped gfx950 kernels (no GPU needed).

Reads the AMDHSA kernel descriptors of the code object inside railgun_amd/librailgun_hip.so
(the .hip_fatbin section, unbundled for gfx950) and checks that no kernel uses scratch
memory: a spill of a decode or prefill kernel to scratch puts a per-lane memory round trip
into its inner loop, and an instantiation that starts spilling (a new GQA ratio, a deeper
prefetch ring) must fail here before it is measured.  Register-to-register moves between
the architectural VGPRs and the accumulation VGPRs are not spills and are allowed.
"""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest
import yaml

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "railgun_amd", "librailgun_hip.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def _tool(name: str) -> str:
    path = os.path.join(LLVM, name)
    if os.path.exists(path):
        return path
    found = shutil.which(name)
    if not found:
        pytest.skip(f"{name} not available")
    return found


def kernel_descriptors(tmp_path) -> dict[str, dict[str, int]]:
    """kernel symbol -> {field: value} from the gfx950 code object's metadata notes."""
    assert os.path.exists(LIB), f"{LIB} missing: run __graft_entry__.build()"
    fatbin = tmp_path / "fatbin.bin"
    subprocess.run([_tool("llvm-objcopy"), "-O", "binary", "--only-section=.hip_fatbin", LIB, str(fatbin)], check=True)
    # One offload bundle per source file with kernels, concatenated in the section.
    data = fatbin.read_bytes()
    starts = [m.start() for m in re.finditer(re.escape(MAGIC), data)]
    assert starts, "no offload bundle in .hip_fatbin"
    kernels: dict[str, dict[str, int]] = {}
    for i, a in enumerate(starts):
        bundle, code = tmp_path / f"bundle{i}.bin", tmp_path / f"gfx950_{i}.co"
        bundle.write_bytes(data[a:starts[i + 1] if i + 1 < len(starts) else len(data)])
        subprocess.run([_tool("clang-offload-bundler"), "--unbundle", "--type=o", f"--input={bundle}",
                        "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={code}"], check=True)
        notes = subprocess.run([_tool("llvm-readelf"), "--notes", str(code)], check=True, capture_output=True,
                               text=True).stdout
        # The metadata note is a YAML document ("---" ... "..."): amdhsa.kernels lists the kernels.
        doc = notes[notes.index("---"):]
        doc = doc[:doc.index("\n...") + 4] if "\n..." in doc else doc
        for k in yaml.safe_load(doc)["amdhsa.kernels"]:
            kernels[k[".name"]] = {key.lstrip("."): val for key, val in k.items() if isinstance(val, int)}
    return kernels


# Scalar registers a kernel may park in VGPR lanes (v_writelane / v_readlane, no memory): the
# 16-bit prefill kernels at head_dim 256, which sit at the 106-SGPR limit and keep about ten
# set-up values there, stored at the unit set-up and none reloaded inside the tile loop; and the
# stream-K decode with the fused RoPE + cache pass (template flag ROPE, "Lb1E" in the name), which
# keeps the pointers used only at segment boundaries there (partials, segment descriptors, the
# cos / sin table), stored at the start and read back at a segment's start or end, not per unit
# (8-12; 13-14 in the G 3 and 5 forms at head_dim 128).  Every other kernel keeps its scalars in
# SGPRs; a count above these means a change pushed live scalars towards the inner loops, and it
# fails here.
MAX_SGPR_LANE_SPILLS = 12
MAX_SGPR_LANE_SPILLS_FUSED_DECODE = 14


def _lane_spill_limit(name: str) -> int:
    if "prefill_mfma_kernel" in name and "Li256E" in name:
        return MAX_SGPR_LANE_SPILLS
    if "decode_stream_kernel" in name and "Lb1EE" in name:
        return MAX_SGPR_LANE_SPILLS_FUSED_DECODE
    return 0


def test_no_kernel_uses_scratch(tmp_path):
    kernels = kernel_descriptors(tmp_path)
    hot = [k for k in kernels if "decode_stream_kernel" in k or "prefill_mfma_kernel" in k]
    assert len(hot) >= 20, sorted(kernels)
    bad = {k: (v["private_segment_fixed_size"], v.get("vgpr_spill_count", 0), v.get("sgpr_spill_count", 0))
           for k, v in kernels.items()
           if v["private_segment_fixed_size"] or v.get("vgpr_spill_count", 0)
           or v.get("sgpr_spill_count", 0) > _lane_spill_limit(k)}
    assert not bad, f"kernels with scratch or spills (bytes/lane, vgpr spills, sgpr spills): {bad}"
