"""In-tree build of the gfx950 library, the CPU oracle and the C++ host tests.

* ``railgun_amd/librailgun_hip.so`` — every ``railgun_amd/csrc/*.hip`` compiled with hipcc
  for gfx950 (objects under ``_build/``), linked as one shared library;
* ``oracle/liboracle.so`` — the C restatement, via ``make -C oracle`` (test infrastructure);
* ``tests/cpp/*`` binaries — C++ tests of the host-side mirror, linked against the library.

Every call compiles from scratch (no up-to-date checks), so a successful build() means the
current sources build.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "railgun_amd")
CSRC = os.path.join(PKG, "csrc")
BUILD_DIR = os.path.join(ROOT, "_build")
LIB_OUT = os.path.join(PKG, "librailgun_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_SOURCES = ["rg_status.hip", "cache_ops.hip", "decode.hip", "prefill.hip", "model_ops.hip", "gemm.hip", "validate.hip"]
# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 on its own.
HIPCC_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++20", f"-I{ROOT}/include",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall",
]
# Per-source additions.  prefill.hip keeps its MFMA accumulators in ordinary VGPRs: with the
# default heuristic they land in AGPRs and are copied to VGPRs around the softmax rescale
# on every key tile.
SOURCE_FLAGS = {"prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}
CPP_TESTS = ["test_paged_attention_op"]


def _run(cmd: list[str], cwd: str | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{err}\n{proc.stdout}")
    if err.strip():
        print(err, file=sys.stderr)


def build_library() -> str:
    os.makedirs(BUILD_DIR, exist_ok=True)
    objs = [os.path.join(BUILD_DIR, os.path.splitext(s)[0] + ".o") for s in HIP_SOURCES]
    jobs = [[HIPCC, *HIPCC_FLAGS, *SOURCE_FLAGS.get(s, []), "-c", os.path.join(CSRC, s), "-o", o]
            for s, o in zip(HIP_SOURCES, objs)]
    with ThreadPoolExecutor(max_workers=min(4, len(jobs))) as ex:
        for f in [ex.submit(_run, j) for j in jobs]:
            f.result()
    tmp = LIB_OUT + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, LIB_OUT)
    return LIB_OUT


def build_oracle() -> str:
    _run(["make", "-B", "-C", os.path.join(ROOT, "oracle")])
    return os.path.join(ROOT, "oracle", "liboracle.so")


def build_cpp_tests() -> list[str]:
    out = []
    src_dir = os.path.join(ROOT, "tests", "cpp")
    for name in CPP_TESTS:
        src = os.path.join(src_dir, name + ".cpp")
        if not os.path.exists(src):
            continue
        exe = os.path.join(src_dir, name)
        _run([HIPCC, "--offload-arch=gfx950", "-O2", "-std=c++20", f"-I{ROOT}/include", src, "-o", exe,
              f"-L{PKG}", "-lrailgun_hip", f"-Wl,-rpath,{PKG}", "-Wl,-rpath,$ORIGIN/../../railgun_amd"])
        out.append(exe)
    return out


def build_all() -> None:
    if shutil.which(HIPCC) is None and not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    build_library()
    build_oracle()
    build_cpp_tests()


if __name__ == "__main__":
    build_all()
    print("built", LIB_OUT)
