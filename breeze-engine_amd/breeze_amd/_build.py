"""Compile the gfx950 C-ABI library in-tree with hipcc.

``python -m breeze_amd._build`` (or ``build()``) writes
``breeze_amd/libbreeze_qmm.so`` next to this file, atomically, so a process
already using the previous library keeps its inode.
"""
import os
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(PKG), "csrc")
SOURCES = ["qmm.hip"]
LIB_NAME = "libbreeze_qmm.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # Loadable by both the ROCm 7.2 runtime and the 7.0 runtime bundled with
    # PyTorch (one of the two serves the whole process).
    "-mcode-object-version=5",
    # The arithmetic contract needs IEEE fp32: no contraction, correctly
    # rounded divide, denormals kept.
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    # No packed-FP32 instructions in any kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the epilogues read every MFMA result
    # with VALU instructions, and the AGPR form adds a copy for each.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # Leading scalar kernel arguments arrive in SGPRs at wave launch, so a
    # kernel's first loads do not wait for a kernarg fetch.
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-Wall",
]


def lib_path():
    return os.path.join(PKG, LIB_NAME)


def build(verbose=False):
    out = lib_path()
    tmp = f"{out}.{os.getpid()}.tmp"
    cmd = [HIPCC, *FLAGS, *(os.path.join(CSRC, s) for s in SOURCES), "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    try:
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stderr[-4000:]}")
        os.replace(tmp, out)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
