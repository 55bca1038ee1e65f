"""Compile the gfx950 C-ABI library in-tree with hipcc.

``python -m breeze_amd._build`` (or ``build()``) writes
``breeze_amd/libbreeze_qmm.so`` next to this file, atomically, so a process
already using the previous library keeps its inode.
"""
import os
import subprocess
import sys
import tempfile

PKG = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(os.path.dirname(PKG), "csrc")
# Host code and small kernels; the decode and prefill kernels, one unit per
# (bits, activation mode) so the device passes run side by side.
SOURCES = ["qmm.hip"] + [f"{k}_w{b}_{m}.hip" for k in ("dec", "pf") for b in (4, 8) for m in ("hp", "lp")]
LIB_NAME = "libbreeze_qmm.so"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# Flags of both passes.
FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Loadable by both the ROCm 7.2 runtime and the 7.0 runtime bundled with
    # PyTorch (one of the two serves the whole process).
    "-mcode-object-version=5",
    # The arithmetic contract needs IEEE fp32: no contraction, correctly
    # rounded divide, denormals kept.
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Wall",
]

# Device pass only: the host target does not know these.
DEVICE_FLAGS = [
    # No packed-FP32 instructions in any kernel.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the epilogues read every MFMA result
    # with VALU instructions, and the AGPR form adds a copy for each.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    # Leading scalar kernel arguments arrive in SGPRs at wave launch, so a
    # kernel's first loads do not wait for a kernarg fetch.
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
]


def lib_path():
    return os.path.join(PKG, LIB_NAME)


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)


def build(verbose=False):
    """Device code objects and host code in two passes (run side by side),
    so device-only flags never reach the host compiler; then one link.
    Intermediates live in a temporary directory, and every compiler process
    is reaped before it goes, so a failed build leaves nothing behind."""
    out = lib_path()
    tmp = f"{out}.{os.getpid()}.tmp"
    srcs = [os.path.join(CSRC, s) for s in SOURCES]
    running = []

    def finish(procs, what):
        for p, s in procs:
            _, err = p.communicate()
            if p.returncode != 0:
                raise RuntimeError(f"hipcc ({what} of {s}) failed ({p.returncode}):\n{err[-4000:]}")

    with tempfile.TemporaryDirectory(prefix="breeze_qmm_build_") as work:
        fatbins = [os.path.join(work, f"{i}.hipfb") for i in range(len(srcs))]
        objs = [os.path.join(work, f"{i}.o") for i in range(len(srcs))]
        try:
            running = [(_run([HIPCC, "-x", "hip", *FLAGS, *DEVICE_FLAGS, "--offload-device-only", "-c", s, "-o", fb],
                             verbose), s) for s, fb in zip(srcs, fatbins)]
            finish(running, "device pass")
            running = [(_run([HIPCC, "-x", "hip", *FLAGS, "--offload-host-only", "-Xclang",
                              "-fcuda-include-gpubinary", "-Xclang", fb, "-c", s, "-o", o], verbose), s)
                       for s, fb, o in zip(srcs, fatbins, objs)]
            finish(running, "host pass")
            running = [(_run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose), "link")]
            finish(running, "link")
            os.replace(tmp, out)
        finally:
            for p, _ in running:
                if p.poll() is None:
                    p.kill()
                p.communicate()
            if os.path.exists(tmp):
                os.unlink(tmp)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
