"""Build recipe for the MI355X backend: the gfx950 code object and the C-ABI
library, both in-tree beside this file (they travel with the repository
snapshot to the GPU box).

  kernels.hsaco          hipcc --genco of csrc/kernels/kernels.hip (gfx950)
  libcajeta_mi355x.so    the runtime + engine (host C++, links amdhip64)
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
HSACO = os.path.join(HERE, "kernels.hsaco")
LIB = os.path.join(HERE, "libcajeta_mi355x.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# -ffp-contract=off: the arithmetic is written in the order it must round;
# packed-fp32-ops off: packed f32 ops are kept out of the code object;
# amdgpu-mfma-vgpr-form: matrix-core results land in ordinary VGPRs (no
# accumulator-register reads before the f32 steps that consume them).
KERNEL_FLAGS = ["--offload-arch=" + ARCH, "-O3", "--genco", "-ffp-contract=off", "-Wno-pass-failed",
                "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-mllvm", "-amdgpu-mfma-vgpr-form"]
HOST_FLAGS = ["--offload-arch=" + ARCH, "-O2", "-fPIC", "-shared", "-std=c++17", "-Wall", "-Wno-unused-function",
              "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-pthread"]

KERNEL_SOURCES = ["kernels/kernels.hip", "kernels/gemv.hip", "kernels/prim.hip", "kernels/attn.hip", "kernels/gemm.hip", "kernels/rows.hip",
                  "kernels/common.h", "kernels/args.h"]
RUNTIME_SOURCES = ["runtime/runtime.cpp", "runtime/engine.cpp", "runtime/gguf.cpp", "runtime/synth.cpp"]


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        raise RuntimeError("build failed: %s\n%s" % (" ".join(cmd), out))
    if verbose and out.strip():
        print(out)


def build(verbose=False):
    """Compile the code object and the library (always, from source)."""
    _run([HIPCC] + KERNEL_FLAGS + ["-o", HSACO + ".tmp", os.path.join(CSRC, "kernels", "kernels.hip")], verbose)
    os.replace(HSACO + ".tmp", HSACO)
    _run([HIPCC] + HOST_FLAGS + ["-o", LIB + ".tmp"] + [os.path.join(CSRC, s) for s in RUNTIME_SOURCES], verbose)
    os.replace(LIB + ".tmp", LIB)
    return HSACO, LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
    print("built", HSACO, LIB)
