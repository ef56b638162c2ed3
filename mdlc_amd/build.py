"""Build libmdlc_hip.so in-tree with hipcc (gfx950 only).

    python -m mdlc_amd.build

The shared library lands in ``mdlc_amd/_lib/`` so it travels with the source
tree. Kernels themselves are not built here: they are generated per model and
compiled at run time with hipRTC through this library.
"""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_DIR = os.path.join(HERE, "_lib")
LIB_PATH = os.path.join(LIB_DIR, "libmdlc_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

# Flags every HIP compile in this project uses: gfx950 only, no packed-fp32
# instruction selection, no fused multiply-add contraction outside MFMA.
HIP_ARCH = "gfx950"
HIPCC_FLAGS = [
    f"--offload-arch={HIP_ARCH}", "-O3", "-std=c++17", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build_shim(verbose: bool = False) -> str:
    os.makedirs(LIB_DIR, exist_ok=True)
    src = os.path.join(HERE, "csrc", "mdlc_hip.cpp")
    tmp = LIB_PATH + ".tmp"
    cmd = [os.path.join(ROCM, "bin", "hipcc"), *HIPCC_FLAGS, "-fPIC", "-shared",
           f"-I{os.path.join(ROOT, 'include')}", src, "-o", tmp,
           f"-L{os.path.join(ROCM, 'lib')}", "-lhiprtc", "-lamdhip64",
           f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}"]
    if verbose:
        print(" ".join(cmd))
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build_shim(verbose="-v" in sys.argv))
