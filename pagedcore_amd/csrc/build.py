"""Compile libpagedcore_hip.so for gfx950 with hipcc (in-tree, next to the package)."""

from __future__ import annotations

import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PACKAGE = os.path.dirname(HERE)
ROOT = os.path.dirname(PACKAGE)
SOURCES = [os.path.join(HERE, name) for name in ("pagedcore_hip.hip", "decode_step.hip", "prefill.hip")]
OUTPUT = os.path.join(PACKAGE, "libpagedcore_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    # Packed fp32 VALU ops are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    # MFMA results stay in VGPRs (no accumulator-register round trip before the VALU
    # uses them).
    "-mllvm",
    "-amdgpu-mfma-vgpr-form",
]


def build(verbose: bool = False) -> str:
    tmp = OUTPUT + ".tmp"
    cmd = [HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), "-o", tmp, *SOURCES]
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops' is not a recognized feature"
    messages = [line for line in (result.stdout + result.stderr).splitlines() if noise not in line]
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + "\n".join(messages))
    if verbose and messages:
        print("\n".join(messages), file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
