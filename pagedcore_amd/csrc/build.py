"""Compile libpagedcore_hip.so for gfx950 with hipcc (in-tree, next to the package).

The build also checks the compiler's resource report of the kernels whose correctness
depends on register allocation or occupancy. The prompt attention kernel and the paged
decode attention kernel issue loads and LDS reads as inline assembly that the compiler does
not track, with hand-counted `vmcnt` waits: that is only correct while no register targeted
by an outstanding load is copied, spilled or reused. The decode attention kernel also relies
on two of its workgroups fitting one CU (empty plan rows then run beside the real ones). A
spill (scratch use) or a register budget below the occupancy a kernel was laid out for fails
the build instead of producing a library whose outputs or speed could silently change.
"""

from __future__ import annotations

import os
import re
import subprocess
import sys
from typing import Dict, Iterable, List, Mapping

HERE = os.path.dirname(os.path.abspath(__file__))
PACKAGE = os.path.dirname(HERE)
ROOT = os.path.dirname(PACKAGE)
SOURCES = [os.path.join(HERE, name) for name in ("pagedcore_hip.hip", "decode_step.hip", "prefill.hip", "skinny_gemm.hip")]
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
    # Leading kernel arguments (up to 14 SGPRs) arrive in SGPRs at wave launch instead of
    # through a scalar load of the argument buffer: one memory round trip less before a
    # kernel's first dependent load.
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    # Per-kernel register, scratch and occupancy report, checked below.
    "-Rpass-analysis=kernel-resource-usage",
]

# Kernels checked after every build: (demangled-name fragment) -> minimum waves per SIMD
# the kernel's launch shape relies on. Each must report no scratch and no spills.
GUARDED_KERNELS: Dict[str, int] = {
    "paged_decode_bin_kernel": 2,
    "prefill_attention_kernel": 6,
}

_NOISE = "packed-fp32-ops' is not a recognized feature"
_REMARK = re.compile(r"remark:\s+(?P<key>[A-Za-z][A-Za-z ]*?(?: \[[^\]]+\])?):\s*(?P<value>\S+)\s+\[-Rpass-analysis")


class ResourceCheckError(RuntimeError):
    """A guarded kernel spills, uses scratch, or needs more registers than its layout allows."""


def parse_resource_usage(text: str) -> Dict[str, Dict[str, str]]:
    """{mangled kernel name: {field: value}} from hipcc's kernel-resource-usage remarks."""
    kernels: Dict[str, Dict[str, str]] = {}
    current = None
    for line in text.splitlines():
        match = _REMARK.search(line)
        if not match:
            continue
        key, value = match.group("key").strip(), match.group("value")
        if key == "Function Name":
            current = kernels.setdefault(value, {})
        elif current is not None:
            current[key] = value
    return kernels


def check_resource_usage(text: str, guarded: Mapping[str, int] = GUARDED_KERNELS) -> List[str]:
    """Raise ResourceCheckError if a guarded kernel (matched by name fragment) is missing
    from the report, reports scratch or spills, or reaches fewer waves per SIMD than its
    minimum. Returns one summary line per guarded kernel."""
    kernels = parse_resource_usage(text)
    problems, summary = [], []
    for fragment, min_waves in guarded.items():
        found = [(name, fields) for name, fields in kernels.items() if fragment in name]
        if not found:
            problems.append(f"{fragment}: no resource report (renamed or not compiled?)")
            continue
        for name, fields in found:
            try:
                scratch = int(fields["ScratchSize [bytes/lane]"])
                vspill = int(fields["VGPRs Spill"])
                sspill = int(fields["SGPRs Spill"])
                waves = int(fields["Occupancy [waves/SIMD]"])
                vgprs = int(fields["VGPRs"])
            except (KeyError, ValueError) as error:
                problems.append(f"{fragment}: incomplete resource report ({error})")
                continue
            line = f"{fragment}: {vgprs} VGPRs, {waves} waves/SIMD, scratch {scratch} B, spills {vspill}/{sspill}"
            summary.append(line)
            if scratch or vspill or sspill:
                problems.append(f"{line}: scratch or spills break the untracked-load bookkeeping")
            if waves < min_waves:
                problems.append(f"{line}: below the {min_waves} waves/SIMD its launch shape assumes")
    if problems:
        raise ResourceCheckError("kernel resource check failed:\n  " + "\n  ".join(problems))
    return summary


def compile_library(sources: Iterable[str], output: str, extra: Iterable[str] = ()) -> str:
    """hipcc the sources into `output`; returns the compiler's messages (remarks included)."""
    cmd = [HIPCC, *FLAGS, *extra, "-I", os.path.join(ROOT, "include"), "-o", output, *sources]
    result = subprocess.run(cmd, capture_output=True, text=True)
    text = "\n".join(line for line in (result.stdout + result.stderr).splitlines() if _NOISE not in line)
    if result.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + text)
    return text


def build(verbose: bool = False) -> str:
    tmp = OUTPUT + ".tmp"
    text = compile_library(SOURCES, tmp)
    try:
        summary = check_resource_usage(text)
    except ResourceCheckError:
        os.remove(tmp)
        raise
    if verbose:
        warnings = [line for line in text.splitlines() if "warning:" in line]
        print("\n".join(warnings + summary), file=sys.stderr)
    os.replace(tmp, OUTPUT)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose=True))
