"""The build's kernel resource check (CPU only: hipcc cross-compiles for gfx950 here).

The decode attention kernel's LDS reads and DMA ring are untracked inline assembly with
hand-counted `vmcnt` waits, correct only while no register with a load in flight is
spilled, copied or reused. The build therefore fails when a guarded kernel reports scratch, spills or fewer
waves per SIMD than its launch shape assumes; these tests show that a spilling build is
refused and the shipped kernels pass."""

from __future__ import annotations

import importlib.util
import os

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _build_module():
    path = os.path.join(ROOT, "pagedcore_amd", "csrc", "build.py")
    spec = importlib.util.spec_from_file_location("pagedcore_build", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    return module


SPILLING_KERNEL = r"""
#include <hip/hip_runtime.h>
// 160 values stay live across a loop under a 32-VGPR budget: the compiler has to spill.
__global__ __launch_bounds__(256) __attribute__((amdgpu_num_vgpr(32))) void spill_probe_kernel(float* p, int n) {
  float v[160];
#pragma unroll
  for (int i = 0; i < 160; ++i) v[i] = p[i * 256 + threadIdx.x];
  float s = 0.f;
  for (int k = 0; k < n; ++k) {
#pragma unroll
    for (int i = 0; i < 160; ++i) s = fmaf(v[i], v[(i * 7 + k) % 160], s);
  }
  p[threadIdx.x] = s;
}

// 100 live values with no budget cap: no spill, but fewer waves per SIMD.
__global__ __launch_bounds__(64) void wide_probe_kernel(float* p, int n) {
  float v[100];
#pragma unroll
  for (int i = 0; i < 100; ++i) v[i] = p[i * 64 + threadIdx.x];
  float s = 0.f;
  for (int k = 0; k < n; ++k) {
#pragma unroll
    for (int i = 0; i < 100; ++i) s = fmaf(v[i], s, v[99 - i]);
  }
  p[threadIdx.x] = s;
}
"""


@pytest.fixture(scope="module")
def probe_report(tmp_path_factory):
    build = _build_module()
    folder = tmp_path_factory.mktemp("guard")
    source = folder / "probe.hip"
    source.write_text(SPILLING_KERNEL)
    return build, build.compile_library([str(source)], str(folder / "probe.so"))


def test_a_spilling_kernel_fails_the_check(probe_report):
    build, text = probe_report
    fields = build.parse_resource_usage(text)
    spill = next(v for k, v in fields.items() if "spill_probe_kernel" in k)
    assert int(spill["ScratchSize [bytes/lane]"]) > 0 and int(spill["VGPRs Spill"]) > 0
    with pytest.raises(build.ResourceCheckError, match="scratch or spills"):
        build.check_resource_usage(text, {"spill_probe_kernel": 1})


def test_low_occupancy_and_missing_kernels_fail_the_check(probe_report):
    build, text = probe_report
    fields = build.parse_resource_usage(text)
    wide = next(v for k, v in fields.items() if "wide_probe_kernel" in k)
    waves = int(wide["Occupancy [waves/SIMD]"])
    assert int(wide["ScratchSize [bytes/lane]"]) == 0
    build.check_resource_usage(text, {"wide_probe_kernel": waves})
    with pytest.raises(build.ResourceCheckError, match="waves/SIMD its launch shape assumes"):
        build.check_resource_usage(text, {"wide_probe_kernel": waves + 1})
    with pytest.raises(build.ResourceCheckError, match="no resource report"):
        build.check_resource_usage(text, {"renamed_kernel": 1})


def test_the_library_kernels_pass_the_check(tmp_path):
    build = _build_module()
    text = build.compile_library(build.SOURCES, str(tmp_path / "lib.so"))
    summary = build.check_resource_usage(text)
    assert len(summary) >= len(build.GUARDED_KERNELS)
    assert all("scratch 0 B, spills 0/0" in line for line in summary)
